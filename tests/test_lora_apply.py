"""hd_lora_apply (include/hd_lora.h; src/model/lora.c:126-375): adapters are
musubi .safetensors files written here with the safetensors package.
CPU: every validation failure returns before the GPU is touched and names
the problem. GPU (marked): the merge of a mixed-dtype adapter, and of two
adapters on one target, against the oracle's merge."""
import ctypes
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from oracle import oracle as O

TARGETS = {   # checkpoint name -> (out, in)
    "model.language_model.layers.0.self_attn.k_proj.weight": (1024, 4096),
    "model.language_model.layers.1.mlp.down_proj.weight": (4096, 12288),
    "model.x_embedder.proj1.weight": (1024, 3072),
    "model.t_embedder1.mlp.0.weight": (4096, 256),
}


def prefix_of(name):
    return "lora_unet_" + name[:-len(".weight")].replace(".", "_")


def fake_store(pkg, names):
    allocs = (pkg.hd_device_alloc * len(names))()
    for i, nm in enumerate(names):
        allocs[i].dev_ptr = 0x100000 * (i + 1)
        allocs[i].nbytes = 16
        allocs[i].name = nm.encode()
    st = pkg.hd_weight_store()
    st.allocs = ctypes.cast(allocs, ctypes.POINTER(pkg.hd_device_alloc))
    st.n_allocs = len(names)
    st.arena_ptr = 0x100000
    return st, allocs


def apply(pkg, lib, store, specs):
    arr = (pkg.hd_lora_spec * max(1, len(specs)))(*[pkg.hd_lora_spec(p.encode(), m) for p, m in specs])
    cfg = pkg.hd_lora_config(ctypes.cast(arr, ctypes.POINTER(pkg.hd_lora_spec)), len(specs))
    return lib.hd_lora_apply(ctypes.byref(cfg), ctypes.byref(store), 0)


def adapter(path, entries):
    """entries: prefix -> (down, up, alpha or None); tensors any dtype."""
    t = {}
    for pfx, (d, u, a) in entries.items():
        t[pfx + ".lora_down.weight"] = d
        t[pfx + ".lora_up.weight"] = u
        if a is not None:
            t[pfx + ".alpha"] = a
    save_file(t, str(path), metadata={"ss_network_module": "networks.lora"})
    return str(path)


def small(out, inp, r=4, dtype=torch.float32):
    return torch.randn(r, inp).to(dtype), torch.randn(out, r).to(dtype)


def test_lora_apply_validation(pkg, lib, tmp_path):
    name = "model.language_model.layers.0.self_attn.k_proj.weight"
    store, keep = fake_store(pkg, [name])
    d, u = small(1024, 4096)
    good = adapter(tmp_path / "good.safetensors", {prefix_of(name): (d, u, torch.tensor(2.0))})
    assert apply(pkg, lib, store, []) == 0                                   # nothing to do
    assert apply(pkg, lib, store, [(str(tmp_path / "none.safetensors"), 1.0)]) == pkg.HD_ERR_IO
    assert apply(pkg, lib, store, [(good, float("nan"))]) == 2               # HD_ERR_PARSE
    cases = {
        "unknown": ({"lora_unet_model_visual_blocks_0_attn_qkv": (d, u, None)}, pkg.HD_ERR_UNSUPPORTED, b"unknown"),
        "shape": ({prefix_of(name): (torch.randn(4, 4000), u, None)}, 2, b"shape mismatch"),
        "rank": ({prefix_of(name): (d, torch.randn(1024, 3), None)}, 2, b"rank mismatch"),
        "alpha0": ({prefix_of(name): (d, u, torch.tensor(0.0))}, 2, b"invalid alpha"),
        "alpha2": ({prefix_of(name): (d, u, torch.tensor([1.0, 2.0]))}, 2, b"malformed alpha"),
        "notinstore": ({prefix_of("model.x_embedder.proj1.weight"): small(1024, 3072) + (None,)},
                       pkg.HD_ERR_MISSING, b"not found in store"),
        "conv": ({prefix_of(name): (torch.randn(4, 4096, 1, 1), u, None)}, pkg.HD_ERR_UNSUPPORTED, b"non-linear"),
    }
    for tag, (ents, code, msg) in cases.items():
        p = adapter(tmp_path / f"{tag}.safetensors", ents)
        assert apply(pkg, lib, store, [(p, 1.0)]) == code, tag
        assert msg in lib.hd_lora_last_error(), (tag, lib.hd_lora_last_error())
    # a down without its up pair
    save_file({prefix_of(name) + ".lora_down.weight": d}, str(tmp_path / "nopair.safetensors"))
    assert apply(pkg, lib, store, [(str(tmp_path / "nopair.safetensors"), 1.0)]) == 2
    assert b"lora_up" in lib.hd_lora_last_error()
    # no LoRA tensors at all
    save_file({"something": d}, str(tmp_path / "empty.safetensors"))
    assert apply(pkg, lib, store, [(str(tmp_path / "empty.safetensors"), 1.0)]) == pkg.HD_ERR_UNSUPPORTED
    # malformed headers: bad length, not JSON, offsets past the end
    bad = tmp_path / "bad.safetensors"
    for blob in (b"\x01\x02", (100).to_bytes(8, "little") + b"{}", (2).to_bytes(8, "little") + b"[]",
                 (64).to_bytes(8, "little") + b'{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}'.ljust(64)):
        bad.write_bytes(blob)
        assert apply(pkg, lib, store, [(str(bad), 1.0)]) == 2, blob
    # an unusable store
    empty = pkg.hd_weight_store()
    assert apply(pkg, lib, empty, [(good, 1.0)]) == pkg.HD_ERR_MISSING
    # the first failing adapter of several stops the call before any merge
    assert apply(pkg, lib, store, [(good, 1.0), (str(tmp_path / "unknown.safetensors"), 1.0)]) == pkg.HD_ERR_UNSUPPORTED


@pytest.mark.gpu
def test_lora_apply_merges(pkg, lib, dev, tmp_path):
    torch.manual_seed(3)
    base = {n: (torch.randn(o, i) * 0.05).to(torch.bfloat16) for n, (o, i) in TARGETS.items()}
    dtypes = [torch.bfloat16, torch.float16, torch.float32, torch.bfloat16]
    r = [16, 8, 64, 4]
    ents_a, ents_b = {}, {}
    want = {n: base[n].float().numpy() for n in TARGETS}
    for k, (n, (o, i)) in enumerate(TARGETS.items()):
        d = (torch.randn(r[k], i) * 0.1).to(dtypes[k])
        u = (torch.randn(o, r[k]) * 0.1).to(dtypes[k])
        alpha = None if k == 1 else torch.tensor(float(r[k]) / 2).to(dtypes[k])
        ents_a[prefix_of(n)] = (d, u, alpha)
        a = float(r[k]) if alpha is None else float(alpha.float())
        want[n] = O.lora_merge(want[n], u.float().numpy(), d.float().numpy(), 0.8 * a / r[k])
    # a second adapter on the first target only (merged after the first)
    n0 = next(iter(TARGETS))
    d2, u2 = (torch.randn(8, 4096) * 0.1), (torch.randn(1024, 8) * 0.1)
    ents_b[prefix_of(n0)] = (d2, u2, torch.tensor(4.0))
    mid = want[n0]
    want[n0] = O.lora_merge(want[n0], u2.numpy(), d2.numpy(), -0.5 * 4.0 / 8)
    pa = adapter(tmp_path / "a.safetensors", ents_a)
    pb = adapter(tmp_path / "b.safetensors", ents_b)
    devw = {n: t.to(dev) for n, t in base.items()}
    ws = pkg.WeightStore(devw)
    ws.store.arena_ptr = next(iter(devw.values())).data_ptr()
    assert apply(pkg, lib, ws.store, [(pa, 0.8), (pb, -0.5)]) == 0, lib.hd_lora_last_error()
    torch.cuda.synchronize()
    for n in TARGETS:
        got = devw[n].float().cpu().numpy()
        diff = np.abs(got - want[n])
        # one bf16 step per rounding: the twice-merged target carries the
        # first merge's step into the second
        step = np.abs(want[n]) * 2.0 ** -7 + 1e-6
        if n == n0:
            step = step * 2 + np.abs(mid) * 2.0 ** -7
        assert np.all(diff <= step), (n, float((diff - step).max()))
        assert np.mean(got == want[n]) > 0.98, (n, float(np.mean(got == want[n])))
    # untouched weights stay bit-identical on a failing call
    snap = {n: t.clone() for n, t in devw.items()}
    bad = adapter(tmp_path / "bad.safetensors", {prefix_of(n0): (d2, u2, torch.tensor(0.0))})
    assert apply(pkg, lib, ws.store, [(pa, 1.0), (bad, 1.0)]) == 2
    for n in TARGETS:
        assert torch.equal(snap[n], devw[n])

"""Vision tower (CPU): the oracle's restatement of the reference's
src/model/vision.c pinned against transformers' Qwen3VLVisionModel
(tests/golden/vision_tiny.npz, written by make_vision_golden.py), its
tables against transformers' own index helpers, its LayerNorm / GELU against
torch, and weight-name resolution of the library against a synthetic store.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden", "vision_tiny.npz")


def _golden():
    d = np.load(GOLD)
    w = {k[2:]: d[k] for k in d.files if k.startswith("w.")}
    return d, w


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_vision_forward_matches_transformers():
    d, w = _golden()
    gh, gw = (int(x) for x in d["grid"])
    emb, ds = O.vision_forward(w, d["pixels"], gh, gw, depth=3, heads=2, ds_layers=[0, 2],
                               faithful=0)
    assert _rel(emb, d["embeds"]) < 1e-5
    assert _rel(ds[0], d["deepstack0"]) < 1e-5
    assert _rel(ds[1], d["deepstack1"]) < 1e-5


def test_vision_forward_pins_each_stage():
    """A dropped or mis-ordered stage moves the output well past the bound:
    swapping the deepstack layers, the rotary coordinates (a transposed
    grid) or the merger norm all fail the comparison above."""
    d, w = _golden()
    gh, gw = (int(x) for x in d["grid"])
    emb, ds = O.vision_forward(w, d["pixels"], gh, gw, depth=3, heads=2, ds_layers=[1, 2],
                               faithful=0)
    assert _rel(ds[0], d["deepstack0"]) > 1e-2
    # grid transposed: same token count, different positions
    emb_t, _ = O.vision_forward(w, d["pixels"], gw, gh, depth=3, heads=2, ds_layers=[0, 2],
                                faithful=0)
    assert _rel(emb_t, d["embeds"]) > 1e-2
    w2 = dict(w)
    w2["merger.norm.bias"] = w["merger.norm.bias"] * 0
    emb_b, _ = O.vision_forward(w2, d["pixels"], gh, gw, depth=3, heads=2, ds_layers=[0, 2],
                                faithful=0)
    assert _rel(emb_b, d["embeds"]) > 1e-2


def test_vision_faithful_rounding_is_small():
    """faithful=1 rounds to bf16 where the reference holds bf16 (and takes
    bf16 rotary angles); on O(1) weights it stays within bf16 noise of fp32."""
    d, w = _golden()
    gh, gw = (int(x) for x in d["grid"])
    emb, _ = O.vision_forward(w, d["pixels"], gh, gw, depth=3, heads=2, ds_layers=[0, 2],
                              faithful=1)
    r = _rel(emb, d["embeds"])
    assert 1e-4 < r < 5e-2
    assert np.array_equal(emb, O.bf16_round(emb))


@pytest.mark.parametrize("grid", [(4, 6), (2, 2), (8, 4), (6, 10)])
def test_vision_tables_match_transformers(grid):
    vu = pytest.importorskip("transformers.vision_utils")
    gh, gw = grid
    idx, wgt, co = O.vision_tables(gh, gw, 48, 2)
    thw = torch.tensor([[1, gh, gw]])
    ti, tw = vu.get_vision_interpolation_indices_and_weights(thw, num_grid_per_side=48,
                                                             mode="bilinear", align_corners=True,
                                                             spatial_merge_size=2)
    pos = vu.get_vision_position_ids(thw, 2)
    assert np.array_equal(co.T, pos.numpy())
    # the same four taps with the same weights (corner order may differ when
    # a weight is zero: compare the weighted tap sets)
    for r in range(gh * gw):
        mine = {}
        for t in range(4):
            mine[int(idx[t, r])] = mine.get(int(idx[t, r]), 0.0) + float(wgt[t, r])
        theirs = {}
        for t in range(ti.shape[1]):
            theirs[int(ti[r, t])] = theirs.get(int(ti[r, t]), 0.0) + float(tw[r, t])
        keys = {k for k, v in mine.items() if v > 1e-6} | {k for k, v in theirs.items() if v > 1e-6}
        for k in keys:
            assert abs(mine.get(k, 0.0) - theirs.get(k, 0.0)) < 1e-5, (grid, r, k)


def test_vision_rotary_closed_form():
    # angle(row r, freq j) = r * 10000^(-2j/36); the column half uses the col
    co = np.array([[0, 3, 5], [0, 7, 2]], np.int32)
    cs = np.empty((3, 72), np.float32)
    sn = np.empty((3, 72), np.float32)
    IP = ctypes.POINTER(ctypes.c_int)
    O.lib().o1o_vision_rotary(co.ctypes.data_as(IP), 3, 72, 0, O.fp(cs), O.fp(sn))
    inv = 1.0 / 10000 ** (np.arange(18) * 2 / 36)
    ang = np.concatenate([co[0][:, None] * inv, co[1][:, None] * inv], 1)
    ang = np.concatenate([ang, ang], 1)
    assert np.allclose(cs, np.cos(ang), atol=2e-6) and np.allclose(sn, np.sin(ang), atol=2e-6)


def test_layernorm_and_gelu_vs_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((7, 1152)) * 2 + 0.5).astype(np.float32)
    w = rng.standard_normal(1152).astype(np.float32)
    b = rng.standard_normal(1152).astype(np.float32)
    want = torch.nn.functional.layer_norm(torch.tensor(x), (1152,), torch.tensor(w), torch.tensor(b),
                                          eps=1e-6).numpy()
    got = O.layernorm(x, w, b, round_=0)
    assert np.abs(got - want).max() < 2e-4
    assert np.array_equal(O.layernorm(x, w, b, round_=1), O.bf16_round(got))
    v = np.linspace(-6, 6, 4001).astype(np.float32)
    assert np.abs(O.gelu_tanh(v, 0) - torch.nn.functional.gelu(torch.tensor(v), approximate="tanh").numpy()).max() < 2e-6
    assert np.abs(O.gelu_erf(v, 0) - torch.nn.functional.gelu(torch.tensor(v)).numpy()).max() < 2e-6


def test_vision_resolve_by_name(pkg, lib):
    """hd_vision_resolve finds every tower tensor under the checkpoint names
    (vision.c:43-130) in a host-side store and fails closed on a gap."""
    names = ["model.visual.patch_embed.proj.weight", "model.visual.patch_embed.proj.bias",
             "model.visual.pos_embed.weight"]
    for i in range(27):
        names += [f"model.visual.blocks.{i}.{k}" for k in O.VISION_BLOCK_KEYS]
    names += [f"model.visual.merger.{k}" for k in O.VISION_MERGER_KEYS]
    for j in range(3):
        names += [f"model.visual.deepstack_merger_list.{j}.{k}" for k in O.VISION_MERGER_KEYS]
    allocs = (pkg.hd_device_alloc * len(names))()
    for i, nm in enumerate(names):
        allocs[i].dev_ptr = 0x10000 + 16 * i
        allocs[i].nbytes = 16
        allocs[i].name = nm.encode()
    store = pkg.hd_weight_store()
    store.allocs = ctypes.cast(allocs, ctypes.POINTER(pkg.hd_device_alloc))
    store.n_allocs = len(names)
    vb = pkg.hd_vision_binding()
    assert lib.hd_vision_resolve(ctypes.byref(store), ctypes.byref(vb)) == 0
    assert vb.patch_proj_w == 0x10000 and vb.pos_embed == 0x10000 + 32
    assert vb.blocks[0].norm1_w == 0x10000 + 16 * 3
    assert vb.blocks[26].fc2_b == 0x10000 + 16 * (3 + 27 * 12 - 1)
    assert vb.deepstack[2].fc2_b == 0x10000 + 16 * (len(names) - 1)
    allocs[100].name = b"model.visual.something_else"
    assert lib.hd_vision_resolve(ctypes.byref(store), ctypes.byref(vb)) == pkg.HD_ERR_MISSING
    assert b"missing" in lib.hd_last_error()


def test_vision_sizes_and_fail_closed(pkg, lib):
    assert lib.hd_vision_tables_bytes(64) == 64 * 40 + 72
    ws_b = lib.hd_vision_workspace_bytes(1024)
    o = pkg.hd_vision_offsets()
    lib.hd_vision_layout(1024, 256, ctypes.byref(o))
    assert o.total_bytes == ws_b and o.h_a > o.patch_out and o.fc1 + 1024 * 4352 * 2 <= ws_b
    vb = pkg.hd_vision_binding()
    ws = pkg.hd_vision_workspace()
    fake = ctypes.c_void_p(0x1000)
    # no workspace base, odd grid, tables not prepared
    assert lib.hd_vision_forward(ctypes.byref(vb), ctypes.byref(ws), fake, 64, 8, 8, fake, None) == pkg.HD_ERR_MISSING
    ws.patch_out = 0x1000
    assert lib.hd_vision_forward(ctypes.byref(vb), ctypes.byref(ws), fake, 63, 7, 9, fake, None) == pkg.HD_ERR_MISSING
    assert lib.hd_vision_forward(ctypes.byref(vb), ctypes.byref(ws), fake, 64, 8, 8, fake, None) == pkg.HD_ERR_MISSING
    assert b"tables" in lib.hd_last_error()
    assert lib.hd_vision_prepare_tables(ctypes.byref(ws), 64, 8, 8) == pkg.HD_ERR_MISSING

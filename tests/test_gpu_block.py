"""Decoder-block parity: hd_decoder_block / hd_decoder_block_batched on the
GPU vs the fp32 CPU oracle of block.c:137-386 (bound rel-L2 <= 1e-2, cosine
>= 0.9999) and vs the oracle's bf16-faithful mode (tighter)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.common import make_block_weights, to_dev, rel_l2, cosine, grid_pos, bf16

pytestmark = pytest.mark.gpu

REL, COS = 1e-2, 0.9999     # north-star bound per block


def run_block(pkg, lib, dev, w, x, pos, H, KV, HID, FF, D, theta, plan=None, internals=False,
              in_place=False):
    pkg.set_block_config(theta=theta)
    S = x.shape[0]
    wd = {k: to_dev(v, dev) for k, v in w.items()}
    bind = pkg.binding_from(wd)
    xd = x.to(dev, torch.bfloat16)
    out = xd if in_place else torch.empty_like(xd)
    posd = torch.from_numpy(pos).to(dev)
    nbytes = lib.hd_decoder_block_scratch_bytes(S, H, KV, HID, FF, D)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    ints = None
    bufs = []
    if internals:
        bufs = [torch.empty_like(xd) for _ in range(3)]
        ints = pkg.hd_block_internals()
        ints.ln0, ints.attn_resid, ints.post_ln = [b.data_ptr() for b in bufs]
    st = lib.hd_decoder_block(pkg.ptr(xd), pkg.ptr(posd), None, bind, None, pkg.ptr(scratch), nbytes,
                              ctypes.byref(ints) if ints else None, pkg.ptr(out), S, H, KV, HID,
                              FF, D, plan.h if plan else None)
    pkg.check_status(st, "hd_decoder_block")
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), [b.float().cpu().numpy() for b in bufs]


def oracle_block(w, x, pos, H, KV, HID, FF, D, theta, faithful, ar_len=0, batch=1, internals=False):
    cfg = orc.block_cfg(H, KV, HID, FF, D, theta=theta, faithful=faithful, ar_len=ar_len)
    return orc.decoder_block(x, pos, {k: v.numpy() for k, v in w.items()}, cfg, batch=batch,
                             internals=internals)


def check(got, ref, x, tag, rel=REL, cos=COS, delta=None):
    """rel-L2 / cosine of the block output; with `delta`, also of the
    residual update (out - x) alone, so the check does not ride on x. The
    update carries the output's bf16 rounding (2^-9 of |out|), so it is only
    meaningful against the bf16-faithful oracle, which rounds there too."""
    r, c = rel_l2(got, ref), cosine(got, ref)
    rd = rel_l2(got - x, ref - x)
    print(f"{tag}: rel_l2={r:.3e} cos={c:.7f} delta_rel_l2={rd:.3e}")
    assert r <= rel and c >= cos, (tag, r, c)
    if delta is not None:
        assert rd <= delta, (tag, rd)


def test_block_small_vs_oracle(pkg, lib, dev):
    H, KV, HID, FF, D = 4, 2, 512, 1024, 128
    T, gh, gw = 32, 8, 16
    S = T + gh * gw
    w = make_block_weights(HID, H, KV, FF, D, seed=0)
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(1)))
    pos = grid_pos(T, gh, gw)
    got, ints = run_block(pkg, lib, dev, w, x, pos, H, KV, HID, FF, D, 1e4, internals=True)
    xn = x.numpy()
    ref32 = oracle_block(w, xn, pos, H, KV, HID, FF, D, 1e4, faithful=0)
    check(got, ref32, xn, "small vs fp32")
    reff, ln0, ar, post = oracle_block(w, xn, pos, H, KV, HID, FF, D, 1e4, faithful=1,
                                       internals=True)
    check(got, reff, xn, "small vs bf16-faithful", rel=5e-3, cos=0.99995, delta=3e-2)
    assert np.array_equal(ints[0], ln0) or rel_l2(ints[0], ln0) < 1e-3   # input_layernorm
    assert rel_l2(ints[1], ar) < 5e-3 and rel_l2(ints[2], post) < 5e-3


def test_block_in_place_and_batched(pkg, lib, dev):
    H, KV, HID, FF, D = 4, 2, 512, 1024, 128
    T, gh, gw = 16, 8, 8
    S = T + gh * gw
    B = 2
    w = make_block_weights(HID, H, KV, FF, D, seed=2)
    x = bf16(torch.randn(B * S, HID, generator=torch.Generator().manual_seed(3)))
    pos = grid_pos(T, gh, gw)
    # in place, batch 1
    got0, _ = run_block(pkg, lib, dev, w, x[:S], pos, H, KV, HID, FF, D, 1e4, in_place=True)
    ref0 = oracle_block(w, x[:S].numpy(), pos, H, KV, HID, FF, D, 1e4, faithful=0)
    check(got0, ref0, x[:S].numpy(), "in-place")
    # batched entry: both sequences in one launch chain
    pkg.set_block_config(theta=1e4)
    wd = {k: to_dev(v, dev) for k, v in w.items()}
    bind = pkg.binding_from(wd)
    xd = x.to(dev, torch.bfloat16)
    out = torch.empty_like(xd)
    posd = torch.from_numpy(pos).to(dev)
    cs = pkg.rope_table(posd, S, D, theta=1e4)
    nbytes = lib.hd_decoder_block_batched_scratch_bytes(B, S, H, KV, HID, FF, D)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    st = lib.hd_decoder_block_batched(pkg.ptr(xd), pkg.ptr(cs), None, 0, bind, pkg.ptr(scratch),
                                      nbytes, None, pkg.ptr(out), B, S, H, KV, HID, FF, D)
    pkg.check_status(st, "batched")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = oracle_block(w, x.numpy(), pos, H, KV, HID, FF, D, 1e4, faithful=0, batch=B)
    check(got, ref, x.numpy(), "batched B=2")
    # sequence 0 of the batch == the single-sequence result (same kernels)
    assert rel_l2(got[:S], got0) < 2e-3


def test_block_split_plan_causal_prefix(pkg, lib, dev):
    H, KV, HID, FF, D = 4, 2, 512, 1024, 128
    T, gh, gw = 40, 8, 12
    S = T + gh * gw
    ar = T - 1
    w = make_block_weights(HID, H, KV, FF, D, seed=4)
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(5)))
    pos = grid_pos(T, gh, gw)
    pos[:, :T] = np.arange(T)[None, :]          # text rows at i on all axes (sequence.c:104-118)
    plan = pkg.SdpaPlan(1, H, KV, S, D, ar_len=ar)
    got, _ = run_block(pkg, lib, dev, w, x, pos, H, KV, HID, FF, D, 5e6, plan=plan)
    ref = oracle_block(w, x.numpy(), pos, H, KV, HID, FF, D, 5e6, faithful=0, ar_len=ar)
    check(got, ref, x.numpy(), "split plan")


def test_block_config0_full_size(pkg, lib, dev):
    """Benchmark configuration 0: 1024 image tokens (32x32) + 128 text, hidden 4096,
    32x128 heads (8 kv), FFN 12288, 2D RoPE theta 1e4, text at position 0."""
    H, KV, HID, FF, D = 32, 8, 4096, 12288, 128
    T, gh, gw = 128, 32, 32
    S = T + gh * gw
    w = make_block_weights(HID, H, KV, FF, D, seed=0)
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(1)))
    pos = grid_pos(T, gh, gw)
    got, _ = run_block(pkg, lib, dev, w, x, pos, H, KV, HID, FF, D, 1e4)
    ref = oracle_block(w, x.numpy(), pos, H, KV, HID, FF, D, 1e4, faithful=0)
    check(got, ref, x.numpy(), "config0 vs fp32")
    reff = oracle_block(w, x.numpy(), pos, H, KV, HID, FF, D, 1e4, faithful=1)
    check(got, reff, x.numpy(), "config0 vs bf16-faithful", rel=5e-3, cos=0.99995, delta=3e-2)


def test_block_config1_full_size(pkg, lib, dev):
    """Benchmark configuration 1's block at its real shape: batch 2 (CFG) x
    (64x64 image tokens + 256 text) = 2 x 4352 rows through
    hd_decoder_block_batched, i.e. the production kernels with every tail
    split active (QKV 816 tiles, o_proj / down 544 tiles, attention 1088
    256-query units over 256 slots), against the fp32 oracle of both
    sequences and the bf16-faithful oracle."""
    H, KV, HID, FF, D = 32, 8, 4096, 12288, 128
    T, gh, gw, B = 256, 64, 64, 2
    S = T + gh * gw
    w = make_block_weights(HID, H, KV, FF, D, seed=10)
    x = bf16(torch.randn(B * S, HID, generator=torch.Generator().manual_seed(11)))
    pos = grid_pos(T, gh, gw)
    pkg.set_block_config(theta=1e4)
    wd = {k: to_dev(v, dev) for k, v in w.items()}
    bind = pkg.binding_from(wd)
    xd = x.to(dev, torch.bfloat16)
    out = torch.empty_like(xd)
    posd = torch.from_numpy(pos).to(dev)
    cs = pkg.rope_table(posd, S, D, theta=1e4)
    nbytes = lib.hd_decoder_block_batched_scratch_bytes(B, S, H, KV, HID, FF, D)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    print(f"config1 block B={B} S={S}", flush=True)
    st = lib.hd_decoder_block_batched(pkg.ptr(xd), pkg.ptr(cs), None, 0, bind, pkg.ptr(scratch),
                                      nbytes, None, pkg.ptr(out), B, S, H, KV, HID, FF, D)
    pkg.check_status(st, "batched config1")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    del wd, bind, xd, out, scratch
    ref = oracle_block(w, x.numpy(), pos, H, KV, HID, FF, D, 1e4, faithful=0, batch=B)
    check(got, ref, x.numpy(), "config1 vs fp32")
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        check(got[rows], ref[rows], x.numpy()[rows], f"config1 seq {b} vs fp32")
    reff = oracle_block(w, x.numpy(), pos, H, KV, HID, FF, D, 1e4, faithful=1, batch=B)
    check(got, reff, x.numpy(), "config1 vs bf16-faithful", rel=5e-3, cos=0.99995, delta=3e-2)


def test_block_reads_device_section(pkg, lib, dev):
    """sec_dev (int64[3] on the device, block.c:233-236) selects the MRoPE
    section: a non-default section through sec_dev equals the same section
    set through the block config bit for bit, and the oracle with that
    section within the bound."""
    H, KV, HID, FF, D = 4, 2, 512, 1024, 128
    T, gh, gw = 16, 8, 12
    S = T + gh * gw
    sec = (16, 24, 24)
    w = make_block_weights(HID, H, KV, FF, D, seed=21)
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(22)))
    pos = grid_pos(T, gh, gw)
    pos[0, T:] = 2000.0                 # a T axis far from H: the section rule matters
    pkg.set_block_config(theta=1e4)
    wd = {k: to_dev(v, dev) for k, v in w.items()}
    bind = pkg.binding_from(wd)
    xd = x.to(dev, torch.bfloat16)
    posd = torch.from_numpy(pos).to(dev)
    secd = torch.tensor(sec, dtype=torch.int64, device=dev)
    nbytes = lib.hd_decoder_block_scratch_bytes(S, H, KV, HID, FF, D)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    outs = []
    for use_dev in (True, False):
        if not use_dev:
            pkg.set_block_config(theta=1e4, section=sec)
        out = torch.empty_like(xd)
        st = lib.hd_decoder_block(pkg.ptr(xd), pkg.ptr(posd), None, bind, pkg.ptr(secd) if use_dev else None,
                                  pkg.ptr(scratch), nbytes, None, pkg.ptr(out), S, H, KV, HID, FF, D, None)
        pkg.check_status(st, "hd_decoder_block sec_dev")
        torch.cuda.synchronize()
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])
    cfg = orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=0, section=sec)
    ref = orc.decoder_block(x.numpy(), pos, {k: v.numpy() for k, v in w.items()}, cfg)
    check(outs[0].float().cpu().numpy(), ref, x.numpy(), "sec_dev block vs fp32")
    cfg_def = orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=0)
    ref_def = orc.decoder_block(x.numpy(), pos, {k: v.numpy() for k, v in w.items()}, cfg_def)
    xn = x.numpy()
    assert rel_l2(ref - xn, ref_def - xn) > 1e-2    # the section changes the block's update

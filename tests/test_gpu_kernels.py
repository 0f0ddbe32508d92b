"""Bandwidth kernels and attention through the C-ABI vs the CPU oracle."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.common import rel_l2, cosine, ulp_diff_bf16, close_bf16, grid_pos, bf16

pytestmark = pytest.mark.gpu


def dbf(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev, torch.bfloat16)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("rows,cols", [(37, 4096), (300, 128), (5, 200), (4, 8), (1031, 4096),
                                       (1030, 1000)])
def test_rmsnorm(pkg, lib, dev, rows, cols):
    rng = np.random.default_rng(rows)
    x = orc.bf16_round(rng.standard_normal((rows, cols)) * 3)
    w = orc.bf16_round(1 + rng.standard_normal(cols) * 0.1)
    y = torch.empty(rows, cols, dtype=torch.bfloat16, device=dev)
    xd, wd = dbf(x, dev), dbf(w, dev)
    lib.hd_rmsnorm(pkg.ptr(xd), pkg.ptr(wd), pkg.ptr(y), rows, cols, 1e-6)
    pkg.check_prim("rmsnorm")
    ref = orc.rmsnorm(x, w, 1e-6, 1)
    assert close_bf16(host(y), ref, ulps=1, atol_rel=0)
    if rows >= 1024:
        # two-rows-per-wave kernel against the one-row kernel (40-row call)
        y40 = torch.empty(40, cols, dtype=torch.bfloat16, device=dev)
        lib.hd_rmsnorm(pkg.ptr(xd), pkg.ptr(wd), pkg.ptr(y40), 40, cols, 1e-6)
        assert torch.equal(y[:40], y40)
        lib.hd_rmsnorm(pkg.ptr(xd[-40:]), pkg.ptr(wd), pkg.ptr(y40), 40, cols, 1e-6)
        assert torch.equal(y[-40:], y40)


@pytest.mark.parametrize("rows", [64, 1033])
def test_add_rmsnorm(pkg, lib, dev, rows):
    rng = np.random.default_rng(1)
    x = orc.bf16_round(rng.standard_normal((rows, 4096)))
    a = orc.bf16_round(rng.standard_normal((rows, 4096)))
    w = orc.bf16_round(1 + rng.standard_normal(4096) * 0.1)
    s = torch.empty(rows, 4096, dtype=torch.bfloat16, device=dev)
    y = torch.empty_like(s)
    xd, ad, wd = dbf(x, dev), dbf(a, dev), dbf(w, dev)
    lib.hd_add_rmsnorm(pkg.ptr(xd), pkg.ptr(ad), pkg.ptr(wd), pkg.ptr(s), pkg.ptr(y), rows, 4096, 1e-6)
    pkg.check_prim("add_rmsnorm")
    sref = orc.residual_add(x, a, 1)
    assert np.array_equal(host(s), sref)
    assert close_bf16(host(y), orc.rmsnorm(sref, w, 1e-6, 1), ulps=1, atol_rel=0)


@pytest.mark.parametrize("n", [16, 1000, 4096 * 3 + 5])
def test_pointwise(pkg, lib, dev, n):
    rng = np.random.default_rng(n)
    g = orc.bf16_round(rng.standard_normal(n) * 3)
    u = orc.bf16_round(rng.standard_normal(n))
    y = torch.empty(n, dtype=torch.bfloat16, device=dev)
    gd, ud = dbf(g, dev), dbf(u, dev)
    lib.hd_swiglu(pkg.ptr(gd), pkg.ptr(ud), pkg.ptr(y), n)
    pkg.check_prim("swiglu")
    assert close_bf16(host(y), orc.swiglu(g, u, 1), ulps=1, atol_rel=0)
    lib.hd_residual_add(pkg.ptr(gd), pkg.ptr(ud), pkg.ptr(y), n)
    assert np.array_equal(host(y), orc.residual_add(g, u, 1))
    lib.hd_silu(pkg.ptr(gd), pkg.ptr(y), n)
    assert close_bf16(host(y), orc.silu(g, 1), ulps=1, atol_rel=0)


def test_mrope_and_rotary(pkg, lib, dev):
    # test_primitives.c:329-388 (seq 4, dim 64, section {6,2,2}, theta 5e6)
    seq, dim = 4, 64
    pos = np.zeros((3, seq), np.float32)
    for i in range(seq):
        pos[:, i] = [10.0 * (i + 1), 100.0 * (i + 1) + 1, 1000.0 * (i + 1) + 2]
    sec = (6, 2, 2)
    c = torch.empty(seq, dim, device=dev)
    s = torch.empty(seq, dim, device=dev)
    secd = torch.tensor(sec, dtype=torch.int64, device=dev)
    posd = torch.from_numpy(pos).to(dev)
    lib.hd_mrope_cos_sin(pkg.ptr(posd), 1, seq, pkg.ptr(secd), 3, dim, 5e6, 1.0, 1, pkg.ptr(c),
                         pkg.ptr(s))
    pkg.check_prim("mrope")
    cr, sr = orc.mrope_cos_sin(pos, seq, dim, 5e6, sec)
    assert rel_l2(c.cpu().numpy(), cr) < 2e-5 and rel_l2(s.cpu().numpy(), sr) < 2e-4
    # rotation with bf16 per-op rounding
    rng = np.random.default_rng(2)
    x = orc.bf16_round(rng.standard_normal((3, seq, dim)))
    y = torch.empty(3, seq, dim, dtype=torch.bfloat16, device=dev)
    xd, cd, sd = dbf(x, dev), torch.from_numpy(cr).to(dev), torch.from_numpy(sr).to(dev)
    lib.hd_apply_rotary(pkg.ptr(xd), pkg.ptr(cd), pkg.ptr(sd), pkg.ptr(y), 3, seq, dim)
    assert np.array_equal(host(y), orc.apply_rotary(x, cr, sr, 1))


@pytest.mark.parametrize("B,S", [(1, 200), (2, 256)])
def test_qkv_epilogue(pkg, lib, dev, B, S):
    H, KV, D = 4, 2, 128
    rng = np.random.default_rng(S)
    qkv = orc.bf16_round(rng.standard_normal((B * S, (H + 2 * KV) * D)) * 2)
    qn = orc.bf16_round(1 + rng.standard_normal(D) * 0.1)
    kn = orc.bf16_round(1 + rng.standard_normal(D) * 0.1)
    pos = grid_pos(S - 10 * 19, 10, 19)
    posd = torch.from_numpy(pos).to(dev)
    cs = pkg.rope_table(posd, S, D, theta=1e4)
    q = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=dev)
    k = torch.empty(B, KV, S, D, dtype=torch.bfloat16, device=dev)
    v = torch.empty(B, KV, S, D, dtype=torch.bfloat16, device=dev)
    qd, qnd, knd = dbf(qkv, dev), dbf(qn, dev), dbf(kn, dev)
    lib.hd_qkv_epilogue(pkg.ptr(qd), pkg.ptr(qnd), pkg.ptr(knd), pkg.ptr(cs),
                        pkg.ptr(q), pkg.ptr(k), pkg.ptr(v), None, B, S, H, KV, D, 1e-6)
    pkg.check_prim("qkv_epilogue")
    cr, sr = orc.mrope_cos_sin(pos, S, D, 1e4)
    for b in range(B):
        rows = qkv[b * S:(b + 1) * S]
        qh = rows[:, :H * D].reshape(S, H, D).transpose(1, 0, 2)
        kh = rows[:, H * D:(H + KV) * D].reshape(S, KV, D).transpose(1, 0, 2)
        vh = rows[:, (H + KV) * D:].reshape(S, KV, D).transpose(1, 0, 2)
        qr = orc.apply_rotary(orc.rmsnorm(qh, qn, 1e-6, 1), cr, sr, 1)
        kr = orc.apply_rotary(orc.rmsnorm(kh, kn, 1e-6, 1), cr, sr, 1)
        # norm sums in another order: rare 1-ulp differences that the
        # per-op rounded rotation can carry to 2 ulps of the larger term
        assert close_bf16(host(q[b]), qr, ulps=2, atol_rel=2e-3)
        assert close_bf16(host(k[b]), kr, ulps=2, atol_rel=2e-3)
        assert np.mean(host(q[b]) == qr) > 0.98
        assert np.array_equal(host(v[b]), vh)
    # V^T layout: same values, transposed, key bits 2/3 exchanged, zero pad
    spad = (S + 63) // 64 * 64
    vt = torch.full((B, KV, D, spad), 7.0, dtype=torch.bfloat16, device=dev)
    lib.hd_qkv_epilogue(pkg.ptr(qd), pkg.ptr(qnd), pkg.ptr(knd), pkg.ptr(cs),
                        pkg.ptr(q), pkg.ptr(k), None, pkg.ptr(vt), B, S, H, KV, D, 1e-6)
    pkg.check_prim("qkv_epilogue vt")
    perm = np.arange(spad)
    perm = (perm & ~12) | ((perm & 4) << 1) | ((perm & 8) >> 1)
    vt_h = host(vt)
    for b in range(B):
        vh = qkv[b * S:(b + 1) * S, (H + KV) * D:].reshape(S, KV, D).transpose(1, 2, 0)
        full = np.zeros((KV, D, spad), np.float32)
        full[:, :, :S] = vh
        assert np.array_equal(vt_h[b], full[:, :, perm])


def _attn_inputs(Hq, Hkv, S, D, seed):
    rng = np.random.default_rng(seed)
    q = orc.bf16_round(rng.standard_normal((Hq, S, D)))
    k = orc.bf16_round(rng.standard_normal((Hkv, S, D)))
    v = orc.bf16_round(rng.standard_normal((Hkv, S, D)))
    return q, k, v


@pytest.mark.parametrize("Hq,Hkv,S,ar", [(8, 2, 256, 0), (4, 4, 200, 0), (4, 1, 333, 50),
                                         (32, 8, 1152, 0)])
def test_flash_vs_oracle(pkg, lib, dev, Hq, Hkv, S, ar):
    D = 128
    q, k, v = _attn_inputs(Hq, Hkv, S, D, S + Hq)
    plan = pkg.SdpaPlan(1, Hq, Hkv, S, D, ar_len=ar)
    out = torch.empty(Hq, S, D, dtype=torch.bfloat16, device=dev)
    qd, kd, vd = dbf(q, dev), dbf(k, dev), dbf(v, dev)
    rc = lib.hd_sdpa_execute(plan.h, pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), None, pkg.ptr(out), None)
    assert rc == 0, lib.hd_cuda_last_error()
    ref = orc.attention(q, k, v, None, ar, round_=0)            # [S, Hq*D] fp32
    got = host(out).transpose(1, 0, 2).reshape(S, Hq * D)
    assert rel_l2(got, ref) < 8e-3 and cosine(got, ref) > 0.99995


def test_flash_dense_mask_and_invariants(pkg, lib, dev):
    Hq, Hkv, S, D = 2, 1, 96, 128
    q, k, v = _attn_inputs(Hq, Hkv, S, D, 11)
    rng = np.random.default_rng(3)
    mask = np.where(rng.random((S, S)) < 0.3, -3.3895e38, 0.0).astype(np.float32)
    np.fill_diagonal(mask, 0.0)
    mb = dbf(mask, dev)
    plan = pkg.SdpaPlan(1, Hq, Hkv, S, D)
    out = torch.empty(Hq, S, D, dtype=torch.bfloat16, device=dev)
    qd, kd, vd = dbf(q, dev), dbf(k, dev), dbf(v, dev)
    rc = lib.hd_sdpa_execute(plan.h, pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), pkg.ptr(mb), pkg.ptr(out),
                             None)
    assert rc == 0
    ref = orc.attention(q, k, v, host(mb), 0, round_=0)
    got = host(out).transpose(1, 0, 2).reshape(S, Hq * D)
    assert rel_l2(got, ref) < 8e-3
    # invariant: q = 0 -> uniform probabilities -> every row is mean(V)
    z = torch.zeros(Hq, S, D, dtype=torch.bfloat16, device=dev)
    rc = lib.hd_sdpa_execute(plan.h, pkg.ptr(z), pkg.ptr(kd), pkg.ptr(vd), None, pkg.ptr(out), None)
    assert rc == 0
    mean_v = v[0].mean(axis=0)
    assert np.abs(host(out)[0] - mean_v[None, :]).max() < 2e-2


def test_eager_matches_oracle(pkg, lib, dev):
    # test_primitives.c:441-535 shape class, fp32 softmax, bf16 probs
    Hq, Hkv, S, D = 2, 1, 3, 4
    q = orc.bf16_round(np.array([(i % 13) * 0.11 for i in range(Hq * S * D)]).reshape(Hq, S, D))
    k = orc.bf16_round(np.array([(i % 7) * 0.13 for i in range(Hkv * S * D)]).reshape(Hkv, S, D))
    v = orc.bf16_round(np.array([(i % 5) * 0.17 for i in range(Hkv * S * D)]).reshape(Hkv, S, D))
    mask = orc.bf16_round(np.array([0.0 if i % 3 == 0 else -3.3895e38 for i in range(S * S)]).reshape(S, S))
    sc = torch.empty(Hq, S, S, dtype=torch.bfloat16, device=dev)
    pr = torch.empty_like(sc)
    out = torch.empty(S, Hq, D, dtype=torch.bfloat16, device=dev)
    qd, kd, vd, md = dbf(q, dev), dbf(k, dev), dbf(v, dev), dbf(mask, dev)
    lib.hd_attention_eager(pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), pkg.ptr(md), pkg.ptr(sc),
                           pkg.ptr(pr), pkg.ptr(out), Hq, Hkv, S, D, D ** -0.5)
    pkg.check_prim("eager")
    ref = orc.attention(q, k, v, host(md), 0, prob_mode=1, round_=1)
    assert close_bf16(host(out).reshape(S, Hq * D), ref, ulps=1, atol_rel=0)


def test_head_split_merge_roundtrip(pkg, lib, dev):
    # test_primitives.c:537-556, bit-exact
    S, H, D = 37, 4, 128
    x = torch.randn(S, H, D, device=dev).to(torch.bfloat16)
    y = torch.empty_like(x)
    z = torch.empty_like(x)
    lib.hd_head_split(pkg.ptr(x), pkg.ptr(y), S, H, D)
    lib.hd_head_merge(pkg.ptr(y), pkg.ptr(z), S, H, D)
    torch.cuda.synchronize()
    assert torch.equal(y.view(H, S, D), x.transpose(0, 1).contiguous())
    assert torch.equal(z, x)


def test_lora_merge(pkg, lib, dev):
    N, K, R = 300, 520, 64
    rng = np.random.default_rng(9)
    w = orc.bf16_round(rng.standard_normal((N, K)) * 0.02)
    up = (rng.standard_normal((N, R)) * 0.01).astype(np.float32)
    down = (rng.standard_normal((R, K)) * 0.01).astype(np.float32)
    wd = dbf(w, dev)
    upd, dnd = torch.from_numpy(up).to(dev), torch.from_numpy(down).to(dev)
    e = pkg.hd_lora_entry()
    e.rank, e.in_dim, e.out_dim, e.alpha, e.multiplier = R, K, N, 32.0, 0.8
    e.down_dev, e.up_dev, e.base_dev = dnd.data_ptr(), upd.data_ptr(), wd.data_ptr()
    st = lib.hd_lora_merge_gpu(ctypes.byref(e), 1, None)
    assert st == 0
    torch.cuda.synchronize()
    ref = orc.lora_merge(w, up, down, 0.8 * 32.0 / R)
    assert close_bf16(host(wd), ref, ulps=1, atol_rel=0)
    assert np.mean(host(wd) == ref) > 0.99


@pytest.mark.parametrize("N,K", [(12288, 4096), (1024, 4096), (4096, 12288)])
def test_lora_merge_real_shapes(pkg, lib, dev, N, K):
    """The configuration-4 targets at their real shapes (gate/up 12288 x 4096,
    k/v 1024 x 4096, down 4096 x 12288), rank 64, A and B ~ N(0, 0.01),
    alpha = rank and multiplier 1 (scale 1): W' = bf16(W + s up.down)
    (lora_merge.cu:35-104 in its documented form, hd_lora.h:11-13) against
    the fp32 oracle; every weight within one bf16 step, > 99 % identical."""
    R = 64
    rng = np.random.default_rng(N + K)
    w = orc.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    up = (rng.standard_normal((N, R)) * 0.01).astype(np.float32)
    down = (rng.standard_normal((R, K)) * 0.01).astype(np.float32)
    wd = dbf(w, dev)
    upd, dnd = torch.from_numpy(up).to(dev), torch.from_numpy(down).to(dev)
    e = pkg.hd_lora_entry()
    e.rank, e.in_dim, e.out_dim, e.alpha, e.multiplier = R, K, N, float(R), 1.0
    e.down_dev, e.up_dev, e.base_dev = dnd.data_ptr(), upd.data_ptr(), wd.data_ptr()
    print(f"lora merge {N}x{K} r={R}", flush=True)
    assert lib.hd_lora_merge_gpu(ctypes.byref(e), 1, None) == 0
    torch.cuda.synchronize()
    got = host(wd)
    ref = orc.lora_merge(w, up, down, 1.0)
    same = float(np.mean(got == ref))
    print(f"lora merge {N}x{K}: identical {same:.5f}, changed by the merge {np.mean(ref != w):.3f}")
    # one bf16 step, plus an absolute floor of 1e-4 x RMS (2e-6 here, 1/40 of
    # a bf16 step at the weights' scale) for sums that cancel to near zero,
    # where the fp32 delta's summation order moves the bf16 exponent
    assert close_bf16(got, ref, ulps=1, atol_rel=1e-4)
    assert same > 0.9999


def test_sched_and_patchify_bit_exact(pkg, lib, dev):
    rng = np.random.default_rng(4)
    n = 3 * 64 * 64
    z = orc.bf16_round(rng.standard_normal(n))
    xp = orc.bf16_round(rng.standard_normal(n))
    mo = torch.empty(n, device=dev)
    zd, xpd = dbf(z, dev), dbf(xp, dev)
    lib.hd_sched_vcond(pkg.ptr(zd), pkg.ptr(xpd), 0.7, pkg.ptr(mo), n)
    assert np.array_equal(mo.cpu().numpy(), orc.sched_vcond(z, xp, 0.7))
    zn = torch.empty(n, dtype=torch.bfloat16, device=dev)
    lib.hd_sched_flow_match_step(pkg.ptr(zd), pkg.ptr(mo), 0.7, 0.6, pkg.ptr(zn), n)
    assert np.array_equal(host(zn), orc.sched_flow_match_step(z, mo.cpu().numpy(), 0.7, 0.6))
    c = rng.standard_normal(n).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    o = torch.empty(n, device=dev)
    cd, ud = torch.from_numpy(c).to(dev), torch.from_numpy(u).to(dev)
    lib.hd_sched_cfg_guided(pkg.ptr(cd), pkg.ptr(ud), 5.0, pkg.ptr(o), n)
    assert np.array_equal(o.cpu().numpy(), orc.sched_cfg_guided(c, u, 5.0))
    img = rng.standard_normal((3, 64, 96)).astype(np.float32)
    tok = torch.empty(2 * 3, 3 * 32 * 32, device=dev)
    imgd = torch.from_numpy(img).to(dev)
    lib.hd_patchify_f32(pkg.ptr(imgd), pkg.ptr(tok), 3, 2, 3, 32)
    assert np.array_equal(tok.cpu().numpy(), orc.patchify(img, 32))
    back = torch.empty_like(imgd)
    lib.hd_unpatchify_f32(pkg.ptr(tok), pkg.ptr(back), 3, 2, 3, 32)
    assert torch.equal(back, imgd)


@pytest.mark.parametrize("Hq,Hkv,S,ar", [(4, 2, 40, 0), (4, 2, 64, 0), (4, 2, 100, 0), (4, 2, 128, 0),
                                         (8, 2, 333, 120), (8, 2, 1024, 0), (8, 2, 1024, 700)])
def test_flash_tile_edges(pkg, lib, dev, Hq, Hkv, S, ar):
    # one and two K/V tiles, ragged tails, causal prefixes ending inside and
    # past the first query tiles
    D = 128
    q, k, v = _attn_inputs(Hq, Hkv, S, D, 3 * S + Hq)
    plan = pkg.SdpaPlan(1, Hq, Hkv, S, D, ar_len=ar)
    qd, kd, vd = dbf(q, dev), dbf(k, dev), dbf(v, dev)
    out = torch.zeros(Hq, S, D, dtype=torch.bfloat16, device=dev)
    rc = lib.hd_sdpa_execute(plan.h, pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), None, pkg.ptr(out), None)
    assert rc == 0, lib.hd_cuda_last_error()
    ref = orc.attention(q, k, v, None, ar, round_=0)
    got = host(out).transpose(1, 0, 2).reshape(S, Hq * D)
    assert rel_l2(got, ref) < 8e-3 and cosine(got, ref) > 0.99995


def test_sdpa_split_passes(pkg, lib, dev):
    """hd_sdpa_execute_split_pass: pass 0 writes the causal head rows into
    the plan's staging and leaves `out` untouched (hd_cudnn_sdpa.cu:455-468),
    pass 1 writes every row with full attention; the staged rows equal the
    causal rows of hd_sdpa_execute_split bit for bit."""
    Hq, Hkv, S, D, ar = 8, 2, 300, 128, 77
    q, k, v = _attn_inputs(Hq, Hkv, S, D, 5)
    plan = pkg.SdpaPlan(1, Hq, Hkv, S, D, ar_len=ar)
    qd, kd, vd = dbf(q, dev), dbf(k, dev), dbf(v, dev)
    full = torch.empty(Hq, S, D, dtype=torch.bfloat16, device=dev)
    assert lib.hd_sdpa_execute_split(plan.h, pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), pkg.ptr(full), None) == 0
    out = torch.full((Hq, S, D), 7.0, dtype=torch.bfloat16, device=dev)
    assert lib.hd_sdpa_execute_split_pass(plan.h, 0, pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), pkg.ptr(out),
                                          None) == 0
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    stage_ptr = lib.hd_sdpa_plan_stage(plan.h)
    assert stage_ptr
    # read the staging through an exact kernel: bf16(x + 0) = x
    stage = torch.empty(ar, Hq, D, dtype=torch.bfloat16, device=dev)
    zeros = torch.zeros_like(stage)
    lib.hd_residual_add(ctypes.c_void_p(stage_ptr), pkg.ptr(zeros), pkg.ptr(stage), stage.numel())
    pkg.check_prim("stage read")
    torch.cuda.synchronize()
    assert torch.equal(stage.transpose(0, 1), full[:, :ar])
    assert lib.hd_sdpa_execute_split_pass(plan.h, 1, pkg.ptr(qd), pkg.ptr(kd), pkg.ptr(vd), pkg.ptr(out),
                                          None) == 0
    torch.cuda.synchronize()
    ref = orc.attention(q, k, v, None, 0, round_=0)
    got = host(out).transpose(1, 0, 2).reshape(S, Hq * D)
    assert rel_l2(got, ref) < 8e-3 and cosine(got, ref) > 0.99995


@pytest.mark.parametrize("order", [1, 2])
def test_unipc_kernels_match_oracle(pkg, lib, dev, order):
    # hd_unipc_* against the C restatement, bit for bit, including the last
    # step (sig_t = 0, where lambda is infinite and the plan's h_phi_1 = -1)
    n = 4099
    rng = np.random.default_rng(order)
    a, b, c, d = (rng.standard_normal(n).astype(np.float32) for _ in range(4))
    da, db, dc, dd = (torch.from_numpy(v).to(dev) for v in (a, b, c, d))
    out = torch.empty(n, dtype=torch.float32, device=dev)
    lib.hd_unipc_convert(pkg.ptr(da), pkg.ptr(db), 0.73, pkg.ptr(out), n)
    torch.cuda.synchronize()
    assert np.array_equal(host(out), orc.unipc_convert(a, b, 0.73))
    for sig_t, sig_s0 in ((0.61, 0.7), (0.0, 0.1)):
        at = 1.0 - sig_t
        phi = -0.3 if sig_t else -1.0
        args = (sig_t, sig_s0, at, phi, phi * 1.01, 0.37, 0.52, 1.0 / -0.9)
        lib.hd_unipc_correct(pkg.ptr(da), pkg.ptr(db), pkg.ptr(dc), pkg.ptr(dd), *args, order, pkg.ptr(out), n)
        torch.cuda.synchronize()
        assert np.array_equal(host(out), orc.unipc_correct(a, b, c, d, *args, order))
        pargs = (sig_t, sig_s0, at, phi, phi * 1.01, 0.5, 1.0 / -0.9)
        lib.hd_unipc_predict(pkg.ptr(da), pkg.ptr(db), pkg.ptr(dc), *pargs, order, pkg.ptr(out), n)
        torch.cuda.synchronize()
        assert np.array_equal(host(out), orc.unipc_predict(a, b, c, *pargs, order))


@pytest.mark.parametrize("B,S,H,KV,HID", [(2, 256, 4, 2, 512), (1, 1152, 32, 8, 4096), (3, 320, 8, 2, 256),
                                          (2, 4352, 32, 8, 1024)])
def test_qkv_rope_fused_matches_unfused(pkg, lib, dev, B, S, H, KV, HID):
    # hd_linear_qkv_rope (norm + rotary + V^T in the GEMM epilogue) against
    # hd_linear_concat3 + hd_qkv_epilogue: the same values, bit for bit,
    # including batches whose sequences share a GEMM tile
    D = 128
    g = torch.Generator(device=dev).manual_seed(S + H)
    x = (torch.randn(B * S, HID, generator=g, device=dev)).to(torch.bfloat16)
    wq = (torch.randn(H * D, HID, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wk = (torch.randn(KV * D, HID, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wv = (torch.randn(KV * D, HID, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    gh, gw = 8, (S - 16) // 8
    posd = torch.from_numpy(grid_pos(S - gh * gw, gh, gw)).to(dev)
    cs = pkg.rope_table(posd, S, D, theta=1e4)
    outs = []
    for fused in (True, False):
        q = torch.zeros(B, H, S, D, dtype=torch.bfloat16, device=dev)
        k = torch.zeros(B, KV, S, D, dtype=torch.bfloat16, device=dev)
        vt = torch.zeros(B, KV, D, S, dtype=torch.bfloat16, device=dev)
        if fused:
            rc = lib.hd_linear_qkv_rope(pkg.ptr(x), pkg.ptr(wq), pkg.ptr(wk), pkg.ptr(wv), pkg.ptr(qn),
                                        pkg.ptr(kn), pkg.ptr(cs), pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt),
                                        B, S, H, KV, HID, 1e-6)
            assert rc == 0
        else:
            qkv = torch.empty(B * S, (H + 2 * KV) * D, dtype=torch.bfloat16, device=dev)
            lib.hd_linear_concat3(pkg.ptr(x), pkg.ptr(wq), H * D, pkg.ptr(wk), KV * D, pkg.ptr(wv), KV * D,
                                  pkg.ptr(qkv), B * S, HID)
            lib.hd_qkv_epilogue(pkg.ptr(qkv), pkg.ptr(qn), pkg.ptr(kn), pkg.ptr(cs), pkg.ptr(q), pkg.ptr(k),
                                None, pkg.ptr(vt), B, S, H, KV, D, 1e-6)
        pkg.check_prim("qkv fused=%s" % fused)
        torch.cuda.synchronize()
        outs.append((q, k, vt))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert float(outs[0][0].float().abs().mean()) > 0.1
    # outside the fused path nothing is launched
    assert lib.hd_linear_qkv_rope(pkg.ptr(x), pkg.ptr(wq), pkg.ptr(wk), pkg.ptr(wv), pkg.ptr(qn), pkg.ptr(kn),
                                  pkg.ptr(cs), pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), B, S - 8, H, KV, HID,
                                  1e-6) == 1


@pytest.mark.parametrize("S,seq_major", [(17 * 128, 1), (2150, 0)])
def test_flash_tail_split_matches_unsplit(pkg, lib, dev, S, seq_major):
    # units = 32 heads x 17 query tiles = 544 > one round of resident blocks:
    # the remainder runs as key-range chunks + merge; it must agree with the
    # unsplit kernel to the fp32 rounding of the merge (a few bf16 ulps)
    B, Hq, Hkv, D = 1, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(S)
    q = torch.randn(B, Hq, S, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B * Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    vt = torch.empty(lib.hd_flash_vt_bytes(B, Hkv, S) // 2, dtype=torch.bfloat16, device=dev)
    lib.hd_flash_make_vt(pkg.ptr(v), pkg.ptr(vt), B * Hkv, S)
    wsb = lib.hd_flash_ws_bytes()
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    shape = (B, S, Hq * D) if seq_major else (B, Hq, S, D)
    a = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    b = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    sc = 1.0 / np.sqrt(D)
    assert lib.hd_flash_attention(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), None, pkg.ptr(a), B, Hq, Hkv, S, D,
                                  0, sc, seq_major) == 0
    assert lib.hd_flash_attention_ws(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), None, pkg.ptr(b), B, Hq, Hkv, S,
                                     D, 0, sc, seq_major, pkg.ptr(ws), wsb) == 0
    torch.cuda.synchronize()
    af, bf = a.float(), b.float()
    assert float((af - bf).norm() / af.norm()) < 2e-3
    # with the workspace the 8-wave kernel runs (256 query rows per unit):
    # 32 of its 32 x 9 units are the split tail, up to 12 % of the rows
    assert float((af == bf).float().mean()) > 0.9
    assert float((af - bf).abs().max()) <= 4 * 2 ** -8 * float(af.abs().max())
    # the split really ran: the last query tiles of the last heads differ
    # in at least a few bits somewhere, or match exactly when the merge
    # reproduces the rounding; both are fine, but nothing may be left zero
    assert float(bf.abs().sum(dim=-1).min()) > 0


@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("bias", [False, True])
def test_gemm_tail_split(pkg, lib, dev, K, bias):
    """hd_linear_residual_ws / hd_linear_ws: M = 8448 gives 33 x 16 = 528
    tiles of 256x256, two rounds of 256 CUs plus 16 tail tiles that run as
    K chunks. Whole tiles equal the unsplit GEMM bit for bit; tail tiles
    differ only by the fp32 reassociation of the K sum (one bf16 step)."""
    M, N = 8448, 4096
    print(f"tail split K={K} bias={bias}", flush=True)
    g = torch.Generator(device=dev).manual_seed(K + bias)
    x = (torch.randn(M, K, device=dev, generator=g)).to(torch.bfloat16)
    w = (torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    r = torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16)
    b = (torch.randn(N, device=dev, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    y0, y1 = torch.empty(M, N, dtype=torch.bfloat16, device=dev), torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    if bias:
        lib.hd_linear(pkg.ptr(x), pkg.ptr(w), pkg.ptr(b), pkg.ptr(y0), M, N, K, 1)
        lib.hd_linear_ws(pkg.ptr(x), pkg.ptr(w), pkg.ptr(b), pkg.ptr(y1), M, N, K, pkg.ptr(ws), ws.numel())
        want = ((x.float() @ w.float().t()).to(torch.bfloat16).float() + b.float())
    else:
        lib.hd_linear_residual(pkg.ptr(x), pkg.ptr(w), pkg.ptr(r), pkg.ptr(y0), M, N, K)
        lib.hd_linear_residual_ws(pkg.ptr(x), pkg.ptr(w), pkg.ptr(r), pkg.ptr(y1), M, N, K,
                                  pkg.ptr(ws), ws.numel())
        want = (x.float() @ w.float().t()).to(torch.bfloat16).float() + r.float()
    pkg.check_prim("tail split")
    torch.cuda.synchronize()
    a, c = y0.float(), y1.float()
    diff = (a - c).abs()
    # one bf16 step of the GEMM sum (rounded before the bias / residual add)
    # plus one of the output
    acc = (x.float() @ w.float().t()).abs()
    step = (acc + a.abs()) * 2.0 ** -7 + 1e-6
    worst = int(torch.argmax(diff - step))
    print("worst", a.flatten()[worst].item(), c.flatten()[worst].item(), acc.flatten()[worst].item())
    assert bool((diff <= step).all())
    same = float((diff == 0).float().mean())
    assert same >= 512 / 528 - 1e-3, same        # whole tiles bit-identical
    assert same < 1.0                            # the tail did run split
    rel = float((c - want).norm() / want.norm())
    assert rel < 5e-3, rel


def test_qkv_rope_tail_split(pkg, lib, dev):
    """hd_linear_qkv_rope_ws at config 1's shape (B = 2, S = 4352: 34 x 24 =
    816 tiles, three rounds of 256 CUs plus 48 tail tiles run as K chunks,
    the merge running the same epilogue): whole tiles equal the unsplit
    fused GEMM bit for bit, tail tiles to the fp32 reassociation of the K
    sum carried through the norm and rotary."""
    B, S, H, KV, HID, D = 2, 4352, 32, 8, 4096, 128
    g = torch.Generator(device=dev).manual_seed(77)
    x = (torch.randn(B * S, HID, generator=g, device=dev)).to(torch.bfloat16)
    wq = (torch.randn(H * D, HID, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wk = (torch.randn(KV * D, HID, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wv = (torch.randn(KV * D, HID, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    posd = torch.from_numpy(grid_pos(256, 64, 64)).to(dev)
    cs = pkg.rope_table(posd, S, D, theta=1e4)
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    outs = []
    for use_ws in (False, True):
        q = torch.zeros(B, H, S, D, dtype=torch.bfloat16, device=dev)
        k = torch.zeros(B, KV, S, D, dtype=torch.bfloat16, device=dev)
        vt = torch.zeros(B, KV, D, S, dtype=torch.bfloat16, device=dev)
        args = [pkg.ptr(x), pkg.ptr(wq), pkg.ptr(wk), pkg.ptr(wv), pkg.ptr(qn), pkg.ptr(kn), pkg.ptr(cs),
                pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), B, S, H, KV, HID, 1e-6]
        rc = lib.hd_linear_qkv_rope_ws(*args, pkg.ptr(ws), ws.numel()) if use_ws else lib.hd_linear_qkv_rope(*args)
        assert rc == 0
        pkg.check_prim("qkv ws=%s" % use_ws)
        torch.cuda.synchronize()
        outs.append((q, k, vt))
    fracs = []
    for a, b in zip(*outs):
        a, b = a.float(), b.float()
        d = (a - b).abs()
        fracs.append(float((d == 0).float().mean()))
        assert float(d.norm() / a.norm()) < 2e-3
        assert bool((d <= a.abs() * 2.0 ** -5 + 1e-2).all())
    print("identical fractions q/k/vt:", fracs)
    assert min(fracs) >= 0.9 and min(fracs) < 1.0


def test_swiglu_tail_split(pkg, lib, dev):
    """hd_linear_swiglu_ws at config 2's row count (M = 16640: 65 x 96 =
    6240 tiles, 24 rounds + 96 tail tiles in K chunks): whole tiles equal
    the unsplit GEMM bit for bit, the tail within the reassociation of the
    K sum carried through silu(gate) * up."""
    M, F, K = 16640, 12288, 4096
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    wg = (torch.randn(F, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(F, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    y0 = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    y1 = torch.empty_like(y0)
    lib.hd_linear_swiglu(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(y0), M, F, K)
    lib.hd_linear_swiglu_ws(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(y1), M, F, K, pkg.ptr(ws), ws.numel())
    pkg.check_prim("swiglu tail split")
    torch.cuda.synchronize()
    a, b = y0.float(), y1.float()
    d = (a - b).abs()
    same = float((d == 0).float().mean())
    print("identical fraction", same)
    assert same >= 6144 / 6240 - 1e-3 and same < 1.0
    assert float(d.norm() / a.norm()) < 1e-3


@pytest.mark.parametrize("S,ar_len,dense,heads,use_ws", [(2176, 0, False, 8, False), (1152, 127, False, 8, False),
                                                         (1000, 0, False, 8, False), (576, 0, True, 8, False),
                                                         (2176, 0, False, 32, True), (1000, 0, False, 32, True),
                                                         (640, 300, False, 32, True)])
def test_flash_launch_paths_vs_fp32(pkg, lib, dev, S, ar_len, dense, heads, use_ws):
    """Every launch path of the flash kernels against fp32 softmax(Q K^T s +
    mask) V on four heads: 4-wave blocks (no workspace, masked launches,
    S % 64 != 0, a dense additive mask), the 8-wave ping-pong blocks with the
    tail split (workspace, full attention, S >= 1024; 32 heads so the last
    round is partial) and the causal text prefix run as its own masked launch
    ahead of the unmasked rows (rows < ar_len see keys <= row,
    hd_cudnn_sdpa.cu:376-441)."""
    B, Hq, Hkv, D = 2, heads, heads // 4, 128
    g = torch.Generator(device=dev).manual_seed(S + ar_len)
    q = torch.randn(B, Hq, S, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B * Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    vt = torch.empty(lib.hd_flash_vt_bytes(B, Hkv, S) // 2, dtype=torch.bfloat16, device=dev)
    lib.hd_flash_make_vt(pkg.ptr(v), pkg.ptr(vt), B * Hkv, S)
    mask = None
    if dense:
        mask = (torch.randn(S, S, generator=g, device=dev) * 2).to(torch.bfloat16)
    print(f"flash paths S={S} ar_len={ar_len} dense={dense} heads={heads} ws={use_ws}", flush=True)
    o = torch.zeros(B, S, Hq * D, dtype=torch.bfloat16, device=dev)
    mp = pkg.ptr(mask) if mask is not None else None
    if use_ws:
        ws = torch.empty(lib.hd_flash_ws_bytes(), dtype=torch.uint8, device=dev)
        rc = lib.hd_flash_attention_ws(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), mp, pkg.ptr(o), B, Hq, Hkv, S, D,
                                       ar_len, D ** -0.5, 1, pkg.ptr(ws), ws.numel())
    else:
        rc = lib.hd_flash_attention(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), mp, pkg.ptr(o), B, Hq, Hkv, S, D,
                                    ar_len, D ** -0.5, 1)
    assert rc == 0
    torch.cuda.synchronize()
    vv = v.view(B, Hkv, S, D).float()
    for b in range(B):
        for h in (0, Hq // 3, Hq // 2 + 1, Hq - 1):
            sc = (q[b, h].float() @ k[b, h // (Hq // Hkv)].float().t()) * D ** -0.5
            if mask is not None:
                sc = sc + mask.float()
            if ar_len:
                r = torch.arange(S, device=dev)
                sc = sc.masked_fill((r[:, None] < ar_len) & (r[None, :] > r[:, None]), float("-inf"))
            ref = torch.softmax(sc, -1) @ vv[b, h // (Hq // Hkv)]
            got = o[b, :, h * D:(h + 1) * D].float()
            rel = float((got - ref).norm() / ref.norm())
            cos = float((got * ref).sum() / (got.norm() * ref.norm()))
            assert rel <= 1e-2 and cos >= 0.9999, (b, h, rel, cos)
    assert float(o.float().abs().sum(dim=-1).min()) > 0


@pytest.mark.parametrize("n,off", [(12291, 0), (12291, 1), (7, 0)])
def test_sched_vector_paths_bit_exact(pkg, lib, dev, n, off):
    """The sampler kernels' 4-wide path (aligned operands; a partial last
    group when n % 4 != 0) and the scalar fallback (operands one element off
    16-byte alignment) both equal the oracle bit for bit; so do the fp32
    denoised / z_next / bf16 upcast pointwise steps against numpy's fp32
    fma (sched.cu:21-72)."""
    rng = np.random.default_rng(n + off)
    z = orc.bf16_round(rng.standard_normal(n))
    xp = orc.bf16_round(rng.standard_normal(n))
    # allocate one element more and view from `off`, so off = 1 misaligns
    zb = torch.zeros(n + 1, dtype=torch.bfloat16, device=dev)
    xb = torch.zeros(n + 1, dtype=torch.bfloat16, device=dev)
    zb[off:off + n] = torch.from_numpy(z.astype(np.float32)).to(torch.bfloat16)
    xb[off:off + n] = torch.from_numpy(xp.astype(np.float32)).to(torch.bfloat16)
    zd, xd = zb[off:off + n], xb[off:off + n]
    mo = torch.empty(n + 1, device=dev)[off:off + n]
    lib.hd_sched_vcond(pkg.ptr(zd), pkg.ptr(xd), 0.7, pkg.ptr(mo), n)
    assert np.array_equal(mo.cpu().numpy(), orc.sched_vcond(z, xp, 0.7))
    zn = torch.empty(n + 1, dtype=torch.bfloat16, device=dev)[off:off + n]
    lib.hd_sched_flow_match_step(pkg.ptr(zd), pkg.ptr(mo), 0.7, 0.6, pkg.ptr(zn), n)
    assert np.array_equal(host(zn), orc.sched_flow_match_step(z, mo.cpu().numpy(), 0.7, 0.6))
    c = rng.standard_normal(n).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    cd = torch.zeros(n + 1, device=dev)
    ud = torch.zeros(n + 1, device=dev)
    cd[off:off + n] = torch.from_numpy(c).to(dev)
    ud[off:off + n] = torch.from_numpy(u).to(dev)
    cv, uv = cd[off:off + n], ud[off:off + n]
    o = torch.empty(n + 1, device=dev)[off:off + n]
    lib.hd_sched_cfg_guided(pkg.ptr(cv), pkg.ptr(uv), 5.0, pkg.ptr(o), n)
    assert np.array_equal(o.cpu().numpy(), orc.sched_cfg_guided(c, u, 5.0))
    f32 = np.float32
    lib.hd_sched_denoised(pkg.ptr(cv), pkg.ptr(uv), 0.3, pkg.ptr(o), n)
    want = (-u.astype(np.float64) * f32(0.3) + c).astype(np.float32)   # one rounding: fma
    assert np.array_equal(o.cpu().numpy(), want)
    lib.hd_sched_z_next(pkg.ptr(cv), pkg.ptr(uv), 0.4, 1.0, pkg.ptr(o), n)
    t = (f32(0.4) * c).astype(np.float32) * f32(1.0)
    want = (f32(1.0) - f32(0.4)).astype(np.float64) * u + t.astype(np.float64)
    assert np.array_equal(o.cpu().numpy(), want.astype(np.float32))
    lib.hd_sched_bf16_upcast(pkg.ptr(zd), pkg.ptr(o), n)
    assert np.array_equal(o.cpu().numpy(), z.astype(np.float32))


def test_patchify_bf16_and_rotary_scalar_path(pkg, lib, dev):
    """patchify_bf16 (4-wide path) equals the oracle's patchify rounded to
    bf16; a head_dim of 24 (not a multiple of 16) takes the scalar rotary
    kernel, which must equal the oracle bit for bit as the 16-byte one does."""
    rng = np.random.default_rng(5)
    img = rng.standard_normal((3, 64, 96)).astype(np.float32)
    tok = torch.empty(2 * 3, 3 * 32 * 32, dtype=torch.bfloat16, device=dev)
    imgd = torch.from_numpy(img).to(dev)
    lib.hd_patchify_bf16(pkg.ptr(imgd), pkg.ptr(tok), 3, 2, 3, 32)
    assert np.array_equal(host(tok), orc.bf16_round(orc.patchify(img, 32)))
    seq, dim = 5, 24
    x = orc.bf16_round(rng.standard_normal((2, seq, dim)))
    cr = rng.standard_normal((seq, dim)).astype(np.float32)
    sr = rng.standard_normal((seq, dim)).astype(np.float32)
    y = torch.empty(2, seq, dim, dtype=torch.bfloat16, device=dev)
    xd, cd, sd = dbf(x, dev), torch.from_numpy(cr).to(dev), torch.from_numpy(sr).to(dev)
    lib.hd_apply_rotary(pkg.ptr(xd), pkg.ptr(cd), pkg.ptr(sd), pkg.ptr(y), 2, seq, dim)
    torch.cuda.synchronize()
    assert np.array_equal(host(y), orc.apply_rotary(x, cr, sr, 1))


def test_lora_merge_batched_entries_vs_oracle(pkg, lib, dev):
    """One hd_lora_merge_gpu call over entries of mixed shapes and ranks, as
    an adapter load makes it: the streaming kernel batches the entries of one
    (out, in, rank) shape into one launch, the other ranks run the fp32
    kernel, and two entries on the same weight (two adapters naming one
    target) merge in entry order, each on the other's result
    (lora_merge.cu:35-104 loops over the entries in order)."""
    rng = np.random.default_rng(77)
    shapes = [(256, 512, 64), (256, 512, 64), (128, 256, 16), (256, 512, 64), (130, 72, 37), (256, 512, 64)]
    ws = [orc.bf16_round(rng.standard_normal((n, k)).astype(np.float32) * 0.02) for n, k, _ in shapes]
    wds = [dbf(w, dev) for w in ws]
    # entry list: every weight once, then weights 1 and 4 a second time
    order = [0, 1, 2, 3, 4, 5, 1, 4]
    ents = (pkg.hd_lora_entry * len(order))()
    keep, refs = [], [w.copy() for w in ws]
    for j, i in enumerate(order):
        n, k, r = shapes[i]
        up = (rng.standard_normal((n, r)) * 0.01).astype(np.float32)
        down = (rng.standard_normal((r, k)) * 0.01).astype(np.float32)
        mult = 0.5 + 0.25 * j
        upd, dnd = torch.from_numpy(up).to(dev), torch.from_numpy(down).to(dev)
        keep += [upd, dnd]
        e = ents[j]
        e.rank, e.in_dim, e.out_dim, e.alpha, e.multiplier = r, k, n, float(r), mult
        e.down_dev, e.up_dev, e.base_dev = dnd.data_ptr(), upd.data_ptr(), wds[i].data_ptr()
        refs[i] = orc.lora_merge(refs[i], up, down, mult)
    assert lib.hd_lora_merge_gpu(ents, len(order), None) == 0
    torch.cuda.synchronize()
    for i, (wd, ref) in enumerate(zip(wds, refs)):
        got = host(wd)
        assert close_bf16(got, ref, ulps=1, atol_rel=1e-4), i
        assert np.mean(got == ref) > 0.999, i


@pytest.mark.parametrize("N,K,R", [(300, 520, 64), (257, 136, 36), (4224, 1032, 64), (130, 72, 8),
                                   (300, 520, 37), (520, 264, 128)])
def test_lora_merge_kernels_vs_oracle(pkg, lib, dev, N, K, R):
    """Both merge kernels against the fp32 oracle (lora_merge.cu:35-104): the
    streaming split-operand kernel (rank <= 64, rank % 4 == 0), including
    ragged tiles and row strips that cross the persistent blocks' ranges,
    and the fp32 matrix-core kernel for the ranks it does not take (37,
    128). Within one bf16 step everywhere, exactly rounded on > 99.9 %."""
    rng = np.random.default_rng(N * 7 + K + R)
    w = orc.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    up = (rng.standard_normal((N, R)) * 0.01).astype(np.float32)
    down = (rng.standard_normal((R, K)) * 0.01).astype(np.float32)
    upd, dnd = torch.from_numpy(up).to(dev), torch.from_numpy(down).to(dev)
    ref = orc.lora_merge(w, up, down, 0.75)
    wd = dbf(w, dev)
    e = pkg.hd_lora_entry()
    e.rank, e.in_dim, e.out_dim, e.alpha, e.multiplier = R, K, N, float(R), 0.75
    e.down_dev, e.up_dev, e.base_dev = dnd.data_ptr(), upd.data_ptr(), wd.data_ptr()
    assert lib.hd_lora_merge_gpu(ctypes.byref(e), 1, None) == 0
    torch.cuda.synchronize()
    got = host(wd)
    assert close_bf16(got, ref, ulps=1, atol_rel=1e-4)
    assert np.mean(got == ref) > 0.999


@pytest.mark.parametrize("B,S,T", [(1, 1152, 128), (2, 640, 300), (1, 2176, 65), (1, 4352, 256)])
def test_flash_causal_prefix_split_launch(pkg, lib, dev, B, S, T):
    """A causal text prefix (rows < ar_len = T - 1 see keys <= row) with the
    tail-split workspace runs as two launches: the prefix rows masked, the
    rows from ar_len on as full attention with a query-row offset and the
    tail split (hd_cudnn_sdpa.cu:376-441 runs the same split as two cuDNN
    passes). Checked against an fp32 torch statement of the attention with
    that mask, and against the single masked launch (no workspace)."""
    g = torch.Generator(device=dev).manual_seed(S + T)
    q = torch.randn(B, 32, S, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, 8, S, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B * 8, S, 128, generator=g, device=dev).to(torch.bfloat16)
    vt = torch.empty(lib.hd_flash_vt_bytes(B, 8, S) // 2, dtype=torch.bfloat16, device=dev)
    lib.hd_flash_make_vt(pkg.ptr(v), pkg.ptr(vt), B * 8, S)
    ws = torch.empty(lib.hd_flash_ws_bytes(), dtype=torch.uint8, device=dev)
    ar = T - 1
    o_split = torch.zeros(B, S, 32 * 128, dtype=torch.bfloat16, device=dev)
    o_one = torch.zeros_like(o_split)
    assert lib.hd_flash_attention_ws(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), None, pkg.ptr(o_split), B, 32, 8, S,
                                     128, ar, 128 ** -0.5, 1, pkg.ptr(ws), ws.numel()) == 0
    assert lib.hd_flash_attention(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), None, pkg.ptr(o_one), B, 32, 8, S, 128,
                                  ar, 128 ** -0.5, 1) == 0
    torch.cuda.synchronize()
    qf = q.float()
    kf = k.float().repeat_interleave(4, 1)
    vf = v.float().view(B, 8, S, 128).repeat_interleave(4, 1)
    sc = qf @ kf.transpose(-1, -2) * 128 ** -0.5
    i = torch.arange(S, device=dev)
    sc = sc.masked_fill((i[:, None] < ar) & (i[None, :] > i[:, None]), float("-inf"))
    ref = (torch.softmax(sc, -1) @ vf).permute(0, 2, 1, 3).reshape(B, S, 32 * 128)
    for got in (o_split, o_one):
        gf = got.float()
        assert float((gf - ref).norm() / ref.norm()) < 5e-3
        assert float((gf[:, :ar] - ref[:, :ar]).norm() / ref[:, :ar].norm()) < 5e-3
    # the prefix rows come from the same masked kernel either way
    assert torch.equal(o_split[:, :ar], o_one[:, :ar])

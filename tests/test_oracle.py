"""Pins the CPU oracle (oracle/o1_oracle.c) before it is trusted as the
checker of the HIP path. Each check is independent of the oracle's own
formula: torch library routines, the reference's known-answer tests and
fixtures (tests/golden/), closed forms, invariants and brute force."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from tests.common import make_block_weights, grid_pos, rel_l2, cosine, bf16

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def test_bf16_rne_matches_torch_fixture():
    g = gold("bf16_rne.json")
    x = np.array(g["f32_bits"], dtype=np.uint32).view(np.float32)
    want = np.array(g["bf16_bits"], dtype=np.uint32)
    got = orc.bf16_round(x).view(np.uint32) >> 16
    assert np.array_equal(got, want)
    lib = orc.lib()
    for v, w in zip(x[:50], want[:50]):
        assert (np.float32(lib.o1o_bf16_round(float(v))).view(np.uint32) >> 16) == w


def test_linear_gemm_smoke_kats():
    for c in gold("gemm_smoke.json")["cases"]:
        X = np.array(c["X"], np.float32).reshape(c["M"], c["K"])
        W = np.array(c["W"], np.float32).reshape(c["N"], c["K"])
        y = orc.linear(X, W, mode=1)
        if "Y" in c:
            assert y.ravel().tolist() == c["Y"]
        else:
            bits = (y.ravel().view(np.uint32) >> 16).tolist()
            assert bits == c["Y_bf16_bits"]


def test_linear_vs_torch_and_bias_modes():
    g = torch.Generator().manual_seed(0)
    for M, N, K in [(7, 5, 6), (65, 33, 130), (4, 3, 5)]:
        x = bf16(torch.randn(M, K, generator=g))
        w = bf16(torch.randn(N, K, generator=g))
        b = bf16(torch.randn(N, generator=g))
        ref = (x.double() @ w.double().t()).float()
        y0 = orc.linear(x.numpy(), w.numpy(), mode=0)
        assert np.allclose(y0, ref.numpy(), rtol=1e-5, atol=1e-5)
        # production bias: bf16(bf16(acc) + b) (gemm.cu:226-235)
        y2 = orc.linear(x.numpy(), w.numpy(), b.numpy(), mode=2)
        want = (bf16(ref) + b).to(torch.bfloat16).float().numpy()
        assert np.mean(y2 == want) > 0.98 and rel_l2(y2, want) < 4e-3


def test_rmsnorm_reference_analytic_and_invariants():
    # test_primitives.c:159-200 input: x = (i+j+1)*0.5, w = j+1
    rows, cols = 4, 8
    x = np.array([[(i + j + 1) * 0.5 for j in range(cols)] for i in range(rows)], np.float32)
    w = np.arange(1, cols + 1, dtype=np.float32)
    y = orc.rmsnorm(x, w, 1e-6, 0)
    ref = F.rms_norm(torch.from_numpy(x), (cols,), torch.from_numpy(w), eps=1e-6).numpy()
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)
    # scale invariance and unit RMS for w = 1
    z = np.random.default_rng(0).standard_normal((16, 4096)).astype(np.float32)
    a = orc.rmsnorm(z, np.ones(4096, np.float32), 0.0, 0)
    b = orc.rmsnorm(z * 37.0, np.ones(4096, np.float32), 0.0, 0)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)
    assert np.allclose(np.sqrt((a.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-5)
    # bf16 output = torch bf16 rms_norm of the same values (one rounding)
    zb = orc.bf16_round(z)
    tb = F.rms_norm(torch.from_numpy(zb), (4096,), eps=1e-6).to(torch.bfloat16).float().numpy()
    assert np.mean(orc.rmsnorm(zb, np.ones(4096, np.float32), 1e-6, 1) == tb) > 0.995


def test_silu_swiglu_vs_torch_bf16_ops():
    # torch bf16 elementwise ops round every op result (what act.cu:29-33 emulates)
    x = np.linspace(-8, 8, 4097).astype(np.float32)
    xb = torch.from_numpy(orc.bf16_round(x)).to(torch.bfloat16)
    u = torch.from_numpy(orc.bf16_round(np.cos(x * 3))).to(torch.bfloat16)
    want_silu = F.silu(xb).float().numpy()
    want_sw = (F.silu(xb) * u).float().numpy()
    got_silu = orc.silu(xb.float().numpy(), 1)
    got_sw = orc.swiglu(xb.float().numpy(), u.float().numpy(), 1)
    assert np.mean(got_silu == want_silu) > 0.99
    assert np.mean(got_sw == want_sw) > 0.99
    assert rel_l2(got_sw, want_sw) < 3e-3


def test_mrope_interleaved_rule_vs_slice_form():
    """The interleaved section rule restated as the slice assignment used by
    the upstream model (T everywhere, then H on indices 1::3 < 3*sec[1], W on
    2::3 < 3*sec[2]); reference test shape test_primitives.c:351."""
    for seq, dim, sec, theta in [(4, 64, (6, 2, 2), 5e6), (23, 128, (24, 20, 20), 5e6),
                                 (40, 128, (24, 20, 20), 1e4)]:
        rng = np.random.default_rng(seq)
        pos = rng.integers(0, 5000, (3, seq)).astype(np.float32)
        half = dim // 2
        inv = 1.0 / (theta ** (np.arange(0, dim, 2, dtype=np.float64) / dim))
        fr = pos[:, :, None].astype(np.float64) * inv[None, None, :]       # [3, seq, half]
        f = fr[0].copy()
        f[:, 1:3 * sec[1]:3] = fr[1][:, 1:3 * sec[1]:3]
        f[:, 2:3 * sec[2]:3] = fr[2][:, 2:3 * sec[2]:3]
        emb = np.concatenate([f, f], -1)
        c, s = orc.mrope_cos_sin(pos, seq, dim, theta, sec)
        assert np.abs(c - np.cos(emb)).max() < 2e-3 and np.abs(s - np.sin(emb)).max() < 2e-3
        # positions with small angles are accurate to fp32 rounding
        small = emb < 10
        assert np.abs(c - np.cos(emb))[small].max() < 1e-5


def test_rotary_invariants():
    rng = np.random.default_rng(1)
    x = orc.bf16_round(rng.standard_normal((3, 20, 128)))
    pos = np.zeros((3, 20), np.float32)
    c, s = orc.mrope_cos_sin(pos, 20, 128, 1e4)
    assert np.array_equal(orc.apply_rotary(x, c, s, 1), x)              # angle 0: identity
    pos = rng.integers(0, 100, (3, 20)).astype(np.float32)
    c, s = orc.mrope_cos_sin(pos, 20, 128, 1e4)
    y = orc.apply_rotary(x, c, s, 0)
    nx = np.hypot(x[..., :64], x[..., 64:])
    ny = np.hypot(y[..., :64], y[..., 64:])
    assert np.allclose(nx, ny, rtol=1e-2)                               # pair norms preserved
    # rotation by +a then -a returns the input (fp32 path, up to bf16 output rounding)
    back = orc.apply_rotary(y, c, -s, 0)
    assert rel_l2(back, x) < 1e-2


def _torch_sdpa(q, k, v, mask=None, ar_len=0):
    Hq, S, D = q.shape
    grp = Hq // k.shape[0]
    kk = torch.from_numpy(k).repeat_interleave(grp, 0)
    vv = torch.from_numpy(v).repeat_interleave(grp, 0)
    bias = torch.zeros(S, S)
    if ar_len:
        causal = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
        causal[ar_len:] = False
        bias = bias.masked_fill(causal, float("-inf"))
    if mask is not None:
        bias = bias + torch.from_numpy(mask)
    o = F.scaled_dot_product_attention(torch.from_numpy(q)[None].double(), kk[None].double(),
                                       vv[None].double(), attn_mask=bias.double())
    return o[0].transpose(0, 1).reshape(S, Hq * D).float().numpy()


@pytest.mark.parametrize("Hq,Hkv,S,ar", [(4, 2, 37, 0), (8, 2, 64, 10), (2, 1, 5, 3)])
def test_attention_vs_torch_sdpa(Hq, Hkv, S, ar):
    rng = np.random.default_rng(S)
    D = 128
    q = rng.standard_normal((Hq, S, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, S, D)).astype(np.float32)
    got = orc.attention(q, k, v, None, ar, round_=0)
    want = _torch_sdpa(q, k, v, None, ar)
    assert np.abs(got - want).max() < 1e-4


def test_attention_invariants():
    rng = np.random.default_rng(2)
    Hq, S, D = 2, 33, 128
    k = rng.standard_normal((1, S, D)).astype(np.float32)
    v = rng.standard_normal((1, S, D)).astype(np.float32)
    out = orc.attention(np.zeros((Hq, S, D), np.float32), k, v, None, 0, round_=0)
    assert np.allclose(out.reshape(S, Hq, D), v[0].mean(0)[None, None, :], atol=1e-5)
    # one-hot: query aligned with key 7 at a large scale -> picks v[7]
    q = np.repeat(k[:, 7:8, :] * 50, S, axis=1).repeat(Hq, 0)
    out = orc.attention(q, k, v, None, 0, round_=0)
    assert np.allclose(out.reshape(S, Hq, D), v[0, 7][None, None, :], atol=1e-4)


def test_timestep_embed_closed_form():
    # test_primitives.c:300-327 (N=3, dim 8) and the forward's dim 256
    for t, dim in [([0.5, 1.0, 2.0], 8), ([500.0], 256)]:
        y = orc.timestep_embed(np.array(t, np.float32), dim)
        half = dim // 2
        fr = np.exp(-np.log(10000.0) * np.arange(half) / half)
        arg = np.array(t)[:, None] * fr[None]
        want = np.concatenate([np.cos(arg), np.sin(arg)], 1)
        assert np.abs(y - want).max() < 2e-4


def test_positions_fixture_layout():
    g = gold("positions_s23.json")
    T, gh, gw, fpnt = g["text_len"], g["grid_h"], g["grid_w"], g["fix_point"]
    pos = grid_pos(T, gh, gw, fix_point=fpnt)
    pos[:, :T] = np.arange(T)[None]
    pos[1, T:] += fpnt
    pos[2, T:] += fpnt
    assert pos.tolist() == g["pos"]


def test_patchify_vs_reshape_and_decode_kat():
    rng = np.random.default_rng(3)
    C, Hp, Wp, p = 3, 3, 5, 4
    img = rng.standard_normal((C, Hp * p, Wp * p)).astype(np.float32)
    tok = orc.patchify(img, p)
    want = img.reshape(C, Hp, p, Wp, p).transpose(1, 3, 0, 2, 4).reshape(Hp * Wp, C * p * p)
    assert np.array_equal(tok, want)
    assert np.array_equal(orc.unpatchify(tok, C, Hp, Wp, p), img)
    # decode.c:14-22 known answers: -1 -> 0, 1 -> 255, 0 -> roundf(127.5) = 128, clamps
    z = np.zeros((1, 3 * 1 * 1), np.float32)
    for val, px in [(-1.0, 0), (1.0, 255), (0.0, 128), (3.0, 255), (-4.0, 0)]:
        z[:] = val
        assert orc.decode_to_rgb(z, 1, 1, 1, 3).ravel().tolist() == [px] * 3


def test_lora_merge_vs_torch():
    rng = np.random.default_rng(4)
    N, K, R = 40, 72, 16
    w = orc.bf16_round(rng.standard_normal((N, K)) * 0.02)
    up = (rng.standard_normal((N, R)) * 0.01).astype(np.float32)
    down = (rng.standard_normal((R, K)) * 0.01).astype(np.float32)
    got = orc.lora_merge(w, up, down, 0.5)
    want = (torch.from_numpy(w) + 0.5 * (torch.from_numpy(up).double() @ torch.from_numpy(down).double()).float()
            ).to(torch.bfloat16).float().numpy()
    assert np.mean(got == want) > 0.99


def test_sched_ops_vs_torch():
    rng = np.random.default_rng(5)
    z = orc.bf16_round(rng.standard_normal(1000))
    xp = orc.bf16_round(rng.standard_normal(1000))
    zt, xt = torch.from_numpy(z), torch.from_numpy(xp)
    assert np.array_equal(orc.sched_vcond(z, xp, 0.3), ((zt - xt) / 0.3).numpy())
    mo = ((zt - xt) / 0.3)
    # fp32 host dt (sched.cu:118); fused multiply-add as the CUDA build
    # contracts it: exact product + sum in float64, one rounding to fp32
    dt = np.float32(0.2) - np.float32(0.3)
    fma = (z.astype(np.float64) + np.float64(dt) * mo.numpy().astype(np.float64)).astype(np.float32)
    want = orc.bf16_round(fma)
    assert np.mean(orc.sched_flow_match_step(z, mo.numpy(), 0.3, 0.2) == want) > 0.999
    c, u = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    want = (np.float64(5.0) * c.astype(np.float64) +
            np.float32(1.0 - 5.0) * u).astype(np.float32)
    assert np.mean(orc.sched_cfg_guided(c, u, 5.0) == want) > 0.999


# ---- composite: an independent torch fp32 statement of the decoder layer ----
def torch_block(x, pos, w, H, KV, D, theta, eps=1e-6, ar_len=0, sec=(24, 20, 20)):
    S, HID = x.shape
    t = {k: v.double() for k, v in w.items()}
    xx = x.double()
    ln = F.rms_norm(xx, (HID,), t["input_ln"], eps)
    q = (ln @ t["q_proj"].T).view(S, H, D)
    k = (ln @ t["k_proj"].T).view(S, KV, D)
    v = (ln @ t["v_proj"].T).view(S, KV, D)
    q = F.rms_norm(q, (D,), t["q_norm"], eps).transpose(0, 1)
    k = F.rms_norm(k, (D,), t["k_norm"], eps).transpose(0, 1)
    v = v.transpose(0, 1)
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    fr = torch.from_numpy(pos).double()[:, :, None] * inv[None, None]
    f = fr[0].clone()
    f[:, 1:3 * sec[1]:3] = fr[1][:, 1:3 * sec[1]:3]
    f[:, 2:3 * sec[2]:3] = fr[2][:, 2:3 * sec[2]:3]
    emb = torch.cat([f, f], -1)
    cos, sin = emb.cos(), emb.sin()

    def rot(a):
        return torch.cat([-a[..., D // 2:], a[..., :D // 2]], -1)
    q = q * cos + rot(q) * sin
    k = k * cos + rot(k) * sin
    bias = torch.zeros(S, S, dtype=torch.float64)
    if ar_len:
        causal = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
        causal[ar_len:] = False
        bias = bias.masked_fill(causal, float("-inf"))
    a = F.scaled_dot_product_attention(q[None], k[None], v[None], attn_mask=bias, enable_gqa=True)[0]
    a = a.transpose(0, 1).reshape(S, H * D)
    ar = xx + a @ t["o_proj"].T
    p = F.rms_norm(ar, (HID,), t["post_ln"], eps)
    m = (F.silu(p @ t["gate_proj"].T) * (p @ t["up_proj"].T)) @ t["down_proj"].T
    return (ar + m).float().numpy()


@pytest.mark.parametrize("ar_len,theta", [(0, 1e4), (23, 5e6)])
def test_block_oracle_vs_torch_layer(ar_len, theta):
    H, KV, HID, FF, D = 4, 2, 256, 512, 128
    T, gh, gw = 24, 6, 7
    S = T + gh * gw
    w = make_block_weights(HID, H, KV, FF, D, seed=3)
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(4)))
    pos = grid_pos(T, gh, gw)
    if ar_len:
        pos[:, :T] = np.arange(T)[None]
    want = torch_block(x, pos, w, H, KV, D, theta, ar_len=ar_len)
    cfg = orc.block_cfg(H, KV, HID, FF, D, theta=theta, faithful=0, ar_len=ar_len)
    got = orc.decoder_block(x.numpy(), pos, {k: v.numpy() for k, v in w.items()}, cfg)
    assert rel_l2(got, want) < 1e-5
    xn = x.numpy()
    assert rel_l2(got - xn, want - xn) < 1e-5
    # the bf16-faithful mode stays inside the north-star bound of the fp32 one
    cfg.faithful = 1
    gf = orc.decoder_block(xn, pos, {k: v.numpy() for k, v in w.items()}, cfg)
    assert rel_l2(gf, want) < 1e-2 and cosine(gf, want) > 0.9999


def test_block_oracle_batch_equals_two_singles():
    H, KV, HID, FF, D = 2, 1, 256, 256, 128
    S = 40
    w = {k: v.numpy() for k, v in make_block_weights(HID, H, KV, FF, D, seed=5).items()}
    x = bf16(torch.randn(2 * S, HID, generator=torch.Generator().manual_seed(6))).numpy()
    pos = grid_pos(4, 6, 6)
    cfg = orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=1)
    both = orc.decoder_block(x, pos, w, cfg, batch=2)
    assert np.array_equal(both[:S], orc.decoder_block(x[:S], pos, w, cfg))
    assert np.array_equal(both[S:], orc.decoder_block(x[S:], pos, w, cfg))

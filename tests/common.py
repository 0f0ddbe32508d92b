"""Shared helpers of the test-suite: seeded synthetic weights (bf16-exact
fp32 on the host), position tables, metrics."""
import numpy as np
import torch

BLOCK_KEYS = ("q_proj", "k_proj", "v_proj", "o_proj", "input_ln", "post_ln", "gate_proj",
              "up_proj", "down_proj", "q_norm", "k_norm")


def bf16(t):
    """Round a float tensor to bf16 values, kept as float32 (torch RNE)."""
    return t.to(torch.bfloat16).float()


def make_block_weights(hidden, heads, kv_heads, ff, head_dim=128, seed=0, std=0.02):
    """Projection weights ~N(0, std); norm gains 1 + N(0, std). bf16 values.
    (A N(0, 0.02) norm gain would make a block an identity map to bf16
    precision and every parity check vacuous.)"""
    g = torch.Generator().manual_seed(seed)
    shapes = {
        "q_proj": (heads * head_dim, hidden), "k_proj": (kv_heads * head_dim, hidden),
        "v_proj": (kv_heads * head_dim, hidden), "o_proj": (hidden, heads * head_dim),
        "gate_proj": (ff, hidden), "up_proj": (ff, hidden), "down_proj": (hidden, ff),
    }
    w = {}
    for k in BLOCK_KEYS:
        if k in shapes:
            w[k] = bf16(torch.randn(*shapes[k], generator=g) * std)
        else:
            n = head_dim if k in ("q_norm", "k_norm") else hidden
            w[k] = bf16(1.0 + torch.randn(n, generator=g) * std)
    return w


def to_dev(t, dev):
    return t.to(dev, torch.bfloat16).contiguous()


def grid_pos(text_len, gh, gw, row_offset=0, fix_point=0):
    """pos [3, S] fp32 for `text_len` text tokens at position 0 followed by a
    gh x gw image grid: (T, H, W) = (fix_point, row + row_offset, col). The
    2D-RoPE layout of the benchmark configurations (text at 0, image rows/cols)."""
    S = text_len + gh * gw
    pos = np.zeros((3, S), np.float32)
    r, c = np.divmod(np.arange(gh * gw), gw)
    pos[0, text_len:] = fix_point
    pos[1, text_len:] = r + row_offset
    pos[2, text_len:] = c
    return pos


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-30))


def close_bf16(got, ref, ulps=2, atol_rel=1e-3):
    """True when every element is within `ulps` bf16 ulps of the reference
    magnitude, plus an absolute floor of atol_rel x RMS(ref) (values near zero
    legitimately differ in sign after fp32 accumulation in another order)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    # one bf16 ulp is at most 2^-7 of the value's magnitude
    tol = ulps * np.abs(ref) * 2.0 ** -7 + atol_rel * rms + 1e-30
    return bool(np.all(np.abs(got - ref) <= tol))


def ulp_diff_bf16(a, b):
    """Max distance in bf16 ulps between two bf16-valued float arrays."""
    ia = np.asarray(a, np.float32).view(np.int32) >> 16
    ib = np.asarray(b, np.float32).view(np.int32) >> 16
    # map sign-magnitude to ordered ints
    ia = np.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFF), ib)
    return int(np.max(np.abs(ia.astype(np.int64) - ib.astype(np.int64)))) if ia.size else 0

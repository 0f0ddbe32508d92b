"""Shared helpers of the test-suite: seeded synthetic weights (bf16-exact
fp32 on the host), position tables, metrics."""
import numpy as np
import torch

VOCAB, TMS = 151936, 151673   # forward.c:274 table rows; the timestep token id

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


class Stepper:
    """One sampler step composed from the library's own calls, as the
    reference's step loops run it (generate.c:855-935, :1314-1455):
    Euler = hd_sched_flow_match_step; flash = host noise from seed + 1
    clipped at `clip` std, then hd_scheduler_step with the ramped s_noise;
    UniPC = the per-step plan and the hd_unipc_* kernels over a three-slot
    history. `step(i, z, m)` updates the bf16 latent z in place from the
    velocity m (fp32, n values)."""

    def __init__(self, pkg, lib, dev, sampler, sch, n, seed, clip=8.0, sn=(8.0, 8.0)):
        import ctypes
        self.pkg, self.lib, self.dev, self.sampler, self.sch, self.n = pkg, lib, dev, sampler, sch, n
        self.clip, self.sn = clip, sn
        self.sig = [sch.sigmas[i] for i in range(sch.num_steps)]
        self.rng = pkg.hd_torch_rng()
        lib.hd_torch_rng_seed(ctypes.byref(self.rng), seed + 1)
        self.fs = pkg.hd_scheduler()
        ctypes.memmove(ctypes.byref(self.fs), ctypes.byref(sch), ctypes.sizeof(sch))
        f = dict(dtype=torch.float32, device=dev)
        self.zf, self.corr_b, self.last, self.pred = (torch.empty(n, **f) for _ in range(4))
        self.slots = [torch.empty(n, **f) for _ in range(3)]
        self.this_order = self.lower = self.have = 0
        self.sscr = torch.empty(3 * n, **f)

    def step(self, i, zr, m):
        import ctypes
        pkg, lib, n, sig = self.pkg, self.lib, self.n, self.sig
        if self.sampler == 0:
            lib.hd_sched_flow_match_step(pkg.ptr(zr), pkg.ptr(m), sig[i], sig[i + 1], pkg.ptr(zr), n)
        elif self.sampler == 1:
            noise = np.empty(n, np.float32)
            lib.hd_step_noise(ctypes.byref(self.rng), pkg.np_ptr(noise), n, self.clip)
            nd = torch.from_numpy(noise).to(self.dev)
            self.fs.step_index = i
            sn = lib.hd_scheduler_noise_scale(ctypes.byref(self.sch), i, self.sn[0], self.sn[1])
            st = lib.hd_scheduler_step(ctypes.byref(self.fs), pkg.ptr(zr), pkg.ptr(m), pkg.ptr(nd), sn,
                                       pkg.ptr(zr), n, pkg.ptr(self.sscr))
            pkg.check_status(st, "scheduler step")
        else:
            pl = pkg.hd_unipc_plan()
            lib.hd_scheduler_unipc_plan(ctypes.byref(self.sch), i, self.this_order, self.lower,
                                        ctypes.byref(pl))
            lib.hd_sched_bf16_upcast(pkg.ptr(zr), pkg.ptr(self.zf), n)
            slots = self.slots
            cur = slots[0]
            lib.hd_unipc_convert(pkg.ptr(self.zf), pkg.ptr(m), sig[i], pkg.ptr(cur), n)
            corr = self.zf
            if i > 0 and self.this_order > 0 and self.have:
                lib.hd_unipc_correct(pkg.ptr(self.last), pkg.ptr(slots[1]), pkg.ptr(slots[2]), pkg.ptr(cur),
                                     pl.c_sig_t, pl.c_sig_s0, pl.c_alpha_t, pl.c_h_phi_1, pl.c_B_h,
                                     pl.c_rhos0, pl.c_rhos1, pl.c_inv_rks0, pl.corr_order,
                                     pkg.ptr(self.corr_b), n)
                corr = self.corr_b
            self.last.copy_(corr)
            lib.hd_unipc_predict(pkg.ptr(corr), pkg.ptr(cur), pkg.ptr(slots[1]), pl.p_sig_t, pl.p_sig_s0,
                                 pl.p_alpha_t, pl.p_h_phi_1, pl.p_B_h, pl.p_rhos_p, pl.p_inv_rks0,
                                 pl.pred_order, pkg.ptr(self.pred), n)
            lib.hd_f32_convert_bf16(pkg.ptr(self.pred), pkg.ptr(zr), n)
            self.slots = [slots[2], slots[0], slots[1]]
            self.this_order, self.lower, self.have = pl.next_this_order, pl.next_lower_order, 1
        pkg.check_prim("step %d" % i)


def make_forward_weights(n_layers, HID, H, KV, FF, D, seed, vocab=None):
    """Global weights of the denoiser (token table of `vocab` rows, t-embedder,
    x_embedder, final norm and head) plus `n_layers` block weight sets."""
    g = torch.Generator().manual_seed(seed)

    def r(*shape, std=0.02):
        return bf16(torch.randn(*shape, generator=g) * std)
    fw = {
        "embed_tokens": r(vocab or VOCAB, HID, std=1.0),
        "te0_w": r(HID, 256), "te0_b": r(HID), "te2_w": r(HID, HID), "te2_b": r(HID),
        "xe1_w": r(1024, 3072), "xe2_w": r(HID, 1024, std=0.05), "xe2_b": r(HID),
        "fl_w": r(3072, HID), "fl_b": r(3072), "fnorm_w": bf16(1 + torch.randn(HID, generator=g) * 0.02),
        "blocks": [make_block_weights(HID, H, KV, FF, D, seed=seed + 1 + i) for i in range(n_layers)],
    }
    return fw

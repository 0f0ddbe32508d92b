"""numpy bindings of liboracle.so - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker / CPU baseline; the product
path (libo1hip) never calls it.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F = ctypes.POINTER(ctypes.c_float)
I64 = ctypes.POINTER(ctypes.c_int64)
c_int, c_float, c_size_t, c_int64 = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_int64


class BlockWeights(ctypes.Structure):
    _fields_ = [(n, F) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "input_ln", "post_ln",
                                 "gate_proj", "up_proj", "down_proj", "q_norm", "k_norm")]


class BlockCfg(ctypes.Structure):
    _fields_ = [("heads", c_int), ("kv_heads", c_int), ("hidden", c_int), ("ff", c_int),
                ("head_dim", c_int), ("eps", c_float), ("theta", c_float),
                ("attention_scaling", c_float), ("section", c_int64 * 3), ("interleaved", c_int),
                ("ar_len", c_int), ("faithful", c_int), ("prob_mode", c_int)]


class ForwardWeights(ctypes.Structure):
    _fields_ = [("embed_tokens", F), ("vocab", c_int64), ("te0_w", F), ("te0_b", F),
                ("te2_w", F), ("te2_b", F), ("xe1_w", F), ("xe2_w", F), ("xe2_b", F),
                ("fl_w", F), ("fl_b", F), ("fnorm_w", F), ("n_layers", c_int),
                ("blocks", ctypes.POINTER(BlockWeights))]


class VisionBlock(ctypes.Structure):
    _fields_ = [(n, F) for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "qkv_w", "qkv_b",
                                 "proj_w", "proj_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class VisionMerger(ctypes.Structure):
    _fields_ = [(n, F) for n in ("norm_w", "norm_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class VisionWeights(ctypes.Structure):
    _fields_ = [("patch_w", F), ("patch_b", F), ("pos_embed", F),
                ("blocks", ctypes.POINTER(VisionBlock)), ("merger", VisionMerger),
                ("deepstack", VisionMerger * 4)]


class VisionCfg(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("depth", "hidden", "heads", "inter", "out_hidden",
                                     "patch_dim", "nside", "merge", "n_ds")] + \
               [("ds_layers", c_int * 4), ("faithful", c_int)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("liboracle.so missing: run make -C oracle")
        _lib = ctypes.CDLL(LIB_PATH)
        L = _lib
        L.o1o_bf16_round.restype = c_float
        L.o1o_bf16_round.argtypes = [c_float]
        L.o1o_num_threads.restype = c_int
        L.o1o_set_threads.argtypes = [c_int]
        L.o1o_linear.argtypes = [F, F, F, F, c_int, c_int, c_int, c_int]
        L.o1o_rmsnorm.argtypes = [F, F, F, c_int, c_int, c_float, c_int]
        L.o1o_silu.argtypes = [F, F, c_size_t, c_int]
        L.o1o_swiglu.argtypes = [F, F, F, c_size_t, c_int]
        L.o1o_residual_add.argtypes = [F, F, F, c_size_t, c_int]
        L.o1o_mrope_cos_sin.argtypes = [F, c_int, I64, c_int, c_int, c_float, c_float, c_int, F, F]
        L.o1o_apply_rotary.argtypes = [F, F, F, F, c_int, c_int, c_int, c_int]
        L.o1o_attention.argtypes = [F, F, F, F, c_int, c_int, c_int, c_int, c_int, c_float, c_int,
                                    c_int, F]
        L.o1o_timestep_embed.argtypes = [F, F, c_int, c_int]
        L.o1o_decoder_block.restype = c_int
        L.o1o_decoder_block.argtypes = [F, F, F, ctypes.POINTER(BlockWeights),
                                        ctypes.POINTER(BlockCfg), c_int, c_int, F, F, F, F]
        L.o1o_forward.restype = c_int
        L.o1o_forward.argtypes = [ctypes.POINTER(ForwardWeights), ctypes.POINTER(BlockCfg), I64,
                                  c_int, F, c_int, c_float, F, F, c_int64, F, F]
        L.o1o_forward_visual.restype = c_int
        L.o1o_forward_visual.argtypes = [ctypes.POINTER(ForwardWeights), ctypes.POINTER(BlockCfg),
                                         I64, c_int, F, c_int, c_float, F, F, c_int64, F,
                                         ctypes.POINTER(F), ctypes.POINTER(ctypes.c_uint8), F, F]
        L.o1o_lora_merge.argtypes = [F, F, F, c_int, c_int, c_int, c_float]
        L.o1o_sched_vcond.argtypes = [F, F, c_float, F, c_int]
        L.o1o_sched_flow_match_step.argtypes = [F, F, c_float, c_float, F, c_int]
        L.o1o_sched_cfg_guided.argtypes = [F, F, c_float, F, c_int]
        L.o1o_unipc_convert.argtypes = [F, F, c_float, F, c_int]
        L.o1o_unipc_correct.argtypes = [F, F, F, F] + [c_float] * 8 + [c_int, F, c_int]
        L.o1o_unipc_predict.argtypes = [F, F, F] + [c_float] * 7 + [c_int, F, c_int]
        L.o1o_patchify.argtypes = [F, F, c_int, c_int, c_int, c_int]
        L.o1o_unpatchify.argtypes = [F, F, c_int, c_int, c_int, c_int]
        L.o1o_layernorm.argtypes = [F, F, F, F, c_int, c_int, c_float, c_int]
        L.o1o_gelu_tanh.argtypes = [F, F, c_size_t, c_int]
        L.o1o_gelu_erf.argtypes = [F, F, c_size_t, c_int]
        IP = ctypes.POINTER(c_int)
        L.o1o_vision_tables.argtypes = [c_int, c_int, c_int, c_int, IP, F, IP]
        L.o1o_vision_rotary.argtypes = [IP, c_int, c_int, c_int, F, F]
        L.o1o_vision_forward.restype = c_int
        L.o1o_vision_forward.argtypes = [ctypes.POINTER(VisionWeights), ctypes.POINTER(VisionCfg), F,
                                         c_int, c_int, F, ctypes.POINTER(F), F]
        L.o1o_decode_to_rgb.argtypes = [F, c_int, c_int, c_int, c_int,
                                        ctypes.POINTER(ctypes.c_uint8)]
    return _lib


def fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(F)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def bf16_round(a):
    """numpy RNE to bf16, kept in fp32 (support.cu:21-28 rule)."""
    u = f32(a).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def linear(x, w, bias=None, mode=1):
    x, w = f32(x), f32(w)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().o1o_linear(fp(x), fp(w), fp(None if bias is None else f32(bias)), fp(y), M, N, K, mode)
    return y


def rmsnorm(x, w, eps=1e-6, round_=1):
    x = f32(x)
    y = np.empty_like(x)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    lib().o1o_rmsnorm(fp(x), fp(f32(w)), fp(y), rows, cols, eps, round_)
    return y


def swiglu(g, u, round_=1):
    g, u = f32(g), f32(u)
    y = np.empty_like(g)
    lib().o1o_swiglu(fp(g), fp(u), fp(y), g.size, round_)
    return y


def silu(x, round_=1):
    x = f32(x)
    y = np.empty_like(x)
    lib().o1o_silu(fp(x), fp(y), x.size, round_)
    return y


def residual_add(x, a, round_=1):
    x, a = f32(x), f32(a)
    y = np.empty_like(x)
    lib().o1o_residual_add(fp(x), fp(a), fp(y), x.size, round_)
    return y


def mrope_cos_sin(pos, seq, dim, theta, section=(24, 20, 20), interleaved=1, scaling=1.0):
    pos = f32(pos)
    c = np.empty((seq, dim), np.float32)
    s = np.empty((seq, dim), np.float32)
    sec = (c_int64 * 3)(*section)
    lib().o1o_mrope_cos_sin(fp(pos), seq, sec, 3, dim, theta, scaling, interleaved, fp(c), fp(s))
    return c, s


def apply_rotary(x, c, s, per_op=1):
    x = f32(x)
    heads, seq, dim = x.shape
    y = np.empty_like(x)
    lib().o1o_apply_rotary(fp(x), fp(f32(c)), fp(f32(s)), fp(y), heads, seq, dim, per_op)
    return y


def attention(q, k, v, mask=None, ar_len=0, scale=None, prob_mode=0, round_=1):
    q, k, v = f32(q), f32(k), f32(v)
    Hq, S, D = q.shape
    Hkv = k.shape[0]
    scale = D ** -0.5 if scale is None else scale
    out = np.empty((S, Hq * D), np.float32)
    lib().o1o_attention(fp(q), fp(k), fp(v), fp(None if mask is None else f32(mask)), Hq, Hkv, S,
                        D, ar_len, scale, prob_mode, round_, fp(out))
    return out


def timestep_embed(t, dim):
    t = f32(np.atleast_1d(t))
    y = np.empty((t.size, dim), np.float32)
    lib().o1o_timestep_embed(fp(t), fp(y), t.size, dim)
    return y


BLOCK_KEYS = ("q_proj", "k_proj", "v_proj", "o_proj", "input_ln", "post_ln", "gate_proj",
              "up_proj", "down_proj", "q_norm", "k_norm")


def block_weights(w):
    """dict of float32 arrays -> (BlockWeights, keepalive list)."""
    keep = [f32(w[k]) for k in BLOCK_KEYS]
    bw = BlockWeights(*[fp(a) for a in keep])
    return bw, keep


def block_cfg(heads, kv_heads, hidden, ff, head_dim=128, eps=1e-6, theta=5e6,
              section=(24, 20, 20), interleaved=1, ar_len=0, faithful=1, prob_mode=0,
              attention_scaling=1.0):
    c = BlockCfg()
    c.heads, c.kv_heads, c.hidden, c.ff, c.head_dim = heads, kv_heads, hidden, ff, head_dim
    c.eps, c.theta, c.attention_scaling = eps, theta, attention_scaling
    for i in range(3):
        c.section[i] = section[i]
    c.interleaved, c.ar_len, c.faithful, c.prob_mode = interleaved, ar_len, faithful, prob_mode
    return c


def decoder_block(x, pos, w, cfg, batch=1, mask=None, internals=False):
    x = f32(x)
    M, HID = x.shape
    seq = M // batch
    bw, keep = block_weights(w)
    out = np.empty_like(x)
    ints = [np.empty_like(x) for _ in range(3)] if internals else [None] * 3
    rc = lib().o1o_decoder_block(fp(x), fp(f32(pos)), fp(None if mask is None else f32(mask)),
                                 ctypes.byref(bw), ctypes.byref(cfg), batch, seq, fp(out),
                                 *[fp(a) for a in ints])
    assert rc == 0
    return (out, *ints) if internals else out


def forward(fw, cfg, ids, vin, t, pos, tms_id, mask=None, keep_blocks=False, visual=None):
    """fw: dict of global arrays + 'blocks' list of per-layer dicts.
    visual: optional (image_embeds [V,hidden], [deepstack0..2 or None], vmask [S] uint8)."""
    keep = []
    blocks = (BlockWeights * len(fw["blocks"]))()
    for i, bwd in enumerate(fw["blocks"]):
        b, k = block_weights(bwd)
        blocks[i] = b
        keep.append(k)
    g = {k: f32(fw[k]) for k in ("embed_tokens", "te0_w", "te0_b", "te2_w", "te2_b", "xe1_w",
                                 "xe2_w", "xe2_b", "fl_w", "fl_b", "fnorm_w")}
    W = ForwardWeights(fp(g["embed_tokens"]), g["embed_tokens"].shape[0], fp(g["te0_w"]),
                       fp(g["te0_b"]), fp(g["te2_w"]), fp(g["te2_b"]), fp(g["xe1_w"]),
                       fp(g["xe2_w"]), fp(g["xe2_b"]), fp(g["fl_w"]), fp(g["fl_b"]),
                       fp(g["fnorm_w"]), len(fw["blocks"]), blocks)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    vin = f32(vin)
    T, I = ids.size, vin.shape[0]
    S = T + I
    out = np.empty((S, 3072), np.float32)
    ab = np.empty((len(fw["blocks"]), S, cfg.hidden), np.float32) if keep_blocks else None
    if visual is None:
        rc = lib().o1o_forward(ctypes.byref(W), ctypes.byref(cfg),
                               ids.ctypes.data_as(I64), T, fp(vin), I, float(t), fp(f32(pos)),
                               fp(None if mask is None else f32(mask)), tms_id, fp(out), fp(ab))
    else:
        emb = f32(visual[0])
        ds = [None if d is None else f32(d) for d in visual[1]] + [None] * (3 - len(visual[1]))
        dsp = (F * 3)(*[fp(d) for d in ds])
        vm = np.ascontiguousarray(visual[2], dtype=np.uint8)
        keep.append((emb, ds, vm))
        rc = lib().o1o_forward_visual(ctypes.byref(W), ctypes.byref(cfg),
                                      ids.ctypes.data_as(I64), T, fp(vin), I, float(t),
                                      fp(f32(pos)), fp(None if mask is None else f32(mask)),
                                      tms_id, fp(emb), dsp,
                                      vm.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), fp(out),
                                      fp(ab))
    assert rc == 0
    return (out, ab) if keep_blocks else out


def lora_merge(w, up, down, scale):
    w = f32(w).copy()
    N, K = w.shape
    R = up.shape[1]
    lib().o1o_lora_merge(fp(w), fp(f32(up)), fp(f32(down)), N, K, R, scale)
    return w


def patchify(img, p):
    img = f32(img)
    C, Hh, W = img.shape
    Hp, Wp = Hh // p, W // p
    tok = np.empty((Hp * Wp, C * p * p), np.float32)
    lib().o1o_patchify(fp(img), fp(tok), C, Hp, Wp, p)
    return tok


def unpatchify(tok, C, Hp, Wp, p):
    tok = f32(tok)
    img = np.empty((C, Hp * p, Wp * p), np.float32)
    lib().o1o_unpatchify(fp(tok), fp(img), C, Hp, Wp, p)
    return img


def decode_to_rgb(z, grid_h, grid_w, patch, channels=3):
    z = f32(z)
    out = np.empty((grid_h * patch, grid_w * patch, channels), np.uint8)
    lib().o1o_decode_to_rgb(fp(z), grid_h, grid_w, patch, channels,
                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    return out


def sched_vcond(z, xp, sigma):
    z, xp = f32(z), f32(xp)
    mo = np.empty_like(z)
    lib().o1o_sched_vcond(fp(z), fp(xp), sigma, fp(mo), z.size)
    return mo


def sched_flow_match_step(z, mo, sigma, sigma_next):
    z, mo = f32(z), f32(mo)
    zn = np.empty_like(z)
    lib().o1o_sched_flow_match_step(fp(z), fp(mo), sigma, sigma_next, fp(zn), z.size)
    return zn


def unipc_convert(smp, mo, sigma):
    smp, mo = f32(smp), f32(mo)
    o = np.empty_like(smp)
    lib().o1o_unipc_convert(fp(smp), fp(mo), sigma, fp(o), smp.size)
    return o


def unipc_correct(last, mo0, mo_old, conv, sig_t, sig_s0, alpha_t, h_phi_1, B_h, rc0, rc1, inv_rk,
                  order):
    last, mo0, mo_old, conv = f32(last), f32(mo0), f32(mo_old), f32(conv)
    o = np.empty_like(last)
    lib().o1o_unipc_correct(fp(last), fp(mo0), fp(mo_old), fp(conv), sig_t, sig_s0, alpha_t, h_phi_1,
                            B_h, rc0, rc1, inv_rk, order, fp(o), last.size)
    return o


def unipc_predict(smp, mo0, mo_old, sig_t, sig_s0, alpha_t, h_phi_1, B_h, rp, inv_rk, order):
    smp, mo0, mo_old = f32(smp), f32(mo0), f32(mo_old)
    o = np.empty_like(smp)
    lib().o1o_unipc_predict(fp(smp), fp(mo0), fp(mo_old), sig_t, sig_s0, alpha_t, h_phi_1, B_h, rp,
                            inv_rk, order, fp(o), smp.size)
    return o


def sched_cfg_guided(c, u, g):
    c, u = f32(c), f32(u)
    o = np.empty_like(c)
    lib().o1o_sched_cfg_guided(fp(c), fp(u), g, fp(o), c.size)
    return o


# ---- vision tower (o1_vision.c) -------------------------------------------
VISION_BLOCK_KEYS = ("norm1.weight", "norm1.bias", "norm2.weight", "norm2.bias", "attn.qkv.weight",
                     "attn.qkv.bias", "attn.proj.weight", "attn.proj.bias",
                     "mlp.linear_fc1.weight", "mlp.linear_fc1.bias", "mlp.linear_fc2.weight",
                     "mlp.linear_fc2.bias")
VISION_MERGER_KEYS = ("norm.weight", "norm.bias", "linear_fc1.weight", "linear_fc1.bias",
                      "linear_fc2.weight", "linear_fc2.bias")


def layernorm(x, w, b, eps=1e-6, round_=1):
    x = f32(x)
    y = np.empty_like(x)
    lib().o1o_layernorm(fp(x), fp(f32(w)), fp(f32(b)) if b is not None else None, fp(y),
                        x.shape[0], x.shape[1], eps, round_)
    return y


def gelu_tanh(x, round_=1):
    x = f32(x)
    y = np.empty_like(x)
    lib().o1o_gelu_tanh(fp(x), fp(y), x.size, round_)
    return y


def gelu_erf(x, round_=1):
    x = f32(x)
    y = np.empty_like(x)
    lib().o1o_gelu_erf(fp(x), fp(y), x.size, round_)
    return y


def vision_tables(gh, gw, nside, merge=2):
    n = gh * gw
    idx = np.empty((4, n), np.int32)
    wgt = np.empty((4, n), np.float32)
    co = np.empty((2, n), np.int32)
    IP = ctypes.POINTER(c_int)
    lib().o1o_vision_tables(gh, gw, nside, merge, idx.ctypes.data_as(IP), fp(wgt),
                            co.ctypes.data_as(IP))
    return idx, wgt, co


def vision_forward(w, pixels, gh, gw, depth, heads, ds_layers, faithful=1, merge=2,
                   keep_blocks=False):
    """w: dict of the vision tower's tensors under their checkpoint names
    without the 'model.visual.' prefix (patch_embed.proj.weight as
    [hidden, patch_dim]). Returns (embeds, [deepstack...]) and, with
    keep_blocks, the [depth, n, hidden] block outputs."""
    keep = []

    def a(name):
        arr = f32(w[name])
        keep.append(arr)
        return fp(arr)

    blocks = (VisionBlock * depth)()
    for i in range(depth):
        blocks[i] = VisionBlock(*[a(f"blocks.{i}.{k}") for k in VISION_BLOCK_KEYS])
    vw = VisionWeights()
    vw.patch_w, vw.patch_b, vw.pos_embed = (a("patch_embed.proj.weight"), a("patch_embed.proj.bias"),
                                            a("pos_embed.weight"))
    vw.blocks = ctypes.cast(blocks, ctypes.POINTER(VisionBlock))
    vw.merger = VisionMerger(*[a(f"merger.{k}") for k in VISION_MERGER_KEYS])
    for j in range(len(ds_layers)):
        vw.deepstack[j] = VisionMerger(*[a(f"deepstack_merger_list.{j}.{k}") for k in VISION_MERGER_KEYS])
    H = w["patch_embed.proj.weight"].shape[0]
    c = VisionCfg()
    c.depth, c.hidden, c.heads = depth, H, heads
    c.inter = w["blocks.0.mlp.linear_fc1.weight"].shape[0]
    c.out_hidden = w["merger.linear_fc2.weight"].shape[0]
    c.patch_dim = w["patch_embed.proj.weight"].shape[1]
    c.nside = int(round(w["pos_embed.weight"].shape[0] ** 0.5))
    c.merge, c.n_ds, c.faithful = merge, len(ds_layers), faithful
    for j, L in enumerate(ds_layers):
        c.ds_layers[j] = L
    m = gh * gw // (merge * merge)
    emb = np.empty((m, c.out_hidden), np.float32)
    ds = [np.empty((m, c.out_hidden), np.float32) for _ in ds_layers]
    dsp = (F * max(1, len(ds)))(*[fp(d) for d in ds])
    px = f32(pixels)
    ab = np.empty((depth, gh * gw, H), np.float32) if keep_blocks else None
    rc = lib().o1o_vision_forward(ctypes.byref(vw), ctypes.byref(c), fp(px), gh, gw, fp(emb),
                                  dsp if ds else None, fp(ab))
    assert rc == 0
    return (emb, ds, ab) if keep_blocks else (emb, ds)

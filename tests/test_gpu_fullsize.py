"""Full-size parity for configuration 2's dominant kernels (S = 16640), each
through the launch the decoder block makes (tail-split workspace), against a
plain torch fp32 reference of the same op on the GPU (reference semantics:
attn.cu:22-127 for attention, gemm.cu:506 + act.cu:22-34 + residual.cu:14-23
for the GEMMs). Bound: the north-star rel-L2 <= 1e-2 / cosine >= 0.9999 per
checked slice; sampled heads / rows keep the fp32 reference small."""
import numpy as np
import pytest
import torch

from tests.common import rel_l2, cosine

pytestmark = pytest.mark.gpu


def check(got, ref, tag, rel=1e-2, cos=0.9999):
    r, c = rel_l2(got, ref), cosine(got, ref)
    print(f"{tag}: rel_l2={r:.3e} cos={c:.7f}", flush=True)
    assert r <= rel and c >= cos, (tag, r, c)


def test_flash_config2_full_size(pkg, lib, dev):
    """32 query heads / 8 kv heads, D = 128, S = 16640 (65 query tiles of
    256 per head: 2080 units over 256 slots, the last partial round split
    8 ways), checked on 4 query heads against fp32 softmax(QK^T / sqrt(D)) V."""
    B, Hq, Hkv, S, D = 1, 32, 8, 16640, 128
    print(f"flash full size S={S}", flush=True)
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(B, Hq, S, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B * Hkv, S, D, generator=g, device=dev).to(torch.bfloat16)
    vt = torch.empty(lib.hd_flash_vt_bytes(B, Hkv, S) // 2, dtype=torch.bfloat16, device=dev)
    lib.hd_flash_make_vt(pkg.ptr(v), pkg.ptr(vt), B * Hkv, S)
    ws = torch.empty(lib.hd_flash_ws_bytes(), dtype=torch.uint8, device=dev)
    out = torch.empty(B, S, Hq * D, dtype=torch.bfloat16, device=dev)
    assert lib.hd_flash_attention_ws(pkg.ptr(q), pkg.ptr(k), pkg.ptr(vt), None, pkg.ptr(out), B, Hq, Hkv, S, D,
                                     0, D ** -0.5, 1, pkg.ptr(ws), ws.numel()) == 0
    torch.cuda.synchronize()
    o = out.view(S, Hq, D)
    for h in (0, 5, 18, 31):           # kv heads 0, 1, 4, 7; the last units are the split ones
        qh, kh, vh = q[0, h].float(), k[0, h // 4].float(), v[h // 4].float()
        ref = torch.empty(S, D, device=dev)
        for r0 in range(0, S, 4160):   # score blocks of 4160 x 16640 fp32
            p = torch.softmax(qh[r0:r0 + 4160] @ kh.t() * D ** -0.5, dim=-1)
            ref[r0:r0 + 4160] = p @ vh
        check(o[:, h].float().cpu().numpy(), ref.cpu().numpy(), f"flash head {h}")


def test_gemms_config2_full_size(pkg, lib, dev):
    """M = 16640: the gate/up + SwiGLU GEMM (65 x 96 tiles, 24 rounds + a
    split tail) and the down projection with its residual (K = 12288, 65 x
    16 tiles, a split tail), checked on rows from every 256-row tile band
    (whole and split tiles) against fp32 matmuls with the reference's bf16
    rounding points."""
    M, H, F = 16640, 4096, 12288
    print(f"gemms full size M={M}", flush=True)
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(M, H, generator=g, device=dev).to(torch.bfloat16)
    wg = (torch.randn(F, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(F, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(H, F, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    res = torch.randn(M, H, generator=g, device=dev).to(torch.bfloat16)
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    sw = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    lib.hd_linear_swiglu_ws(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(sw), M, F, H, pkg.ptr(ws), ws.numel())
    y = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    lib.hd_linear_residual_ws(pkg.ptr(sw), pkg.ptr(wd), pkg.ptr(res), pkg.ptr(y), M, H, F, pkg.ptr(ws), ws.numel())
    pkg.check_prim("full-size gemms")
    torch.cuda.synchronize()
    rows = torch.from_numpy(np.concatenate([np.arange(b, min(b + 256, M), 37) for b in range(0, M, 256)])).to(dev)
    xs = x[rows].float()
    gt = (xs @ wg.float().t()).to(torch.bfloat16).float()
    up = (xs @ wu.float().t()).to(torch.bfloat16).float()
    s_ref = ((gt * torch.sigmoid(gt)).to(torch.bfloat16).float() * up).to(torch.bfloat16)
    check(sw[rows].float().cpu().numpy(), s_ref.float().cpu().numpy(), "swiglu gemm")
    # down projection on the kernel's own SwiGLU rows (isolates the GEMM)
    d_ref = (sw[rows].float() @ wd.float().t()).to(torch.bfloat16).float() + res[rows].float()
    check(y[rows].float().cpu().numpy(), d_ref.to(torch.bfloat16).float().cpu().numpy(), "down + residual")


# ---- whole blocks and a full-width step at the benchmark configurations ----
from oracle import oracle as orc                       # noqa: E402
from tests.common import (make_block_weights, make_forward_weights, grid_pos, bf16,  # noqa: E402
                          TMS)

H_, KV_, HID_, FF_, D_ = 32, 8, 4096, 12288, 128


def multi_grid_pos(T, gh, gw, refs):
    """Text at 0, the target grid, then `refs` reference grids of the same
    size with a +64 row offset per reference (the edit configuration)."""
    parts = [grid_pos(T, gh, gw)] + [grid_pos(0, gh, gw, row_offset=64 * r) for r in range(1, refs + 1)]
    return np.ascontiguousarray(np.concatenate(parts, 1))


def block_full(pkg, lib, dev, S, pos, seed, tag):
    import ctypes  # noqa: F401
    w = make_block_weights(HID_, H_, KV_, FF_, D_, seed=seed)
    x = bf16(torch.randn(S, HID_, generator=torch.Generator().manual_seed(seed + 1)))
    pkg.set_block_config(theta=1e4)
    wd = {k: v.to(dev, torch.bfloat16).contiguous() for k, v in w.items()}
    bind = pkg.binding_from(wd)
    xd = x.to(dev, torch.bfloat16)
    out = torch.empty_like(xd)
    posd = torch.from_numpy(pos).to(dev)
    cs = pkg.rope_table(posd, S, D_, theta=1e4)
    nbytes = lib.hd_decoder_block_batched_scratch_bytes(1, S, H_, KV_, HID_, FF_, D_)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    print(f"{tag}: block S={S}", flush=True)
    st = lib.hd_decoder_block_batched(pkg.ptr(xd), pkg.ptr(cs), None, 0, bind, pkg.ptr(scratch), nbytes,
                                      None, pkg.ptr(out), 1, S, H_, KV_, HID_, FF_, D_)
    pkg.check_status(st, tag)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    del wd, bind, xd, out, scratch
    cfg = orc.block_cfg(H_, KV_, HID_, FF_, D_, theta=1e4, faithful=0)
    ref = orc.decoder_block(x.numpy(), pos, {k: v.numpy() for k, v in w.items()}, cfg)
    check(got, ref, f"{tag} vs fp32 oracle")
    xn = x.numpy()
    r = rel_l2(got - xn, ref - xn)
    print(f"{tag}: residual update rel_l2={r:.3e} (vs fp32)", flush=True)
    # the image rows and the text rows each hold the bound on their own
    check(got[256:], ref[256:], f"{tag} image rows")
    # the residual update (block output - input) against the bf16-faithful
    # oracle (the reference's rounding points), at the bound the S = 1152
    # and S = 4352 blocks hold in test_gpu_block.py
    cfgf = orc.block_cfg(H_, KV_, HID_, FF_, D_, theta=1e4, faithful=1)
    reff = orc.decoder_block(xn, pos, {k: v.numpy() for k, v in w.items()}, cfgf)
    check(got, reff, f"{tag} vs bf16-faithful oracle", rel=5e-3, cos=0.99995)
    rd = rel_l2(got - xn, reff - xn)
    print(f"{tag}: residual update rel_l2={rd:.3e} (vs bf16-faithful)", flush=True)
    assert rd <= 3e-2, (tag, rd)


@pytest.mark.timeout(400)
def test_block_config2_full_size(pkg, lib, dev):
    """Configuration 2's block: 128x128 image tokens + 256 text = 16640 rows,
    hidden 4096, 32/8 heads, FFN 12288, through the production launches
    (fused QKV epilogue with q/k norm + rotary + V^T, 8-wave flash with the
    split tail, SwiGLU and residual GEMMs with split tails) against the fp32
    oracle of block.c:137-386."""
    block_full(pkg, lib, dev, 16640, grid_pos(256, 128, 128), 30, "config2")


@pytest.mark.timeout(400)
def test_block_config3_full_size(pkg, lib, dev):
    """Configuration 3's block: 512 text + a 64x64 target + 3 references of
    64x64 at +64 rows each = 16896 rows, full bidirectional attention."""
    block_full(pkg, lib, dev, 16896, multi_grid_pos(512, 64, 64, 3), 40, "config3")


@pytest.mark.timeout(400)
def test_forward_config1_full_width(pkg, lib, dev):
    """Configuration 1's step at full width with 2 of its 36 layers: batch 2
    (CFG) x (256 text + 64x64 image) tokens through hd_forward_batched
    (t-embedder, token table of 151936 rows with the timestep token,
    x_embedder, blocks, final norm and head) against the oracle's forward of
    each sequence (forward.c:253-397). The two sequences differ in ids,
    latents and timestep."""
    import ctypes
    from tests.test_gpu_forward import store_names
    nL, T, gh, gw, B = 2, 256, 64, 64, 2
    I = gh * gw
    S = T + I
    fw = make_forward_weights(nL, HID_, H_, KV_, FF_, D_, seed=50)
    rng = np.random.default_rng(51)
    ids = rng.integers(0, 151643, (B, T)).astype(np.int64)
    ids[:, -1] = TMS
    ids[1, 7] = -3                   # padding row 0
    vin = bf16(torch.from_numpy(rng.standard_normal((B, I, 3072)).astype(np.float32))).numpy()
    ts = np.array([0.5, 0.25], np.float32)
    pos = grid_pos(T, gh, gw)
    pkg.set_block_config(theta=1e4)
    tens = {k: v.to(dev, torch.bfloat16) for k, v in store_names(fw).items()}
    store = pkg.WeightStore(tens)
    fb = pkg.hd_forward_binding()
    pkg.check_status(lib.hd_forward_resolve(ctypes.byref(store.store), nL, ctypes.byref(fb)), "resolve")
    wsb = lib.hd_forward_batched_workspace_bytes(B, S, I, H_, KV_, HID_, FF_, D_)
    wsbuf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    idsd = torch.from_numpy(ids).to(dev)
    vind = torch.from_numpy(vin).to(dev, torch.bfloat16)
    tsd = torch.from_numpy(ts).to(dev)
    posd = torch.from_numpy(pos).to(dev)
    out = torch.empty(B, S, 3072, dtype=torch.bfloat16, device=dev)
    print(f"config1 forward B={B} S={S} layers={nL}", flush=True)
    st = lib.hd_forward_batched(ctypes.byref(fb), ctypes.byref(ws), B, pkg.ptr(idsd), T, pkg.ptr(posd), 0,
                                pkg.ptr(vind), I, pkg.ptr(tsd), S, H_, KV_, HID_, FF_, D_, TMS, None,
                                pkg.ptr(out), None)
    pkg.check_status(st, "forward_batched config1")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    del tens, store, wsbuf, out
    ofw = {k: v.numpy() for k, v in fw.items() if k != "blocks"}
    ofw["blocks"] = [{k: v.numpy() for k, v in b.items()} for b in fw["blocks"]]
    cfg = orc.block_cfg(H_, KV_, HID_, FF_, D_, theta=1e4, faithful=0)
    for b in range(B):
        ref = orc.forward(ofw, cfg, ids[b], vin[b], float(ts[b]), pos, TMS)
        check(got[b], ref, f"config1 step seq {b}")

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


def check(got, ref, tag):
    r, c = rel_l2(got, ref), cosine(got, ref)
    print(f"{tag}: rel_l2={r:.3e} cos={c:.7f}", flush=True)
    assert r <= 1e-2 and c >= 0.9999, (tag, r, c)


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

"""GEMM parity: MFMA kernels through the C-ABI vs a torch fp32 reference of
the same op (x.float() @ w.float().T, one bf16 rounding) and vs the
reference's known-answer tests (test_gemm_smoke.c:15-20)."""
import pytest
import torch

from tests.common import rel_l2, cosine, ulp_diff_bf16, close_bf16

pytestmark = pytest.mark.gpu


def rnd(shape, g, std=1.0):
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


SHAPES = [(1152, 6144, 4096), (300, 1024, 512), (1, 4096, 256), (7, 512, 1024), (513, 3072, 1024),
          (2048, 4096, 12288)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_linear_matches_fp32(pkg, lib, dev, M, N, K):
    g = torch.Generator().manual_seed(M * 7 + N)
    x = rnd((M, K), g).to(dev)
    w = rnd((N, K), g, 0.02).to(dev)
    y = pkg.linear(x, w)
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    got = y.float()
    assert rel_l2(got.cpu(), ref.cpu()) < 4e-3
    assert cosine(got.cpu(), ref.cpu()) > 0.99999
    # fp32 accumulation in another order: at most a couple of bf16 ulps apart
    assert close_bf16(got.cpu().numpy(), ref.cpu().numpy(), ulps=2)


def test_linear_bias_two_roundings(pkg, lib, dev):
    g = torch.Generator().manual_seed(3)
    M, N, K = 130, 1024, 256
    x, w, b = rnd((M, K), g).to(dev), rnd((N, K), g, 0.05).to(dev), rnd((N,), g).to(dev)
    y = pkg.linear(x, w, b)
    torch.cuda.synchronize()
    acc = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    ref = (acc + b.float()).to(torch.bfloat16).float()   # gemm.cu:226-235
    assert close_bf16(y.float().cpu().numpy(), ref.cpu().numpy(), ulps=2)
    assert rel_l2(y.float().cpu(), ref.cpu()) < 4e-3


def test_gemm_smoke_kat(pkg, lib, dev):
    # test_gemm_smoke.c:15-20: X=[[1,2],[3,4]], W=[[5,6],[7,8]] -> [[17,23],[39,53]]
    x = torch.tensor([[1., 2.], [3., 4.]], dtype=torch.bfloat16, device=dev)
    w = torch.tensor([[5., 6.], [7., 8.]], dtype=torch.bfloat16, device=dev)
    y = pkg.linear(x, w)
    torch.cuda.synchronize()
    assert y.float().cpu().tolist() == [[17., 23.], [39., 53.]]
    # the same KAT through the MFMA path: zero-pad K to 64, N to 256
    xp = torch.zeros(2, 64, dtype=torch.bfloat16, device=dev)
    wp = torch.zeros(256, 64, dtype=torch.bfloat16, device=dev)
    xp[:, :2] = x
    wp[:2, :2] = w
    y = pkg.linear(xp, wp)
    torch.cuda.synchronize()
    assert y[:, :2].float().cpu().tolist() == [[17., 23.], [39., 53.]]
    assert float(y[:, 2:].abs().max()) == 0.0


def test_linear_residual(pkg, lib, dev):
    g = torch.Generator().manual_seed(5)
    M, N, K = 777, 4096, 1024
    x, w, r = rnd((M, K), g).to(dev), rnd((N, K), g, 0.02).to(dev), rnd((M, N), g).to(dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    lib.hd_linear_residual(pkg.ptr(x), pkg.ptr(w), pkg.ptr(r), pkg.ptr(y), M, N, K)
    pkg.check_prim("linear_residual")
    torch.cuda.synchronize()
    o = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    ref = (r.float() + o).to(torch.bfloat16).float()          # residual.cu:20-22
    assert rel_l2(y.float().cpu(), ref.cpu()) < 4e-3
    # o may differ by an ulp of |o| (fp32 accumulation order); the sum is
    # rounded once more, so the bound is in ulps of |o| + |sum|
    err = (y.float() - ref).abs()
    assert bool((err <= 2.0 ** -7 * (o.abs() + ref.abs()) + 1e-6).all())


@pytest.mark.parametrize("M", [1152, 70])
def test_linear_swiglu(pkg, lib, dev, M):
    g = torch.Generator().manual_seed(6)
    F, K = 1536, 512
    x, wg, wu = rnd((M, K), g).to(dev), rnd((F, K), g, 0.05).to(dev), rnd((F, K), g, 0.05).to(dev)
    y = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    lib.hd_linear_swiglu(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(y), M, F, K)
    pkg.check_prim("linear_swiglu")
    torch.cuda.synchronize()
    gt = (x.float() @ wg.float().t()).to(torch.bfloat16).float()
    up = (x.float() @ wu.float().t()).to(torch.bfloat16).float()
    s = (gt * torch.sigmoid(gt)).to(torch.bfloat16).float()   # act.cu:29-33
    ref = (s * up).to(torch.bfloat16).float()
    assert rel_l2(y.float().cpu(), ref.cpu()) < 5e-3
    assert cosine(y.float().cpu(), ref.cpu()) > 0.99999


def test_linear_concat3(pkg, lib, dev):
    g = torch.Generator().manual_seed(7)
    M, K = 520, 1024
    w0, w1, w2 = rnd((1024, K), g, .02).to(dev), rnd((256, K), g, .02).to(dev), rnd((512, K), g, .02).to(dev)
    x = rnd((M, K), g).to(dev)
    y = torch.empty(M, 1792, dtype=torch.bfloat16, device=dev)
    lib.hd_linear_concat3(pkg.ptr(x), pkg.ptr(w0), 1024, pkg.ptr(w1), 256, pkg.ptr(w2), 512,
                          pkg.ptr(y), M, K)
    pkg.check_prim("concat3")
    torch.cuda.synchronize()
    ref = (x.float() @ torch.cat([w0, w1, w2]).float().t()).to(torch.bfloat16).float()
    assert close_bf16(y.float().cpu().numpy(), ref.cpu().numpy(), ulps=2)


def test_linear_reference_backend(pkg, lib, dev):
    g = torch.Generator().manual_seed(8)
    M, N, K = 7, 5, 6     # test_primitives.c:273 shape
    x, w = rnd((M, K), g).to(dev), rnd((N, K), g).to(dev)
    y = pkg.linear(x, w)
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    assert close_bf16(y.float().cpu().numpy(), ref.cpu().numpy(), ulps=1)


@pytest.mark.parametrize("M", [1152, 8704, 700])
def test_gemm_epilogues_with_and_without_tail_split(pkg, lib, dev, M):
    """Plain, residual (K = 3072) and SwiGLU GEMMs through the production
    tiles, each with and without the tail-split workspace (M = 8704 splits
    its last round; M = 700 exercises partial row tiles), against fp32
    products of the same bf16 operands rounded at the kernels' rounding
    points: residual y = bf16(res + bf16(x.W^T)), SwiGLU
    bf16(bf16(silu(bf16(g))) * bf16(u))."""
    g = torch.Generator(device=dev).manual_seed(M)
    K, N, F = 1024, 2048, 1536
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(N, 3 * K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    xd = torch.randn(M, 3 * K, generator=g, device=dev).to(torch.bfloat16)
    wg = (torch.randn(F, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(F, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    r = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    print(f"gemm epilogues M={M}", flush=True)
    outs = []
    for use_ws in (False, True):
        wp, wn = (pkg.ptr(ws), ws.numel()) if use_ws else (None, 0)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        yr = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        ys = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
        lib.hd_linear_ws(pkg.ptr(x), pkg.ptr(w), None, pkg.ptr(y), M, N, K, wp, wn)
        lib.hd_linear_residual_ws(pkg.ptr(xd), pkg.ptr(wd), pkg.ptr(r), pkg.ptr(yr), M, N, 3 * K, wp, wn)
        lib.hd_linear_swiglu_ws(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(ys), M, F, K, wp, wn)
        pkg.check_prim("gemm epilogues ws=%d" % use_ws)
        torch.cuda.synchronize()
        outs.append((y, yr, ys))
    xf = x.float()
    ref = (xf @ w.float().t()).to(torch.bfloat16).float()
    prod = (xd.float() @ wd.float().t()).to(torch.bfloat16).float()
    refr = (prod + r.float()).to(torch.bfloat16).float()
    gt = (xf @ wg.float().t()).to(torch.bfloat16).float()
    up = (xf @ wu.float().t()).to(torch.bfloat16).float()
    refs = ((gt * torch.sigmoid(gt)).to(torch.bfloat16).float() * up).to(torch.bfloat16).float()
    for y, yr, ys in outs:
        for got, want, tag in ((y, ref, "plain"), (ys, refs, "swiglu")):
            assert close_bf16(got.float().cpu().numpy(), want.cpu().numpy(), ulps=2, atol_rel=1e-3), tag
        # two roundings: one bf16 step of the product (its fp32 sum order
        # differs from the reference's) and one of the sum, which may cancel
        err = (yr.float() - refr).abs()
        tol = 2.0 ** -7 * (refr.abs() + prod.abs()) + 1e-3 * float(refr.pow(2).mean().sqrt())
        assert bool((err <= tol).all()), ("residual", float((err - tol).max()))
    # the split launch's tail tiles differ from the unsplit launch by the
    # fp32 reassociation of their K sums (one bf16 step of the plain output)
    assert close_bf16(outs[0][0].float().cpu().numpy(), outs[1][0].float().cpu().numpy(), ulps=1, atol_rel=1e-3)
    assert float(outs[0][2].float().abs().mean()) > 0


def test_swiglu_epilogue_vs_exact_division(pkg, lib, dev):
    """The fused SwiGLU epilogue uses the hardware reciprocal for
    1/(1 + e^-g); hd_linear twice + hd_swiglu compute the same bf16 gate and
    up projections (same K order) and the sigmoid with an IEEE division
    (act.cu:29-33). After the bf16 rounding of silu(g) the two agree except
    near rounding boundaries: >= 99.9 % identical, the rest one bf16 step."""
    M, F, K = 1024, 3072, 1024
    g = torch.Generator(device=dev).manual_seed(21)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    wg = (torch.randn(F, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(F, K, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    fused = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    gt = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    up = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    sep = torch.empty(M, F, dtype=torch.bfloat16, device=dev)
    lib.hd_linear_swiglu(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(fused), M, F, K)
    lib.hd_linear(pkg.ptr(x), pkg.ptr(wg), None, pkg.ptr(gt), M, F, K, 1)
    lib.hd_linear(pkg.ptr(x), pkg.ptr(wu), None, pkg.ptr(up), M, F, K, 1)
    lib.hd_swiglu(pkg.ptr(gt), pkg.ptr(up), pkg.ptr(sep), M * F)
    pkg.check_prim("swiglu epilogue vs exact")
    torch.cuda.synchronize()
    a, b = fused.cpu().float().numpy(), sep.cpu().float().numpy()
    same = float((a == b).mean())
    print("identical fraction", same)
    assert same >= 0.999
    assert close_bf16(a, b, ulps=1)


@pytest.mark.parametrize("shape", [32, 16])
def test_mfma_probe_checksums(pkg, lib, dev, shape):
    """The matrix-core ceiling probe (diagnostic) on constant operands: every
    lane's checksum is the closed form of its 8 (or 16) accumulator chains,
    iters rounds of dot products of 16 (32) products of 0.5 x 0.5 per step,
    and the returned FLOP count is blocks x 8 waves x 8 x iters x 32768;
    bad arguments return 0."""
    blocks, iters = 4, 8
    ops = torch.full((1 << 16,), 0.5, device=dev).to(torch.bfloat16)
    out = torch.zeros(blocks * 512, dtype=torch.float32, device=dev)
    fl = lib.hd_mfma_probe(pkg.ptr(ops), ops.numel(), blocks, iters, shape, pkg.ptr(out))
    torch.cuda.synchronize()
    assert fl == blocks * 8 * 8 * iters * 32768
    # each output element of one chain accumulates iters MFMAs of K products
    # of 0.25; a lane holds 16 (32x32) or 4 (16x16) elements of 8 (16) chains
    k, per_lane = (16, 8 * 16) if shape == 32 else (32, 16 * 4)
    want = iters * k * 0.25 * per_lane
    assert torch.allclose(out, torch.full_like(out, want))
    for bad_iters, bad_shape in ((6, shape), (iters, 8)):
        assert lib.hd_mfma_probe(pkg.ptr(ops), ops.numel(), blocks, bad_iters, bad_shape,
                                 pkg.ptr(out)) == 0
        with pytest.raises(RuntimeError, match="mfma_probe: bad args"):
            pkg.check_prim("mfma_probe")   # reports through the error buffer, then clears it


@pytest.mark.parametrize("M,N,K,epi,use_ws", [(1728, 1152, 1152, 0, False), (1728, 3456, 1152, 2, True),
                                              (1728, 1152, 4352, 0, True), (700, 1536, 1024, 3, True),
                                              (1152, 4096, 4096, 2, True)])
def test_small_grid_128_tiles(pkg, lib, dev, M, N, K, epi, use_ws):
    """Small grids run on 128x128 tiles (two blocks per CU, 16x16x32 MFMA):
    without a K split when the 256-row grid fits one round and K <= 4096, and
    through the cost model (with its tail split when a workspace is given)
    otherwise: the vision tower's M = 1728 shapes, a ragged SwiGLU and the
    one-block o_proj shape, against torch fp32 (one bf16 rounding of the
    product, then the epilogue's own)."""
    print(f"small grid M={M} N={N} K={K} epi={epi} ws={use_ws} "
          f"cfg={lib.hd_gemm_config_name(M, N, K, epi).decode()}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    r = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    wp, wn = (pkg.ptr(ws), ws.numel()) if use_ws else (None, 0)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    prod = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    if epi == 0:
        lib.hd_linear_ws(pkg.ptr(x), pkg.ptr(w), None, pkg.ptr(y), M, N, K, wp, wn)
        want = prod
    elif epi == 2:
        lib.hd_linear_residual_ws(pkg.ptr(x), pkg.ptr(w), pkg.ptr(r), pkg.ptr(y), M, N, K, wp, wn)
        want = (prod + r.float()).to(torch.bfloat16).float()
    else:
        lib.hd_linear_swiglu_ws(pkg.ptr(x), pkg.ptr(w), pkg.ptr(wu), pkg.ptr(y), M, N, K, wp, wn)
        up = (x.float() @ wu.float().t()).to(torch.bfloat16).float()
        sg = (prod * torch.sigmoid(prod)).to(torch.bfloat16).float()
        want = (sg * up).to(torch.bfloat16).float()
    pkg.check_prim("small grid gemm")
    torch.cuda.synchronize()
    got = y.float().cpu()
    want = want.cpu()
    assert rel_l2(got, want) < 5e-3
    assert cosine(got, want) > 0.99999
    if epi == 2:
        # a step of the rounded product survives the residual add even
        # where the sum cancels: the bound scales with |product| + |sum|
        step = (prod.abs().cpu() + want.abs()) * 2.0 ** -7 * 2 + 1e-6
        assert bool(((got - want).abs() <= step).all())
    else:
        assert close_bf16(got.numpy(), want.numpy(), ulps=2 if epi == 0 else 4, atol_rel=1e-3)

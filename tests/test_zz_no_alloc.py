"""hd_linear_noalloc (the GEMM with its tail-split workspace in a static
device array) against hd_linear_ws with a caller workspace: bit-identical on
two calls in a row, the second smaller, both shapes with a split tail (the
split result differs from the unsplit hd_linear in the tail tiles, which
shows the static scratch was used)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def run_pair(pkg, lib, dev, M, N, K, bias, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g, device=dev).to(torch.bfloat16) if bias else None
    bp = pkg.ptr(b) if bias else None
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    y_ws = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    y_plain = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    print(f"no-alloc linear M={M} N={N} K={K} bias={bias}", flush=True)
    lib.hd_linear_ws(pkg.ptr(x), pkg.ptr(w), bp, pkg.ptr(y_ws), M, N, K, pkg.ptr(ws), ws.numel())
    lib.hd_linear_noalloc(pkg.ptr(x), pkg.ptr(w), bp, pkg.ptr(y_na), M, N, K)
    lib.hd_linear(pkg.ptr(x), pkg.ptr(w), bp, pkg.ptr(y_plain), M, N, K, 1)
    pkg.check_prim("linear noalloc")
    torch.cuda.synchronize()
    assert torch.equal(y_na, y_ws)
    return int((y_na != y_plain).sum())


def test_linear_noalloc_matches_workspace_entry(pkg, lib, dev):
    assert lib.hd_linear_noalloc_scratch_bytes() >= lib.hd_gemm_ws_bytes()
    # o_proj at configuration 1 (34 x 16 tiles: two rounds + a split tail),
    # then the down projection at configuration 0 (K = 12288, 72 tiles split)
    d1 = run_pair(pkg, lib, dev, 8704, 4096, 4096, True, 1)
    d2 = run_pair(pkg, lib, dev, 1152, 4096, 12288, False, 2)
    print(f"elements that differ from the unsplit GEMM: {d1}, {d2}", flush=True)
    assert d1 > 0 and d2 > 0

"""Benchmark of the o1 denoiser step on MI355X (one GPU).

Workload (benchmark configuration 1): one full denoising-step forward at
1024x1024 - 36 decoder blocks (hidden 4096, 32x128 heads, 8 kv heads, FFN
12288), 4096 image tokens (64x64 grid) + 256 text tokens = 4352 per
sequence, batch 2 (CFG cond/uncond), t-embedder MLP at t=0.5, x_embedder,
final norm + head. Random-init bf16 weights, synthetic seeded inputs.
A "step" = one hd_forward_batched call over both CFG sequences.

Prints ONE JSON line (driver contract) with roofline and cpu_baseline.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15      # dense bf16 MFMA, MI355X
PEAK_HBM = 8.0e12

CFGS = {
    "c1": dict(name="denoise_step_1024sq_cfg2", batch=2, text=256, gh=64, gw=64),
    "c2": dict(name="denoise_step_2048sq", batch=1, text=256, gh=128, gw=128),
}
HID, NH, NKV, FF, D, L = 4096, 32, 8, 12288, 128, 36


def step_flops(S, B, I, T):
    gemm_tok = 2 * (HID * NH * D + 2 * HID * NKV * D + NH * D * HID + 3 * HID * FF)
    blocks = L * (B * S * gemm_tok + B * 4 * S * S * NH * D)
    embed = B * (2 * I * (3072 * 1024 + 1024 * HID) + 2 * (256 * HID + HID * HID))
    head = B * S * 2 * HID * 3072
    return blocks + embed + head


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c1", choices=sorted(CFGS))
    ap.add_argument("--layers", type=int, default=L)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only the dominant kernel (gate/up GEMM + SwiGLU at the step's "
                         "shape) and a 1 GiB device copy, for rocprofv3 counter passes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on exactly one GPU (the reference has no multi-GPU "
              "path; sharding is a design note only). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    lib = pkg.load()
    from importlib import import_module
    synth = import_module("o1c_amd.synthetic")

    cfg = CFGS[args.config]
    B, T, gh, gw = cfg["batch"], cfg["text"], cfg["gh"], cfg["gw"]
    I = gh * gw
    S = T + I
    dev = torch.device("cuda:0")
    torch.cuda.init()
    pkg.bind_torch_stream()
    if args.kernel_only:
        kernel_only(pkg, lib, B * S, args.kernel_iters)
        return
    print(f"[bench] building {args.layers}-layer synthetic model", file=sys.stderr, flush=True)
    tensors = synth.build_model(n_layers=args.layers, seed=0, device="cuda:0")
    model = synth.Model(tensors, args.layers)
    pkg.set_block_config(theta=1e4)          # 2D RoPE, theta 1e4 (synthetic benchmark configurations)

    # synthetic inputs: text ids (last = timestep token), latents N(0,1) seed 42
    g = torch.Generator().manual_seed(42)
    lat = torch.randn(I, 3072, generator=g)
    vin = lat.to(torch.bfloat16).unsqueeze(0).repeat(B, 1, 1).contiguous().to(dev)
    gi = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 151643, (B, T), generator=gi, dtype=torch.int64)
    ids[:, -1] = synth.TMS_ID
    ids = ids.to(dev)
    tsd = torch.full((B,), 0.5, dtype=torch.float32, device=dev)
    pos = np.zeros((3, S), np.float32)
    r, c = np.divmod(np.arange(I), gw)
    pos[1, T:], pos[2, T:] = r, c
    posd = torch.from_numpy(pos).to(dev)
    wsb = lib.hd_forward_batched_workspace_bytes(B, S, I, NH, NKV, HID, FF, D)
    wsbuf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    out = torch.empty(B, S, 3072, dtype=torch.bfloat16, device=dev)
    import ctypes

    def step():
        st = lib.hd_forward_batched(ctypes.byref(model.binding), ctypes.byref(ws), B, pkg.ptr(ids), T,
                                    pkg.ptr(posd), 0, pkg.ptr(vin), I, pkg.ptr(tsd), S, NH, NKV,
                                    HID, FF, D, synth.TMS_ID, None, pkg.ptr(out), None)
        if st != 0:
            raise RuntimeError(lib.hd_last_error().decode())

    print("[bench] warmup", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), "non-finite output"
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    steps_per_s = 1000.0 / ms
    flops = step_flops(S, B, I, T) * args.layers / L if args.layers != L else step_flops(S, B, I, T)

    # ---- dominant kernel: gate/up GEMM with SwiGLU epilogue, timed alone ----
    M = B * S
    blk = model.binding.blocks[0]
    xln = torch.randn(M, HID, device=dev).to(torch.bfloat16)
    swi = torch.empty(M, FF, dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        lib.hd_linear_swiglu(pkg.ptr(xln), ctypes.c_void_p(blk.gate_proj), ctypes.c_void_p(blk.up_proj),
                             pkg.ptr(swi), M, FF, HID)
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record()
    for _ in range(args.kernel_iters):
        lib.hd_linear_swiglu(pkg.ptr(xln), ctypes.c_void_p(blk.gate_proj), ctypes.c_void_p(blk.up_proj),
                             pkg.ptr(swi), M, FF, HID)
    k1.record()
    torch.cuda.synchronize()
    kms = k0.elapsed_time(k1) / args.kernel_iters
    kflop = 2.0 * M * (2 * FF) * HID
    achieved = kflop / (kms * 1e-3) / 1e12

    # attention kernel alone (flash, full non-causal) at the step's shape
    q = torch.randn(B, NH, S, D, device=dev).to(torch.bfloat16)
    kk = torch.randn(B, NKV, S, D, device=dev).to(torch.bfloat16)
    vt = torch.zeros(lib.hd_flash_vt_bytes(B, NKV, S) // 2, dtype=torch.bfloat16, device=dev)
    ao = torch.empty(B, S, NH * D, dtype=torch.bfloat16, device=dev)
    for _ in range(2):
        lib.hd_flash_attention(pkg.ptr(q), pkg.ptr(kk), pkg.ptr(vt), None, pkg.ptr(ao), B, NH, NKV, S,
                               D, 0, D ** -0.5, 1)
    torch.cuda.synchronize()
    k0.record()
    for _ in range(args.kernel_iters):
        lib.hd_flash_attention(pkg.ptr(q), pkg.ptr(kk), pkg.ptr(vt), None, pkg.ptr(ao), B, NH, NKV, S,
                               D, 0, D ** -0.5, 1)
    k1.record()
    torch.cuda.synchronize()
    ams = k0.elapsed_time(k1) / args.kernel_iters
    aflop = 4.0 * B * S * S * NH * D
    attn_tf = aflop / (ams * 1e-3) / 1e12

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(S, T, gh, gw, B, args.layers)

    res = {
        "metric": "DiT denoise steps/sec (1024^2, CFG batch 2, 36 blocks)" if args.config == "c1"
                  else "DiT denoise steps/sec (2048^2, 36 blocks)",
        "value": round(steps_per_s, 4),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights seed 0, N(0,1) latents seed 42)",
        "config": {"workload": cfg["name"], "batch": B, "seq_len": S, "image_tokens": I,
                   "text_tokens": T, "layers": args.layers, "hidden": HID, "heads": NH,
                   "kv_heads": NKV, "ffn": FF, "parallelism": "single GPU"},
        "step_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "step_mfma_frac": round(flops / (ms * 1e-3) / PEAK_BF16, 4),
        "wall_s": round(wall, 3),
        "roofline": {"kernel": "gemm_bf16 gate/up + SwiGLU epilogue", "bound": "mfma",
                     "achieved": round(achieved, 1), "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved * 1e12 / PEAK_BF16, 4), "traffic": read_traffic(),
                     "launch_ms": round(kms, 4), "shape": [M, 2 * FF, HID]},
        "attention": {"kernel": "flash_fwd (full, GQA 32/8, D=128)", "achieved": round(attn_tf, 1),
                      "unit": "TFLOP/s", "frac": round(attn_tf * 1e12 / PEAK_BF16, 4),
                      "launch_ms": round(ams, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


def kernel_only(pkg, lib, M, iters):
    """Dominant kernel alone + a copy of known size (the counter calibration)."""
    import ctypes
    import torch
    dev = torch.device("cuda:0")
    x = torch.randn(M, HID, device=dev).to(torch.bfloat16)
    wg = (torch.randn(FF, HID, device=dev) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(FF, HID, device=dev) * 0.02).to(torch.bfloat16)
    y = torch.empty(M, FF, dtype=torch.bfloat16, device=dev)
    src = torch.ones(1 << 29, dtype=torch.int16, device=dev)     # 1 GiB
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(iters):
        lib.hd_linear_swiglu(pkg.ptr(x), pkg.ptr(wg), pkg.ptr(wu), pkg.ptr(y), M, FF, HID)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"kernel_only": True, "M": M, "iters": iters, "copy_bytes": 1 << 30}))


def read_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed counter
    summary (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by
    a 1 GiB copy's counters); None when absent."""
    path = os.path.join(ROOT, "profiles", "gemm_swiglu_c1_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_baseline(S, T, gh, gw, B, layers):
    """The fp32 C oracle of one decoder block on the host cores, for one CFG
    sequence at the step's real shape; steps/s extrapolated x(layers * B)."""
    import numpy as np
    import torch
    from oracle import oracle as orc
    from tests.common import make_block_weights, grid_pos, bf16
    threads = min(os.cpu_count() or 1, 16)
    orc.lib().o1o_set_threads(threads)
    w = {k: v.numpy() for k, v in make_block_weights(HID, NH, NKV, FF, D, seed=0).items()}
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(1))).numpy()
    pos = grid_pos(T, gh, gw)
    cfg = orc.block_cfg(NH, NKV, HID, FF, D, theta=1e4, faithful=0)
    t0 = time.perf_counter()
    orc.decoder_block(x, pos, w, cfg)
    dt = time.perf_counter() - t0
    return {"value": round(1.0 / (dt * layers * B), 6), "unit": "steps/s", "cores": threads,
            "kind": "port",
            "sample": f"1 decoder block, 1 sequence of S={S} (fp32 C oracle, OpenMP); "
                      f"steps/s = 1/(t_block x {layers} blocks x {B} CFG sequences); "
                      f"t_block={dt:.2f}s; cpu={platform.processor() or platform.machine()}"}


if __name__ == "__main__":
    main()

"""Benchmark of the o1 denoiser step on MI355X (one GPU).

Workload (benchmark configuration 1): one full denoising-step forward at
1024x1024 - 36 decoder blocks (hidden 4096, 32x128 heads, 8 kv heads, FFN
12288), 4096 image tokens (64x64 grid) + 256 text tokens = 4352 per
sequence, batch 2 (CFG cond/uncond), t-embedder MLP at t=0.5, x_embedder,
final norm + head. Random-init bf16 weights, synthetic seeded inputs.
A "step" = one hd_forward_batched call over both CFG sequences.

Prints ONE JSON line (driver contract) with roofline and cpu_baseline. The
default run also times, on the same weights, configuration 2 (2048x2048,
16640 tokens, batch 1) as a `c2` object, configuration 0 (one block,
S = 1152) as a `c0` object, configuration 3 (the edit step: 1024^2 target
+ 3 references, 16896 tokens, vision conditioning) as a `c3` object and,
last because it rewrites the weights, configuration 4 (GPU LoRA merge into
all 252 projection weights + one 28-step CFG image) as a `c4` object.
"""
import argparse
import ctypes
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
    # one decoder block (the reference's CPU-runnable case): 32x32 image
    # tokens + 128 text tokens, batch 1
    "c0": dict(name="block_forward_s1152", batch=1, text=128, gh=32, gw=32, refs=0),
    "c1": dict(name="denoise_step_1024sq_cfg2", batch=2, text=256, gh=64, gw=64, refs=0),
    "c2": dict(name="denoise_step_2048sq", batch=1, text=256, gh=128, gw=128, refs=0),
    # multi-reference edit: 64x64 target + 3 references of 64x64 (+64 RoPE
    # rows each, x_embedder rows cached) + 512 text tokens = 16896
    "c3": dict(name="edit_step_3refs_1024sq", batch=1, text=512, gh=64, gw=64, refs=3),
    # LoRA merge (r=64, all q/k/v/o/gate/up/down of 36 blocks) + 28-step
    # flow-match Euler sampler, CFG batch 2, guidance 5, shift 3
    "c4": dict(name="lora_merge_plus_28step_euler_cfg_1024sq", batch=2, text=256, gh=64, gw=64,
               refs=0, steps=28, guidance=5.0, shift=3.0, rank=64),
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
    ap.add_argument("--no-c2", action="store_true",
                    help="with the default configuration 1, skip the configuration 2 (2048^2) timing "
                         "that the same run adds as its `c2` object")
    ap.add_argument("--c2-steps", type=int, default=10)
    ap.add_argument("--no-c0", action="store_true",
                    help="with the default configuration 1, skip the configuration 0 (one block, "
                         "S = 1152) timing that the same run adds as its `c0` object")
    ap.add_argument("--c0-steps", type=int, default=200)
    ap.add_argument("--no-c3", action="store_true",
                    help="with the default configuration 1, skip the configuration 3 (edit step, "
                         "1024^2 target + 3 references, vision conditioning) object")
    ap.add_argument("--c3-steps", type=int, default=5)
    ap.add_argument("--no-c4", action="store_true",
                    help="with the default configuration 1, skip the configuration 4 (LoRA merge + "
                         "28-step CFG image) object; it merges into the model's weights, so it runs last")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--flash-only", action="store_true",
                    help="run only the flash attention kernel at the configuration's shape "
                         "(--kernel-iters launches), for rocprofv3 counter passes")
    ap.add_argument("--vision-only", action="store_true",
                    help="run only the vision tower of configuration 3 (3 references of 24x24 "
                         "patches, one multi-image call, 10 untimed + 10 timed), for rocprofv3")
    ap.add_argument("--elementwise", action="store_true",
                    help="time each HBM-bound kernel of the path (norms, rotary, QKV epilogue, "
                         "SwiGLU, residual, head permutes, sampler pointwise, patchify) at "
                         "configuration 2's sizes and print its HBM rate against 8 TB/s")
    ap.add_argument("--ceilings", action="store_true",
                    help="measure, in one process, the matrix-core ceiling probe on random and "
                         "constant operands, hipBLASLt (torch.matmul) on the gate/up shape and this "
                         "build's gate/up GEMMs at configurations 1 and 2")
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

    # random-init weights leave the reference's [-2, 2] final-latent range:
    # the 28-step image keeps only the NaN/Inf part of the fail-closed check
    lib.hd_denoise_set_output_check(1)
    cfg = CFGS[args.config]
    B, T, gh, gw, R = cfg["batch"], cfg["text"], cfg["gh"], cfg["gw"], cfg["refs"]
    I = gh * gw * (1 + R)
    S = T + I
    dev = torch.device("cuda:0")
    torch.cuda.init()
    pkg.bind_torch_stream()
    if args.elementwise:
        elementwise_bench(pkg, lib, args.kernel_iters)
        return
    if args.kernel_only:
        kernel_only(pkg, lib, B * S, args.kernel_iters)
        return
    if args.ceilings:
        print(json.dumps(ceilings(pkg, lib, dev)))
        return
    if args.config == "c0":
        run_c0(pkg, lib, cfg, args, dev)
        return
    if args.flash_only:
        q = torch.randn(B, NH, S, D, device=dev).to(torch.bfloat16)
        kk = torch.randn(B, NKV, S, D, device=dev).to(torch.bfloat16)
        vt = torch.randn(lib.hd_flash_vt_bytes(B, NKV, S) // 2, device=dev).to(torch.bfloat16)
        ao = torch.empty(B, S, NH * D, dtype=torch.bfloat16, device=dev)
        # with the tail-split workspace, as the decoder block launches it
        fws = torch.empty(lib.hd_flash_ws_bytes(), dtype=torch.uint8, device=dev)
        for _ in range(args.kernel_iters):
            rc = lib.hd_flash_attention_ws(pkg.ptr(q), pkg.ptr(kk), pkg.ptr(vt), None, pkg.ptr(ao), B, NH,
                                           NKV, S, D, 0, D ** -0.5, 1, pkg.ptr(fws), fws.numel())
            if rc != 0:
                raise RuntimeError(lib.hd_cuda_last_error().decode())
        torch.cuda.synchronize()
        return
    if args.vision_only:
        from importlib import import_module as _im
        vids = torch.zeros(1, 512, dtype=torch.int64, device=dev)
        _, info = run_vision(pkg, lib, _im("o1c_amd.synthetic"), vids, 3, 512, 512 + 3 * 4096, dev,
                             iters=10)
        print(json.dumps(info))
        return
    print(f"[bench] building {args.layers}-layer synthetic model", file=sys.stderr, flush=True)
    tensors = synth.build_model(n_layers=args.layers, seed=0, device="cuda:0")
    model = synth.Model(tensors, args.layers)
    pkg.set_block_config(theta=1e4)          # 2D RoPE, theta 1e4 (synthetic benchmark configurations)

    r = time_config(pkg, lib, synth, model, tensors, args.config, args.steps, args.warmup,
                    args.layers, args.kernel_iters, dev, args)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(S, T, gh, gw, B, args.layers)
    metric = {"c0": "DiT block forwards/sec (config 0)",
              "c1": "DiT denoise steps/sec (1024^2, CFG batch 2, 36 blocks)",
              "c2": "DiT denoise steps/sec (2048^2, 36 blocks)",
              "c3": "DiT edit steps/sec (1024^2 target + 3 references, 36 blocks)",
              "c4": "DiT denoise steps/sec (1024^2, CFG batch 2) + LoRA merge and 28-step image"}
    res = {
        "metric": metric[args.config],
        "value": round(1000.0 / r["ms"], 4),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights seed 0, N(0,1) latents seed 42)",
        "config": {"workload": cfg["name"], "batch": B, "seq_len": S, "image_tokens": I,
                   "text_tokens": T, "layers": args.layers, "hidden": HID, "heads": NH,
                   "kv_heads": NKV, "ffn": FF, "parallelism": "single GPU"},
        "step_tflops": r["step_tflops"],
        "step_mfma_frac": r["step_mfma_frac"],
        "wall_s": r["wall_s"],
        "roofline": dict(r["gemm"], traffic=read_traffic(args.config)),
        "attention": r["attention"],
        "cpu_baseline": cpu,
    }
    res.update(r["extra"])
    if args.config == "c1" and not args.no_c2:
        # the north-star configuration in the same run, on the same weights:
        # 2048^2, 16384 image + 256 text tokens, batch 1
        print("[bench] configuration 2 (2048^2) on the same model", file=sys.stderr, flush=True)
        r2 = time_config(pkg, lib, synth, model, tensors, "c2", args.c2_steps, min(args.warmup, 3),
                         args.layers, args.kernel_iters, dev, args)
        c2 = CFGS["c2"]
        res["c2"] = {"workload": c2["name"], "seq_len": c2["text"] + c2["gh"] * c2["gw"], "batch": 1,
                     "steps": args.c2_steps, "ms_per_step": round(r2["ms"], 3),
                     "steps_per_s": round(1000.0 / r2["ms"], 4), "step_tflops": r2["step_tflops"],
                     "step_mfma_frac": r2["step_mfma_frac"], "wall_s": r2["wall_s"],
                     "gemm": dict(r2["gemm"], traffic=read_traffic("c2")), "attention": r2["attention"]}
    if args.config == "c1" and not args.no_c0:
        # configuration 0 (one block, S = 1152) on layer 0 of the same weights
        print("[bench] configuration 0 (one block, S = 1152) on layer 0", file=sys.stderr, flush=True)
        r0 = time_c0(pkg, lib, ctypes.byref(model.binding.blocks[0]), model.binding.blocks[0], dev,
                     args.c0_steps, 20, args.kernel_iters)
        res["c0"] = {"workload": CFGS["c0"]["name"], "seq_len": r0["S"], "batch": 1, "steps": args.c0_steps,
                     "ms_per_block": round(r0["ms"], 4), "blocks_per_s": round(1000.0 / r0["ms"], 2),
                     "block_tflops": round(r0["flops"] / (r0["ms"] * 1e-3) / 1e12, 1),
                     "block_mfma_frac": round(r0["flops"] / (r0["ms"] * 1e-3) / PEAK_BF16, 4),
                     "wall_s": round(r0["wall"], 3), "gemm": r0["gemm"]}
    if args.config == "c1" and not args.no_c3:
        # configuration 3: the edit step (512 text + 64x64 target + 3
        # references of 64x64, S = 16896) with vision conditioning
        print("[bench] configuration 3 (edit step, 3 references) on the same model", file=sys.stderr, flush=True)
        r3 = time_config(pkg, lib, synth, model, tensors, "c3", args.c3_steps, 2, args.layers,
                         args.kernel_iters, dev, args)
        c3 = CFGS["c3"]
        res["c3"] = {"workload": c3["name"], "seq_len": c3["text"] + c3["gh"] * c3["gw"] * (1 + c3["refs"]),
                     "batch": 1, "steps": args.c3_steps, "ms_per_step": round(r3["ms"], 3),
                     "steps_per_s": round(1000.0 / r3["ms"], 4), "step_tflops": r3["step_tflops"],
                     "step_mfma_frac": r3["step_mfma_frac"], "wall_s": r3["wall_s"],
                     "gemm": r3["gemm"], "attention": r3["attention"], **r3["extra"]}
    if args.config == "c1" and not args.no_c4:
        # configuration 4 last: the LoRA merge rewrites the model's weights
        print("[bench] configuration 4 (LoRA merge + 28-step image) on the same model", file=sys.stderr,
              flush=True)
        r4 = time_config(pkg, lib, synth, model, tensors, "c4", 3, 1, args.layers, args.kernel_iters, dev, args)
        c4 = CFGS["c4"]
        res["c4"] = {"workload": c4["name"], "seq_len": c4["text"] + c4["gh"] * c4["gw"], "batch": 2,
                     "ms_per_step": round(r4["ms"], 3), **r4["extra"]}
    print(json.dumps(res))


def time_config(pkg, lib, synth, model, tensors, name, steps, warmup, layers, kernel_iters, dev, args):
    """Times `steps` denoiser steps of configuration `name` on `model`
    (untimed `warmup` steps first), then the step's dominant GEMM (gate/up +
    SwiGLU at M = B*S) and its attention launch alone, each over
    `kernel_iters` launches between HIP events on the library's stream."""
    import numpy as np
    import torch
    cfg = CFGS[name]
    B, T, gh, gw, R = cfg["batch"], cfg["text"], cfg["gh"], cfg["gw"], cfg["refs"]
    I = gh * gw * (1 + R)
    S = T + I
    # synthetic inputs: text ids (last = timestep token), latents N(0,1) seed 42
    g = torch.Generator().manual_seed(42)
    lat = torch.randn(I, 3072, generator=g)
    vin = lat.to(torch.bfloat16).unsqueeze(0).repeat(B, 1, 1).contiguous().to(dev)
    gi = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 151643, (B, T), generator=gi, dtype=torch.int64)
    ids[:, -1] = synth.TMS_ID
    ids = ids.to(dev)
    tsd = torch.full((B,), 0.5, dtype=torch.float32, device=dev)
    # 2D RoPE positions: text at 0; target grid, then each reference grid
    # with a +64 row offset per reference
    pos = np.zeros((3, S), np.float32)
    segs = 1 + R
    gha = (ctypes.c_int * segs)(*([gh] * segs))
    gwa = (ctypes.c_int * segs)(*([gw] * segs))
    roa = (ctypes.c_int * segs)(*[64 * k for k in range(segs)])
    assert lib.hd_seq_grid_positions(T, segs, gha, gwa, roa, None, 0.0, pkg.np_ptr(pos)) == S
    posd = torch.from_numpy(pos).to(dev)
    wsb = lib.hd_forward_batched_workspace_bytes(B, S, I, NH, NKV, HID, FF, D)
    wsbuf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    out = torch.empty(B, S, 3072, dtype=torch.bfloat16, device=dev)
    extra = {}
    if R:
        # reference rows are clean fixed N(0,1) content: their x_embedder rows
        # are computed once and reused every step (forward.c:301-313)
        n_ref = gh * gw * R
        ref_rows = vin[0, I - n_ref:].contiguous()
        xs = pkg.linear(ref_rows, tensors["model.x_embedder.proj1.weight"])
        xe_ref = pkg.linear(xs, tensors["model.x_embedder.proj2.weight"],
                            tensors["model.x_embedder.proj2.bias"])
        ws.xe_ref = xe_ref.data_ptr()
        ws.n_ref = n_ref
    if name == "c4":
        extra = run_c4(pkg, lib, model, tensors, cfg, ws, ids, posd, vin, T, I, S, dev, args)
    vis = None
    if R:
        vis, extra = run_vision(pkg, lib, synth, ids, R, T, S, dev)

    def step():
        if vis is not None:
            # edit step: vision conditioning on the text rows (image pads
            # replaced, DeepStack into blocks 0-2) through hd_forward
            st = lib.hd_forward(ctypes.byref(model.binding), ctypes.byref(ws), pkg.ptr(ids), T,
                                pkg.ptr(posd), None, pkg.ptr(vin), I, ctypes.addressof(vis["cond"]),
                                pkg.ptr(tsd), None, S, NH, NKV, HID, FF, D, synth.TMS_ID, None,
                                pkg.ptr(out), None)
        else:
            st = lib.hd_forward_batched(ctypes.byref(model.binding), ctypes.byref(ws), B, pkg.ptr(ids),
                                        T, pkg.ptr(posd), 0, pkg.ptr(vin), I, pkg.ptr(tsd), S, NH,
                                        NKV, HID, FF, D, synth.TMS_ID, None, pkg.ptr(out), None)
        if st != 0:
            raise RuntimeError(lib.hd_last_error().decode())

    print(f"[bench] {name}: warmup", file=sys.stderr, flush=True)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), "non-finite output"
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    print(f"[bench] {name}: timing {steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    flops = step_flops(S, B, I, T) * layers / L if layers != L else step_flops(S, B, I, T)
    del wsbuf, out

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
    for _ in range(kernel_iters):
        lib.hd_linear_swiglu(pkg.ptr(xln), ctypes.c_void_p(blk.gate_proj), ctypes.c_void_p(blk.up_proj),
                             pkg.ptr(swi), M, FF, HID)
    k1.record()
    torch.cuda.synchronize()
    kms = k0.elapsed_time(k1) / kernel_iters
    kflop = 2.0 * M * (2 * FF) * HID
    achieved = kflop / (kms * 1e-3) / 1e12
    del xln, swi

    # attention kernel alone (flash, full non-causal) at the step's shape
    # N(0,1) operands, V included: matrix-core power (and so the clock the
    # chip holds) depends on the data, and all-zero V runs ~10 % faster
    q = torch.randn(B, NH, S, D, device=dev).to(torch.bfloat16)
    kk = torch.randn(B, NKV, S, D, device=dev).to(torch.bfloat16)
    vt = torch.randn(lib.hd_flash_vt_bytes(B, NKV, S) // 2, device=dev).to(torch.bfloat16)
    ao = torch.empty(B, S, NH * D, dtype=torch.bfloat16, device=dev)
    # the launch the block makes: with the tail-split workspace (8-wave
    # blocks at these sequence lengths, the last partial round split)
    fws = torch.empty(lib.hd_flash_ws_bytes(), dtype=torch.uint8, device=dev)

    def attn():
        rc = lib.hd_flash_attention_ws(pkg.ptr(q), pkg.ptr(kk), pkg.ptr(vt), None, pkg.ptr(ao), B, NH, NKV, S,
                                       D, 0, D ** -0.5, 1, pkg.ptr(fws), fws.numel())
        assert rc == 0, lib.hd_cuda_last_error()

    for _ in range(2):
        attn()
    torch.cuda.synchronize()
    k0.record()
    for _ in range(kernel_iters):
        attn()
    k1.record()
    torch.cuda.synchronize()
    ams = k0.elapsed_time(k1) / kernel_iters
    aflop = 4.0 * B * S * S * NH * D
    attn_tf = aflop / (ams * 1e-3) / 1e12
    del q, kk, vt, ao, fws
    return {
        "ms": ms, "wall_s": round(wall, 3),
        "step_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "step_mfma_frac": round(flops / (ms * 1e-3) / PEAK_BF16, 4),
        "gemm": {"kernel": "gemm_bf16 gate/up + SwiGLU epilogue", "bound": "mfma",
                 "achieved": round(achieved, 1), "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                 "frac": round(achieved * 1e12 / PEAK_BF16, 4), "launch_ms": round(kms, 4),
                 "shape": [M, 2 * FF, HID]},
        "attention": {"kernel": "flash_pp16_kernel (8-wave ping-pong on 16x16x32 MFMA tiles; full, GQA 32/8, D=128; tail-split workspace as in the block)",
                      "achieved": round(attn_tf, 1), "unit": "TFLOP/s",
                      "frac": round(attn_tf * 1e12 / PEAK_BF16, 4), "launch_ms": round(ams, 4)},
        "extra": extra,
    }


def time_c0(pkg, lib, block, b0, dev, steps, warmup, kernel_iters):
    """Time configuration 0 on one decoder block's weights: the block through
    hd_decoder_block_batched (B = 1, S = 1152: 32x32 image tokens + 128 text
    tokens at position 0, 2-D RoPE theta 1e4) on an N(0,1) input (seed 1),
    and the block's dominant kernel (gate/up GEMM + SwiGLU at M = 1152).
    `block` is the ctypes reference of the block binding, `b0` the binding."""
    import numpy as np
    import torch
    cfg = CFGS["c0"]
    T, gh, gw = cfg["text"], cfg["gh"], cfg["gw"]
    S = T + gh * gw
    pos = np.zeros((3, S), np.float32)
    one = (ctypes.c_int * 1)
    assert lib.hd_seq_grid_positions(T, 1, one(gh), one(gw), one(0), None, 0.0, pkg.np_ptr(pos)) == S
    cs = pkg.rope_table(torch.from_numpy(pos).to(dev), S, D, theta=1e4)
    x = torch.randn(S, HID, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    out = torch.empty_like(x)
    sb = lib.hd_decoder_block_batched_scratch_bytes(1, S, NH, NKV, HID, FF, D)
    scr = torch.empty(sb, dtype=torch.uint8, device=dev)

    def step():
        st = lib.hd_decoder_block_batched(pkg.ptr(x), pkg.ptr(cs), None, 0, block, pkg.ptr(scr), sb, None,
                                          pkg.ptr(out), 1, S, NH, NKV, HID, FF, D)
        if st != 0:
            raise RuntimeError(lib.hd_last_error().decode())

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    gemm_tok = 2 * (HID * NH * D + 2 * HID * NKV * D + NH * D * HID + 3 * HID * FF)
    flops = S * gemm_tok + 4 * S * S * NH * D
    xl = torch.randn(S, HID, device=dev).to(torch.bfloat16)
    sw = torch.empty(S, FF, dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        lib.hd_linear_swiglu(pkg.ptr(xl), ctypes.c_void_p(b0.gate_proj), ctypes.c_void_p(b0.up_proj), pkg.ptr(sw), S, FF, HID)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(kernel_iters):
        lib.hd_linear_swiglu(pkg.ptr(xl), ctypes.c_void_p(b0.gate_proj), ctypes.c_void_p(b0.up_proj), pkg.ptr(sw), S, FF, HID)
    e1.record()
    torch.cuda.synchronize()
    kms = e0.elapsed_time(e1) / kernel_iters
    kflop = 2.0 * S * 2 * FF * HID
    return {"S": S, "T": T, "gh": gh, "gw": gw, "ms": ms, "wall": wall, "flops": flops,
            "gemm": {"kernel": "gemm_bf16 gate/up + SwiGLU epilogue", "bound": "mfma",
                     "achieved": round(kflop / (kms * 1e-3) / 1e12, 1), "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": round(kflop / (kms * 1e-3) / PEAK_BF16, 4),
                     "traffic": read_traffic("c0"), "launch_ms": round(kms, 4), "shape": [S, 2 * FF, HID]}}


def run_c0(pkg, lib, cfg, args, dev):
    """Configuration 0: one decoder block (random-init bf16 weights, seed 0).
    A step is one block forward."""
    from importlib import import_module
    synth = import_module("o1c_amd.synthetic")
    tensors = synth.build_model(n_layers=1, seed=0, device="cuda:0")
    model = synth.Model(tensors, 1)
    pkg.set_block_config(theta=1e4)
    r = time_c0(pkg, lib, ctypes.byref(model.binding.blocks[0]), model.binding.blocks[0], dev, args.steps,
                args.warmup, args.kernel_iters)
    S, T, gh, gw, ms = r["S"], r["T"], r["gh"], r["gw"], r["ms"]
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(S, T, gh, gw, 1, 1)
        cpu["unit"] = "blocks/s"
        cpu["sample"] = cpu["sample"].replace("steps/s = 1/(t_block x 1 blocks x 1 CFG sequences)",
                                              "blocks/s = 1/t_block")
    res = {
        "metric": "DiT block forwards/sec (config 0: one decoder block, S=1152)",
        "value": round(1000.0 / ms, 3), "unit": "blocks/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights seed 0, N(0,1) input seed 1)",
        "config": {"workload": cfg["name"], "batch": 1, "seq_len": S, "image_tokens": gh * gw,
                   "text_tokens": T, "layers": 1, "hidden": HID, "heads": NH, "kv_heads": NKV,
                   "ffn": FF, "parallelism": "single GPU"},
        "step_tflops": round(r["flops"] / (ms * 1e-3) / 1e12, 1),
        "step_mfma_frac": round(r["flops"] / (ms * 1e-3) / PEAK_BF16, 4),
        "wall_s": round(r["wall"], 3),
        "roofline": r["gemm"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


def run_vision(pkg, lib, synth, ids, R, T, S, dev, iters=5):
    """Reference images through the Qwen3-VL vision tower: R condition
    images of 384x384 (24x24 patches of 16 px, 144 merged tokens each,
    generate.c:65, :313-330), random-init tower weights, N(0,1) patchified
    pixels. The text rows get R x (vision_start, 144 image pads, vision_end)
    after a 3-token header; the tower runs once per image (before the
    steps) and its embeddings condition every step."""
    import torch
    gh = gw = 24
    n, m = gh * gw, gh * gw // 4
    V = R * m
    print(f"[bench] vision tower: {R} references of {n} patches", file=sys.stderr, flush=True)
    vt = synth.build_vision(seed=3, device="cuda:0")
    # all R references in one hd_vision_forward_multi call (same grid)
    tower = synth.VisionTower(vt, gh, gw, images=R)
    g = torch.Generator(device=dev).manual_seed(11)
    px = torch.randn(R * n, synth.V_PATCH, device=dev, generator=g).to(torch.bfloat16)
    emb = torch.empty(V, synth.V_OUT, dtype=torch.bfloat16, device=dev)
    ds = [torch.empty(V, synth.V_OUT, dtype=torch.bfloat16, device=dev) for _ in range(3)]

    def run_all():
        tower(px, emb, ds)

    run_all()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        run_all()
    e1.record()
    torch.cuda.synchronize()
    ms_ref = e0.elapsed_time(e1) / iters / R
    assert torch.isfinite(emb.float()).all()
    # text rows: header(3) | R x (vs, m pads, vend) | caption ... | tms
    VS, PAD, VEND = 151652, 151655, 151653
    ids_h = ids[0].cpu()
    vmask = torch.zeros(S, dtype=torch.uint8)
    at = 3
    for r in range(R):
        ids_h[at] = VS
        ids_h[at + 1:at + 1 + m] = PAD
        vmask[at + 1:at + 1 + m] = 1
        ids_h[at + 1 + m] = VEND
        at += m + 2
    assert at < T - 1 and int(vmask.sum()) == V
    ids[0].copy_(ids_h)
    vmd = vmask.to(dev)
    cond = pkg.hd_visual_cond()
    cond.image_embeds = emb.data_ptr()
    for j in range(3):
        cond.deepstack[j] = ds[j].data_ptr()
    cond.visual_mask = vmd.data_ptr()
    cond.v_tokens = V
    fl = synth.vision_flops(n)
    keep = {"cond": cond, "tensors": vt, "tower": tower, "emb": emb, "ds": ds, "vmask": vmd, "px": px}
    info = {"vision": {"kernel": "vision tower (27 blocks + 4 mergers), R references per call",
                       "patches": n, "merged_tokens": m, "references": R,
                       "ms_per_reference": round(ms_ref, 3),
                       "tflops": round(fl / (ms_ref * 1e-3) / 1e12, 1),
                       "frac": round(fl / (ms_ref * 1e-3) / PEAK_BF16, 4),
                       "gflop_per_reference": round(fl / 1e9, 1)}}
    return keep, info


def run_c4(pkg, lib, model, tensors, cfg, ws, ids, posd, vin, T, I, S, dev, args):
    """LoRA merge of every q/k/v/o/gate/up/down weight of the 36 blocks on the
    GPU (rank 64, A,B ~ N(0, 0.01), scale 1.0), then one image: 28-step
    flow-match Euler with CFG (guidance 5, sigmas linear 1 -> 0 with shift 3)
    from the seeded initial latent, all through the C-ABI."""
    import numpy as np
    import torch
    r = cfg["rank"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
             "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    entries = (pkg.hd_lora_entry * (len(names) * L))()
    keep = []
    k = 0
    for layer in range(L):
        for nm in names:
            w = tensors[f"model.language_model.layers.{layer}.{nm}.weight"]
            N, K = w.shape
            up = torch.empty(N, r, device=dev).normal_(0, 0.01, generator=gen)
            down = torch.empty(r, K, device=dev).normal_(0, 0.01, generator=gen)
            keep += [up, down]
            e = entries[k]
            e.rank, e.in_dim, e.out_dim, e.alpha, e.multiplier = r, K, N, float(r), 1.0
            e.up_dev, e.down_dev, e.base_dev = up.data_ptr(), down.data_ptr(), w.data_ptr()
            k += 1
    # one merge into a small scratch weight first, so the timed call does
    # not include loading the kernels' code on their first launch
    wx = torch.zeros(256, 256, dtype=torch.bfloat16, device=dev)
    ux, dx = torch.zeros(256, r, device=dev), torch.zeros(r, 256, device=dev)
    ex = pkg.hd_lora_entry()
    ex.rank, ex.in_dim, ex.out_dim, ex.alpha, ex.multiplier = r, 256, 256, float(r), 1.0
    ex.up_dev, ex.down_dev, ex.base_dev = ux.data_ptr(), dx.data_ptr(), wx.data_ptr()
    if lib.hd_lora_merge_gpu(ctypes.byref(ex), 1, None) != 0:
        raise RuntimeError(lib.hd_last_error().decode())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    st = lib.hd_lora_merge_gpu(entries, k, None)
    e1.record()
    torch.cuda.synchronize()
    if st != 0:
        raise RuntimeError(lib.hd_last_error().decode())
    merge_ms = e0.elapsed_time(e1)
    welems = sum(int(tensors[f"model.language_model.layers.0.{nm}.weight"].numel()) for nm in names) * L
    # sampler
    steps, g, shift = cfg["steps"], cfg["guidance"], cfg["shift"]
    sch = pkg.hd_scheduler()
    n = lib.hd_scheduler_derive_default(ctypes.byref(sch), steps, shift, 8.0)
    sig = (ctypes.c_float * n)(*sch.sigmas[:n])
    side = cfg["gh"] * 32      # 3072-d patch features = 3 x 32 x 32 pixels
    noise = np.empty(3 * side * side, np.float32)
    lib.hd_initial_noise(42, side, side, pkg.np_ptr(noise))
    noised = torch.from_numpy(noise).to(dev)
    z = torch.empty(I, 3072, dtype=torch.bfloat16, device=dev)
    lib.hd_patchify_bf16(pkg.ptr(noised), pkg.ptr(z), 3, cfg["gh"], cfg["gw"], 32)
    sb = lib.hd_denoise_scratch_bytes(S, I, steps)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    st = lib.hd_denoise_euler_cfg(ctypes.byref(model.binding), ctypes.byref(ws), pkg.ptr(ids), T,
                                  pkg.ptr(posd), 0, pkg.ptr(z), I, sig, steps, g, S, NH, NKV, HID,
                                  FF, D, 151673, pkg.ptr(scratch), sb, None)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if st != 0:
        raise RuntimeError(lib.hd_last_error().decode())
    img_s = e0.elapsed_time(e1) / 1000.0
    zf = z.float()
    assert torch.isfinite(zf).all(), "non-finite latent"
    lora = {"targets": k, "rank": r, "merge_ms": round(merge_ms, 3), "weight_elems": welems,
            "hbm_gb_s": round(welems * 4 / (merge_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(welems * 4 / (merge_ms * 1e-3) / 8e12, 4),
            "fp32_tflops": round(welems * 2 * r / (merge_ms * 1e-3) / 1e12, 2),
            "fp32_matrix_frac": round(welems * 2 * r / (merge_ms * 1e-3) / 157.3e12, 4),
            "kernel": "lora_merge_stream_kernel (rank product on bf16 MFMA, fp32 operands split in 3 bf16 parts)"}
    if not args.no_cpu_baseline:
        lora["cpu_baseline"] = cpu_lora_baseline(r, welems)
    return {"lora": lora,
            "sampler": {"steps": steps, "guidance": g, "shift": shift,
                        "sigmas_first_last": [round(sch.sigmas[0], 6), round(sch.sigmas[steps - 1], 6)],
                        "s_per_image": round(img_s, 3), "wall_s": round(wall, 3),
                        "latent_std": round(float(zf.std()), 4)}}


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


def ceilings(pkg, lib, dev, reps=5):
    """What the matrix cores sustain here, measured in one process: the MFMA
    probe (8 independent 32x32x16 bf16 chains per wave, or 16 of 16x16x32,
    8 waves per CU, no memory traffic) on N(0,1) and on constant operands; hipBLASLt's plain
    GEMM (torch.matmul) on the gate/up shape (M x 4096 -> 24576); this
    build's plain GEMM and its gate/up GEMM with the SwiGLU epilogue on the
    same shapes (M = 8704: configuration 1, M = 16640: configuration 2).
    Best of `reps` timed groups, each on the library's stream."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def best(fn, n):
        fn()
        torch.cuda.synchronize()
        t = []
        for _ in range(reps):
            e0, e1 = ev(), ev()
            e0.record()
            for _ in range(n):
                fn()
            e1.record()
            torch.cuda.synchronize()
            t.append(e0.elapsed_time(e1) / n * 1e-3)
        return min(t)

    out = {"cus": cus, "peak_pf": PEAK_BF16 / 1e15}
    chk = torch.empty(cus * 512, dtype=torch.float32, device=dev)
    for name, ops in (("random", torch.randn(1 << 16, device=dev).to(torch.bfloat16)),
                      ("constant", torch.full((1 << 16,), 0.5, device=dev).to(torch.bfloat16))):
        for shape in (32, 16):
            fl = [0.0]

            def probe():
                fl[0] = lib.hd_mfma_probe(pkg.ptr(ops), ops.numel(), cus, 4096, shape, pkg.ptr(chk))
            t = best(probe, 5)
            out[f"mfma{shape}_probe_{name}"] = {"pf": round(fl[0] / t / 1e15, 4),
                                               "frac": round(fl[0] / t / PEAK_BF16, 4)}
    ws = torch.empty(lib.hd_gemm_ws_bytes(), dtype=torch.uint8, device=dev)
    for M in (8704, 16640):
        g = torch.Generator(device=dev).manual_seed(M)
        x = torch.randn(M, HID, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(2 * FF, HID, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        y = torch.empty(M, 2 * FF, dtype=torch.bfloat16, device=dev)
        ys = torch.empty(M, FF, dtype=torch.bfloat16, device=dev)
        flop = 2.0 * M * 2 * FF * HID
        res = {}
        t = best(lambda: torch.matmul(x, w.t(), out=y), 5)
        res["hipblaslt_plain"] = round(flop / t / 1e15, 4)
        t = best(lambda: lib.hd_linear_ws(pkg.ptr(x), pkg.ptr(w), None, pkg.ptr(y), M, 2 * FF, HID,
                                          pkg.ptr(ws), ws.numel()), 5)
        res["this_build_plain"] = round(flop / t / 1e15, 4)
        t = best(lambda: lib.hd_linear_swiglu_ws(pkg.ptr(x), pkg.ptr(w), pkg.ptr(w[FF:]), pkg.ptr(ys), M, FF,
                                                 HID, pkg.ptr(ws), ws.numel()), 5)
        res["this_build_swiglu"] = round(flop / t / 1e15, 4)
        res["unit"] = "PFLOP/s"
        out[f"gate_up_M{M}"] = res
    return out


def elementwise_bench(pkg, lib, iters):
    """HBM-bound kernels at configuration 2's sizes (S = 16640 rows, hidden
    4096, FFN 12288; 16384 image tokens x 3072 patch features; a 4096^2 RGB
    image at 32-px patches), each launched `iters` times between HIP events
    on the library's stream. Bytes are algorithmic: every operand read once
    and every result written once."""
    import torch
    dev = torch.device("cuda:0")
    S, I, P = 16640, 16384, 3072
    g = torch.Generator(device=dev).manual_seed(0)
    bfr = lambda *sh: torch.randn(*sh, generator=g, device=dev).to(torch.bfloat16)
    f32 = lambda *sh: torch.randn(*sh, generator=g, device=dev)
    x, a, y, sm = bfr(S, HID), bfr(S, HID), torch.empty(S, HID, dtype=torch.bfloat16, device=dev), \
        torch.empty(S, HID, dtype=torch.bfloat16, device=dev)
    w = bfr(HID)
    gt, up, sw = bfr(S, FF), bfr(S, FF), torch.empty(S, FF, dtype=torch.bfloat16, device=dev)
    qkv = bfr(S, (NH + 2 * NKV) * D)
    qn, kn = bfr(D), bfr(D)
    pos = torch.zeros(3, S, device=dev)
    cs = pkg.rope_table(pos, S, D, theta=1e4)
    q, k = torch.empty(NH, S, D, dtype=torch.bfloat16, device=dev), torch.empty(NKV, S, D, dtype=torch.bfloat16, device=dev)
    vt = torch.empty(NKV, D, S, dtype=torch.bfloat16, device=dev)
    qh, qo = bfr(NH, S, D), torch.empty(NH, S, D, dtype=torch.bfloat16, device=dev)
    cc, ss = f32(S, D), f32(S, D)
    hs = torch.empty(S, NH * D, dtype=torch.bfloat16, device=dev)
    z, xp = bfr(I * P), bfr(I * P)
    mo, mu, mg = f32(I * P), f32(I * P), torch.empty(I * P, device=dev)
    zn = torch.empty(I * P, dtype=torch.bfloat16, device=dev)
    img, tok = f32(3, 128 * 32, 128 * 32), torch.empty(I, P, dtype=torch.bfloat16, device=dev)
    pt = pkg.ptr
    E = S * HID
    cases = [
        ("rmsnorm [16640 x 4096]", 4 * E, lambda: lib.hd_rmsnorm(pt(x), pt(w), pt(y), S, HID, 1e-6)),
        ("add_rmsnorm [16640 x 4096] (sum and norm out)", 8 * E,
         lambda: lib.hd_add_rmsnorm(pt(x), pt(a), pt(w), pt(sm), pt(y), S, HID, 1e-6)),
        ("residual_add [16640 x 4096]", 6 * E, lambda: lib.hd_residual_add(pt(x), pt(a), pt(y), E)),
        ("swiglu [16640 x 12288]", 6 * S * FF, lambda: lib.hd_swiglu(pt(gt), pt(up), pt(sw), S * FF)),
        ("qkv_epilogue [16640 x 6144] -> q, k, V^T", 4 * S * (NH + 2 * NKV) * D + S * 64 * 8,
         lambda: lib.hd_qkv_epilogue(pt(qkv), pt(qn), pt(kn), pt(cs), pt(q), pt(k), None, pt(vt), 1, S,
                                     NH, NKV, D, 1e-6)),
        ("apply_rotary [32 x 16640 x 128] (fp32 cos/sin tables)", 4 * NH * S * D + 8 * S * D,
         lambda: lib.hd_apply_rotary(pt(qh), pt(cc), pt(ss), pt(qo), NH, S, D)),
        ("head_split [16640 x 32 x 128]", 4 * E, lambda: lib.hd_head_split(pt(hs), pt(qo), S, NH, D)),
        ("sched_vcond [16384 x 3072] bf16, bf16 -> fp32", 8 * I * P,
         lambda: lib.hd_sched_vcond(pt(z), pt(xp), 0.5, pt(mo), I * P)),
        ("sched_cfg_guided [16384 x 3072] fp32", 12 * I * P,
         lambda: lib.hd_sched_cfg_guided(pt(mo), pt(mu), 5.0, pt(mg), I * P)),
        ("sched_flow_match_step [16384 x 3072] bf16 + fp32 -> bf16", 8 * I * P,
         lambda: lib.hd_sched_flow_match_step(pt(z), pt(mo), 0.5, 0.45, pt(zn), I * P)),
        ("patchify_bf16 3 x 4096^2 fp32 -> [16384 x 3072] bf16", 6 * I * P,
         lambda: lib.hd_patchify_bf16(pt(img), pt(tok), 3, 128, 128, 32)),
    ]
    rows = []
    for name, nbytes, fn in cases:
        for _ in range(3):
            fn()
        pkg.check_prim(name)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / iters
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append({"kernel": name, "bytes": int(nbytes), "us": round(ms * 1e3, 2),
                     "GB_s": round(gbs, 1), "frac_of_8TBs": round(gbs / (PEAK_HBM / 1e9), 3)})
    print(json.dumps({"elementwise": rows, "peak_GB_s": PEAK_HBM / 1e9}))


def read_traffic(config):
    """HBM bytes per launch of the dominant kernel at `config`'s shape, from
    the committed counter summary (two rocprofv3 --pmc passes, FETCH_SIZE and
    WRITE_SIZE, scaled by a 1 GiB copy's counters); None when absent."""
    name = {"c4": "c1"}.get(config, config)
    path = os.path.join(ROOT, "profiles", f"gemm_swiglu_{name}_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def host_cpu():
    """Threads this process may run on (nproc), the CPU model, and the
    OpenMP thread count the baseline uses (all of them)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    model = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return n, model


def cpu_lora_baseline(r, welems):
    """The fp32 C oracle merging one gate-sized target (12288 x 4096, rank r)
    on the host cores, extrapolated by element count to the whole merge."""
    import numpy as np
    from oracle import oracle as orc
    threads, model = host_cpu()
    orc.lib().o1o_set_threads(threads)
    N, K = FF, HID
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    up = (rng.standard_normal((N, r)) * 0.01).astype(np.float32)
    down = (rng.standard_normal((r, K)) * 0.01).astype(np.float32)
    t0 = time.perf_counter()
    orc.lora_merge(w, up, down, 1.0)
    dt = time.perf_counter() - t0
    return {"value": round(dt * 1e3 * welems / (N * K), 1), "unit": "ms (whole merge)", "cores": threads,
            "kind": "port", "nproc": threads, "cpu_model": model,
            "omp_threads": orc.lib().o1o_num_threads(),
            "sample": f"1 target {N}x{K} rank {r} merged by the fp32 C oracle (OpenMP) in {dt:.2f}s, "
                      f"x {welems / (N * K):.1f} for all targets"}


def cpu_baseline(S, T, gh, gw, B, layers):
    """The fp32 C oracle of one decoder block on the host cores, for one CFG
    sequence at the step's real shape; steps/s extrapolated x(layers * B)."""
    import numpy as np
    import torch
    from oracle import oracle as orc
    from tests.common import make_block_weights, grid_pos, bf16
    threads, model = host_cpu()
    orc.lib().o1o_set_threads(threads)
    w = {k: v.numpy() for k, v in make_block_weights(HID, NH, NKV, FF, D, seed=0).items()}
    x = bf16(torch.randn(S, HID, generator=torch.Generator().manual_seed(1))).numpy()
    pos = grid_pos(T, gh, gw)
    cfg = orc.block_cfg(NH, NKV, HID, FF, D, theta=1e4, faithful=0)
    t0 = time.perf_counter()
    orc.decoder_block(x, pos, w, cfg)
    dt = time.perf_counter() - t0
    return {"value": round(1.0 / (dt * layers * B), 6), "unit": "steps/s", "cores": threads,
            "kind": "port", "nproc": threads, "cpu_model": model,
            "omp_threads": orc.lib().o1o_num_threads(),
            "sample": f"1 decoder block, 1 sequence of S={S} (fp32 C oracle: packed-panel AVX2 FMA "
                      f"SGEMM, OpenMP on every host thread); steps/s = 1/(t_block x {layers} blocks x "
                      f"{B} CFG sequences), a labelled extrapolation; t_block={dt:.2f}s"}


if __name__ == "__main__":
    main()

"""Benchmark configuration 4 at its real shape, as a property test: the
LoRA-merged 28-step flow-match Euler sampler with classifier-free guidance
(generate.c:1314-1455; merge lora_merge.cu:35-104) at 1024x1024 - batch 2
(cond / uncond), S = 256 text + 4096 image tokens, hidden 4096, 32 x 128
heads, 8 kv heads, FFN 12288 - on a 2-layer random-init model (the step's
per-layer work is the 36-layer model's; the layer count only scales it).
The oracle cannot run 28 steps at this size, so the checks are the ones
that do not depend on it: every value of the final latent finite, two runs
from the same seeded latent bit-identical, the general loop (hd_denoise)
bit-identical to the dedicated Euler-CFG loop (hd_denoise_euler_cfg), and
the latent moved away from the initial noise. The per-step arithmetic of
the same loops is held to the oracle in test_gpu_loop_oracle.py."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HID, NH, NKV, FF, D, NL = 4096, 32, 8, 12288, 128, 2
T, GH, GW = 256, 64, 64
I = GH * GW
S = T + I
STEPS, G, SHIFT, RANK = 28, 5.0, 3.0, 64


def test_c4_lora_merged_28_step_cfg_loop(pkg, lib, dev):
    from importlib import import_module
    synth = import_module("o1c_amd.synthetic")
    tensors = synth.build_model(n_layers=NL, seed=0, device="cuda:0")
    # rank-64 LoRA on every q/k/v/o/gate/up/down weight, merged on the GPU
    names = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
             "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    entries = (pkg.hd_lora_entry * (len(names) * NL))()
    keep = []
    k = 0
    for layer in range(NL):
        for nm in names:
            w = tensors[f"model.language_model.layers.{layer}.{nm}.weight"]
            N, K = w.shape
            up = torch.empty(N, RANK, device=dev).normal_(0, 0.01, generator=gen)
            down = torch.empty(RANK, K, device=dev).normal_(0, 0.01, generator=gen)
            keep += [up, down]
            e = entries[k]
            e.rank, e.in_dim, e.out_dim, e.alpha, e.multiplier = RANK, K, N, float(RANK), 1.0
            e.up_dev, e.down_dev, e.base_dev = up.data_ptr(), down.data_ptr(), w.data_ptr()
            k += 1
    before = tensors["model.language_model.layers.1.mlp.down_proj.weight"].clone()
    pkg.check_status(lib.hd_lora_merge_gpu(entries, k, None), "hd_lora_merge_gpu")
    torch.cuda.synchronize()
    after = tensors["model.language_model.layers.1.mlp.down_proj.weight"]
    assert not torch.equal(before, after)
    model = synth.Model(tensors, NL)
    pkg.set_block_config(theta=1e4)

    # inputs: text ids (last = timestep token), 2-D RoPE grid positions,
    # the seeded initial latent patchified to bf16 (generate.c:1295)
    gi = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 151643, (2, T), generator=gi, dtype=torch.int64)
    ids[:, -1] = synth.TMS_ID
    idsd = ids.to(dev)
    pos = np.zeros((3, S), np.float32)
    one = ctypes.c_int * 1
    assert lib.hd_seq_grid_positions(T, 1, one(GH), one(GW), one(0), None, 0.0, pkg.np_ptr(pos)) == S
    posd = torch.from_numpy(pos).to(dev)
    sch = pkg.hd_scheduler()
    n = lib.hd_scheduler_derive_default(ctypes.byref(sch), STEPS, SHIFT, 8.0)
    assert n == STEPS + 1 and sch.sigmas[0] > 0.999 and sch.sigmas[STEPS] == 0.0
    side = GH * 32
    noise = np.empty(3 * side * side, np.float32)
    lib.hd_initial_noise(42, side, side, pkg.np_ptr(noise))
    z0 = torch.empty(I, 3072, dtype=torch.bfloat16, device=dev)
    lib.hd_patchify_bf16(pkg.ptr(torch.from_numpy(noise).to(dev)), pkg.ptr(z0), 3, GH, GW, 32)
    torch.cuda.synchronize()

    wsb = torch.empty(lib.hd_forward_batched_workspace_bytes(2, S, I, NH, NKV, HID, FF, D),
                      dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsb.data_ptr()
    sb = lib.hd_denoise_run_scratch_bytes(2, S, I, STEPS)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)

    def run_general():
        z = z0.clone()
        st = lib.hd_denoise(ctypes.byref(model.binding), ctypes.byref(ws), 0, ctypes.byref(sch), STEPS, 2,
                            pkg.ptr(idsd), T, pkg.ptr(posd), 0, pkg.ptr(z), I, G, 0, 1.0, 1.0, 0.0, S, NH,
                            NKV, HID, FF, D, synth.TMS_ID, pkg.ptr(scratch), sb, None)
        pkg.check_status(st, "hd_denoise (configuration 4)")
        torch.cuda.synchronize()
        return z

    za, zb = run_general(), run_general()
    assert torch.isfinite(za.float()).all()
    assert torch.equal(za, zb), "two runs from the same latent differ"
    sig = (ctypes.c_float * (STEPS + 1))(*[sch.sigmas[i] for i in range(STEPS + 1)])
    sbe = lib.hd_denoise_scratch_bytes(S, I, STEPS)
    scr_e = torch.empty(sbe, dtype=torch.uint8, device=dev)
    ze = z0.clone()
    st = lib.hd_denoise_euler_cfg(ctypes.byref(model.binding), ctypes.byref(ws), pkg.ptr(idsd), T,
                                  pkg.ptr(posd), 0, pkg.ptr(ze), I, sig, STEPS, G, S, NH, NKV, HID, FF, D,
                                  synth.TMS_ID, pkg.ptr(scr_e), sbe, None)
    pkg.check_status(st, "hd_denoise_euler_cfg (configuration 4)")
    torch.cuda.synchronize()
    assert torch.equal(ze, za), "hd_denoise and hd_denoise_euler_cfg differ"
    d = (za.float() - z0.float())
    print(f"c4 loop: |z_final - z0| rms {float(d.pow(2).mean().sqrt()):.4f}, "
          f"z_final std {float(za.float().std()):.4f}", flush=True)
    assert float(d.abs().max()) > 0.1

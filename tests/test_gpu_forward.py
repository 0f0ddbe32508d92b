"""Whole-denoiser parity: hd_forward / hd_forward_batched (t-embedder, token
embedding + timestep-token substitution, x_embedder, blocks, final norm and
head; forward.c:190-404) on the GPU vs the CPU oracle's forward."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.common import (make_block_weights, make_forward_weights, rel_l2, cosine, grid_pos, bf16,
                          Stepper, VOCAB, TMS)

pytestmark = pytest.mark.gpu


def store_names(fw):
    L = "model.language_model."
    names = {L + "embed_tokens.weight": fw["embed_tokens"],
             "model.t_embedder1.mlp.0.weight": fw["te0_w"], "model.t_embedder1.mlp.0.bias": fw["te0_b"],
             "model.t_embedder1.mlp.2.weight": fw["te2_w"], "model.t_embedder1.mlp.2.bias": fw["te2_b"],
             "model.x_embedder.proj1.weight": fw["xe1_w"], "model.x_embedder.proj2.weight": fw["xe2_w"],
             "model.x_embedder.proj2.bias": fw["xe2_b"], "model.final_layer2.linear.weight": fw["fl_w"],
             "model.final_layer2.linear.bias": fw["fl_b"], L + "norm.weight": fw["fnorm_w"]}
    slot = {"q_proj": "self_attn.q_proj.weight", "k_proj": "self_attn.k_proj.weight",
            "v_proj": "self_attn.v_proj.weight", "o_proj": "self_attn.o_proj.weight",
            "input_ln": "input_layernorm.weight", "post_ln": "post_attention_layernorm.weight",
            "gate_proj": "mlp.gate_proj.weight", "up_proj": "mlp.up_proj.weight",
            "down_proj": "mlp.down_proj.weight", "q_norm": "self_attn.q_norm.weight",
            "k_norm": "self_attn.k_norm.weight"}
    for i, b in enumerate(fw["blocks"]):
        for k, v in b.items():
            names[f"{L}layers.{i}.{slot[k]}"] = v
    return names


@pytest.mark.parametrize("split", [False, True])
def test_forward_vs_oracle(pkg, lib, dev, split):
    nL, HID, H, KV, FF, D = 2, 512, 4, 2, 1024, 128
    T, gh, gw = 24, 8, 10
    I = gh * gw
    S = T + I
    theta = 5e6 if split else 1e4
    fw = make_forward_weights(nL, HID, H, KV, FF, D, seed=11)
    rng = np.random.default_rng(3)
    ids = rng.integers(0, 151643, T).astype(np.int64)
    ids[-1] = TMS
    ids[3] = -5          # out of range -> padding row 0 (embed.cu:24)
    vin = bf16(torch.from_numpy(rng.standard_normal((I, 3072)).astype(np.float32))).numpy()
    pos = grid_pos(T, gh, gw)
    ar = 0
    if split:
        pos[:, :T] = np.arange(T)[None]
        pos[:, T:] += 4096
        ar = T - 1
    t = 0.37
    # GPU
    pkg.set_block_config(theta=theta)
    tens = {k: v.to(dev, torch.bfloat16) for k, v in store_names(fw).items()}
    ws_store = pkg.WeightStore(tens)
    fb = pkg.hd_forward_binding()
    pkg.check_status(lib.hd_forward_resolve(ctypes.byref(ws_store.store), nL, ctypes.byref(fb)), "resolve")
    assert lib.hd_forward_num_layers(ctypes.byref(fb)) == nL
    nbytes = lib.hd_forward_workspace_bytes(S, I, H, KV, HID, FF, D, None)
    wsbuf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    plan = pkg.SdpaPlan(1, H, KV, S, D, ar_len=ar) if split else None
    if plan:
        ws.sdpa = plan.h.value
    idsd = torch.from_numpy(ids).to(dev)
    posd = torch.from_numpy(pos).to(dev)
    vind = torch.from_numpy(vin).to(dev, torch.bfloat16)
    td = torch.tensor([t], dtype=torch.float32, device=dev)
    out = torch.empty(S, 3072, dtype=torch.bfloat16, device=dev)
    diag = pkg.hd_forward_diagnostics()
    blk0 = torch.empty(S, HID, dtype=torch.bfloat16, device=dev)
    diag.after_block_0 = blk0.data_ptr()
    st = lib.hd_forward(ctypes.byref(fb), ctypes.byref(ws), pkg.ptr(idsd), T, pkg.ptr(posd), None,
                        pkg.ptr(vind), I, None, pkg.ptr(td), None, S, H, KV, HID, FF, D, TMS,
                        ctypes.byref(diag), pkg.ptr(out), None)
    pkg.check_status(st, "hd_forward")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    lib.hd_forward_binding_free(ctypes.byref(fb))
    # oracle
    ofw = {k: (v.numpy() if not isinstance(v, list) else [{kk: vv.numpy() for kk, vv in b.items()}
                                                           for b in v]) for k, v in fw.items()}
    for faithful, bound in ((1, 5e-3), (0, 1e-2)):
        cfg = orc.block_cfg(H, KV, HID, FF, D, theta=theta, faithful=faithful, ar_len=ar)
        ref, blocks = orc.forward(ofw, cfg, ids, vin, t, pos, TMS, keep_blocks=True)
        r, c = rel_l2(got, ref), cosine(got, ref)
        rb = rel_l2(blk0.float().cpu().numpy(), blocks[0])
        print(f"forward split={split} faithful={faithful}: rel_l2={r:.3e} cos={c:.7f} block0={rb:.3e}")
        assert r <= bound and c >= 0.9999 and rb <= bound


def test_forward_device_section_matches_config(pkg, lib, dev):
    """hd_forward's sec_dev (the MRoPE section in device memory, as the
    reference passes secd to every forward, generate.c:1341) gives the
    forward the same values as that section set through the block config,
    bit for bit; a non-default section ([32, 16, 16] against the default [24,
    20, 20]) changes the output, so the argument is not ignored."""
    nL, HID, H, KV, FF, D = 2, 512, 4, 2, 1024, 128
    T, gh, gw = 24, 8, 10
    I = gh * gw
    S = T + I
    fw = make_forward_weights(nL, HID, H, KV, FF, D, seed=12)
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 151643, T).astype(np.int64)
    ids[-1] = TMS
    vin = bf16(torch.from_numpy(rng.standard_normal((I, 3072)).astype(np.float32))).numpy()
    pos = grid_pos(T, gh, gw)
    tens = {k: v.to(dev, torch.bfloat16) for k, v in store_names(fw).items()}
    ws_store = pkg.WeightStore(tens)
    fb = pkg.hd_forward_binding()
    pkg.check_status(lib.hd_forward_resolve(ctypes.byref(ws_store.store), nL, ctypes.byref(fb)), "resolve")
    wsbuf = torch.empty(lib.hd_forward_workspace_bytes(S, I, H, KV, HID, FF, D, None), dtype=torch.uint8,
                        device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    idsd, posd = torch.from_numpy(ids).to(dev), torch.from_numpy(pos).to(dev)
    vind = torch.from_numpy(vin).to(dev, torch.bfloat16)
    td = torch.tensor([0.61], dtype=torch.float32, device=dev)
    sec = (32, 16, 16)
    secd = torch.tensor(sec, dtype=torch.int64, device=dev)

    def run(sec_ptr):
        out = torch.empty(S, 3072, dtype=torch.bfloat16, device=dev)
        st = lib.hd_forward(ctypes.byref(fb), ctypes.byref(ws), pkg.ptr(idsd), T, pkg.ptr(posd), None,
                            pkg.ptr(vind), I, None, pkg.ptr(td), sec_ptr, S, H, KV, HID, FF, D, TMS, None,
                            pkg.ptr(out), None)
        pkg.check_status(st, "hd_forward")
        torch.cuda.synchronize()
        return out

    pkg.set_block_config(theta=1e4)                   # default section [24, 20, 20]
    dflt = run(None)
    via_dev = run(pkg.ptr(secd))
    pkg.set_block_config(theta=1e4, section=sec)
    via_cfg = run(None)
    lib.hd_forward_binding_free(ctypes.byref(fb))
    assert torch.equal(via_dev, via_cfg)
    assert not torch.equal(via_dev, dflt)


def test_forward_batched_matches_single(pkg, lib, dev):
    import importlib
    synth = importlib.import_module("o1c_amd.synthetic")
    nL, HID, H, KV, FF, D = 2, 512, 4, 2, 1024, 128
    T, I = 16, 64
    S = T + I
    B = 2
    tens = synth.build_model(n_layers=nL, hidden=HID, heads=H, kv_heads=KV, ff=FF, seed=5)
    model = synth.Model(tens, nL)
    pkg.set_block_config(theta=1e4)
    pos = grid_pos(T, 8, 8)
    posd = torch.from_numpy(pos).to(dev)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 151643, (B, T), generator=g)
    ids[:, -1] = TMS
    idsd = ids.to(dev)
    vin = torch.randn(B, I, 3072, generator=g).to(dev, torch.bfloat16)
    td = torch.tensor([0.5, 0.8], device=dev)
    wsb = lib.hd_forward_batched_workspace_bytes(B, S, I, H, KV, HID, FF, D)
    buf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = buf.data_ptr()
    out = torch.empty(B, S, 3072, dtype=torch.bfloat16, device=dev)
    st = lib.hd_forward_batched(ctypes.byref(model.binding), ctypes.byref(ws), B, pkg.ptr(idsd), T,
                                pkg.ptr(posd), 0, pkg.ptr(vin), I, pkg.ptr(td), S, H, KV, HID, FF, D,
                                TMS, None, pkg.ptr(out), None)
    pkg.check_status(st, "batched")
    for b in range(B):
        w1 = torch.empty(lib.hd_forward_workspace_bytes(S, I, H, KV, HID, FF, D, None),
                         dtype=torch.uint8, device=dev)
        ws1 = pkg.hd_forward_workspace()
        ws1.hidden_a = w1.data_ptr()
        o1 = torch.empty(S, 3072, dtype=torch.bfloat16, device=dev)
        idb = idsd[b].contiguous()
        vb = vin[b].contiguous()
        tb = td[b:b + 1].contiguous()
        st = lib.hd_forward(ctypes.byref(model.binding), ctypes.byref(ws1), pkg.ptr(idb), T,
                            pkg.ptr(posd), None, pkg.ptr(vb), I, None, pkg.ptr(tb), None, S, H, KV,
                            HID, FF, D, TMS, None, pkg.ptr(o1), None)
        pkg.check_status(st, "single")
        torch.cuda.synchronize()
        # same kernels, M differs (B*S vs S rows): GEMM tiles differ -> a few ulps
        assert rel_l2(out[b].float().cpu(), o1.float().cpu()) < 5e-3


def test_denoise_loop_matches_stepwise(pkg, lib, dev):
    """hd_denoise_euler_cfg (device loop): (1) one step equals the step
    composed by hand from hd_forward_batched + the sampler formulas
    (sched.cu:50-72, :137-145) up to division/fma rounding; (2) a 3-step loop
    equals three chained 1-step loops bit for bit (guidance 5 and 1/sigma
    amplify any single-ulp difference chaotically, so multi-step agreement
    with a restatement is not a meaningful bound)."""
    import importlib
    synth = importlib.import_module("o1c_amd.synthetic")
    nL, HID, H, KV, FF, D = 1, 512, 4, 2, 1024, 128
    T, gh, gw = 16, 8, 8
    I = gh * gw
    S = T + I
    tens = synth.build_model(n_layers=nL, hidden=HID, heads=H, kv_heads=KV, ff=FF, seed=9)
    model = synth.Model(tens, nL)
    pkg.set_block_config(theta=1e4)
    posd = torch.from_numpy(grid_pos(T, gh, gw)).to(dev)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, 151643, (2, T), generator=g)
    ids[:, -1] = TMS
    idsd = ids.to(dev)
    z0 = torch.randn(I, 3072, generator=g).to(dev, torch.bfloat16)
    sch = pkg.hd_scheduler()
    steps = 3
    n = lib.hd_scheduler_derive_default(ctypes.byref(sch), steps, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(n)]
    wsb = lib.hd_forward_batched_workspace_bytes(2, S, I, H, KV, HID, FF, D)
    buf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = buf.data_ptr()
    sb = lib.hd_denoise_scratch_bytes(S, I, steps)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)

    def loop(z, sigmas):
        k = len(sigmas) - 1
        st = lib.hd_denoise_euler_cfg(ctypes.byref(model.binding), ctypes.byref(ws), pkg.ptr(idsd),
                                      T, pkg.ptr(posd), 0, pkg.ptr(z), I,
                                      (ctypes.c_float * len(sigmas))(*sigmas), k, 5.0, S, H, KV,
                                      HID, FF, D, TMS, pkg.ptr(scratch), sb, None)
        pkg.check_status(st, "denoise")

    z3 = z0.clone()
    loop(z3, sig)
    zc = z0.clone()
    for i in range(steps):
        loop(zc, sig[i:i + 2])
    torch.cuda.synchronize()
    assert torch.equal(z3, zc)
    assert float((z3.float() - z0.float()).abs().mean()) > 1e-3      # the latent moved
    # one step by hand
    z1 = z0.clone()
    loop(z1, sig[:2])
    out = torch.empty(2, S, 3072, dtype=torch.bfloat16, device=dev)
    vin = z0.unsqueeze(0).repeat(2, 1, 1).contiguous()
    td = torch.full((2,), float(np.float32(1.0) - np.float32(sig[0])), dtype=torch.float32, device=dev)
    st = lib.hd_forward_batched(ctypes.byref(model.binding), ctypes.byref(ws), 2, pkg.ptr(idsd), T,
                                pkg.ptr(posd), 0, pkg.ptr(vin), I, pkg.ptr(td), S, H, KV, HID, FF,
                                D, TMS, None, pkg.ptr(out), None)
    pkg.check_status(st, "forward")
    zf = z0.float()
    s32 = torch.tensor(sig[0], dtype=torch.float32)
    mo_c = (zf - out[0, T:].float()) / s32
    mo_u = (zf - out[1, T:].float()) / s32
    mo = (5.0 * mo_c.double() + ((1.0 - 5.0) * mo_u).double()).float()      # fma(g, c, (1-g) u)
    dt = float(np.float32(sig[1]) - np.float32(sig[0]))
    zr = (zf.double() + dt * mo.double()).float().to(torch.bfloat16)       # bf16(fma(dt, mo, z))
    torch.cuda.synchronize()
    assert rel_l2(z1.float().cpu(), zr.float().cpu()) < 2e-3
    assert (z1 == zr).float().mean().item() > 0.99


def test_scheduler_step_device(pkg, lib, dev):
    sch = pkg.hd_scheduler()
    lib.hd_scheduler_derive_flash(ctypes.byref(sch), 28, 1.0, 8.0)
    n = 4096
    g = torch.Generator().manual_seed(4)
    z = torch.randn(n, generator=g).to(dev, torch.bfloat16)
    mo = torch.randn(n, generator=g).to(dev)
    noise = torch.randn(n, generator=g).to(dev)
    zn = torch.empty(n, dtype=torch.bfloat16, device=dev)
    scratch = torch.empty(3 * n, device=dev)
    st = lib.hd_scheduler_step(ctypes.byref(sch), pkg.ptr(z), pkg.ptr(mo), pkg.ptr(noise), 1.0,
                               pkg.ptr(zn), n, pkg.ptr(scratch))
    pkg.check_status(st, "step")
    assert sch.step_index == 1
    sg, sn = np.float32(sch.sigmas[0]), np.float32(sch.sigmas[1])
    zf = z.float().cpu().double()
    den = (zf - mo.cpu().double() * sg).float()                       # fma(-mo, sigma, z)
    want = ((noise.cpu().double() * sn).float().double() + (1 - sn) * den.double()).float()
    want = want.to(torch.bfloat16).float()
    assert rel_l2(zn.float().cpu(), want) < 3e-3


@pytest.mark.parametrize("sampler,batch", [(0, 1), (0, 2), (1, 1), (2, 2), (2, 1)])
def test_denoise_samplers_match_stepwise(pkg, lib, dev, sampler, batch):
    """hd_denoise (Euler / flash SDE / UniPC, with and without CFG) equals the
    same steps composed by hand from the library's own calls, bit for bit:
    forward at t = 1 - sigma, velocity, CFG, then the sampler (flash: host
    noise from seed + 1 clipped at 8 std and hd_scheduler_step; UniPC: the
    per-step plan and the hd_unipc_* kernels with the three-slot history)."""
    import importlib
    synth = importlib.import_module("o1c_amd.synthetic")
    nL, HID, H, KV, FF, D = 1, 512, 4, 2, 1024, 128
    T, gh, gw = 16, 8, 8
    I = gh * gw
    S = T + I
    n = I * 3072
    tens = synth.build_model(n_layers=nL, hidden=HID, heads=H, kv_heads=KV, ff=FF, seed=9)
    model = synth.Model(tens, nL)
    pkg.set_block_config(theta=1e4)
    posd = torch.from_numpy(grid_pos(T, gh, gw)).to(dev)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 151643, (batch, T), generator=g)
    ids[:, -1] = TMS
    idsd = ids.to(dev)
    z0 = torch.randn(I, 3072, generator=g).to(dev, torch.bfloat16)
    sch = pkg.hd_scheduler()
    steps = 4
    if sampler == 1:
        lib.hd_scheduler_derive_flash(ctypes.byref(sch), steps, 3.0, 8.0)
    else:
        lib.hd_scheduler_derive_default(ctypes.byref(sch), steps, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(sch.num_steps)]
    wsb = lib.hd_forward_batched_workspace_bytes(batch, S, I, H, KV, HID, FF, D)
    buf = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = buf.data_ptr()
    sb = lib.hd_denoise_run_scratch_bytes(batch, S, I, steps)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    seed, guidance = 77, 4.0
    z = z0.clone()
    st = lib.hd_denoise(ctypes.byref(model.binding), ctypes.byref(ws), sampler, ctypes.byref(sch), steps,
                        batch, pkg.ptr(idsd), T, pkg.ptr(posd), 0, pkg.ptr(z), I, guidance, seed, 8.0, 8.0,
                        8.0, S, H, KV, HID, FF, D, TMS, pkg.ptr(scratch), sb, None)
    pkg.check_status(st, "denoise")
    torch.cuda.synchronize()
    assert float((z.float() - z0.float()).abs().mean()) > 1e-3

    # the same steps by hand
    zr = z0.clone()
    out = torch.empty(batch, S, 3072, dtype=torch.bfloat16, device=dev)
    mo_c = torch.empty(n, dtype=torch.float32, device=dev)
    mo_u = torch.empty_like(mo_c)
    mo = torch.empty_like(mo_c)
    stepper = Stepper(pkg, lib, dev, sampler, sch, n, seed)
    for i in range(steps):
        s_i = np.float32(sig[i])
        vin = zr.unsqueeze(0).repeat(batch, 1, 1).contiguous()
        td = torch.full((batch,), float(np.float32(1.0) - s_i), dtype=torch.float32, device=dev)
        st = lib.hd_forward_batched(ctypes.byref(model.binding), ctypes.byref(ws), batch, pkg.ptr(idsd), T,
                                    pkg.ptr(posd), 0, pkg.ptr(vin), I, pkg.ptr(td), S, H, KV, HID, FF,
                                    D, TMS, None, pkg.ptr(out), None)
        pkg.check_status(st, "forward")
        sg = max(float(s_i), 1e-6)
        lib.hd_sched_vcond(pkg.ptr(zr), pkg.ptr(out[0, T:]), sg, pkg.ptr(mo_c), n)
        m = mo_c
        if batch == 2:
            lib.hd_sched_vcond(pkg.ptr(zr), pkg.ptr(out[1, T:]), sg, pkg.ptr(mo_u), n)
            lib.hd_sched_cfg_guided(pkg.ptr(mo_c), pkg.ptr(mo_u), guidance, pkg.ptr(mo), n)
            m = mo
        stepper.step(i, zr, m)
    torch.cuda.synchronize()
    assert torch.equal(z, zr)

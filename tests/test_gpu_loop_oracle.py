"""The device denoise loops against an independent CPU loop (generate.c:
1314-1455): each step feeds t = 1 - sigma_i to the oracle's forward
(forward.c:253-397) of the conditional and unconditional sequences, forms
mo = (z - x_pred[img]) / max(sigma_i, 1e-6) (sched.cu:35-41), combines
(1 - g) mo_u + g mo_c (sched.cu:137-145) and steps z with the flow-match
Euler update (sched.cu:44-52) or the flash SDE step: noise from torch's CPU
generator seeded with seed + 1 and clipped at clip x its sample std
(generate.c:1295-1296, :1419-1437), s_noise ramped over the steps
(scheduler.c:197-208), z' = bf16(sigma' n s + (1 - sigma') (z - sigma mo))
(sched.cu:14-28, scheduler.c:71-99). The oracle runs in its bf16-faithful
mode; the loop's own calls (hd_forward, hd_sched_*) are not used on the CPU
side.

Bound: the accumulated update z_final - z0 within rel-L2 1e-2 of the oracle
loop's, or, when guidance amplifies the per-forward rounding (g = 5 turns
the two branches' bf16 noise into 6.4x their size: 5 mo_c - 4 mo_u), within
1.5x the spread between the oracle's own fp32 and bf16-faithful loops on
the same inputs - the rounding the reference itself carries."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.common import make_forward_weights, grid_pos, rel_l2, cosine, bf16, TMS

pytestmark = pytest.mark.gpu

nL, HID, H, KV, FF, D = 2, 512, 4, 2, 1024, 128
GH, GW = 8, 8
I = GH * GW
STEPS = 3


def oracle_loop(fw, cfg, seqs, z0, sig, guidance, sampler, seed=0, clip=0.0, sn=(1.0, 1.0), unipc=None):
    """seqs: [(ids, pos, T)] or [(ids, pos, T, cfg)] - one (conditional) or
    two (+ unconditional); a fourth item overrides `cfg` for that sequence
    (its own causal prefix).
    unipc: (lib, pkg, sched) for sampler 2 - the per-step plan comes from
    hd_scheduler_unipc_plan (host code pinned bit-exact against the
    reference's scheduler.c by the CPU tests)."""
    z = z0.copy()
    gen = torch.Generator().manual_seed(seed + 1)
    n = z.size
    this_order = lower = have = 0
    last = slot1 = slot2 = None
    for i in range(STEPS):
        s_i = np.float32(sig[i])
        sg = max(float(s_i), 1e-6)
        t = float(np.float32(1.0) - s_i)
        mos = []
        for sq in seqs:
            ids, pos, T = sq[:3]
            xp = orc.forward(fw, sq[3] if len(sq) > 3 else cfg, ids, z, t, pos, TMS)[T:]
            mos.append(orc.sched_vcond(z, xp, sg))
        mo = orc.sched_cfg_guided(mos[0], mos[1], guidance) if len(mos) == 2 else mos[0]
        if sampler == 0:
            z = orc.sched_flow_match_step(z, mo, sig[i], sig[i + 1])
        elif sampler == 2:
            # generate.c:1360-1410: convert, correct (from step 1 on, with
            # history), predict, z = bf16(prediction), rotate the history
            lib, pkg, sch = unipc
            pl = pkg.hd_unipc_plan()
            lib.hd_scheduler_unipc_plan(ctypes.byref(sch), i, this_order, lower, ctypes.byref(pl))
            conv = orc.unipc_convert(z, mo, float(s_i))
            corr = z
            if i > 0 and this_order > 0 and have:
                corr = orc.unipc_correct(last, slot1, slot2, conv, pl.c_sig_t, pl.c_sig_s0, pl.c_alpha_t,
                                         pl.c_h_phi_1, pl.c_B_h, pl.c_rhos0, pl.c_rhos1, pl.c_inv_rks0,
                                         pl.corr_order)
            last = corr.copy()
            pred = orc.unipc_predict(corr, conv, slot1 if slot1 is not None else conv, pl.p_sig_t,
                                     pl.p_sig_s0, pl.p_alpha_t, pl.p_h_phi_1, pl.p_B_h, pl.p_rhos_p,
                                     pl.p_inv_rks0, pl.pred_order)
            z = bf16(torch.from_numpy(pred)).numpy()
            slot2, slot1 = slot1, conv
            this_order, lower, have = pl.next_this_order, pl.next_lower_order, 1
        else:
            noise = torch.randn(n, generator=gen).numpy().astype(np.float64)
            if clip > 0:
                cv = np.float32(clip) * np.float32(np.std(noise, ddof=1))
                noise = np.clip(noise, -float(cv), float(cv))
            noise = noise.astype(np.float32).reshape(z.shape)
            s_noise = np.float32(sn[0] + (sn[1] - sn[0]) * i / (STEPS - 1))
            sn1 = np.float32(sig[i + 1])
            den = z - mo * s_i
            z = bf16(torch.from_numpy((sn1 * noise) * s_noise + (np.float32(1) - sn1) * den)).numpy()
    return z


def setup(pkg, lib, dev):
    from tests.test_gpu_forward import store_names
    fw = make_forward_weights(nL, HID, H, KV, FF, D, seed=71)
    pkg.set_block_config(theta=1e4)
    tens = {k: v.to(dev, torch.bfloat16) for k, v in store_names(fw).items()}
    store = pkg.WeightStore(tens)
    fb = pkg.hd_forward_binding()
    pkg.check_status(lib.hd_forward_resolve(ctypes.byref(store.store), nL, ctypes.byref(fb)), "resolve")
    ofw = {k: v.numpy() for k, v in fw.items() if k != "blocks"}
    ofw["blocks"] = [{k: v.numpy() for k, v in b.items()} for b in fw["blocks"]]
    cfg = orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=1)
    cfg32 = orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=0)
    return (tens, store), fb, ofw, (cfg, cfg32)


def workspace(pkg, lib, dev, B, S):
    buf = torch.empty(lib.hd_forward_batched_workspace_bytes(B, S, I, H, KV, HID, FF, D),
                      dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = buf.data_ptr()
    return ws, buf


def compare(z, z0, zo, zo32, tag):
    d, do, d32 = z - z0, zo - z0, zo32 - z0
    r, c = rel_l2(d, do), cosine(d, do)
    spread = rel_l2(d32, do)
    print(f"{tag}: update rel_l2={r:.3e} cos={c:.7f} (oracle fp32 vs faithful: {spread:.3e}; "
          f"vs fp32 {rel_l2(d, d32):.3e})", flush=True)
    assert r <= max(1e-2, 1.5 * spread), (tag, r, spread)
    assert c >= 0.9997, (tag, c)


def ids_for(T, seed):
    ids = np.random.default_rng(seed).integers(0, 151643, T).astype(np.int64)
    ids[-1] = TMS
    return ids


@pytest.mark.parametrize("sampler", [0, 1, 2])
def test_denoise_cfg_equal_length_vs_oracle_loop(pkg, lib, dev, sampler):
    """hd_denoise, batch 2: cond and uncond ids of one length (Euler, flash
    SDE, FlowUniPC over the default schedule)."""
    keep, fb, ofw, cfg = setup(pkg, lib, dev)
    T = 16
    S = T + I
    ids = np.stack([ids_for(T, 1), ids_for(T, 2)])
    pos = grid_pos(T, GH, GW)
    sch = pkg.hd_scheduler()
    if sampler == 2:
        lib.hd_scheduler_derive_default(ctypes.byref(sch), STEPS, 3.0, 8.0)
    else:
        lib.hd_scheduler_derive_flash(ctypes.byref(sch), STEPS, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(sch.num_steps)]
    z0 = bf16(torch.randn(I, 3072, generator=torch.Generator().manual_seed(5))).numpy()
    g, seed, clip, sn = 5.0, 77, 2.0, (1.0, 0.5)
    ws, wbuf = workspace(pkg, lib, dev, 2, S)
    sb = lib.hd_denoise_run_scratch_bytes(2, S, I, STEPS)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    zd = torch.from_numpy(z0).to(dev, torch.bfloat16)
    idsd, posd = torch.from_numpy(ids).to(dev), torch.from_numpy(pos).to(dev)
    st = lib.hd_denoise(ctypes.byref(fb), ctypes.byref(ws), sampler, ctypes.byref(sch), STEPS, 2, pkg.ptr(idsd),
                        T, pkg.ptr(posd), 0, pkg.ptr(zd), I, g, seed, sn[0], sn[1], clip, S, H, KV, HID, FF,
                        D, TMS, pkg.ptr(scratch), sb, None)
    pkg.check_status(st, "hd_denoise")
    torch.cuda.synchronize()
    z = zd.float().cpu().numpy()
    sq = [(ids[0], pos, T), (ids[1], pos, T)]
    up = (lib, pkg, sch)
    zo = oracle_loop(ofw, cfg[0], sq, z0, sig, g, sampler, seed, clip, sn, unipc=up)
    zo32 = oracle_loop(ofw, cfg[1], sq, z0, sig, g, sampler, seed, clip, sn, unipc=up)
    compare(z, z0, zo, zo32, f"hd_denoise sampler {sampler}")
    lib.hd_forward_binding_free(ctypes.byref(fb))


@pytest.mark.parametrize("sampler", [0, 1, 2])
def test_denoise_cfg_own_uncond_sequence_vs_oracle_loop(pkg, lib, dev, sampler):
    """hd_denoise_cfg: the unconditional branch is a shorter sequence of its
    own (the reference's " " caption), with its own positions and
    workspace."""
    keep, fb, ofw, cfg = setup(pkg, lib, dev)
    T, Tu = 20, 6
    S, Su = T + I, Tu + I
    ids, idu = ids_for(T, 3), ids_for(Tu, 4)
    pos, posu = grid_pos(T, GH, GW), grid_pos(Tu, GH, GW)
    sch = pkg.hd_scheduler()
    if sampler == 2:   # FlowUniPC: the reference's default schedule (generate.c:1335-1345)
        lib.hd_scheduler_derive_default(ctypes.byref(sch), STEPS, 3.0, 8.0)
    else:
        lib.hd_scheduler_derive_flash(ctypes.byref(sch), STEPS, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(sch.num_steps)]
    z0 = bf16(torch.randn(I, 3072, generator=torch.Generator().manual_seed(6))).numpy()
    g, seed, clip, sn = 5.0, 91, 2.0, (1.0, 0.5)
    ws, wb = workspace(pkg, lib, dev, 1, S)
    wsu, wbu = workspace(pkg, lib, dev, 1, Su)
    sb = lib.hd_denoise_cfg_scratch_bytes(S, Su, I, STEPS)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    zd = torch.from_numpy(z0).to(dev, torch.bfloat16)
    dv = lambda a: torch.from_numpy(a).to(dev)
    idsd, idud, posd, posud = dv(ids), dv(idu), dv(pos), dv(posu)
    st = lib.hd_denoise_cfg(ctypes.byref(fb), ctypes.byref(ws), ctypes.byref(wsu), sampler, ctypes.byref(sch),
                            STEPS, pkg.ptr(idsd), T, pkg.ptr(posd), 0, S, pkg.ptr(idud), Tu, pkg.ptr(posud), 0,
                            Su, pkg.ptr(zd), I, g, seed, sn[0], sn[1], clip, H, KV, HID, FF, D, TMS,
                            pkg.ptr(scratch), sb, None)
    pkg.check_status(st, "hd_denoise_cfg")
    torch.cuda.synchronize()
    z = zd.float().cpu().numpy()
    sq = [(ids, pos, T), (idu, posu, Tu)]
    up = (lib, pkg, sch)
    zo = oracle_loop(ofw, cfg[0], sq, z0, sig, g, sampler, seed, clip, sn, unipc=up)
    zo32 = oracle_loop(ofw, cfg[1], sq, z0, sig, g, sampler, seed, clip, sn, unipc=up)
    compare(z, z0, zo, zo32, f"hd_denoise_cfg sampler {sampler}")
    # padding the unconditional prompt to the conditional length is not the same
    zp = oracle_loop(ofw, cfg[0], [(ids, pos, T), (np.concatenate([idu, ids_for(T - Tu, 4)]), pos, T)],
                     z0, sig, g, sampler, seed, clip, sn, unipc=up)
    assert rel_l2(zp - z0, zo - z0) > 2e-2
    # argument checks return before any device call
    assert lib.hd_denoise_cfg(ctypes.byref(fb), ctypes.byref(ws), ctypes.byref(ws), sampler, ctypes.byref(sch),
                              STEPS, pkg.ptr(idsd), T, pkg.ptr(posd), 0, S, pkg.ptr(idud), Tu, pkg.ptr(posud),
                              0, Su, pkg.ptr(zd), I, g, seed, 1.0, 1.0, 0.0, H, KV, HID, FF, D, TMS,
                              pkg.ptr(scratch), sb, None) == pkg.HD_ERR_MISMATCH
    assert lib.hd_denoise_cfg(ctypes.byref(fb), ctypes.byref(ws), ctypes.byref(wsu), sampler, ctypes.byref(sch),
                              STEPS, pkg.ptr(idsd), T, pkg.ptr(posd), 0, S, pkg.ptr(idud), Tu, pkg.ptr(posud),
                              0, Su + 1, pkg.ptr(zd), I, g, seed, 1.0, 1.0, 0.0, H, KV, HID, FF, D, TMS,
                              pkg.ptr(scratch), sb, None) == pkg.HD_ERR_MISMATCH
    lib.hd_forward_binding_free(ctypes.byref(fb))


def test_denoise_unguided_vs_oracle_loop(pkg, lib, dev):
    """hd_denoise, batch 1 (no guidance, no amplification): the plain
    per-step bound holds for the update."""
    keep, fb, ofw, cfg = setup(pkg, lib, dev)
    T = 16
    S = T + I
    ids = ids_for(T, 8)
    pos = grid_pos(T, GH, GW)
    sch = pkg.hd_scheduler()
    lib.hd_scheduler_derive_flash(ctypes.byref(sch), STEPS, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(sch.num_steps)]
    z0 = bf16(torch.randn(I, 3072, generator=torch.Generator().manual_seed(9))).numpy()
    ws, wbuf = workspace(pkg, lib, dev, 1, S)
    sb = lib.hd_denoise_run_scratch_bytes(1, S, I, STEPS)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    zd = torch.from_numpy(z0).to(dev, torch.bfloat16)
    idsd, posd = torch.from_numpy(ids).to(dev), torch.from_numpy(pos).to(dev)
    st = lib.hd_denoise(ctypes.byref(fb), ctypes.byref(ws), 0, ctypes.byref(sch), STEPS, 1, pkg.ptr(idsd),
                        T, pkg.ptr(posd), 0, pkg.ptr(zd), I, 1.0, 0, 1.0, 1.0, 0.0, S, H, KV, HID, FF,
                        D, TMS, pkg.ptr(scratch), sb, None)
    pkg.check_status(st, "hd_denoise B=1")
    torch.cuda.synchronize()
    z = zd.float().cpu().numpy()
    zo = oracle_loop(ofw, cfg[0], [(ids, pos, T)], z0, sig, 1.0, 0)
    d, do = z - z0, zo - z0
    r, c = rel_l2(d, do), cosine(d, do)
    print(f"unguided: update rel_l2={r:.3e} cos={c:.7f}", flush=True)
    assert r <= 1e-2 and c >= 0.9999, (r, c)
    lib.hd_forward_binding_free(ctypes.byref(fb))


def test_denoise_cfg_causal_prefixes_vs_oracle_loop(pkg, lib, dev):
    """hd_denoise_cfg with the reference's text-to-image masks on both
    branches: each sequence's text rows attend causally (rows < T - 1 see
    keys <= row; generate.c:1119-1120 builds maskd[0] and maskd[1] with
    ar_len = text_len - 1 each), through each workspace's own split plan."""
    keep, fb, ofw, cfg = setup(pkg, lib, dev)
    T, Tu = 20, 6
    S, Su = T + I, Tu + I
    ids, idu = ids_for(T, 13), ids_for(Tu, 14)
    pos, posu = grid_pos(T, GH, GW), grid_pos(Tu, GH, GW)
    sch = pkg.hd_scheduler()
    lib.hd_scheduler_derive_flash(ctypes.byref(sch), STEPS, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(sch.num_steps)]
    z0 = bf16(torch.randn(I, 3072, generator=torch.Generator().manual_seed(16))).numpy()
    g = 5.0
    ws, wb = workspace(pkg, lib, dev, 1, S)
    wsu, wbu = workspace(pkg, lib, dev, 1, Su)
    sb = lib.hd_denoise_cfg_scratch_bytes(S, Su, I, STEPS)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    zd = torch.from_numpy(z0).to(dev, torch.bfloat16)
    dv = lambda a: torch.from_numpy(a).to(dev)
    idsd, idud, posd, posud = dv(ids), dv(idu), dv(pos), dv(posu)
    st = lib.hd_denoise_cfg(ctypes.byref(fb), ctypes.byref(ws), ctypes.byref(wsu), 0, ctypes.byref(sch),
                            STEPS, pkg.ptr(idsd), T, pkg.ptr(posd), T - 1, S, pkg.ptr(idud), Tu, pkg.ptr(posud),
                            Tu - 1, Su, pkg.ptr(zd), I, g, 0, 1.0, 1.0, 0.0, H, KV, HID, FF, D, TMS,
                            pkg.ptr(scratch), sb, None)
    pkg.check_status(st, "hd_denoise_cfg (causal prefixes)")
    torch.cuda.synchronize()
    z = zd.float().cpu().numpy()
    mk = lambda ar, faithful: orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=faithful, ar_len=ar)
    sq = [(ids, pos, T, mk(T - 1, 1)), (idu, posu, Tu, mk(Tu - 1, 1))]
    sq32 = [(ids, pos, T, mk(T - 1, 0)), (idu, posu, Tu, mk(Tu - 1, 0))]
    zo = oracle_loop(ofw, cfg[0], sq, z0, sig, g, 0)
    zo32 = oracle_loop(ofw, cfg[1], sq32, z0, sig, g, 0)
    compare(z, z0, zo, zo32, "hd_denoise_cfg causal prefixes")
    # the prefixes matter: the same loop with full attention is a different result
    zf = oracle_loop(ofw, cfg[0], [(ids, pos, T), (idu, posu, Tu)], z0, sig, g, 0)
    assert rel_l2(zf - z0, zo - z0) > 1e-3
    lib.hd_forward_binding_free(ctypes.byref(fb))


@pytest.mark.parametrize("loop", ["hd_denoise", "hd_denoise_cfg"])
def test_first_guided_velocity_vs_oracle(pkg, lib, dev, loop):
    """The guided velocity of one step, where the device loop and the oracle
    see the same latent, at the north-star bound (rel-L2 <= 1e-2, cosine >=
    0.9999). One Euler step from sigma 1 to 0 gives z1 = bf16(z0 - mo), so
    z0 - z1 is the guided velocity (5 mo_c - 4 mo_u) up to the bf16 rounding
    of z1, which the oracle applies too."""
    keep, fb, ofw, cfg = setup(pkg, lib, dev)
    sch = pkg.hd_scheduler()
    pkg.check_status(lib.hd_scheduler_init(ctypes.byref(sch), (ctypes.c_float * 2)(1.0, 0.0), 2, 0.0),
                     "scheduler")
    z0 = bf16(torch.randn(I, 3072, generator=torch.Generator().manual_seed(21))).numpy()
    zd = torch.from_numpy(z0).to(dev, torch.bfloat16)
    dv = lambda a: torch.from_numpy(a).to(dev)
    g = 5.0
    if loop == "hd_denoise":
        T = Tu = 16
        ids, idu = ids_for(T, 22), ids_for(T, 23)
        pos = posu = grid_pos(T, GH, GW)
        S = T + I
        ws, wbuf = workspace(pkg, lib, dev, 2, S)
        sb = lib.hd_denoise_run_scratch_bytes(2, S, I, 1)
        scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
        idsd, posd = dv(np.stack([ids, idu])), dv(pos)
        st = lib.hd_denoise(ctypes.byref(fb), ctypes.byref(ws), 0, ctypes.byref(sch), 1, 2, pkg.ptr(idsd), T,
                            pkg.ptr(posd), 0, pkg.ptr(zd), I, g, 0, 1.0, 1.0, 0.0, S, H, KV, HID, FF, D, TMS,
                            pkg.ptr(scratch), sb, None)
    else:
        T, Tu = 20, 6
        ids, idu = ids_for(T, 24), ids_for(Tu, 25)
        pos, posu = grid_pos(T, GH, GW), grid_pos(Tu, GH, GW)
        S, Su = T + I, Tu + I
        ws, wb = workspace(pkg, lib, dev, 1, S)
        wsu, wbu = workspace(pkg, lib, dev, 1, Su)
        sb = lib.hd_denoise_cfg_scratch_bytes(S, Su, I, 1)
        scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
        idsd, idud, posd, posud = dv(ids), dv(idu), dv(pos), dv(posu)
        st = lib.hd_denoise_cfg(ctypes.byref(fb), ctypes.byref(ws), ctypes.byref(wsu), 0, ctypes.byref(sch), 1,
                                pkg.ptr(idsd), T, pkg.ptr(posd), 0, S, pkg.ptr(idud), Tu, pkg.ptr(posud), 0, Su,
                                pkg.ptr(zd), I, g, 0, 1.0, 1.0, 0.0, H, KV, HID, FF, D, TMS, pkg.ptr(scratch),
                                sb, None)
    pkg.check_status(st, loop)
    torch.cuda.synchronize()
    v = z0 - zd.float().cpu().numpy()
    xc = orc.forward(ofw, cfg[0], ids, z0, 0.0, pos, TMS)[T:]
    xu = orc.forward(ofw, cfg[0], idu, z0, 0.0, posu, TMS)[Tu:]
    mo = orc.sched_cfg_guided(orc.sched_vcond(z0, xc, 1.0), orc.sched_vcond(z0, xu, 1.0), g)
    vo = z0 - orc.sched_flow_match_step(z0, mo, 1.0, 0.0)
    r, c = rel_l2(v, vo), cosine(v, vo)
    print(f"{loop}: first guided velocity rel_l2={r:.3e} cos={c:.7f}", flush=True)
    assert r <= 1e-2 and c >= 0.9999, (r, c)
    lib.hd_forward_binding_free(ctypes.byref(fb))


def test_final_latent_fails_closed(pkg, lib, dev):
    """generate.c:1474-1496: a NaN/Inf in the final latent, or (the
    reference's default check) a value outside [-2, 2], fails the loop with
    HD_ERR_MISSING (generate.c:1546) and the reference's message. One Euler
    step with sigma 1 -> 1 leaves z = bf16(z + 0 * mo) = z, so the final
    latent is the input the test chose."""
    keep, fb, ofw, cfg = setup(pkg, lib, dev)
    sch = pkg.hd_scheduler()
    pkg.check_status(lib.hd_scheduler_init(ctypes.byref(sch), (ctypes.c_float * 2)(1.0, 1.0), 2, 0.0),
                     "scheduler")
    T = 16
    S = T + I
    ids, pos = ids_for(T, 31), grid_pos(T, GH, GW)
    ws, wbuf = workspace(pkg, lib, dev, 1, S)
    sb = lib.hd_denoise_run_scratch_bytes(1, S, I, 1)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    idsd, posd = torch.from_numpy(ids).to(dev), torch.from_numpy(pos).to(dev)
    base = torch.rand(I, 3072, generator=torch.Generator().manual_seed(32)) * 3.0 - 1.5   # [-1.5, 1.5)

    def run(z, mode):
        assert lib.hd_denoise_set_output_check(mode) in (0, 1, 2)
        zd = z.to(dev, torch.bfloat16)
        st = lib.hd_denoise(ctypes.byref(fb), ctypes.byref(ws), 0, ctypes.byref(sch), 1, 1, pkg.ptr(idsd), T,
                            pkg.ptr(posd), 0, pkg.ptr(zd), I, 1.0, 0, 1.0, 1.0, 0.0, S, H, KV, HID, FF, D, TMS,
                            pkg.ptr(scratch), sb, None)
        torch.cuda.synchronize()
        return st, lib.hd_last_error().decode(), zd

    st, msg, zd = run(base, 2)
    assert st == pkg.HD_OK, msg
    assert torch.equal(zd.cpu(), base.to(torch.bfloat16))      # sigma 1 -> 1 keeps z
    hi = base.clone()
    hi[10, 7] = 2.5
    st, msg, _ = run(hi, 2)
    assert st == pkg.HD_ERR_MISSING and "out of bounds" in msg and "2.5000" in msg, (st, msg)
    lo = base.clone()
    lo[5, 3000] = -2.25
    st, msg, _ = run(lo, 2)
    assert st == pkg.HD_ERR_MISSING and "[-2.2500," in msg, (st, msg)
    assert run(hi, 1)[0] == pkg.HD_OK           # mode 1: NaN/Inf only
    nan = base.clone()
    nan[I - 1, 3071] = float("nan")
    st, msg, _ = run(nan, 1)
    assert st == pkg.HD_ERR_MISSING and "NaN/Inf" in msg, (st, msg)
    inf = base.clone()
    inf[0, 0] = float("inf")
    st, msg, _ = run(inf, 2)
    assert st == pkg.HD_ERR_MISSING and "NaN/Inf" in msg, (st, msg)
    assert run(nan, 0)[0] == pkg.HD_OK          # mode 0: off
    assert lib.hd_denoise_set_output_check(3) == -1
    lib.hd_forward_binding_free(ctypes.byref(fb))

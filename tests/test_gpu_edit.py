"""hd_denoise_visual: the edit / personalize loop (generate.c:792-935) on the
device. GPU (marked): the loop equals the same steps composed by hand from
hd_forward with vision conditioning over [text | target | references], the
target rows' velocity and the sampler, bit for bit; with the references'
x_embedder rows cached in the workspace (generate.c:792-805) it equals its
own composition bit for bit and the patch path within bf16 noise. CPU: the
argument checks, which return before any device call."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

from tests.common import Stepper, grid_pos, rel_l2

TMS, IMG_PAD = 151673, 151655
nL, HID, H, KV, FF, D = 1, 512, 4, 2, 1024, 128
T, GH, GW, NREF = 16, 8, 8, 32
IT = GH * GW
S = T + IT + NREF


def _visual(pkg, dev, g):
    vrows = [3, 4, 5, 6]
    emb = torch.randn(len(vrows), HID, generator=g).to(dev, torch.bfloat16)
    ds = [(torch.randn(len(vrows), HID, generator=g) * 0.5).to(dev, torch.bfloat16) for _ in range(3)]
    vmask = torch.zeros(S, dtype=torch.uint8)
    vmask[vrows] = 1
    vmask = vmask.to(dev)
    vc = pkg.hd_visual_cond()
    vc.image_embeds = emb.data_ptr()
    for j in range(3):
        vc.deepstack[j] = ds[j].data_ptr()
    vc.visual_mask = vmask.data_ptr()
    vc.v_tokens = len(vrows)
    return vc, vrows, (emb, ds, vmask)


def _cache_refs(pkg, lib, dev, bw, ref):
    """The references' x_embedder rows, as generate.c:792-805 computes them."""
    stg = torch.empty(NREF, 1024, dtype=torch.bfloat16, device=dev)
    xe = torch.empty(NREF, HID, dtype=torch.bfloat16, device=dev)
    lib.hd_linear(pkg.ptr(ref), bw.xe1_w, None, pkg.ptr(stg), NREF, 1024, 3072, 1)
    lib.hd_linear(pkg.ptr(stg), bw.xe2_w, bw.xe2_b, pkg.ptr(xe), NREF, HID, 1024, 1)
    pkg.check_prim("x_embedder cache")
    return xe


@pytest.mark.gpu
@pytest.mark.parametrize("sampler,cached", [(1, False), (0, True), (2, False), (1, True)])
def test_denoise_visual_matches_stepwise(pkg, lib, dev, sampler, cached):
    synth = importlib.import_module("o1c_amd.synthetic")
    tens = synth.build_model(n_layers=nL, hidden=HID, heads=H, kv_heads=KV, ff=FF, seed=21)
    model = synth.Model(tens, nL)
    pkg.set_block_config(theta=1e4)
    g = torch.Generator().manual_seed(8)
    # text rows, the target grid and the reference grid after it
    pos = np.concatenate([grid_pos(T, GH, GW), grid_pos(0, 4, 8, row_offset=GH)[:, :NREF]], 1)
    assert pos.shape[1] == S
    posd = torch.from_numpy(np.ascontiguousarray(pos)).to(dev)
    vc, vrows, keep = _visual(pkg, dev, g)
    ids = torch.randint(0, 151643, (T,), generator=g)
    ids[vrows] = IMG_PAD
    ids[-1] = TMS
    idsd = ids.to(dev)
    z0 = torch.randn(IT, 3072, generator=g).to(dev, torch.bfloat16)
    ref = torch.randn(NREF, 3072, generator=g).to(dev, torch.bfloat16)
    sch = pkg.hd_scheduler()
    steps = 3
    # the edit loop's default runs the flash step over the default schedule;
    # UniPC takes the default schedule, Euler the flash ramp
    if sampler == 0:
        lib.hd_scheduler_derive_flash(ctypes.byref(sch), steps, 3.0, 8.0)
    else:
        lib.hd_scheduler_derive_default(ctypes.byref(sch), steps, 3.0, 8.0)
    sig = [sch.sigmas[i] for i in range(sch.num_steps)]
    wsbuf = torch.empty(lib.hd_forward_workspace_bytes(S, IT + NREF, H, KV, HID, FF, D, None),
                        dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    xe = None
    if cached:
        xe = _cache_refs(pkg, lib, dev, model.binding, ref)
        ws.xe_ref, ws.n_ref = xe.data_ptr(), NREF
    sb = lib.hd_denoise_run_scratch_bytes(1, S, IT + NREF, steps)
    scratch = torch.empty(sb, dtype=torch.uint8, device=dev)
    seed = 123

    def run(ws_):
        z = z0.clone()
        st = lib.hd_denoise_visual(ctypes.byref(model.binding), ctypes.byref(ws_), sampler, ctypes.byref(sch),
                                   steps, pkg.ptr(idsd), T, pkg.ptr(posd), None, ctypes.byref(vc), pkg.ptr(z),
                                   IT, pkg.ptr(ref), NREF, seed, 8.0, 8.0, 8.0, S, H, KV, HID, FF, D, TMS,
                                   pkg.ptr(scratch), sb, None)
        pkg.check_status(st, "denoise_visual")
        torch.cuda.synchronize()
        return z

    z = run(ws)
    assert float((z.float() - z0.float()).abs().mean()) > 1e-3

    # the same steps by hand: vinputs = cat(z, ref), target rows of the output
    n = IT * 3072
    zr = z0.clone()
    out = torch.empty(S, 3072, dtype=torch.bfloat16, device=dev)
    mo = torch.empty(n, dtype=torch.float32, device=dev)
    stepper = Stepper(pkg, lib, dev, sampler, sch, n, seed)
    for i in range(steps):
        s_i = np.float32(sig[i])
        vin = torch.cat([zr, ref]).contiguous()
        td = torch.tensor([float(np.float32(1.0) - s_i)], dtype=torch.float32, device=dev)
        st = lib.hd_forward(ctypes.byref(model.binding), ctypes.byref(ws), pkg.ptr(idsd), T, pkg.ptr(posd),
                            None, pkg.ptr(vin), IT + NREF, ctypes.byref(vc), pkg.ptr(td), None, S, H, KV,
                            HID, FF, D, TMS, None, pkg.ptr(out), None)
        pkg.check_status(st, "forward")
        lib.hd_sched_vcond(pkg.ptr(zr), pkg.ptr(out[T:T + IT]), max(float(s_i), 1e-6), pkg.ptr(mo), n)
        stepper.step(i, zr, mo)
    torch.cuda.synchronize()
    assert torch.equal(z, zr)

    if cached:
        # the cache stands in for the patches: same loop without it
        plain = pkg.hd_forward_workspace()
        plain.hidden_a = wsbuf.data_ptr()
        zp = run(plain)
        r = rel_l2(z.float().cpu().numpy(), zp.float().cpu().numpy())
        print(f"cached vs patches: rel_l2={r:.3e}")
        assert r < 1e-2


def test_denoise_visual_argument_checks(pkg, lib):
    bw = pkg.hd_forward_binding()
    ws = pkg.hd_forward_workspace()
    sch = pkg.hd_scheduler()
    lib.hd_scheduler_derive_flash(ctypes.byref(sch), 4, 3.0, 8.0)
    fake = ctypes.c_void_p(0x1000)

    def call(ws_, T_, it, ref, nref, S_, sampler=1, z=fake):
        return lib.hd_denoise_visual(ctypes.byref(bw), ctypes.byref(ws_), sampler, ctypes.byref(sch), 4, fake,
                                     T_, fake, None, None, z, it, ref, nref, 0, 1.0, 1.0, 0.0, S_, H, KV,
                                     HID, FF, D, TMS, fake, 1 << 20, None)

    assert call(ws, 8, 64, fake, 16, 88, z=None) == pkg.HD_ERR_MISSING
    assert call(ws, 8, 64, fake, 16, 88, sampler=3) == pkg.HD_ERR_UNSUPPORTED
    assert call(ws, 8, 64, fake, 16, 90) == pkg.HD_ERR_MISMATCH          # 8 + 64 + 16 != 90
    assert b"reference" in lib.hd_last_error()
    assert call(ws, 8, 64, None, 16, 88) == pkg.HD_ERR_MISSING           # no patches, no cache
    ws.xe_ref, ws.n_ref = 0x2000, 8
    assert call(ws, 8, 64, fake, 16, 88) == pkg.HD_ERR_MISMATCH          # cache of another size
    assert b"caches 8" in lib.hd_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("cached", [True, False])
def test_edit_forward_multi_reference_vs_oracle(pkg, lib, dev, cached):
    """The edit configuration's layout at reduced width through hd_forward:
    text rows at position 0 with image-pad rows (vision conditioning:
    masked scatter + DeepStack into blocks 0-2) and the timestep token, the
    target grid, then two reference grids at +64 and +128 rows
    (hd_seq_grid_positions), full bidirectional attention; the references'
    x_embedder rows cached in the workspace (forward.c:301-313) or computed
    from the patches. Against the oracle's forward, which embeds every
    image row itself (forward.c:253-397)."""
    from tests.common import make_forward_weights, bf16, cosine
    from tests.test_gpu_forward import store_names
    from oracle import oracle as orc
    nLf, Tf, gh, gw, R = 4, 24, 8, 8, 2
    It = gh * gw
    nref = R * It
    I = It + nref
    Sf = Tf + I
    fw = make_forward_weights(nLf, HID, H, KV, FF, D, seed=61)
    rng = np.random.default_rng(62)
    ids = rng.integers(0, 151643, Tf).astype(np.int64)
    vrows = [2, 3, 4, 5, 6, 7, 8, 9]
    ids[vrows] = IMG_PAD
    ids[-1] = TMS
    vmask = np.zeros(Sf, np.uint8)
    vmask[vrows] = 1
    g = torch.Generator().manual_seed(63)
    emb = bf16(torch.randn(len(vrows), HID, generator=g))
    dsl = [bf16(torch.randn(len(vrows), HID, generator=g) * 0.5) for _ in range(3)]
    vin = bf16(torch.from_numpy(rng.standard_normal((I, 3072)).astype(np.float32))).numpy()
    pos = np.zeros((3, Sf), np.float32)
    segs = 1 + R
    arr = lambda v: (ctypes.c_int * segs)(*v)
    assert lib.hd_seq_grid_positions(Tf, segs, arr([gh] * segs), arr([gw] * segs),
                                     arr([64 * k for k in range(segs)]), None, 0.0, pkg.np_ptr(pos)) == Sf
    assert pos[1, Tf + It] == 64 and pos[1, Tf + 2 * It] == 128 and pos[2, Tf + It + 1] == 1
    t = 0.42
    pkg.set_block_config(theta=1e4)
    tens = {k: v.to(dev, torch.bfloat16) for k, v in store_names(fw).items()}
    store = pkg.WeightStore(tens)
    fb = pkg.hd_forward_binding()
    pkg.check_status(lib.hd_forward_resolve(ctypes.byref(store.store), nLf, ctypes.byref(fb)), "resolve")
    wsbuf = torch.empty(lib.hd_forward_workspace_bytes(Sf, I, H, KV, HID, FF, D, None),
                        dtype=torch.uint8, device=dev)
    ws = pkg.hd_forward_workspace()
    ws.hidden_a = wsbuf.data_ptr()
    vind = torch.from_numpy(vin).to(dev, torch.bfloat16)
    if cached:
        xe = _cache_refs_n(pkg, lib, dev, fb, vind[It:].contiguous(), nref)
        ws.xe_ref, ws.n_ref = xe.data_ptr(), nref
    embd, dsd = emb.to(dev, torch.bfloat16), [d.to(dev, torch.bfloat16) for d in dsl]
    vmd = torch.from_numpy(vmask).to(dev)
    vc = pkg.hd_visual_cond()
    vc.image_embeds = embd.data_ptr()
    for j in range(3):
        vc.deepstack[j] = dsd[j].data_ptr()
    vc.visual_mask = vmd.data_ptr()
    vc.v_tokens = len(vrows)
    idsd, posd = torch.from_numpy(ids).to(dev), torch.from_numpy(pos).to(dev)
    td = torch.tensor([t], dtype=torch.float32, device=dev)
    out = torch.empty(Sf, 3072, dtype=torch.bfloat16, device=dev)
    st = lib.hd_forward(ctypes.byref(fb), ctypes.byref(ws), pkg.ptr(idsd), Tf, pkg.ptr(posd), None,
                        pkg.ptr(vind), I, ctypes.addressof(vc), pkg.ptr(td), None, Sf, H, KV, HID,
                        FF, D, TMS, None, pkg.ptr(out), None)
    pkg.check_status(st, "hd_forward edit layout")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    lib.hd_forward_binding_free(ctypes.byref(fb))
    ofw = {k: v.numpy() for k, v in fw.items() if k != "blocks"}
    ofw["blocks"] = [{k: v.numpy() for k, v in b.items()} for b in fw["blocks"]]
    cfg = orc.block_cfg(H, KV, HID, FF, D, theta=1e4, faithful=0)
    ref = orc.forward(ofw, cfg, ids, vin, t, pos, TMS,
                      visual=(emb.numpy(), [d.numpy() for d in dsl], vmask))
    r, c = rel_l2(got, ref), cosine(got, ref)
    print(f"edit forward (cached={cached}): rel_l2={r:.3e} cos={c:.7f}", flush=True)
    assert r <= 1e-2 and c >= 0.9999
    # the target rows (the ones the sampler reads) hold the bound on their own
    rt, ct = rel_l2(got[Tf:Tf + It], ref[Tf:Tf + It]), cosine(got[Tf:Tf + It], ref[Tf:Tf + It])
    assert rt <= 1e-2 and ct >= 0.9999, (rt, ct)


def _cache_refs_n(pkg, lib, dev, bw, ref, n):
    stg = torch.empty(n, 1024, dtype=torch.bfloat16, device=dev)
    xe = torch.empty(n, HID, dtype=torch.bfloat16, device=dev)
    lib.hd_linear(pkg.ptr(ref), bw.xe1_w, None, pkg.ptr(stg), n, 1024, 3072, 1)
    lib.hd_linear(pkg.ptr(stg), bw.xe2_w, bw.xe2_b, pkg.ptr(xe), n, HID, 1024, 1)
    pkg.check_prim("x_embedder cache")
    return xe

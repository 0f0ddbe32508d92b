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

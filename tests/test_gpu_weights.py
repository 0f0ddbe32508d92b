"""GGUF pack loader on the GPU: a synthetic model written as a GGUF pack
(tests/gguf_writer.py), loaded with hd_weights_to_device_gguf, must hold the
same bytes as the source tensors, and a forward resolved from the loaded
store must equal the forward resolved from the source tensors bit for bit."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

from tests import gguf_writer as gw
from tests.common import grid_pos

pytestmark = pytest.mark.gpu
TMS = 151673


def test_device_info(pkg, lib, dev):
    s = pkg.hd_weight_store()
    assert lib.hd_device_info(0, ctypes.byref(s)) == 0
    assert s.device_name and s.device_mem_bytes > (100 << 30) and s.compute_major == 9
    assert lib.hd_device_info(99, ctypes.byref(s)) == 3      # HD_ERR_PROFILE
    assert lib.hd_weights_last_error()


def test_gguf_pack_loads_and_runs(pkg, lib, dev, tmp_path):
    synth = importlib.import_module("o1c_amd.synthetic")
    nL, HID, H, KV, FF, D = 2, 512, 4, 2, 1024, 128
    tens = synth.build_model(n_layers=nL, hidden=HID, heads=H, kv_heads=KV, ff=FF, seed=13)
    entries = []
    for name, t in tens.items():
        c = t.detach().cpu()
        if c.dtype == torch.bfloat16:
            data, gt = c.view(torch.int16).numpy().view(np.uint16).tobytes(), gw.GGML_BF16
        else:
            data, gt = c.float().numpy().tobytes(), gw.GGML_F32
        entries.append((name, list(reversed(c.shape)), gt, data))
    kvs = [("general.architecture", gw.GGUF_STR, "hidream_o1"), ("general.name", gw.GGUF_STR, "synthetic"),
           ("general.alignment", gw.GGUF_U32, 256), ("hidream.dtype", gw.GGUF_STR, "bf16"),
           ("hidream.num_layers", gw.GGUF_STR, str(nL))]
    path = str(tmp_path / "model.gguf")
    gw.write(path, kvs, entries, alignment=256)
    print("pack bytes", __import__("os").path.getsize(path), flush=True)

    store = pkg.hd_weight_store()
    st = lib.hd_weights_to_device_gguf(path.encode(), 0, ctypes.byref(store))
    assert st == 0, lib.hd_weights_last_error()
    try:
        assert store.n_allocs == len(tens) and store.arena_ptr and store.gemm and store.upload_stream
        assert store.arena_bytes % 256 == 0
        for i in range(store.n_allocs):
            a = store.allocs[i]
            src = tens[a.name.decode()]
            assert a.nbytes == src.numel() * src.element_size()
            assert (a.dev_ptr - store.arena_ptr) % 256 == 0
            # read back through exact library conversions (bf16 -> f32 widening, f32 * 1)
            got = torch.empty(src.numel(), dtype=torch.float32, device=dev)
            if src.dtype == torch.bfloat16:
                lib.hd_sched_bf16_upcast(a.dev_ptr, pkg.ptr(got), src.numel())
            else:
                lib.hd_scale_f32(a.dev_ptr, pkg.ptr(got), 1.0, src.numel())
            pkg.check_prim("read back")
            torch.cuda.synchronize()
            assert torch.equal(got, src.float().flatten()), a.name

        # forward from the loaded store vs from the source tensors
        binding = pkg.hd_forward_binding()
        pkg.check_status(lib.hd_forward_resolve(ctypes.byref(store), nL, ctypes.byref(binding)),
                         "resolve loaded")
        model = synth.Model(tens, nL)
        pkg.set_block_config(theta=1e4)
        T, I = 16, 64
        S = T + I
        posd = torch.from_numpy(grid_pos(T, 8, 8)).to(dev)
        g = torch.Generator().manual_seed(3)
        ids = torch.randint(0, 151643, (1, T), generator=g)
        ids[:, -1] = TMS
        idsd = ids.to(dev)
        vin = torch.randn(1, I, 3072, generator=g).to(dev, torch.bfloat16)
        td = torch.tensor([0.4], device=dev)
        wsb = lib.hd_forward_batched_workspace_bytes(1, S, I, H, KV, HID, FF, D)
        buf = torch.empty(wsb, dtype=torch.uint8, device=dev)
        ws = pkg.hd_forward_workspace()
        ws.hidden_a = buf.data_ptr()
        outs = []
        for b in (binding, model.binding):
            out = torch.empty(1, S, 3072, dtype=torch.bfloat16, device=dev)
            st = lib.hd_forward_batched(ctypes.byref(b), ctypes.byref(ws), 1, pkg.ptr(idsd), T, pkg.ptr(posd),
                                        0, pkg.ptr(vin), I, pkg.ptr(td), S, H, KV, HID, FF, D, TMS, None,
                                        pkg.ptr(out), None)
            pkg.check_status(st, "forward")
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1])
        lib.hd_forward_binding_free(ctypes.byref(binding))
    finally:
        lib.hd_weight_store_free(ctypes.byref(store))
    assert not store.arena_ptr and store.n_allocs == 0

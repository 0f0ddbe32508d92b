"""CPU-side checks of the C-ABI: the library loads, exports every symbol
include/*.h declares, and the host-side argument checks fail closed (no
compute call reaches the GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(ROOT, "include", fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b(hd_[a-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported(lib, pkg):
    names = declared_functions()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    untyped = [n for n in names if n not in pkg.SIGNATURES]
    assert not untyped, untyped


def test_host_bf16_helpers(lib):
    # test_primitives.c:142-157
    assert lib.hd_f32_to_bf16(1.0) == 0x3F80
    assert lib.hd_f32_to_bf16(0.0) == 0
    assert lib.hd_bf16_to_f32(lib.hd_f32_to_bf16(1.0)) == 1.0
    for v in (0.5, 3.14159, 1e-3, 1e3, -2.5):
        back = lib.hd_bf16_to_f32(lib.hd_f32_to_bf16(v))
        assert abs(back - v) / abs(v) < 1e-2


def test_block_fails_closed(lib, pkg):
    b = pkg.hd_block_binding()
    st = lib.hd_decoder_block(None, None, None, ctypes.byref(b), None, None, 0, None, None, 16, 4,
                              2, 512, 1024, 128, None)
    assert st == pkg.HD_ERR_MISSING
    assert b"null" in lib.hd_last_error()
    # a resolved-looking binding with too little scratch -> HD_ERR_OOM
    for n, _ in pkg.hd_block_binding._fields_[1:]:
        setattr(b, n, 0x1000)
    fake = ctypes.c_void_p(0x1000)
    st = lib.hd_decoder_block(fake, fake, None, ctypes.byref(b), None, fake, 10, None, fake, 16, 4,
                              2, 512, 1024, 128, None)
    assert st == pkg.HD_ERR_OOM
    st = lib.hd_decoder_block(fake, fake, None, ctypes.byref(b), None, fake, 1 << 40, None, fake,
                              16, 4, 2, 512, 1024, 64, None)
    assert st == pkg.HD_ERR_UNSUPPORTED


def test_sdpa_create_rejects_bad_shapes(lib):
    h = ctypes.c_void_p()
    assert lib.hd_sdpa_create_prod(ctypes.byref(h), 1, 32, 7, 128, 0, 128, 0.08) != 0
    assert b"head counts" in lib.hd_cuda_last_error()
    assert lib.hd_sdpa_create_split(ctypes.byref(h), 1, 32, 8, 128, 128, 128, 0.08) != 0
    assert lib.hd_sdpa_create(ctypes.byref(h), 1, 32, 8, 128, 128, 64, 0.08) != 0
    lib.hd_cuda_clear_error()
    assert lib.hd_cuda_last_error() == b""


def test_scratch_sizes_scale(lib):
    one = lib.hd_decoder_block_scratch_bytes(16640, 32, 8, 4096, 12288, 128)
    # no S^2 term: the whole block scratch at S=16640 stays ~1.2 GB
    assert 1.0e9 < one < 1.4e9
    two = lib.hd_decoder_block_batched_scratch_bytes(2, 4352, 32, 8, 4096, 12288, 128)
    assert two > lib.hd_decoder_block_batched_scratch_bytes(1, 4352, 32, 8, 4096, 12288, 128)
    ws = lib.hd_forward_workspace_bytes(4352, 4096, 32, 8, 4096, 12288, 128, None)
    assert ws > lib.hd_decoder_block_scratch_bytes(4352, 32, 8, 4096, 12288, 128) // 2


def test_block_config_roundtrip(lib, pkg):
    c = pkg.hd_block_config()
    lib.hd_block_get_config(ctypes.byref(c))
    assert abs(c.eps - 1e-6) < 1e-12 and c.rope_theta == 5e6 and list(c.section) == [24, 20, 20]
    pkg.set_block_config(theta=1e4)
    lib.hd_block_get_config(ctypes.byref(c))
    assert c.rope_theta == 1e4
    pkg.set_block_config()


def test_forward_fails_closed(lib, pkg):
    fb = pkg.hd_forward_binding()
    ws = pkg.hd_forward_workspace()
    st = lib.hd_forward(ctypes.byref(fb), ctypes.byref(ws), None, 4, None, None, None, 4, None, None,
                        None, 8, 4, 2, 512, 1024, 128, 151673, None, None, None)
    assert st == pkg.HD_ERR_MISSING


def test_gemm_config_names(lib):
    assert lib.hd_gemm_config_name(16640, 6144, 4096, 0).startswith(b"bf16_")
    assert lib.hd_gemm_config_name(7, 5, 6, 0) == b"reference"

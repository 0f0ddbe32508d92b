"""GGUF v3 reader (include/hd_gguf.h) on packs written by tests/gguf_writer.py:
header fields, tensor table and payload bytes against what was written, and
every field against the reference's own gguf.c built into oracle/_ref (when
that build exists). CPU only."""
import ctypes
import os

import numpy as np
import pytest

from tests import gguf_writer as gw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")

PACK_KVS = [
    ("general.architecture", gw.GGUF_STR, "hidream_o1"),
    ("general.name", gw.GGUF_STR, "synthetic pack"),
    ("general.alignment", gw.GGUF_U32, 256),
    ("hidream.profile", gw.GGUF_STR, "base"),
    ("hidream.variant", gw.GGUF_STR, "full"),
    ("hidream.revision", gw.GGUF_STR, "r1"),
    ("hidream.dtype", gw.GGUF_STR, "bf16"),
    ("hidream.num_layers", gw.GGUF_STR, "36"),
    ("hidream.layout_version", gw.GGUF_STR, "2"),
    # keys and types the reader skips
    ("general.file_type", gw.GGUF_U32, 32),
    ("x.u8", gw.GGUF_U8, 7), ("x.i16", gw.GGUF_I16, -3), ("x.f32", gw.GGUF_F32, 1.5),
    ("x.bool", gw.GGUF_BOOL, 1), ("x.u64", gw.GGUF_U64, 1 << 40), ("x.f64", gw.GGUF_F64, -2.25),
    ("x.arr_str", gw.GGUF_ARR, (gw.GGUF_STR, ["a", "bc", ""])),
    ("x.arr_u32", gw.GGUF_ARR, (gw.GGUF_U32, [1, 2, 3])),
    ("x.arr_arr", gw.GGUF_ARR, (gw.GGUF_ARR, [(gw.GGUF_I8, [1, -1]), (gw.GGUF_I8, [])])),
]


def _tensors(rng):
    out = []
    for name, shape, gt in (("model.a.weight", (5, 3), gw.GGML_BF16), ("model.b.bias", (7,), gw.GGML_F32),
                            ("model.c.weight", (2, 3, 4), gw.GGML_F16), ("model.d.scale", (), gw.GGML_F32),
                            ("model.e.weight", (300, 2), gw.GGML_BF16)):
        if gt == gw.GGML_BF16:
            arr = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
        else:
            arr = rng.standard_normal(shape)
        out.append((name, list(reversed(shape)), gt, gw.tensor_bytes(arr, gt)))
    return out


@pytest.fixture(scope="module")
def packs(tmp_path_factory):
    d = tmp_path_factory.mktemp("gguf")
    rng = np.random.default_rng(0)
    ts = _tensors(rng)
    files = {}
    files["pack"] = (str(d / "pack.gguf"), PACK_KVS, ts, 256)
    gw.write(*files["pack"][:3], alignment=256)
    kv_noalign = [kv for kv in PACK_KVS if kv[0] != "general.alignment"]
    files["default_align"] = (str(d / "a32.gguf"), kv_noalign, ts, 32)
    gw.write(*files["default_align"][:3], alignment=32)
    kv64 = [kv if kv[0] != "general.alignment" else (kv[0], gw.GGUF_U32, 64) for kv in PACK_KVS]
    files["align64"] = (str(d / "a64.gguf"), kv64, ts, 64)
    gw.write(*files["align64"][:3], alignment=64)
    return files


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (no /root/reference here)")
    return ctypes.CDLL(REF_SO, mode=os.RTLD_LAZY | os.RTLD_LOCAL)


def _open(lib, pkg, path):
    f = pkg.hd_gguf_file()
    st = lib.hd_gguf_open(path.encode(), ctypes.byref(f))
    return st, f


def _fields(f):
    head = tuple(getattr(f, n) for n in ("n_tensors", "alignment", "tensor_data_off", "payload_bytes",
                                          "arch", "name", "profile", "variant", "revision", "dtype",
                                          "quantization", "num_layers", "layout_version"))
    ts = tuple((f.tensors[i].name, f.tensors[i].n_dims, tuple(f.tensors[i].dims), f.tensors[i].type,
                f.tensors[i].offset, f.tensors[i].nbytes) for i in range(f.n_tensors))
    return head, ts


@pytest.mark.parametrize("which", ["pack", "default_align", "align64"])
def test_gguf_roundtrip(pkg, lib, packs, which):
    path, kvs, ts, al = packs[which]
    st, f = _open(lib, pkg, path)
    assert st == 0, lib.hd_gguf_last_error()
    try:
        assert f.alignment == al and f.n_tensors == len(ts)
        assert (f.arch, f.profile, f.dtype) == (b"hidream_o1", b"base", b"bf16")
        assert (f.num_layers, f.layout_version, f.quantization) == (36, 2, None)
        off = 0
        for i, (name, dims, gt, data) in enumerate(ts):
            t = f.tensors[i]
            off = (off + al - 1) // al * al
            assert (t.name.decode(), t.n_dims, list(t.dims)[:t.n_dims], t.type) == (name, len(dims), dims, gt)
            assert (t.offset, t.nbytes) == (off, len(data))
            off += len(data)
            buf = (ctypes.c_uint8 * len(data))()
            assert lib.hd_gguf_read_tensor(ctypes.byref(f), ctypes.byref(f.tensors[i]), buf) == 0
            assert bytes(buf) == data
        assert f.payload_bytes == (off + al - 1) // al * al
        assert f.tensor_data_off % al == 0 and f.tensor_data_off + f.payload_bytes == os.path.getsize(path)
    finally:
        lib.hd_gguf_close(ctypes.byref(f))
    assert f.tensors is None or not f.tensors


@pytest.mark.parametrize("which", ["pack", "default_align", "align64"])
def test_gguf_matches_reference_build(pkg, lib, ref, packs, which):
    ref.hd_gguf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(pkg.hd_gguf_file)]
    ref.hd_gguf_close.argtypes = [ctypes.POINTER(pkg.hd_gguf_file)]
    path = packs[which][0]
    st, a = _open(lib, pkg, path)
    b = pkg.hd_gguf_file()
    assert ref.hd_gguf_open(path.encode(), ctypes.byref(b)) == st == 0
    try:
        assert _fields(a) == _fields(b)
    finally:
        lib.hd_gguf_close(ctypes.byref(a))
        ref.hd_gguf_close(ctypes.byref(b))


def _malformed(tmp_path):
    rng = np.random.default_rng(1)
    ts = _tensors(rng)[:2]
    cases = {}
    p = str(tmp_path / "magic.gguf"); gw.write(p, PACK_KVS, ts, magic=b"GGUX"); cases["bad magic"] = p
    p = str(tmp_path / "v2.gguf"); gw.write(p, PACK_KVS, ts, version=2); cases["version 2"] = p
    p = str(tmp_path / "zero.gguf"); gw.write(p, PACK_KVS, [], raw_infos=(0, b"")); cases["no tensors"] = p
    nine = gw._str("t") + (9).to_bytes(4, "little") + b"\1\0\0\0\0\0\0\0" * 9 + (0).to_bytes(12, "little")
    p = str(tmp_path / "nine.gguf"); gw.write(p, PACK_KVS, ts[:1], raw_infos=(1, nine)); cases["9 dims"] = p
    q40 = gw._str("t") + (1).to_bytes(4, "little") + (32).to_bytes(8, "little") + (2).to_bytes(4, "little") \
        + (0).to_bytes(8, "little")
    p = str(tmp_path / "q40.gguf"); gw.write(p, PACK_KVS, ts[:1], raw_infos=(1, q40)); cases["type Q4_0"] = p
    bad_kv = PACK_KVS[:2] + [("x.bad", 13, b"")]
    p = str(tmp_path / "kv13.gguf")
    import struct
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 1, 1) + gw._str("x.bad") + struct.pack("<I", 13) + b"\0" * 64)
    cases["KV type 13"] = p
    return cases


def test_gguf_malformed_headers(pkg, lib, tmp_path):
    for what, path in _malformed(tmp_path).items():
        st, f = _open(lib, pkg, path)
        lib.hd_gguf_close(ctypes.byref(f))
        assert st == 2, (what, st)          # HD_ERR_PARSE
        assert lib.hd_gguf_last_error()
    st, f = _open(lib, pkg, str(tmp_path / "missing.gguf"))
    assert st == 1                           # HD_ERR_IO


def test_gguf_malformed_match_reference_build(pkg, lib, ref, tmp_path):
    ref.hd_gguf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(pkg.hd_gguf_file)]
    ref.hd_gguf_close.argtypes = [ctypes.POINTER(pkg.hd_gguf_file)]
    for what, path in _malformed(tmp_path).items():
        st, f = _open(lib, pkg, path)
        lib.hd_gguf_close(ctypes.byref(f))
        g = pkg.hd_gguf_file()
        rs = ref.hd_gguf_open(path.encode(), ctypes.byref(g))
        ref.hd_gguf_close(ctypes.byref(g))
        assert st == rs, (what, st, rs)

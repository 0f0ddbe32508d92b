"""Sequence builders (CPU): hd_seq_t2i, hd_seq_build_tokens, hd_resolution_snap.

Pinned by the reference's own expectations: the S=23 position fixture
(src/runtime/sequence.c:97-100), the structural assertions of
tests/unit/test_seq_ref.c:60-238 (K=1 edit and K=2 personalize geometry and
positions, which that test states were checked against transformers'
get_rope_index_fix_point), and the bucket table of sequence.c:28-33.
The reference's hd_seq_build itself runs its tokenizer first; here the
tokenized template is an input (template ids below follow the token layout
test_seq_ref.c:8-12 describes: 3 header tokens, per reference a
vision_start / image_pad / vision_end triple, the caption, a 5-token tail).
"""
import ctypes
import json
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")

PATCH = 32
IMG, VID, VS, VEND, TMS, BOI = 151655, 151656, 151652, 151653, 151673, 151669
FIX = 4096
HEADER = [151644, 872, 198]                       # <|im_start|> user \n
TAIL = [151645, 198, 151644, 77091, 198]          # <|im_end|> \n <|im_start|> assistant \n


def _template(k, caption_len):
    ids = list(HEADER)
    for _ in range(k):
        ids += [VS, IMG, VEND]
    ids += [1000 + i for i in range(caption_len)]
    return np.array(ids + TAIL, np.int64)


def _build(pkg, lib, tpl, refs, h=1024, w=1024, tms_n=1):
    geo = (pkg.hd_ref_geom * max(1, len(refs)))(*[pkg.hd_ref_geom(*r) for r in refs])
    seq = pkg.hd_sequence()
    st = lib.hd_seq_build_tokens(pkg.np_ptr(tpl), len(tpl), len(refs), PATCH, IMG, VID, VS, TMS,
                                 tms_n, 1, FIX, h, w, geo, ctypes.byref(seq))
    return st, seq


def _arrays(seq):
    S = seq.S
    pos = np.ctypeslib.as_array(seq.pos_f32, (3, S)).copy()
    mask = np.ctypeslib.as_array(seq.mask_bf16, (S * S * 2,)).view(np.uint16).reshape(S, S).copy()
    vm = np.ctypeslib.as_array(seq.vinput_mask, (S,)).copy()
    ids = np.ctypeslib.as_array(seq.input_ids, (S,)).copy()
    return ids, pos, mask, vm


def _check_mask(mask, token_rows):
    want = np.triu(np.full(mask.shape, 0xFF7F, np.uint16), 1)
    want[token_rows] = 0
    assert np.array_equal(mask, want)


def test_t2i_matches_fixture(pkg, lib):
    g = json.load(open(os.path.join(GOLD, "positions_s23.json")))
    T = g["text_len"]
    ids = np.arange(T, dtype=np.int64) + 7
    seq = pkg.hd_sequence()
    assert lib.hd_seq_t2i(pkg.np_ptr(ids), T, g["grid_h"] * PATCH, g["grid_w"] * PATCH, PATCH,
                          IMG, VID, VS, TMS, 1, 1, g["fix_point"], ctypes.byref(seq)) == 0
    try:
        assert (seq.S, seq.text_len, seq.image_len, seq.img_begin) == (g["S"], T, 4, T)
        assert list(seq.sec) == [24, 20, 20] and seq.n_refs == 0
        S = seq.S
        pos = np.ctypeslib.as_array(seq.pos_f32, (3, S))
        assert pos.tolist() == g["pos"]
        mask = np.ctypeslib.as_array(seq.mask_bf16, (S * S * 2,)).view(np.uint16).reshape(S, S)
        tok = np.zeros(S, bool)
        tok[T - 1:] = True
        _check_mask(mask, tok)
        # the per-table entry points agree with the assembled sequence
        m2 = np.empty((S, S), np.uint16)
        assert lib.hd_seq_t2i_mask(T, S, pkg.np_ptr(m2)) == 0
        assert np.array_equal(mask, m2)
        vm = np.ctypeslib.as_array(seq.vinput_mask, (S,))
        assert vm.tolist() == [0] * T + [1] * 4
        assert np.ctypeslib.as_array(seq.input_ids, (T,)).tolist() == ids.tolist()
        assert lib.hd_seq_diag(ctypes.byref(seq), b"t2i") == 0
    finally:
        lib.hd_sequence_free(ctypes.byref(seq))
    assert not seq.pos_f32 and seq.S == 0


def test_build_edit_k1(pkg, lib):
    """test_seq_ref.c:60-165: 1024^2 target, one 512^2 reference (16x16,
    condition grid 12x12), caption of 4 tokens."""
    tpl = _template(1, 4)
    st, seq = _build(pkg, lib, tpl, [(256, 16, 16, 12, 12)])
    assert st == 0, lib.hd_last_error()
    try:
        exp_n = len(tpl) + 144 - 1
        T = exp_n + 2
        S = T + 1024 + 256
        assert (seq.text_len, seq.image_len, seq.S, seq.n_refs) == (T, 1024, S, 1)
        assert seq.ref_len[0] == 256 and seq.ref_begin[0] == T + 1024
        ids, pos, mask, vm = _arrays(seq)
        assert vm.sum() == 1024 + 256 and vm[T:].all() and not vm[:T].any()
        d0 = pos[0]
        assert d0[0] == 0 and d0[3] == 3 and d0[148] == 16 and d0[T - 1] == 27
        tgt0, tgt_last = T, T + 1023
        assert pos[:, tgt0].tolist() == [FIX] * 3
        assert pos[1, tgt_last] == FIX + 31 and pos[2, tgt_last] == FIX + 31
        ref0, ref_last = T + 1024, S - 1
        assert pos[:, ref0].tolist() == [4128] * 3
        assert pos[1, ref_last] == 4128 + 15 and pos[2, ref_last] == 4128 + 15
        # template grid: rows 4..147 at 4 + (0, r, c) over the 12x12 condition grid
        r, c = np.divmod(np.arange(144), 12)
        assert np.array_equal(pos[0, 4:148], np.full(144, 4.0))
        assert np.array_equal(pos[1, 4:148], 4.0 + r) and np.array_equal(pos[2, 4:148], 4.0 + c)
        # text after the template grid runs on from 16 on all three axes
        assert np.array_equal(pos[:, 148:T], np.tile(np.arange(16, 28, dtype=np.float32), (3, 1)))
        tok = np.zeros(S, bool)
        tok[exp_n + 1:] = True                     # tms rows, target, reference
        _check_mask(mask, tok)
        vs0 = int(np.argmax(ids == VS))
        assert vs0 == 3 and ids[vs0 + 1] == IMG and ids[vs0 + 145] == VEND
        assert ids[exp_n] == BOI and ids[exp_n + 1] == TMS
        assert ids[T] == VS and ids[T + 1] == IMG and ids[ref0] == VS and ids[ref0 + 1] == IMG
        assert (ids[T + 1:ref0] == IMG).all() and (ids[ref0 + 1:] == IMG).all()
    finally:
        lib.hd_sequence_free(ctypes.byref(seq))


def test_build_personalize_k2(pkg, lib):
    """test_seq_ref.c:166-238: two 384^2 references (12x12 each), caption of
    5 tokens."""
    tpl = _template(2, 5)
    st, seq = _build(pkg, lib, tpl, [(144, 12, 12, 12, 12)] * 2)
    assert st == 0, lib.hd_last_error()
    try:
        exp_n = len(tpl) + 2 * 144 - 2
        T = exp_n + 2
        S = T + 1024 + 288
        assert (seq.text_len, seq.S, seq.n_refs) == (T, S, 2)
        assert seq.ref_begin[0] == T + 1024 and seq.ref_begin[1] == T + 1024 + 144
        ids, pos, mask, vm = _arrays(seq)
        assert pos[0, 0] == 0 and pos[0, 148] == 16 and pos[0, T - 1] == 42
        assert pos[0, T] == FIX and pos[1, T + 1023] == FIX + 31
        r1, r2 = seq.ref_begin[0], seq.ref_begin[1]
        assert pos[0, r1] == 4128 and pos[0, r2] == 4140
        assert pos[1, r2 + 143] == 4140 + 11 and pos[2, r2 + 143] == 4140 + 11
        assert vm.sum() == 1024 + 288
        vs0 = int(np.argmax(ids == VS))
        assert vs0 == 3 and ids[vs0 + 145] == VEND
        vs1 = vs0 + 146
        assert ids[vs1] == VS and ids[vs1 + 145] == VEND
        assert ids[exp_n] == BOI and ids[exp_n + 1] == TMS
        assert ids[T] == VS and ids[r1] == VS and ids[r2] == VS
        tok = np.zeros(S, bool)
        tok[exp_n + 1:] = True
        _check_mask(mask, tok)
    finally:
        lib.hd_sequence_free(ctypes.byref(seq))


def test_build_text_only_and_several_tms(pkg, lib):
    """K=0 reduces to the text-to-image layout with the target's
    vision_start counted as its first grid row; N timestep tokens all
    attend fully."""
    tpl = _template(0, 6)
    st, seq = _build(pkg, lib, tpl, [], h=256, w=320, tms_n=3)
    assert st == 0, lib.hd_last_error()
    try:
        T = len(tpl) + 1 + 3
        assert (seq.text_len, seq.image_len, seq.S, seq.n_refs) == (T, 8 * 10, T + 80, 0)
        ids, pos, mask, vm = _arrays(seq)
        assert np.array_equal(pos[:, :T], np.tile(np.arange(T, dtype=np.float32), (3, 1)))
        r, c = np.divmod(np.arange(80), 10)
        assert np.array_equal(pos[0, T:], np.full(80, float(FIX)))
        assert np.array_equal(pos[1, T:], FIX + r) and np.array_equal(pos[2, T:], FIX + c)
        assert (ids[len(tpl) + 1:T] == TMS).all()
        tok = np.zeros(seq.S, bool)
        tok[len(tpl) + 1:] = True
        _check_mask(mask, tok)
    finally:
        lib.hd_sequence_free(ctypes.byref(seq))


def test_build_rejects_bad_requests(pkg, lib):
    seq = pkg.hd_sequence()
    tpl = _template(1, 3)
    # template with one placeholder, two references asked
    assert _build(pkg, lib, tpl, [(144, 12, 12, 12, 12)] * 2)[0] != 0
    assert _build(pkg, lib, tpl, [(144, 12, 12, 0, 12)])[0] != 0
    assert lib.hd_seq_build_tokens(None, 0, 0, PATCH, IMG, VID, VS, TMS, 1, 1, FIX, 1024, 1024,
                                   None, ctypes.byref(seq)) != 0
    assert lib.hd_seq_t2i(None, 0, 64, 64, PATCH, IMG, VID, VS, TMS, 1, 1, FIX, ctypes.byref(seq)) != 0
    lib.hd_sequence_free(ctypes.byref(seq))       # freeing an empty sequence is a no-op


BUCKETS = [(2048, 2048), (2304, 1728), (1728, 2304), (2560, 1440), (1440, 2560), (2496, 1664),
           (1664, 2496), (3104, 1312), (1312, 3104), (2304, 1792), (1792, 2304)]


@pytest.mark.parametrize("wh", [(1024, 1024), (1920, 1080), (1080, 1920), (4000, 3000),
                                (3000, 4000), (3000, 2000), (5000, 2000), (1, 1000),
                                (1000, 1), (1300, 1000), (0, 512), (512, -3)])
def test_resolution_snap(pkg, lib, wh):
    w, h = ctypes.c_int(), ctypes.c_int()
    lib.hd_resolution_snap(wh[0], wh[1], ctypes.byref(w), ctypes.byref(h))
    if wh[0] <= 0 or wh[1] <= 0:
        assert (w.value, h.value) == (2048, 2048)
        return
    # brute force: the first bucket of least aspect-ratio distance
    d = [abs(bw / bh - wh[0] / wh[1]) for bw, bh in BUCKETS]
    assert (w.value, h.value) == BUCKETS[int(np.argmin(d))]
    assert w.value % 32 == 0 and h.value % 32 == 0

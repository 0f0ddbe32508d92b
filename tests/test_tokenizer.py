"""Prompt tokenizer (hd_tokenizer_*, replaces src/model/tokenizer.c) on the
CPU: the reference's own frozen token ids (tests/golden/tokenizer_frozen.json,
from its tests/unit/test_tokenizer.c, which froze transformers' output), and
equality with the reference tokenizer itself (oracle/_ref/libref.so, built
from tokenizer.c where it lies) on a corpus that exercises every
pre-tokenizer rule, special tokens and invalid UTF-8. The vocabulary, merges
and special tokens come from the reference's tables written by
oracle/_ref/tok_dump into oracle/_ref/tok (never committed); without the
reference build those tests skip."""
import ctypes
import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOK = os.path.join(ROOT, "oracle", "_ref", "tok")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")
HAVE_TABLES = all(os.path.exists(os.path.join(TOK, f)) for f in ("vocab.json", "merges.txt", "added_tokens.json"))
HD_OK, HD_ERR_IO, HD_ERR_PARSE, HD_ERR_MISSING = 0, 1, 2, 6

needs_tables = pytest.mark.skipif(not HAVE_TABLES, reason="reference tokenizer tables not built (oracle/ref.mk)")


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.load()


@pytest.fixture(scope="module")
def loaded(lib):
    if not HAVE_TABLES:
        pytest.skip("reference tokenizer tables not built (oracle/ref.mk)")
    st = lib.hd_tokenizer_load(*(os.path.join(TOK, f).encode() for f in ("vocab.json", "merges.txt",
                                                                           "added_tokens.json")))
    assert st == HD_OK, lib.hd_last_error()
    yield lib
    lib.hd_tokenizer_unload()


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libref.so not built")
    r = ctypes.CDLL(REF_SO, mode=os.RTLD_LAZY | os.RTLD_LOCAL)
    try:
        r.hd_tokenizer_encode
    except AttributeError:
        pytest.skip("libref.so built without the tokenizer")
    pi = ctypes.POINTER(ctypes.c_int)
    r.hd_tokenizer_encode.argtypes = [ctypes.c_char_p, ctypes.POINTER(pi), ctypes.POINTER(ctypes.c_size_t)]
    r.hd_tokenizer_encode.restype = ctypes.c_int
    r.hd_tokenizer_encode_prompt.argtypes = r.hd_tokenizer_encode.argtypes
    r.hd_tokenizer_encode_prompt.restype = ctypes.c_int
    r.hd_tokenizer_free_ids.argtypes = [pi]
    r.hd_tokenizer_build_ref_template.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
    r.hd_tokenizer_build_ref_template.restype = ctypes.c_int
    r.hd_tokenizer_build_template.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]
    r.hd_tokenizer_build_template.restype = ctypes.c_int
    r.hd_tokenizer_special_id.argtypes = [ctypes.c_char_p]
    r.hd_tokenizer_special_id.restype = ctypes.c_int
    return r


def encode(l, text, prompt=False):
    ids = ctypes.POINTER(ctypes.c_int)()
    n = ctypes.c_size_t()
    fn = l.hd_tokenizer_encode_prompt if prompt else l.hd_tokenizer_encode
    st = fn(text, ctypes.byref(ids), ctypes.byref(n))
    out = [ids[i] for i in range(n.value)] if st == HD_OK else None
    if ids:
        l.hd_tokenizer_free_ids(ids)
    return st, out


def template(l, fn, *args):
    out = ctypes.c_void_p()
    st = fn(*args, ctypes.byref(out))
    s = ctypes.string_at(out.value) if st == HD_OK else None
    if out.value:
        ctypes.CDLL(None).free(out)
    return st, s


@needs_tables
def test_frozen_vectors(loaded):
    """The reference's frozen ids (canonical, empty and teapot prompts)."""
    gold = json.load(open(os.path.join(ROOT, "tests", "golden", "tokenizer_frozen.json")))
    for case in gold["cases"]:
        st, ids = encode(loaded, case["prompt"].encode("utf-8"), prompt=True)
        assert st == HD_OK
        assert ids == case["ids"], case["prompt"]


CORPUS = [
    "a red fox sits under a cherry blossom tree", "Hello, world!", "it's they're we've I'm you'll he'd",
    "IT'S  Dont' 's 't", "x'sy", "12345 67 8", "v1.2.3-beta_4", "  leading", "trailing   ", "a  b   c    d",
    "tab\there", "new\nline", "cr\r\nlf", "\n\n\n", " \n \n", "mix \t\n end", "!!!???...", " ,;: -- __",
    "price: $19.99 (20% off)", "email@example.com #tag @user", "path/to/file.txt", "x=y+z*2^3",
    "café naïve résumé", "中文 文本", "emoji 😀🎉 ok", "Ünïcödé—dash", "tabs\t\t\tand spaces   ",
    "<|im_start|>user\nhi<|im_end|>", "a<|image_pad|>b<|vision_start|><|vision_end|>c",
    "<|endoftext|><|endoftext|>", "<|im_start", "<think>reason</think> done", "<|not_special|>",
    "'", "''", "'s's", " 's", "   's", "9's", "Mr. O'Neil's 2nd dog", "A" * 40, "ab" * 30, "1" * 25,
    " " * 7, "end with space ", "x y", "zero​width", "\x7f\x01ctrl",
]


@needs_tables
def test_matches_reference_corpus(loaded, ref):
    """hd_tokenizer_encode equals the reference's on every corpus string,
    as raw text and inside the im-chat / reference templates."""
    for s in CORPUS:
        b = s.encode("utf-8")
        for prompt in (False, True):
            got, want = encode(loaded, b, prompt), encode(ref, b, prompt)
            assert got == want, (s, prompt)
        for k in (0, 2):
            st1, t1 = template(loaded, loaded.hd_tokenizer_build_ref_template, b, k)
            st2, t2 = template(ref, ref.hd_tokenizer_build_ref_template, b, k)
            assert (st1, t1) == (st2, t2)
            assert encode(loaded, t1) == encode(ref, t2)


@needs_tables
def test_invalid_utf8_matches_reference(loaded, ref):
    """Byte sequences that are not UTF-8 (stray continuation bytes, truncated
    and broken sequences) are split and BPE'd exactly as the reference does."""
    cases = [b"\x80abc", b"a\xc3", b"a\xc3b", b"\xe4\xb8", b"\xe4\xb8a\xb8", b"\xff\xfe x", b"\xf0\x9f\x98",
             b"ok \xed\xa0\x80 surrogate", b"\xc3\xa9\xc3"]
    for b in cases:
        assert encode(loaded, b) == encode(ref, b), b


@needs_tables
def test_special_ids_and_templates(loaded, ref):
    for s in ("<|im_start|>", "<|im_end|>", "<|vision_start|>", "<|image_pad|>", "<|video_pad|>", "nope", ""):
        assert loaded.hd_tokenizer_special_id(s.encode()) == ref.hd_tokenizer_special_id(s.encode())
    assert loaded.hd_tokenizer_special_id(b"<|im_start|>") == 151644
    st, t = template(loaded, loaded.hd_tokenizer_build_template, b"hi")
    assert st == HD_OK and t == b"<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n"
    assert template(loaded, loaded.hd_tokenizer_build_ref_template, b"cap", -1)[0] == HD_ERR_PARSE


def test_errors_fail_closed(lib, tmp_path):
    """Nothing loaded -> HD_ERR_MISSING; unreadable / malformed files; a piece
    missing from the vocabulary fails the whole encode (tokenizer.c:392-399)."""
    lib.hd_tokenizer_unload()
    assert encode(lib, b"abc")[0] == HD_ERR_MISSING
    assert lib.hd_tokenizer_special_id(b"<|im_start|>") == -1
    v, m, a = tmp_path / "vocab.json", tmp_path / "merges.txt", tmp_path / "added.json"
    v.write_text(json.dumps({"a": 0, "b": 1, "ab": 2, "Ġ": 3, "Ġa": 4}))
    m.write_text("#version: 0.2\na b\nĠ a\n")
    a.write_text(json.dumps({"version": "1.0", "added_tokens": [{"id": 9, "content": "<s>", "special": True}]}))
    p = [str(x).encode() for x in (v, m, a)]
    assert lib.hd_tokenizer_load(p[0], b"/nonexistent/merges.txt", p[2]) == HD_ERR_IO
    bad = tmp_path / "bad.json"
    bad.write_text('{"a": 0,')
    assert lib.hd_tokenizer_load(bytes(str(bad), "utf-8"), p[1], p[2]) == HD_ERR_PARSE
    assert lib.hd_tokenizer_load(*p) == HD_OK
    assert encode(lib, b"ab a<s>ab") == (HD_OK, [2, 4, 9, 2])
    st, ids = encode(lib, b"abc")
    assert st == HD_ERR_PARSE and ids is None
    assert b"not in vocab" in lib.hd_last_error()
    assert encode(lib, None)[0] == HD_ERR_PARSE
    lib.hd_tokenizer_unload()

"""Writes tokenizer_frozen.json: the reference's own golden tokenizer vectors
(prompt -> ids) from its unit test, tests/unit/test_tokenizer.c (canonical
prompt :18-25, empty prompt :64-72, teapot prompt :111-125). Those ids were
frozen from transformers' AutoTokenizer on the model (apply_chat_template +
encode(add_special_tokens=False)). Only the data (C string literals and int
arrays) is extracted; run here, where /root/reference exists."""
import json
import os
import re
import sys

SRC = "/root/reference/tests/unit/test_tokenizer.c"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tokenizer_frozen.json")


def c_strings(block):
    """Concatenates adjacent C string literals (octal escapes decoded as bytes)."""
    raw = b""
    for lit in re.findall(r'"((?:[^"\\]|\\.)*)"', block):
        b = lit.encode("latin-1")
        raw += b.decode("unicode_escape").encode("latin-1")
    return raw.decode("utf-8")


def ints(block):
    return [int(x) for x in re.findall(r"\d+", block)]


def main():
    src = open(SRC, encoding="utf-8").read()
    canon = c_strings(re.search(r"CANONICAL_PROMPT\s*=\s*(.*?);", src, re.S).group(1))
    canon_ids = ints(re.search(r"FROZEN_IDS\[\d+\]\s*=\s*\{(.*?)\}", src, re.S).group(1))
    empty_ids = ints(re.search(r"want\[8\]\s*=\s*\{(.*?)\}", src, re.S).group(1))
    tea = c_strings(re.search(r"static const char \*PROMPT\s*=\s*(.*?);", src, re.S).group(1))
    tea_ids = ints(re.search(r"FROZEN\[\d+\]\s*=\s*\{(.*?)\}", src, re.S).group(1))
    cases = [{"prompt": canon, "ids": canon_ids}, {"prompt": "", "ids": empty_ids},
             {"prompt": tea, "ids": tea_ids}]
    assert [len(c["ids"]) for c in cases] == [17, 8, 51], [len(c["ids"]) for c in cases]
    json.dump({"source": "tests/unit/test_tokenizer.c (reference)", "cases": cases}, open(OUT, "w"), indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    sys.exit(main())

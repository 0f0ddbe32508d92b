# Builds the reference's own pure-C host modules into oracle/_ref/ as a
# checker (test infrastructure only). Sources are compiled where they lie
# under /root/reference; nothing is copied and no header is stubbed.
#   src/runtime/torch_rng.c  - torch CPU MT19937 randn
#   src/model/scheduler.c    - sigma derivations (its device-step wrappers
#                              stay unresolved and are never called)
#   src/runtime/decode.c     - latent -> RGB uint8 decode
#   src/io/gguf.c            - GGUF v3 header / tensor-table reader
#   src/model/tokenizer.c    - Qwen2 byte-level BPE prompt tokenizer (with
#                              model.c for hd_set_error / hd_last_error and
#                              json.c, both plain C)
# and tok_dump (oracle/tok_dump.c, compiled against the reference's
# tokenizer_tables.h) that writes those tables as vocab.json / merges.txt /
# added_tokens.json into _ref/tok for the library's file-based tokenizer.
REF ?= /root/reference
OUT := _ref
CC ?= gcc
CFLAGS = -O2 -fPIC -std=gnu11 -w -I$(REF)/include -I$(REF)/src/cuda -I$(REF)/src/model -I$(REF)/src/runtime \
         -I$(REF)/src/io

all: $(OUT)/libref.so $(OUT)/tok/vocab.json

$(OUT)/libref.so: $(REF)/src/runtime/torch_rng.c $(REF)/src/model/scheduler.c \
                  $(REF)/src/runtime/decode.c $(REF)/src/io/gguf.c \
                  $(REF)/src/model/tokenizer.c $(REF)/src/model/model.c $(REF)/src/io/json.c
	@mkdir -p $(OUT)
	$(CC) $(CFLAGS) -shared -o $@ $^ -lm

$(OUT)/tok_dump: tok_dump.c $(REF)/src/model/tokenizer_tables.h
	@mkdir -p $(OUT)
	$(CC) -O1 -w -I$(REF)/src/model -o $@ tok_dump.c

$(OUT)/tok/vocab.json: $(OUT)/tok_dump
	@mkdir -p $(OUT)/tok
	./$(OUT)/tok_dump $(OUT)/tok

clean:
	rm -rf $(OUT)
.PHONY: all clean

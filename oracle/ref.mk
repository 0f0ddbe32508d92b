# Builds the reference's own pure-C host modules into oracle/_ref/ as a
# checker (test infrastructure only). Sources are compiled where they lie
# under /root/reference; nothing is copied and no header is stubbed.
#   src/runtime/torch_rng.c  - torch CPU MT19937 randn
#   src/model/scheduler.c    - sigma derivations (its device-step wrappers
#                              stay unresolved and are never called)
#   src/runtime/decode.c     - latent -> RGB uint8 decode
#   src/io/gguf.c            - GGUF v3 header / tensor-table reader
REF ?= /root/reference
OUT := _ref
CC ?= gcc
CFLAGS = -O2 -fPIC -std=gnu11 -w -I$(REF)/include -I$(REF)/src/cuda -I$(REF)/src/model -I$(REF)/src/runtime \
         -I$(REF)/src/io

$(OUT)/libref.so: $(REF)/src/runtime/torch_rng.c $(REF)/src/model/scheduler.c \
                  $(REF)/src/runtime/decode.c $(REF)/src/io/gguf.c
	@mkdir -p $(OUT)
	$(CC) $(CFLAGS) -shared -o $@ $^ -lm

clean:
	rm -rf $(OUT)
.PHONY: clean

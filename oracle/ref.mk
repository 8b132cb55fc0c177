# Builds forword.c's own sources, where they lie, into oracle/_ref/ (git-ignored,
# never committed).  Flags are the reference Makefile's (Makefile:3,5).  The
# driver ref_driver.c is this repository's code: it calls the reference's
# exported functions to write golden vectors.
#   make -f ref.mk            (from oracle/)
REF     ?= /root/reference
OUT     := _ref
CC      ?= gcc
RFLAGS  := -O2 -std=c11 -march=native -fPIC -w
SRCS    := transformer attention ffn tokenizer chat_template sampler rope norm linear \
           gguf gguf_raw model_config quant quant_matvec tensor_data tensor_ops
REF_C   := $(addprefix $(REF)/,$(addsuffix .c,$(SRCS)))

all: $(OUT)/libforword_ref.so $(OUT)/ref_driver

$(OUT)/libforword_ref.so: $(REF_C)
	mkdir -p $(OUT)
	$(CC) $(RFLAGS) -shared -o $@ $(REF_C) -lm

$(OUT)/ref_driver: ref_driver.c $(OUT)/libforword_ref.so
	$(CC) -O2 -std=c11 -march=native -Wall -I$(REF) -o $@ ref_driver.c \
	    -L$(OUT) -lforword_ref -Wl,-rpath,'$$ORIGIN' -lm

clean:
	rm -rf $(OUT)

.PHONY: all clean

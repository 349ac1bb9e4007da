# Builds the reference's CPU path from its own sources, in place under
# $(REF), into oracle/_ref/libpicograd_ref.so.  This is the checker's
# reference build: it is never linked into the product library.
#
# Flags follow the reference's x86_64 build (Makefile:6-7, :21-28): C11,
# -O3 -ffast-math, -mavx2 globally, per-file ISA flags for the
# mixed-precision micros.  clang is used because gcc 11 rejects
# -mavx512fp16.
REF     ?= /root/reference
OUT     ?= $(dir $(lastword $(MAKEFILE_LIST)))_ref
CC_REF  ?= clang
CFLAGS_REF := -O3 -std=c11 -ffast-math -funroll-loops -ftree-vectorize -fPIC \
              -mavx2 -w -I$(REF)/src -D_POSIX_C_SOURCE=200809L -DPG_ARCH_X86_64 -pthread
ASFLAGS_REF := -mavx2 -mavx512f

REF_C := $(shell find $(REF)/src -name '*.c' -not -path '*/backend/cuda/*' \
            -not -path '*/backend/metal/*' -not -path '*/backend/hip/*' \
            -not -name gemm_neon.c -not -name gemm_sve.c -not -name gemm_generic.c 2>/dev/null)
REF_S := $(shell find $(REF)/src -name '*.S' 2>/dev/null)
REF_O := $(patsubst $(REF)/src/%.c,$(OUT)/obj/%.o,$(REF_C)) \
         $(patsubst $(REF)/src/%.S,$(OUT)/obj/%.So,$(REF_S))

$(OUT)/obj/backend/cpu/hgemm_avx512fp16.o: XFLAGS = -mavx512fp16
$(OUT)/obj/backend/cpu/bgemm_avx512bf16.o: XFLAGS = -mavx512bf16
$(OUT)/obj/backend/cpu/amx_bf16.o: XFLAGS = -mamx-tile -mamx-bf16 -mavx512bf16

$(OUT)/libpicograd_ref.so: $(REF_O)
	$(CC_REF) $(CFLAGS_REF) -shared -o $@ $^ -lm -ldl -pthread

$(OUT)/obj/%.o: $(REF)/src/%.c
	@mkdir -p $(dir $@)
	$(CC_REF) $(CFLAGS_REF) $(XFLAGS) -c $< -o $@

$(OUT)/obj/%.So: $(REF)/src/%.S
	@mkdir -p $(dir $@)
	$(CC_REF) $(ASFLAGS_REF) -c $< -o $@

$(OUT)/libref_convert.so: $(dir $(lastword $(MAKEFILE_LIST)))ref_convert_shim.c
	@mkdir -p $(OUT)
	$(CC_REF) $(CFLAGS_REF) -shared -o $@ $<

# compiler and flags of this build, reported beside the CPU timings
$(OUT)/build_info.txt: $(OUT)/libpicograd_ref.so
	@{ $(CC_REF) --version | head -1; echo "CFLAGS $(CFLAGS_REF)"; } > $@

ref: $(OUT)/libpicograd_ref.so $(OUT)/libref_convert.so $(OUT)/build_info.txt
.PHONY: ref
.DEFAULT_GOAL := ref

# ref.mk — compile the reference's own C sources (read in place, never copied)
# into oracle/_ref/. Test and baseline infrastructure only: nothing in the
# product links these libraries.
#
#   make -f oracle/ref.mk            (from the repo root)
#
# Flags follow the reference Makefile:7-8 (-O3 -std=c11 -ffast-math -pthread),
# with ARCH overridden from -march=native to -march=x86-64-v3 (the Makefile's
# own ARCH knob): the libraries are built in one container and executed on
# another host, so they must not carry instructions of the build machine
# (AVX-512) that the other host may lack. x86-64-v3 keeps AVX2+FMA+F16C, so
# quant.c still selects its __AVX2__ kernel (quant.c:17-19).

REF      ?= /root/reference
OUT      := oracle/_ref
CC       ?= gcc
REFFLAGS := -O3 -std=c11 -Wall -Wextra -ffast-math -pthread -march=x86-64-v3 -fPIC
LDFLAGS  := -shared -Wl,-Bsymbolic -lm -lpthread

# Whole reference hot path + caller: quant.c, nn.c, loader.c, model.c, sample.c.
REF_ALL   := $(REF)/src/quant.c $(REF)/src/nn.c $(REF)/src/loader.c \
             $(REF)/src/model.c $(REF)/src/sample.c
# Caller only (model.c + loader.c): matmul, deq_row, rmsnorm, softmax, silu_f
# and rope_neox stay undefined and bind, at load time, to whichever library
# exporting the nn.h surface was loaded RTLD_GLOBAL first (the drop-in test).
REF_MODEL := $(REF)/src/model.c $(REF)/src/loader.c

# The same sources without -ffast-math: a second build of the reference whose
# rounding differs from the first only by the compiler's fast-math rewrites —
# the yardstick of how far two correct builds drift on a sensitive model.
NOFAST   := -O2 -std=c11 -Wall -Wextra -pthread -march=x86-64-v3 -fPIC

all: $(OUT)/libhakm_ref.so $(OUT)/libhakm_ref_model.so $(OUT)/libhakm_ref_nofast.so $(OUT)/build_info.txt

$(OUT):
	mkdir -p $(OUT)

$(OUT)/libhakm_ref.so: $(REF_ALL) | $(OUT)
	$(CC) $(REFFLAGS) -o $@ $(REF_ALL) $(LDFLAGS)

$(OUT)/libhakm_ref_nofast.so: $(REF_ALL) | $(OUT)
	$(CC) $(NOFAST) -o $@ $(REF_ALL) $(LDFLAGS)

$(OUT)/libhakm_ref_model.so: $(REF_MODEL) | $(OUT)
	$(CC) $(REFFLAGS) -o $@ $(REF_MODEL) $(LDFLAGS)

# compiler and flags of the build, for the CPU-baseline records
$(OUT)/build_info.txt: $(OUT)/libhakm_ref.so | $(OUT)
	{ $(CC) --version | head -n 1; echo "$(REFFLAGS)"; } > $@

clean:
	rm -rf $(OUT)

.PHONY: all clean

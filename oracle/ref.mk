# Builds the reference CPU library (hadilq/mfft-bench src/*.c, minus main.c)
# from the sources where they lie, into oracle/_ref/.  Test infrastructure:
# the library is only ever loaded by tests/ and by bench.py's CPU-baseline leg.
#
#   make -f oracle/ref.mk REF=/root/reference
#
# Two code paths are built so the library also loads on a host CPU that lacks
# AVX-512: x86-64-v4 (AVX-512, what the reference's -march=native selects on
# an AVX-512 host) and x86-64-v3 (AVX2).  Flags otherwise follow the
# reference's Makefile:2,6-8,14-17 (-O3 -funroll-loops -std=gnu11
# -DLIMB_BITS=16, OpenMP on).
REF     ?= /root/reference
OUT     ?= $(dir $(lastword $(MAKEFILE_LIST)))_ref
SRCS    := kernel.c bigmat.c roots.c methods.c mfft.c lowprec.c fpfixed.c mlgemm.c
CFLAGS  := -O3 -funroll-loops -std=gnu11 -DLIMB_BITS=16 -fopenmp -fPIC -w

all: $(OUT)/libmfftref_v4.so $(OUT)/libmfftref_v3.so

$(OUT)/libmfftref_v4.so: $(addprefix $(REF)/src/,$(SRCS))
	mkdir -p $(OUT)
	gcc $(CFLAGS) -march=x86-64-v4 -shared -o $@ $^ -lm

$(OUT)/libmfftref_v3.so: $(addprefix $(REF)/src/,$(SRCS))
	mkdir -p $(OUT)
	gcc $(CFLAGS) -march=x86-64-v3 -shared -o $@ $^ -lm

.PHONY: all

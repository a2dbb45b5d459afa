# Builds the reference C library from its own sources where they lie under
# /root/reference/src (every file except the CLI's main.c, as its Makefile's
# `lib` target does: Makefile:27-46), into oracle/_ref/.  Test
# infrastructure only: it validates the restatement in oracle.c and serves
# as the "reference" CPU baseline.  Nothing is copied into this repository.
#   _ref/libember_ref_debug.so  flags of `make debug` (Makefile:57-59)
#   _ref/libember_ref.so        flags of the optimized build (Makefile:23),
#                               -march=x86-64-v3 in place of -march=native
#   _ref/libember_ref_v4.so     the same with -march=x86-64-v4 (AVX-512), for
#                               hosts that have it (the build host's
#                               -march=native need not match the GPU host)
#   _ref/ember_cli              the reference's command-line program, every
#                               source file, `make debug` flags (the CPU side
#                               the product library's build of the same
#                               program is compared with)
#   _ref/ember_cli_o3           the same program with the optimized flags (its
#                               own build-to-build deviation, the bar for
#                               sampled completions)
# -Wl,-Bsymbolic keeps the library's internal calls inside itself, since its
# exported ember_* names equal the product library's.
REF ?= /root/reference
CC  ?= gcc
SRC := $(filter-out $(REF)/src/main.c,$(wildcard $(REF)/src/*.c))
COMMON = -std=c11 -D_DEFAULT_SOURCE -fPIC -shared -pthread -Wl,-Bsymbolic -w

.PHONY: all
all: _ref/libember_ref_debug.so _ref/libember_ref.so _ref/libember_ref_v4.so _ref/ember_cli _ref/ember_cli_o3

_ref:
	mkdir -p _ref

_ref/libember_ref_debug.so: $(SRC) | _ref
	$(CC) $(COMMON) -O2 -fno-fast-math -ffp-contract=off -o $@ $(SRC) -lm

_ref/libember_ref.so: $(SRC) | _ref
	$(CC) $(COMMON) -O3 -ffast-math -march=x86-64-v3 -funroll-loops -o $@ $(SRC) -lm

_ref/libember_ref_v4.so: $(SRC) | _ref
	$(CC) $(COMMON) -O3 -ffast-math -march=x86-64-v4 -funroll-loops -o $@ $(SRC) -lm

_ref/ember_cli: $(wildcard $(REF)/src/*.c) | _ref
	$(CC) -std=c11 -D_DEFAULT_SOURCE -pthread -w -O2 -fno-fast-math -ffp-contract=off -o $@ $(wildcard $(REF)/src/*.c) -lm

_ref/ember_cli_o3: $(wildcard $(REF)/src/*.c) | _ref
	$(CC) -std=c11 -D_DEFAULT_SOURCE -pthread -w -O3 -ffast-math -march=x86-64-v3 -funroll-loops -o $@ $(wildcard $(REF)/src/*.c) -lm

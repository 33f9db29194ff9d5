# Builds the reference engine's own sources, where they lie under
# /root/reference, into oracle/_ref/ (git-ignored).  This is a checker and
# the CPU baseline only; nothing in the product links it.
#
#   make -f oracle/ref.mk            (from the repo root)
#
# Two variants of the same engine sources:
#   oracle/  -DLZ_GDN_STATE_F32=1   the fp32-state float arm the GPU path
#                                   restates (run with --fixed off --fastfp off)
#   ship/    default defines        the reference's shipping build, timed as
#                                   the CPU baseline
# Flags follow the reference Makefile's native flavour (Makefile:137,174,183,
# 327-333): -O2 -march=x86-64 -mtune=alderlake -ffp-contract=off, the MMX/SSE
# translation units with -mmmx -msse -msse2, the AVX2 one with -mavx2.

REF      ?= /root/reference
OUT      := oracle/_ref
CC       := gcc
ENG      := err compat lfn json safetensors model ops ops_kernel ops_rope ops_moe \
            ops_epi ops_quant ops_sched ops_matmul ops_t2_arm ops_arm ops_t2_scalar \
            ops_norm ops_gdn ops_conv1d fwht forward forward_attn forward_moe \
            forward_ssm forward_kda forward_engram forward_csa2 forward_mtp \
            forward_rope forward_ckpt forward_state engram_keys sampler generate \
            lz_mathf lz_bf16 lz4d tokenizer unicode chat gbk cpucheck
MMX      := ops_mmx ops_mmx_sse ops_sse2
AVX2     := ops_avx2
BASEFL   := -O2 -std=c99 -w -march=x86-64 -mtune=alderlake -ffp-contract=off \
            -fPIC -I$(REF)/src -DLZ_MMX_TU=1 -DLZ_SSE2_TU=1 -DLZ_AVX2_TU=1

ORA_DEFS := -DLZ_GDN_STATE_F32=1
SHIP_DEFS :=

ORA_OBJS  := $(addprefix $(OUT)/oracle/,$(addsuffix .o,$(ENG) $(MMX) $(AVX2)))
SHIP_OBJS := $(addprefix $(OUT)/ship/,$(addsuffix .o,$(ENG) $(MMX) $(AVX2)))

all: $(OUT)/l98ref_oracle $(OUT)/l98ref_ship $(OUT)/libl98ref.so $(OUT)/libl98ref_subn.so

$(OUT)/oracle/%.o: $(REF)/src/%.c
	@mkdir -p $(OUT)/oracle
	$(CC) $(BASEFL) $(ORA_DEFS) -c -o $@ $<
$(addprefix $(OUT)/oracle/,$(addsuffix .o,$(MMX))): $(OUT)/oracle/%.o: $(REF)/src/%.c
	@mkdir -p $(OUT)/oracle
	$(CC) $(BASEFL) $(ORA_DEFS) -mmmx -msse -msse2 -c -o $@ $<
$(OUT)/oracle/$(AVX2).o: $(REF)/src/$(AVX2).c
	@mkdir -p $(OUT)/oracle
	$(CC) $(BASEFL) $(ORA_DEFS) -mavx2 -c -o $@ $<

$(OUT)/ship/%.o: $(REF)/src/%.c
	@mkdir -p $(OUT)/ship
	$(CC) $(BASEFL) $(SHIP_DEFS) -c -o $@ $<
$(addprefix $(OUT)/ship/,$(addsuffix .o,$(MMX))): $(OUT)/ship/%.o: $(REF)/src/%.c
	@mkdir -p $(OUT)/ship
	$(CC) $(BASEFL) $(SHIP_DEFS) -mmmx -msse -msse2 -c -o $@ $<
$(OUT)/ship/$(AVX2).o: $(REF)/src/$(AVX2).c
	@mkdir -p $(OUT)/ship
	$(CC) $(BASEFL) $(SHIP_DEFS) -mavx2 -c -o $@ $<

# The harness is this repo's own code; it drives the reference API.
$(OUT)/l98ref_oracle: oracle/ref_harness.c $(ORA_OBJS)
	$(CC) $(BASEFL) $(ORA_DEFS) -DHARNESS_ORACLE=1 -o $@ oracle/ref_harness.c $(ORA_OBJS) -lm
$(OUT)/l98ref_ship: oracle/ref_harness.c $(SHIP_OBJS)
	$(CC) $(BASEFL) $(SHIP_DEFS) -DHARNESS_ORACLE=0 -o $@ oracle/ref_harness.c $(SHIP_OBJS) -lm
$(OUT)/libl98ref.so: $(ORA_OBJS)
	$(CC) -shared -o $@ $(ORA_OBJS) -lm

.PHONY: all

# The reference's static subn_fwht_quant / subn_rot_f32 exported by a
# wrapper translation unit that compiles src/forward_kda.c in place
# (oracle/ref_subn.c), linked with every other oracle-mode object.
SUBN_OBJS := $(filter-out $(OUT)/oracle/forward_kda.o,$(ORA_OBJS))
$(OUT)/ref_subn.o: oracle/ref_subn.c $(REF)/src/forward_kda.c
	@mkdir -p $(OUT)
	$(CC) $(BASEFL) $(ORA_DEFS) -c -o $@ oracle/ref_subn.c
$(OUT)/libl98ref_subn.so: $(OUT)/ref_subn.o $(SUBN_OBJS)
	$(CC) -shared -o $@ $(OUT)/ref_subn.o $(SUBN_OBJS) -lm

# Tap build: the reference's own LZ_TAP hook (src/forward.h:27-36) routed to
# a recorder in the harness, to localise a divergence layer by layer.
TAP_DEFS := -DLZ_GDN_STATE_F32=1 '-DLZ_TAP(tag,li,ptr,n)=l98_tap(tag,li,(const float*)(ptr),n)' \
            '-Dl98_tap_decl=1' -include oracle/tap.h
TAP_OBJS := $(addprefix $(OUT)/tap/,$(addsuffix .o,$(ENG) $(MMX) $(AVX2)))
$(OUT)/tap/%.o: $(REF)/src/%.c oracle/tap.h
	@mkdir -p $(OUT)/tap
	$(CC) $(BASEFL) $(TAP_DEFS) -c -o $@ $<
$(addprefix $(OUT)/tap/,$(addsuffix .o,$(MMX))): $(OUT)/tap/%.o: $(REF)/src/%.c
	@mkdir -p $(OUT)/tap
	$(CC) $(BASEFL) $(TAP_DEFS) -mmmx -msse -msse2 -c -o $@ $<
$(OUT)/tap/$(AVX2).o: $(REF)/src/$(AVX2).c
	@mkdir -p $(OUT)/tap
	$(CC) $(BASEFL) $(TAP_DEFS) -mavx2 -c -o $@ $<
$(OUT)/l98ref_tap: oracle/ref_harness.c $(TAP_OBJS)
	$(CC) $(BASEFL) $(TAP_DEFS) -DHARNESS_ORACLE=1 -DHARNESS_TAP=1 -o $@ oracle/ref_harness.c $(TAP_OBJS) -lm
tap: $(OUT)/l98ref_tap
.PHONY: tap

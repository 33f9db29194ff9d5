/* llama98_hip.h -- C ABI of the MI355X (gfx950) implementation of the
 * llama98 MTP speculative-decoding step.
 *
 * The entry points keep the reference's names, argument meaning, return
 * conventions and error codes (reference src/forward.h:1883-2150,
 * src/llama_zh.h:520-640, llama98.def:14-60), so a caller of the
 * reference's spec path links against libl98hip.so instead.  All compute
 * runs on the GPU; the structs below carry the fields callers of the
 * reference read (LZRunState's mtp_* buffers, ssm_slot, mtp_pos, ...) as
 * host mirrors, refreshed by the entry point that returns them.
 *
 * Numerics: the reference's float-oracle mode (--fixed off --fastfp off,
 * fp32 KDA state, Q8 KV cache, no attention window).  Results are
 * bit-identical to that mode of the reference engine.
 *
 * Threading: like the reference, one LZRunState is used by one thread at a
 * time; distinct states may run concurrently on distinct HIP streams.
 */
#ifndef LLAMA98_HIP_H
#define LLAMA98_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef unsigned long long lz_u64;

/* Reference error codes (src/err.h:19-380) that this path returns. */
enum {
    LZ_ERR_OK = 0,
    LZ_ERR_NULL_ARG = 6,
    LZ_ERR_STATE_ALLOC = 7,
    LZ_ERR_FORWARD = 20,
    LZ_ERR_SPEC_NO_HEAD = 24,
    LZ_ERR_SPEC_K_RANGE = 25,
    LZ_ERR_BIN_OPEN = 81,
    LZ_ERR_BIN_MAGIC = 83,
    LZ_ERR_BIN_VERSION = 84
};

#define LZ_KVF_Q8 0           /* src/forward.h:428 */
#define LZ_PROF_N 7           /* src/forward.h:502 */
#define LZ_SPEC_K_MAX 6      /* src/ops.h:2098 */
/* This library's own draft-width cap: the l98_* generation loops run k up to
 * 7 (a verify of M = 8 = LZ_BATCH_MAX rows).  The reference-named entry
 * points keep the reference's LZ_SPEC_K_MAX check and error. */
#define L98_SPEC_K_GPU 7
#define LZ_BATCH_MAX 8       /* src/ops.h:1457 */

/* The LZModelConfig fields the spec path reads (src/model.h:237-874). */
typedef struct {
    int vocab_size, hidden_size, n_layers, seq_len;
    int n_heads, n_kv_heads, head_dim, rotary_dim;
    int lin_n_k_heads, lin_n_v_heads, lin_k_head_dim, lin_v_head_dim, conv_kernel;
    int n_linear_layers, n_full_layers;
    int attn_q_dim, attn_qgate_dim, attn_kv_dim, lin_key_dim, lin_value_dim, lin_conv_dim;
    int kda_gate_rank, num_experts, num_experts_per_token, moe_latent_dim;
    int moe_intermediate_size, moe_shared_width, mtp_intermediate_size, mtp_n_layers;
    float rms_norm_eps, rope_theta;
    int layer_types[128];
    int use_subn, hadamard_o, hadamard_down;   /* SubLN (src/model.h: use_subn, hadamard_o/_down) */
    int mtp_n_draft, mtp_markov_rank;          /* DSpark (src/model.h:359-375): > 1 draft slots; a
                                                  model.bin carries no Markov rank (0) */
    int kda_has_gate_lower_bound;              /* src/model.h:264-265: the KDA gate is */
    float kda_gate_lower_bound;                /* lb * sigmoid(exp(A_log) * pre) when set */
} LZModelConfig;

/* Caller-allocated, as in the reference: LZModel m; lz_open(&m, dir, ...). */
typedef struct {
    LZModelConfig config;
    long long bytes_device;        /* device memory held by the weights */
    void *impl;                    /* device weights */
} LZModel;

typedef struct {
    int seq_len;
    int ssm_slot;                  /* KDA/conv ring slot (src/forward.h:1153) */
    int ssm_ring_depth;            /* spec_k_max + 1 (src/forward.h:1164) */
    int mtp_pos;                   /* next MTP KV row (src/forward.h:897) */
    int nt_cap;                    /* tokens per forward chunk */
    /* host mirrors, refreshed by the call that returns or fills them */
    float *logits;                 /* vocab: lz_forward_capture */
    float *mtp_logits;             /* (L98_SPEC_K_GPU+1) x vocab: lz_forward_verify */
    float *mtp_verify_hidden;      /* (L98_SPEC_K_GPU+1) x hidden: lz_forward_verify */
    float *mtp_chain;              /* hidden: after capture / draft / round */
    float *mtp_draft_logits;       /* vocab: lz_mtp_draft_step */
    float *mtp_kdraft_logits;      /* LZ_SPEC_K_MAX x vocab: lz_mtp_draft_batch (DSpark models; NULL
                                      otherwise, src/forward.h:866) */
    long long bytes_device;
    void *impl;
} LZRunState;

/* LZSampleParams / LZSampler subset (src/sampler.h:150-190).  Penalties
 * are outside this path: a sampler whose penalties are active is refused. */
typedef struct {
    float temperature;
    float temp_think;
    int think_temp_enabled;
    float topp;
    float minp;
    int topk;
    float presence_penalty;
    float frequency_penalty;
    float repetition_penalty;
    int repeat_last_n;
    int minp_llamacpp;
} LZSampleParams;

typedef struct {
    int vocab_size;
    LZSampleParams p;
    lz_u64 rng_state;
} LZSampler;

/* ---- model (src/model.h:1327-1341) ---- */
/* lz_load_config (src/model.h:1327): the model's configuration without
 * loading it.  This path reads model.bin only: path is a model.bin or a
 * directory holding one (a config.json is refused).  Returns 0, or 1 with a
 * message. */
int lz_load_config(LZModelConfig *c, const char *path, char *errbuf, int errlen);
/* Reads <dir>/model.bin and uploads the weights to the current HIP device
 * (the reference also reads a model.bin whole in lz_open,
 * src/model.c:3264-3266).  Returns 0, or 1 with a message in errbuf. */
int lz_open(LZModel *m, const char *dir, char *errbuf, int errlen);
/* lz_read_weights (src/model.h:1337): the weights of a model.bin are loaded
 * by lz_open, so this returns 0 for an open model, 1 otherwise. */
int lz_read_weights(LZModel *m, char *errbuf, int errlen);
void lz_free(LZModel *m);

/* ---- run state (src/forward.h:1883-1933) ---- */
/* Returns 0, or 1 with a message. Ring depth is spec_k_max + 1 (spec_k_max
 * clamped to L98_SPEC_K_GPU).  seq_len <= 0 takes the model's. */
int lz_state_alloc(LZRunState *s, const LZModel *m, int seq_len, int spec_k_max,
                   char *errbuf, int errlen);
void lz_state_free(LZRunState *s);
void lz_state_reset(LZRunState *s, const LZModel *m);

/* ---- forward (src/forward.h:1937-2150) ---- */
/* lz_forward (src/forward.h:1937): one token at pos; returns the host
 * logits mirror s->logits (do not free), or NULL.  mtp_chain is untouched. */
float *lz_forward(const LZModel *m, LZRunState *s, int token, int pos);
/* One token; its final-normed hidden goes to mtp_chain.  Returns the host
 * logits mirror, or NULL on a bad token/position. */
float *lz_forward_capture(const LZModel *m, LZRunState *s, int token, int pos);
/* Prefill of n tokens at pos0.. with every row's final-normed hidden copied
 * to hidden_out (host, n x hidden).  Returns s->logits (last row's logits are
 * not computed, as in the reference: the pointer is only a success flag), or
 * NULL. */
float *lz_forward_batch_capture(const LZModel *m, LZRunState *s, const int *tokens, int n,
                                int pos0, float *hidden_out);
/* Verify forward of n <= LZ_BATCH_MAX tokens at pos0..: every row's logits
 * into s->mtp_logits and hidden into s->mtp_verify_hidden; advances the ring
 * by n.  Returns 0, or 1 on failure. */
int lz_forward_verify(const LZModel *m, LZRunState *s, const int *tokens, int n, int pos0);
/* One MTP draft step; returns s->mtp_draft_logits, or NULL (also on a
 * DSpark head, which binds no fc). */
float *lz_mtp_draft_step(const LZModel *m, LZRunState *s, int next_token, int pos);
/* DSpark (mtp_n_draft > 1): lz_mtp_draft_batch (src/forward.h:2033, body
 * src/forward_mtp.c:385-505): k <= mtp_n_draft independent slots from
 * s->mtp_chain, slot 0 fed next_token, the rest the mask row; their base
 * logits into s->mtp_kdraft_logits (returned), or NULL.  The chain is not
 * changed.  lz_mtp_markov_correct (src/forward.h:2046, body
 * src/forward_mtp.c:510-531) adds markov_proj(markov_embed[x_prev]) to
 * logits in place: the rank of a model.bin head is 0, so it adds zeros. */
float *lz_mtp_draft_batch(const LZModel *m, LZRunState *s, int next_token, int k);
void lz_mtp_markov_correct(const LZModel *m, LZRunState *s, int x_prev, float *logits);
/* MTP KV rows from (hidden, next token) pairs.  Returns 0, or 1 (also on a
 * DSpark head). */
int lz_mtp_prefill(const LZModel *m, LZRunState *s, const float *h_body_all,
                   const int *next_tokens, int n, int pos0);
int lz_mtp_catchup(const LZModel *m, LZRunState *s, const float *h_body_all,
                   const int *next_tokens, int n, int pos0);

/* ---- acceptance and rounds (src/llama_zh.h:520-640) ---- */
int lz_spec_accept(const int *draft, const int *targ, int n_draft, int bonus, int *out);
int lz_spec_accept_temp(const float *p, const float *q, int x, int vocab, float u,
                        lz_u64 *residual_rng, int *out_accepted);
/* Greedy round.  Returns n_accept + 1 (tokens in out), 0 on discard
 * (k_eff < n_min), or -LZErr. */
int lz_spec_round(const LZModel *m, LZRunState *s, int anchor, int anchor_pos, int k,
                  float p_min, int n_min, const LZSampler *samp, int debug_break_rollback,
                  int debug_skip_catchup, int *out, int *out_n_accept, int *out_new_pos,
                  int *out_k_eff, char *errbuf, int errlen);
/* Temperature / top-p round (src/generate.c:1234-1377). */
int lz_spec_round_temp(const LZModel *m, LZRunState *s, int anchor, int anchor_pos, int k,
                       float p_min, int n_min, LZSampler *samp, int debug_break_rollback,
                       int debug_skip_catchup, int *out, int *out_n_accept, int *out_new_pos,
                       int *out_k_eff, char *errbuf, int errlen);
/* DSpark rounds (src/llama_zh.h:629-660; src/generate.c:1000-1133 and
 * 1382-1505): one draft batch, each slot corrected and argmax'd (greedy) or
 * sampled (temperature) in order with the p_min cut, the verify,
 * acceptance, ring rollback and the chain reseed; no catch-up and no
 * mtp_pos advance.  k <= mtp_n_draft.  lz_spec_round / lz_spec_round_temp
 * refuse a DSpark head, these refuse a one-slot head. */
int lz_spec_round_dspark(const LZModel *m, LZRunState *s, int anchor, int anchor_pos, int k,
                         float p_min, int n_min, const LZSampler *samp, int debug_break_rollback,
                         int *out, int *out_n_accept, int *out_new_pos, int *out_k_eff,
                         char *errbuf, int errlen);
int lz_spec_round_dspark_temp(const LZModel *m, LZRunState *s, int anchor, int anchor_pos, int k,
                              float p_min, int n_min, LZSampler *samp, int debug_break_rollback,
                              int *out, int *out_n_accept, int *out_new_pos, int *out_k_eff,
                              char *errbuf, int errlen);

/* ---- sampler (src/sampler.h:200-230) ---- */
void lz_sample_defaults(LZSampleParams *p);
int lz_sampler_init(LZSampler *s, int vocab_size, const LZSampleParams *p, lz_u64 seed);
void lz_sampler_free(LZSampler *s);
float lz_random_f32(lz_u64 *state);
int lz_sample_argmax(const float *logits, int n);
int lz_argmax_p1(const float *logits, int n, float *out_p);

/* ---- exported data (llama98.def:117-157; src/forward.c:29-448,
 * src/generate.c:226) ----
 * Counters, updated as the reference's are: lz_debug_us_draft / _verify /
 * _capture / _catchup (microseconds; device time between stream marks for
 * the device-resident round), lz_debug_n_capture / _catchup /
 * _ring_rollback / _chunks / _lmhead.  The device-resident loops
 * (l98_greedy_rounds, l98_generate) add their rounds' rollback, catch-up,
 * chunk and lm_head counts but no per-phase times.
 * Knobs: this path implements one setting of each, which is the value they
 * hold: Q8 K and V caches, no KV rotation, no attention sink or window
 * (lz_attn_window 0; the reference's default -1 selects an automatic
 * window), the model's own top-k (lz_moe_topk 0) at lz_moe_tau 1, and no
 * MTP attention probes.  lz_state_alloc and every forward or round entry
 * point refuse to run when a caller has set another value.  lz_prof_us
 * stays zero: per-section times come from rocprofv3 on this path. */
extern long long lz_debug_us_draft, lz_debug_us_verify, lz_debug_us_capture, lz_debug_us_catchup;
extern long long lz_debug_n_capture, lz_debug_n_catchup, lz_debug_n_ring_rollback;
extern long long lz_debug_n_chunks, lz_debug_n_lmhead, lz_debug_n_kv_rot, lz_debug_attn_skip;
extern long long lz_debug_mtp_attn_rows;
extern float lz_debug_mtp_attn_scale;
extern int lz_debug_mtp_attn_window;
extern int lz_kv_kfmt, lz_kv_vfmt, lz_kv_rot_enable, lz_attn_sink, lz_attn_window;
extern int lz_moe_topk;
extern float lz_moe_tau;
extern int lz_prof_enable;
extern float lz_prof_us[LZ_PROF_N];

/* ---- this implementation's own additions (no reference counterpart) ---- */
/* The whole generation loop of lz_generate's --spec path
 * (src/generate.c:1822-2106, penalties off): prefill + MTP prefill, then
 * rounds until n_new tokens are emitted.  Greedy rounds run back to back on
 * the device with no host round trip.  tokens receives up to cap ids
 * (whole last round).  With a temperature sampler, samp->rng_state is
 * advanced as the run consumed it.  Returns the number of tokens emitted,
 * or -LZErr. */
int l98_generate(const LZModel *m, LZRunState *s, const int *prompt, int n_prompt, int k,
                 int n_new, LZSampler *samp, int *tokens, int cap, int *k_eff_out,
                 int *n_accept_out, int *n_rounds);
/* Prefill + MTP prefill + first capture forward of a prompt, seeding the
 * device round state.  Returns the first emitted token, or -LZErr. */
int l98_session_start(const LZModel *m, LZRunState *s, const int *prompt, int n_prompt,
                      const LZSampler *samp);
/* The sampler of the session l98_session_start began (its parameters and
 * the generator state after the first token's draw), for a caller that
 * drives the session's rounds itself (lz_spec_round_temp).  Returns 0, or
 * 1 on a null argument. */
int l98_session_sampler(const LZRunState *s, LZSampler *out);
/* n greedy rounds after l98_session_start (or a previous call), back to back
 * on the device: every scalar of a round (positions, ring slot, drafts,
 * acceptance) stays in device memory, and with use_graph each round is one
 * HIP graph launch.  tokens receives the emitted ids, n_accept_out each
 * round's acceptance, device_ms the hipEvent time of the n rounds.  Returns
 * the number of tokens emitted, or -LZErr. */
int l98_greedy_rounds(const LZModel *m, LZRunState *s, int k, int n_rounds, int use_graph, int *tokens,
                      int cap, int *n_accept_out, float *device_ms);
/* l98_greedy_rounds plus, per round, the distinct (layer, expert) weight
 * sets its verify streamed and its new_pos (for byte accounting). */
int l98_greedy_rounds_ex(const LZModel *m, LZRunState *s, int k, int n_rounds, int use_graph, int *tokens,
                         int cap, int *n_accept_out, int *experts_out, int *new_pos_out, float *device_ms);
/* Session batches (configs[4]'s server-style verify).  No counterpart in the
 * reference, which keeps one sequence per LZRunState and has no batching;
 * the reference-equivalent result is n_seq independent calls.  Each session
 * is enqueued on its own stream and the calls return when all are done.
 *
 * l98_verify_batch: lz_forward_verify (src/forward.h:2060) of n_tok
 * tokens for each of n_seq sessions of one model; session i verifies
 * tokens[i*n_tok ..] at positions pos0[i]...  With copy_out the logits and
 * captured hidden rows land in each state's mtp_logits / mtp_verify_hidden
 * as lz_forward_verify leaves them.  wall_ms: host time of the batch.
 * Returns 0, or 1 on a bad argument or a device error. */
int l98_verify_batch(const LZModel *m, LZRunState **states, int n_seq, const int *tokens, int n_tok,
                     const int *pos0, int copy_out, float *wall_ms);
/* l98_greedy_rounds for n_seq sessions started with l98_session_start:
 * n_rounds rounds each.  tokens[i*cap ..] receives session i's emitted ids,
 * n_out[i] their count.  Returns the total tokens emitted, or -LZErr.
 * The rounds run batched across the sessions when the model allows it (a
 * one-slot MTP head, no SubLN, one scale per weight row, (k+1)*n_seq <= 512
 * rows): each draft step is one many-row pass over every session's row, the
 * verify one many-row forward, then every session's acceptance, catch-up
 * and round record in one launch each; otherwise each session's round graph
 * is replayed on its own stream.  Either way each session emits exactly what
 * it emits alone. */
int l98_greedy_rounds_batch(const LZModel *m, LZRunState **states, int n_seq, int k, int n_rounds, int *tokens,
                            int cap, int *n_out, float *wall_ms);
/* l98_greedy_rounds_batch with the path chosen: mode 0 as above, mode 1
 * each session's own round graph (the reference for the batched path's
 * tests). */
int l98_greedy_rounds_batch_ex(const LZModel *m, LZRunState **states, int n_seq, int k, int n_rounds, int *tokens,
                               int cap, int *n_out, float *wall_ms, int mode);
/* 1 when l98_greedy_rounds_batch runs n_seq sessions of this model at
 * draft width k as batched rounds, else 0. */
int l98_batched_rounds_ok(const LZModel *m, int n_seq, int k);
/* The attention path of a session's chunk (verify, draft step, capture
 * chunk): 0 chosen by the session's capacity (past 2048 positions two
 * launches: the scores of every 64-position slice, kv head and token, then
 * the softmax and value chains of every (q head, token, 32-wide output
 * group); else one launch per (q head, token)); 1 always the one launch;
 * 2 the two launches wherever their LDS fits.  Both give the same bits.
 * Process-wide; applies to launches enqueued and graphs captured
 * afterwards.  No counterpart in the reference (a tuning and test
 * control). */
void l98_set_attn_path(int mode);
/* Mean duration of `iters` launches, hipEvent-timed on the state's stream.
 * which = 0: the tied lm_head GEMV with mrows token rows, back to back;
 * 1: the verify forward of mrows tokens; 2: a device copy of the lm_head's
 * int8 bytes (calibration for byte counters); 3: the lm_head GEMV after a
 * cache-evicting 512 MiB copy each time (only the GEMV timed); 4, 5, 6: the
 * RMSNorm-prologue GEMV of every KDA layer's, attention layer's and layer's
 * MoE input projections in order, back to back (mean per launch); 7-10:
 * the launch floor, per launch of a chain of 64 dependent launches: 7 an
 * empty kernel of 1 block, 8 of 256 blocks, 9 a kernel of 256 blocks each
 * reading the mrows x hidden floats the previous launch wrote (7-9 captured
 * as one HIP graph and replayed), 10 mode 8 launched without a graph, 11
 * mode 9 plus a last-block reduction per 8 blocks (device-scope release,
 * counter, acquire, the group's partials read back), as a graph.
 * Returns 0 (1 on a bad argument or a device error). */
int l98_time_kernel(const LZModel *m, LZRunState *s, int which, int mrows, int iters, float *avg_ms);
/* Per-CU streaming probe: 16 dependent launches of `blocks` blocks of
 * `threads` (256, 512 or 1024) threads, each block streaming its own
 * kb_per_block KiB (non-temporal 16-byte loads, 16 per thread in flight),
 * each launch on a fresh region of a 1 GiB buffer.  *us_per_launch: the mean
 * per launch.  Returns 0 (1 on a bad argument or a device error). */
int l98_time_stream(LZRunState *s, int blocks, int threads, int kb_per_block, int iters, float *us_per_launch);
/* For each of `rows` rows of n (<= 2048) non-negative floats (host
 * arrays), the float the serial loop s = 0; s += x[i] gives, computed on the
 * device by the parallel routine the RMSNorm kernels use for their sums of
 * squares.  No reference counterpart: a check of that routine on arbitrary
 * inputs.  Returns 0 (1 on a bad argument or a device error). */
int l98_row_sums(const float *x, int rows, int n, float *out);

/* Block-diagonal Walsh-Hadamard transforms of the SubLN variant
 * (use_subn = 1, hadamard_o / hadamard_down > 0), on the device, over host
 * arrays of `rows` rows of n <= 8192 elements; blk is a power of two
 * dividing n.  Each returns 0 (1 on a bad argument or a device error).
 *
 * l98_fwht_i32 replaces lz_fwht_i32 (src/fwht.c:65, src/fwht.h), applied to
 * each blk-block of each row: y = H x in wrapping int32. */
int l98_fwht_i32(const int32_t *x, int32_t *y, int rows, int n, int blk);
/* l98_fwht_f32 replaces lz_fwht (src/fwht.c:198, declared in src/ops.h) on
 * each blk-block, in place; rot = 1 then multiplies every element by
 * rsqrt(blk) (lz_rsqrt_float_body), which is subn_rot_f32
 * (src/forward_kda.c:130-135). */
int l98_fwht_f32(float *v, int rows, int n, int blk, int rot);
/* subn_fwht_quant (src/forward_kda.c:43-92, a static function of the
 * reference, so no FFI binds it today): each row of n (n % 32 == 0) floats
 * to n int8 codes in q and n / 32 scales in s, one scale per gw elements
 * (gw = n unless gw is a multiple of 32 dividing n), repeated in each of
 * the group's 32-element slots, as lz_matmul_xq_nt reads them. */
int l98_subn_fwht_quant(const float *x, int rows, int n, int blk, int gw, int8_t *q, float *s);
/* Index-order prefix queries over `rows` rows of n non-negative floats
 * (host arrays), answered on the device by the routine the temperature
 * sampler uses for its softmax sums and cdf scans: mode 0 gives in outv[r]
 * the float the serial loop s = 0; s += x[i] ends with (out[r] = -1);
 * mode 1 the first index i whose running sum exceeds c[r], mode 2 the first
 * whose running sum reaches c[r], in out[r] with that running sum in
 * outv[r] (-1 and the total when there is none).  No reference
 * counterpart: a check of that routine.  Returns 0 (1 on a bad argument or
 * a device error). */
int l98_prefix_query(const float *x, int rows, int n, int mode, const float *c, int *out, float *outv);
/* MoE routing of nt (<= 8) tokens over E (<= 128) experts, top-k (<= 8),
 * computed on the device by the routine the expert kernels run in each
 * block: host logits[nt][E] and bias[E] (NULL: zeros) in, idx[nt][topk]
 * and renormalized weights w[nt][topk] out, as lz_moe_route
 * (src/ops_moe.c:12-163, sigmoid scores, no temperature) fills idx_out /
 * w_out per token.  A check of that routine on arbitrary logits; the
 * reference routes inside forward_moe (src/forward_moe.c:96-98).  Returns 0
 * (1 on a bad argument or a device error). */
int l98_moe_route(const float *logits, const float *bias, int nt, int E, int topk, int *idx, float *w);
/* The device argmax of the draft steps and verify rows, on `rows` (<= 8)
 * host rows of n floats: mode 0 is lz_sample_argmax (src/sampler.c:226-243,
 * order-preserving key, first index wins), mode 1 the index lz_argmax_p1
 * returns (src/sampler.c:279-295: float '>' from element 0, so a NaN at 0
 * stays the answer).  A check of the kernel the rounds run; the reference
 * has no device.  Returns 0 (1 on a bad argument or a device error). */
int l98_argmax_rows(const float *x, int rows, int n, int mode, int *out);
/* The top-p candidates' order on host keys: a stable descending sort of n
 * (<= 2^20) keys below 2^30 (the bits of probabilities in [0, 1]) with
 * their indices, by the library's radix sort, as select_all orders the
 * candidates (src/sampler.c:526-538: descending, equal keys in index
 * order).  Returns 0 (1 on a bad argument or a device error). */
int l98_sort_desc(const uint32_t *keys, int n, uint32_t *keys_out, int *idx_out);
/* The rounds' argmax path on host inputs: the tied lm_head GEMV's epilogue
 * (per-tile packed maxima of N rows of K int8 weights with scales ws, one
 * per row for gs = 0 or K, else K/gs per row in groups of gs) over M rows of
 * per-32 quantized activations, then the reduction of the tile candidates;
 * logits (M x N) and the argmax of each row (mode as l98_argmax_rows) come
 * back.  A check of the kernels the rounds run (src/sampler.c:226-295); the
 * reference has no device.  Returns 0 (1 on a bad argument or a device
 * error). */
int l98_gemv_argmax(const int8_t *w, const float *ws, int N, int K, int gs, const int8_t *xq, const float *xqs,
                    int M, int mode, float *logits, int *out);
/* lz_spec_accept_temp (src/generate.c:283-346) on host rows with no device
 * allocation: no counterpart in the reference; for callers that cannot call
 * hipMalloc (tight serving loops, harnesses that forbid it).  It copies
 * synchronously and waits for its kernel, so it is not for code under HIP
 * graph capture.  The rows, the generator state and the result are staged
 * in a static device array of 2 * L98_NOALLOC_MAX_VOCAB floats + 256 bytes
 * per GPU, held until the process ends; calls that overlap on one GPU race
 * on it.  Returns what lz_spec_accept_temp returns (the token, -1 on bad
 * input), -2 when vocab > L98_NOALLOC_MAX_VOCAB, -3 on a device error. */
#define L98_NOALLOC_MAX_VOCAB 262144
int l98_spec_accept_temp_noalloc(const float *p, const float *q, int x, int vocab, float u,
                                 lz_u64 *residual_rng, int *out_accepted);
/* The wide int8 GEMM of the many-row forwards (prefill chunks, batched
 * verify) on host arrays: out[t][n] = (sum_s float(acc[t,n,s]) * xqs[t][s])
 * * ws[n] for M token rows of K (K % 32 == 0) int8 codes against N weight
 * rows, acc the exact int32 group sums, as lz_matmul_xq_nt computes it
 * (src/ops_matmul.c:336-466, src/ops_epi.c:983-1017).  A check of the
 * matrix-core kernel; returns 0 (1 on a bad argument or a device error). */
int l98_gemm_q8(const int8_t *w, const float *ws, int N, int K, const int8_t *xq, const float *xqs, int M,
                float *out);
/* Device and build facts, for logs. */
const char *l98_device_name(void);
/* Seconds of device time of the last l98_generate call's round loop
 * (hipEvent-timed), and its round count. */
double l98_last_loop_seconds(void);

#ifdef __cplusplus
}
#endif
#endif

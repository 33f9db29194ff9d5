// Host-side launchers of the gfx950 kernels (l98_k_*.hip).  Each returns
// 0, a HIP error code, or -1 when the arguments do not fit the kernel's
// shape limits (checked on the host before any launch).
#ifndef L98_LAUNCH_H
#define L98_LAUNCH_H
#include <hip/hip_runtime.h>

#include "l98_dev.h"

extern "C" {
int l98k_upload_exp_table(const float *tab);
// per translation unit (l98k_upload_exp_table runs all of them)
int l98k_upload_exp_table_misc(const float *tab);
int l98k_upload_exp_table_gemv(const float *tab);
int l98k_upload_exp_table_moe(const float *tab);
int l98k_upload_exp_table_kda(const float *tab);
int l98k_upload_exp_table_attn(const float *tab);
int l98k_upload_exp_table_smp(const float *tab);
int l98k_upload_exp_table_mfma(const float *tab);
// Wide int8 GEMM on the matrix cores (l98_k_mfma.hip): out[t][n] for M
// token rows, bit-identical to the GEMV path per token.
int l98k_mfma_gemm(const int8_t *W, const float *ws, int N, int K, const int8_t *X, const float *Xs, int M, float *out,
                   int out_stride, hipStream_t st);
// Up to six dense GEMMs over the same M rows in one launch (each its own
// weights, input rows of width K[j] and output).
int l98k_mfma_gemm_multi(int n_jobs, const int8_t *const *W, const float *const *ws, const int *N, float *const *out,
                         const int *out_stride, const int *K, const int8_t *const *X, const float *const *Xs, int M,
                         hipStream_t st);
// Grouped over experts: group g < *ng multiplies expert gexp[g]'s bank rows
// with its columns list[goff[g] .. + gcnt[g]] (activation row xmap[col] or
// col, output row col).  mean_cols, the host's estimate of the columns per
// group, picks the tile shape (the same bits either way).
int l98k_mfma_gemm_grouped(const int8_t *bank, const float *bank_s, int N, int K, const int8_t *X, const float *Xs,
                           const int *ng, int max_groups, const int *gexp, const int *goff, const int *gcnt,
                           const int *list, const int *xmap, int max_cols, int mean_cols, float *out, int out_stride,
                           hipStream_t st);
// Two grouped GEMMs over the same columns and groups (w1 and w3), one
// launch where the tiles allow.
int l98k_mfma_gemm_grouped2(const int8_t *bank1, const float *bank1_s, float *out1, const int8_t *bank3,
                            const float *bank3_s, float *out3, int N, int K, const int8_t *X, const float *Xs,
                            const int *ng, int max_groups, const int *gexp, const int *goff, const int *gcnt,
                            const int *list, const int *xmap, int max_cols, int mean_cols, int out_stride,
                            hipStream_t st);
// Quantized GEMM inputs of `rows` rows: mode 0 quantize, 1 silu(src)*src2,
// 2 slot-ordered expert combine; the GEMV prologues' arithmetic.
int l98k_wide_pro(int mode, const float *src, const float *src2, int src_stride, const int *sel_idx,
                  const float *sel_w, int topk, int n, int rows, int8_t *xq, float *xqs, hipStream_t st);
// The same rows left in float (fout, row stride n), for a norm before the
// quantization (the SubLN routed-up and shared-down inputs).
int l98k_wide_pro_f(int mode, const float *src, const float *src2, int src_stride, const int *sel_idx,
                    const float *sel_w, int topk, int n, int rows, float *fout, hipStream_t st);
// Temperature sampling (one block per call; l98_k_sample.hip).
// The launches that take `skip` (a device flag) do nothing when it is set
// (null: never).
// probs = softmax(logits * inv_t); with keys: the top-p candidate keys for
// l98k_smp_sort_desc and their count.
int l98k_smp_softmax(const float *logits, int n, float inv_t, float *probs, float cutoff, uint32_t *keys,
                     int *n_cand, const int *skip, hipStream_t st);
// A draw from p by the cdf (rng advanced on the device); ctl_tok optional.
int l98k_smp_draw(const float *p, int n, unsigned long long *rng, int *out_tok, float *out_p, int *ctl_tok,
                  const int *skip, hipStream_t st);
// Scratch bytes of l98k_smp_sort_desc for n keys.
size_t l98k_smp_sort_tmp_bytes(int n);
// Stable descending sort of n keys (below 2^30) with their indices: a
// radix sort of this library's own, three passes of three launches; keys
// is overwritten.
int l98k_smp_sort_desc(uint32_t *keys, uint32_t *keys_out, int *vals_out, int n, void *tmp, const int *skip,
                       hipStream_t st);
// Top-p target distribution from the softmax and the sorted candidates.
int l98k_smp_topp_dist(const float *probs, int n, const uint32_t *skeys, const int *svals, const int *n_cand,
                       float topp, float *p_out, const int *skip, hipStream_t st);
// Speculative acceptance of draft x with residual resampling (u given, or
// drawn when u is null): out[0] token, out[1] accepted.
int l98k_smp_accept(const float *p, const float *q, int n, int x, const float *u, unsigned long long *rng, int *out,
                    hipStream_t st);
// The same for row `row` of a device-resident round: the draft token from
// x_dev, the emitted token to *ctl_out; a rejection sets *ctl_n = row and
// *done (nothing runs once *done is set).
int l98k_smp_accept_row(const float *p, const float *q, int n, const int *x_dev, unsigned long long *rng,
                        int *ctl_out, int *ctl_n, int *done, int row, hipStream_t st);
// lz_sample_ex's top-p draw after the candidate sort.
int l98k_smp_sample_topp(const float *probs, int n, const uint32_t *skeys, const int *svals, const int *n_cand,
                         float topp, unsigned long long *rng, int *out_tok, hipStream_t st);
// Exact index-order prefix queries over rows of n (mode 0 total, 1 first
// prefix > c, 2 first prefix >= c): out = index (-1 none), outv = value.
int l98k_smp_xprefix(const float *x, int rows, int n, int mode, const float *c, int *out, float *outv,
                     hipStream_t st);
// Fused GEMV of b->n jobs over m <= MAX_CHUNK activation rows; each job's
// prologue builds its int8 input rows.
int l98k_gemv(GemvBatch *b, int m, hipStream_t st);
// Tiles of a GEMV over `rows` rows of in_dim with m token rows (the grid of
// l98k_gemv; an argmax epilogue needs tiles * m partial entries).
int l98k_gemv_tiles(int rows, int in_dim, int m);
// 1 when a GEMV with an RMSNorm prologue over m rows of in_dim fits the kernel.
int l98k_gemv_norm_fits(int in_dim, int m);
// Grouped expert GEMV: n_jobs (<= 2) projections over the groups in grp.
int l98k_expert_gemv(const ExpertJob *jobs, int n_jobs, const MoeGroups *grp, int max_groups, int in_dim,
                     int out_rows, int nt, hipStream_t st);
int l98k_embed(const int8_t *q, const float *s, const int *toks, int d, int gs, int nt, float *x, hipStream_t st);
// x += a (+ b) (when a), RMSNorm(1+w) -> out (when out) and per-32 int8 (when xq).
int l98k_rmsnorm(float *x, int x_stride, const float *a, const float *b, const float *w, int n, float eps,
                 int rows, float *out, int out_stride, int8_t *xq, float *xqs, hipStream_t st);
// The same with w == nullptr allowed (no norm: the folded row is only stored
// and/or quantized) and tok = 1 for one int8 scale per row
// (lz_quantize_q8_tok) instead of one per 32 elements.
int l98k_rmsnorm_ex(float *x, int x_stride, const float *a, const float *b, const float *w, int n, float eps,
                    int rows, float *out, int out_stride, int8_t *xq, float *xqs, int tok, hipStream_t st);
// MTP input rows: [norm_e(embed(tok)) | norm_h(h)] quantized per 32 into xq [rows][2d].
// DSpark main_proj input rows: [norm(chain) | norm(emb(tok[0]) or mask) | depth row], quantized per 32
int l98k_dspark_pre(const int8_t *emb_q, const float *emb_s, int gs, const int *tok, const float *chain,
                    const float *mask, const float *depth, int d, const float *w_e, const float *w_h, float eps,
                    int rows, int8_t *xq, float *xqs, hipStream_t st);
int l98k_mtp_pre(const int8_t *emb_q, const float *emb_s, int gs, const int *toks, const float *h, int d,
                 const float *w_e, const float *w_h, float eps, int rows, int8_t *xq, float *xqs,
                 hipStream_t st);
// One KDA layer step for a chunk: conv, gate up-projection, recurrence,
// gated norm and o_proj quantization (kd in {32, 64, 128}, conv taps K in 2..4).
int l98k_kda_step(const KdaStepArgs *a, int kd, int K, hipStream_t st);
// The KDA step of several sessions' rows in one launch (items in device
// memory; state_off / conv_off: the layer's offsets inside each ring slot).
int l98k_kda_items(const KdaStepArgs *a, const KdaItem *items, int n_items, int max_n, size_t state_off,
                   size_t conv_off, int kd, int K, hipStream_t st);
// One session's prefill of n > MAX_CHUNK rows (no ring advance) as three
// launches: the state-free work of every row and head at once, the
// recurrence (one block per head), the gated norm and quantization of every
// row and head at once.  a->rec and a->orow: scratch of n * nv * (5*kd + 4)
// and n * value floats; a->state / conv_ring / ctl_slot as for one session.
int l98k_kda_split(const KdaStepArgs *a, int n, int kd, int K, hipStream_t st);
int l98k_attn_prep(const AttnArgs *a, int nt, hipStream_t st);
// DSpark slot attention (mtp_attn_t1): rows slot rows of qg [rows][qg_dim]
// and vp [rows][kv_dim]; the last row's V quantization also goes to the MTP
// plane's row 0 (vc0, vs0); output float rows (out) or quantized (oq, oqs).
int l98k_attn_t1(const float *qg, int qg_dim, const float *vp, int kv_dim, int nh, int nkv, int hd, int q_dim,
                 int rows, int8_t *vc0, float *vs0, float *out, int8_t *oq, float *oqs, hipStream_t st);
// Attention of several sessions' rows in one launch per kernel (items in
// device memory); att: n_items blocks of att_item floats.  kv_cached: every
// row's K and V are already in the cache (a prefill after its K/V launch).
int l98k_attn_prep_items(const AttnArgs *a, const AttnItem *items, int n_items, int plane, hipStream_t st);
int l98k_attn_items(const AttnArgs *a, const AttnItem *items, int n_items, int plane, int max_len, int nmax,
                    float *att, size_t att_item, int kv_cached, hipStream_t st);
// Attention of nt tokens (positions *ctl_pos + pos_off + t) against the KV
// plane: scores with the q/k preparation and the chunk's own K/V cache rows,
// then softmax, value sum, output gate and quantization into oq / oqs.
// att: scratch [MAX_CHUNK][nh][round4(max_len)] floats.
int l98k_attn(const AttnArgs *a, int nt, int max_len, float *att, hipStream_t st);
// l98k_attn's chunk path: 0 by capacity, 1 one launch, 2 two launches.
void l98k_set_attn_path(int mode);
// Routing of nt tokens (computed in every block) and the routed experts'
// first projections (n_jobs <= 2, e.g. w1 and w3 over the latent rows);
// publishes sel_idx / sel_w / grp (and adds the distinct-expert count to
// *tally) for the down projection and the combine.
// routing only (the tables k_moe_up computes in each block), for checks
int l98k_moe_route(const float *logits, const float *bias, int E, int topk, int nt, int *sel_idx, float *sel_w,
                   hipStream_t st);
int l98k_moe_up(const ExpertJob *jobs, int n_jobs, const float *logits, const float *bias, int E, int topk, int nt,
                int *sel_idx, float *sel_w, MoeGroups *grp, int *tally, int in_dim, int out_rows, hipStream_t st);
// Routing of `rows` token rows (8-row groups through the in-block router);
// with lx, the rows' latent lx[rows][lat] quantized per 32 into lq / lqs in
// the same launch.
int l98k_moe_route_wide(const float *logits, const float *bias, int E, int topk, int rows, int *sel_idx, float *sel_w,
                        const float *lx, int lat, int8_t *lq, float *lqs, hipStream_t st);
// The pairs of a wide routing grouped by expert (tables of the grouped GEMM).
int l98k_moe_group(const int *sel_idx, int npairs, int topk, int E, int *ng, int *gexp, int *goff, int *gcnt,
                   int *list, int *pair_token, hipStream_t st);
int l98k_row_sums(const float *x, int rows, int n, float *out, hipStream_t st);
// Block-diagonal Walsh-Hadamard transforms, one block per row of n <= 8192
// (blk a power of two dividing n): lz_fwht_i32 / lz_fwht on each block,
// rot = 1 adds subn_rot_f32's rsqrt(blk) factor; l98k_subn_quant is
// subn_fwht_quant (n % 32 == 0; q: rows x n, s: rows x n / 32).
int l98k_fwht_i32(const int32_t *x, int32_t *y, int rows, int n, int blk, hipStream_t st);
int l98k_fwht_f32(float *v, int rows, int n, int blk, int rot, hipStream_t st);
int l98k_subn_quant(const float *x, int rows, int n, int blk, int gw, int8_t *q, float *s, hipStream_t st);
// Per row argmax of rows x n floats, one block per row (mode 0:
// sample_argmax's key order, 1: lz_argmax_p1's compare).
int l98k_argmax(const float *x, int n, int rows, int mode, int *out, hipStream_t st);
// The same from a GEMV's argmax-epilogue candidates (GemvBatch.amax_part,
// tiles per row; x: the GEMV's output rows of n, read for mode 1's rule).
int l98k_argmax_part(const unsigned long long *part, int tiles, const float *x, int n, int rows, int mode, int *out,
                     hipStream_t st);
// flags: 1 debug_break_rollback, 2 a DSpark round (no catch-up, mtp_pos kept)
int l98k_accept(DevCtl *ctl, const float *vhidden, int d, float *chain, int depth, int flags, hipStream_t st);
int l98k_set_tokens(DevCtl *ctl, int op, RoundRec *hist, int hist_cap, hipStream_t st);
int l98k_put_ctl(const DevCtl *src, DevCtl *const *dst, int n, hipStream_t st);
// Two quantizing producers in one launch (a: mode 0 or 1, b: any mode).
int l98k_wide_pro2(int mode_a, const float *src_a, const float *src2_a, int stride_a, int n_a, int rows_a,
                   int8_t *xq_a, float *xqs_a, int mode_b, const float *src_b, const float *src2_b, int stride_b,
                   const int *sel_idx_b, const float *sel_w_b, int topk_b, int n_b, int rows_b, int8_t *xq_b,
                   float *xqs_b, hipStream_t st);
// Item i's per floats (per % 4 == 0) from src + i * per to dst[i] (device
// table), one launch.
int l98k_scatter_rows(const float *src, size_t per, float *const *dst, int n, hipStream_t st);
// Session-batch round control (op 0 draft rows in, 1 draft argmaxes and
// chains out, 2 verify rows in, 3 acceptance, 4 catch-up rows in, 5 round
// record and advance), block r for session r.
int l98k_batch_round(int op, const BatchSess *bs, int n, int j, int K1, int nc, int d, const int *am,
                     const float *rows, int *toks, float *h, hipStream_t st);
// Launch-floor probes: `launches` dependent launches of an empty kernel
// (kind 0) or of a kernel whose `grid` blocks each read the n floats the
// previous launch wrote (kind 1, buffers a and b alternating; 256 <= n <=
// 8192), or kind 1 plus a last-block reduction per 8 blocks (kind 2: b is
// followed by grid x 256 floats of partials and grid counters).
int l98k_launch_chain(int kind, int launches, int grid, float *a, float *b, int n, hipStream_t st);
// Streaming probe: `blocks` blocks of `threads` threads, each streaming its
// own `chunks` 16-byte chunks of w.
int l98k_stream(const void *w, int blocks, int threads, int chunks, int *out, hipStream_t st);
}

#endif

// Device-side argument blocks shared by the kernels and the host engine.
#ifndef L98_DEV_H
#define L98_DEV_H
#include <stddef.h>
#include <stdint.h>

#define MAX_GEMV_JOBS 8
#define MAX_EXPERTS 128
#define MAX_TOPK 8
#define MAX_CHUNK 8          // tokens per forward chunk (the reference's LZ_BATCH_MAX)
#define MAX_PAIRS (MAX_CHUNK * MAX_TOPK)
#define KDA_MAX_RANK 128     // gate low-rank width handled by the KDA step kernel

// How a GEMV tile builds its int8 activation rows (in LDS, per block).
enum {
    PRO_XQ = 0,        // rows already quantized: xq / xqs
    PRO_QUANT = 1,     // quantize float rows src
    PRO_NORM = 2,      // x = src (+ a (+ b)); RMSNorm(1+w); quantize
    PRO_SILU = 3,      // silu(src) * src2; quantize
    PRO_COMBINE = 4,   // sum over slots of sel_w * src[pair]; quantize
    PRO_FOLD = 5       // x = src (+ a (+ b)); quantize (PRO_NORM without the norm)
};

// Prologue of one GEMV job.  Rows are addressed by the tile's activation
// row index xr (the token, or for grouped experts the token or the pair).
typedef struct {
    int mode;
    int src_stride;          // floats between rows of src / src2 / x_out
    const float *src;        // QUANT, NORM, SILU: rows; COMBINE: per-pair rows [pairs][in_dim]
    const float *src2;       // SILU: second operand
    const float *a, *b;      // NORM: optional residual addends [rows][in_dim]
    const float *w;          // NORM: weight [in_dim]
    float eps;
    int topk;                // COMBINE
    const int *sel_idx;      // COMBINE: [rows][topk]
    const float *sel_w;      // COMBINE: [rows][topk]
    float *x_out;            // NORM: the updated residual rows (written by one block)
    float *o_out;            // NORM: the normed rows (written by one block)
    int o_stride;
    int pad;
} Prologue;

// One weight matrix of a fused GEMV launch.  Jobs of one launch may differ
// in input width and prologue.
typedef struct {
    const int8_t *w;         // [rows][in_dim] int8, row-major
    const float *ws;         // [rows][in_dim/gs] scales (one per row when gs is 0)
    float *out;              // out[t * out_stride + row]
    const int8_t *xq;        // PRO_XQ activations [M][in_dim]
    const float *xqs;        // PRO_XQ activation scales [M][in_dim/32]
    int32_t *acc_out;        // optional exact group sums [M][rows][in_dim/32] (tests)
    int rows;
    int in_dim;
    int out_stride;
    int tiles;               // tiles of this job: blocks (0..tiles-1, job) of the launch grid (set by the launcher)
    int R;                   // rows per tile (set by the launcher)
    int gs;                  // weight scale group (a multiple of 32 dividing in_dim; 0: the row)
    Prologue pro;
} GemvJob;

// A fused GEMV launch: block (x, y) is tile x of job y, so a block's job is
// known at entry and its fields load with the kernel's first scalar loads.
// amax_part (one job only): the launch also stores, per tile and output
// row t, the packed argmax candidate of the tile's rows (amax_mode 0:
// sample_argmax's key order, 1: lz_argmax_p1's) at amax_part[t * tiles +
// tile] (amax_cap entries; tiles * m needed), for l98k_argmax_part.
typedef struct {
    int n;
    int amax_mode, amax_cap, pad;
    unsigned long long *amax_part;
    GemvJob job[MAX_GEMV_JOBS];
} GemvBatch;

// All experts of one projection (w1, w2 or w3) of a layer, stacked:
// expert e occupies rows [e*out_rows, (e+1)*out_rows).
typedef struct {
    const int8_t *q;
    const float *s;          // expert e: [out_rows][in/gs] from e*out_rows*(in/gs)
    int gs;                  // weight scale group (0: the row)
} ExpertBank;

// One projection of a grouped expert GEMV launch (up to two per launch,
// e.g. w1 and w3 over the same activations).
typedef struct {
    const int8_t *q;         // bank: expert e rows [e*out_rows, (e+1)*out_rows)
    const float *s;
    float *out;              // out[pair * out_rows + row]
    const int8_t *xq;        // PRO_XQ activation rows (by token or by pair)
    const float *xqs;
    int xq_by_pair;          // 1: activation row = pair index, 0: = the pair's token
    int gs;                  // weight scale group (0: the row)
    Prologue pro;            // PRO_XQ, PRO_QUANT or PRO_SILU
} ExpertJob;

// Distinct experts selected by a chunk and their (token, slot) members.
typedef struct {
    int n_groups;
    int expert[MAX_PAIRS];
    int n_members[MAX_PAIRS];
    int member[MAX_PAIRS][MAX_CHUNK];   // pair index t*topk + slot
    int pair_token[MAX_PAIRS];
} MoeGroups;

// Per-round control block in device memory.  The host seeds it; the
// draft/verify/accept kernels read and update it, so a round needs no host
// round trip and can be captured as a graph.
typedef struct {
    int anchor, anchor_pos, mtp_pos, slot_base;
    int k_eff, n_accept, new_pos, ssm_slot;
    int catch_n, catch_pos, mtp_pos_next, pos_scratch;
    int tok[16];             // tok[0] = anchor, tok[1..k] = drafts
    int targ[16];            // verify argmaxes (targ[k_eff] = bonus)
    int out[16];             // accepted tokens of the round
    int catch_tok[16];       // catch-up tokens; rows past catch_n carry a valid stand-in id
    int round;               // rounds completed since the history was cleared
    int expert_tally;        // distinct experts streamed by the MoE layers since the last round record
    int smp_done;            // temperature round: a verify row rejected its draft (later rows do nothing)
    int pad[13];
} DevCtl;

// One finished round as the host reads it back.
typedef struct {
    int n_accept, k_eff, new_pos, ssm_slot;
    int experts;             // distinct (layer, expert) weight sets the round's verify streamed
    int out[8];
} RoundRec;

// One KDA layer's token step (conv, gate up-projection, recurrence, gated
// norm) for a chunk of nt tokens; one block per head.
typedef struct {
    const float *pq, *pk, *pv;          // projections before the conv [nt][key | key | value]
    const float *pfa;                   // gate low-rank projection [nt][rank]
    const int8_t *fb_q;                 // gate up-projection [nv*kd][rank] int8
    const float *fb_s;                  // its scales [nv*kd][rank/fb_gs]
    const float *conv_w;                // [conv_dim][K] taps, channels [q | k | v]
    float *conv_ring;                   // the layer's history inside ring slot 0, [conv_dim][K-1]
    size_t conv_slot_stride;            // floats between ring slots
    const float *bvec;                  // b projection [nt][nv]
    const float *gz;                    // g projection [nt][value]
    const float *a_log, *dt_bias, *o_norm;
    float *state;                       // layer's head block inside slot 0
    size_t slot_stride;                 // floats between ring slots
    const int *ctl_slot;
    float *raw_out;                     // optional recurrence output (tests)
    float *normed_out;                  // optional gated-norm output (tests)
    int8_t *xq;                         // o_proj activations [nt][value]
    float *xqs;
    int nv, key, value, rank, depth, advance, nt;
    float scale, eps;
    float gate_lb;                      // gate lower bound (has_lb): g = lb * sigmoid(exp(A_log) * pre)
    int has_lb;                         // 0: g = -exp(A_log) * softplus(pre)
    int fb_gs;                          // f_b scale group (0: the row)
    int hist_rows;                      // conv history from the rows before row 0, not the ring (split prefill)
    float *rec;                         // split prefill: token records [n][nv][5*kd + 4]
    float *orow;                        // split prefill: recurrence outputs [n][value]
} KdaStepArgs;

typedef struct {
    const float *qg;                    // [nt][qg_dim] interleaved per head [q | gate]
    const float *kp, *vp;               // [nt][kv_dim] projections
    const float *q_norm, *k_norm;
    const float *rope_cs;               // [seq][rot/2][2]
    float *qh;                          // [nt][q_dim] normed + rotated q
    int8_t *kcache, *vcache;            // plane base [seq][kv_dim]
    float *kscale, *vscale;             // plane base [seq][kv_dim/32]
    float *out;                         // optional [nt][q_dim] gated attention output (tests)
    int8_t *oq;                         // [nt][q_dim] its per-32 quantization (o_proj input)
    float *oqs;                         // [nt][q_dim/32]
    const int *ctl_pos;                 // position of token 0 = *ctl_pos + pos_off
    int pos_off;
    int nh, nkv, hd, rot, q_dim, qg_dim, kv_dim, kv_only;
    float eps, attn_scale;
} AttnArgs;

// One session of a batched round (l98k_batch_round): its control block,
// draft chain, round history and KDA ring depth.
typedef struct {
    DevCtl *ctl;
    float *chain;
    RoundRec *hist;
    int hist_cap, depth;
} BatchSess;

// One session's rows of a many-session attention launch (l98k_attn_items).
typedef struct {
    int8_t *kq, *vq;                    // the session's KV planes, plane 0 base [planes][seq][kv_dim]
    float *ks, *vs;                     // their scales [planes][seq][kv_dim/32]
    const int *ctl_pos;                 // position of the item's first row = *ctl_pos + pos_off
    int row0, n, seq_len, pos_off;
} AttnItem;

// One session's rows of a many-session KDA launch (l98k_kda_items).
typedef struct {
    float *state;                       // the session's KDA ring, layer 0 head block of slot 0
    float *conv_ring;                   // its conv history ring, layer 0 of slot 0
    const int *ctl_slot;                // ring slot base
    size_t slot_stride, conv_slot_stride;
    int row0, n, depth, pad;
} KdaItem;

#endif

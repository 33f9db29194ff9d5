/* Seeded random-init KunMoe checkpoints in the reference's model.bin format.
 *
 * The writer follows the reference loader: header words in the order
 * lz_open_bin reads them (reference src/model.c:3993-4200, version 5), then
 * tensors in model_walk order (src/model.c:2240-2625, LAYER_SPECS
 * src/model.c:1496-1665).  Every matrix is LZ_FMT_Q8_0 with one fp32 scale
 * per output row (gs = in_dim); norms, A_log, dt_bias, the depthwise conv
 * filters and the router bias are LZ_FMT_F32.
 *
 * Randomness is splitmix64 per (tensor, row) stream with a Box-Muller normal
 * built from basic IEEE double operations only (no libm), so the same seed
 * gives the same bytes on every x86-64 host and thread count.
 */
#ifndef L98_SYNTH_H
#define L98_SYNTH_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int vocab, hidden, n_layers, seq_len;
    int attn_period;            /* layer i is full attention iff i % period == period-1 */
    int n_heads, n_kv_heads, head_dim;
    int kda_heads, kd, vd;      /* lin_n_k_heads == lin_n_v_heads == kda_heads */
    int conv_kernel, gate_rank;
    int n_experts, topk, latent, moe_inter, shared_w;
    int mtp_inter;
    float w_std;                /* N(0, w_std) for every matrix except the router */
    float router_std;           /* router weight std (0: use w_std) */
    float bias_std;             /* router selection bias std */
    float gate_lb;              /* KDA gate lower bound (kda_gate_lower_bound; 0:
                                   none, the softplus gate) */
    float resid_std;            /* std of the matrices that write the residual stream
                                   (attention / KDA o_proj, routed up_proj, shared
                                   down_proj); 0: use w_std */
    int mtp_echo;               /* 1: MTP fc = [I | N(0, w_std)], MTP o_proj and
                                   down_proj zero, so the head drafts its own input
                                   token */
    int use_subn;               /* 1: SubLN - no pre-layer norms; every projection
                                   normalizes its own input with its own weight */
    int hadamard_o;             /* SubLN block Hadamard of the KDA o_proj input (0 off) */
    int hadamard_down;          /* SubLN block Hadamard of the dense FFN down_proj
                                   input (the MTP head's FFN; 0 off) */
    int bin_version;            /* model.bin version word: 4..9 (0: 5).  4 is the
                                   published shape: the 13-word tail only, so no
                                   MTP head and none of its tensors; 6..9 append
                                   the application table (identity), mtp_n_draft
                                   1, no rotated vocabulary, the scale layout, and
                                   from 7 / 8 / 9 loop_input_mix 0, ced_local 0,
                                   loop_input_mix_from 2 */
    int gs;                     /* Q8_0 group size (a multiple of 32 dividing the
                                   row; 0: one group per row) */
    int scale_layout;           /* Q8_0 scale plane (version >= 6): 0 f32 per
                                   group, 1 binary16 per group, 2 a binary16 base
                                   per row and a u8 per group (base * u / 255) */
    int bf16_small;             /* 1: the F32 tensors (norms, conv taps, A_log,
                                   dt_bias, router bias) stored as BF16 */
    int mtp_n_draft;            /* DSpark draft slots (version >= 6; 0 or 1: the
                                   fc head).  > 1 writes main_proj [d][3d],
                                   depth_embed [n_draft][d], mask_embed [d] and
                                   the two Markov tensors [vocab][0] (a model.bin
                                   carries no Markov rank, so they are empty) in
                                   place of fc; with mtp_echo, main_proj =
                                   [I | I | N(0, w_std)] */
} L98SynthConfig;

/* Named configurations:
 *   0  tiny    d=256, 4 layers (3 KDA + 1 attn), E=16 top-2, V=8192
 *   1  base    d=1024, 24 layers (3:1), 16 KDA heads x64, E=64 top-6, V=65536
 *   2  tiny    same shapes as 0 (k-sweep config uses config 0's model)
 *   3  large   d=2048, 32 layers (3:1), 16 KDA heads x128, E=128 top-8, V=131072
 *   4  server  config 0's shapes, router N(0,1/d), bias N(0,0.5)
 *  10  micro   d=64 toy for fast unit tests
 *  11  echo    micro's shapes with a small vocabulary, an echoing MTP head and
 *              damped residual writers: greedy drafts are accepted at every
 *              depth, so the accepted-draft path of a round runs
 *   5  subln   config 0's shapes with use_subn = 1, hadamard_o = 64,
 *              hadamard_down = 256 (the survey's C1s variant)
 *  12  micro-subln  micro's shapes with use_subn = 1, hadamard_o = 32,
 *              hadamard_down = 64
 *  13  micro's shapes as a version-9 file: Q8_0 groups of 32, binary16
 *              scales, BF16 small tensors
 *  14  tiny's shapes as a version-6 file: Q8_0 groups of 128, scale layout 2
 *              (row base + u8 codes), BF16 small tensors
 *  15  tiny's shapes as a version-4 file (no MTP head): groups of 64
 *  16  micro's shapes as a version-7 file, per-row groups, f32 scales
 *  17  micro's shapes as a version-8 file, groups of 32, scale layout 2
 *  18  micro's shapes with a DSpark head of 4 slots (version 6)
 *  19  echo's shapes with a DSpark head of 6 slots (version 6), echoing
 *  20  tiny's shapes with a DSpark head of 3 slots (version 7), groups of
 *              64, BF16 small tensors
 *  21  micro-subln's shapes with a DSpark head of 3 slots (version 6)
 *  22  base's shapes with a DSpark head of 6 slots (version 6)
 * Returns 0 on success, 1 for an unknown id. */
int l98_synth_config(int id, L98SynthConfig *out);

/* Writes <dir>/model.bin.  seq_len in cfg is what the state allocator sizes
 * for.  Returns 0 on success, nonzero with a message in err otherwise. */
int l98_synth_write(const char *dir, const L98SynthConfig *cfg, uint64_t seed,
                    int n_threads, char *err, int errlen);

/* Deterministic N(0,1) stream used by the writer, exposed for tests. */
double l98_synth_normal(uint64_t *state);

#ifdef __cplusplus
}
#endif
#endif

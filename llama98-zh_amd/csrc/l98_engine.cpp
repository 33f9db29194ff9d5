// Host engine of the MI355X MTP speculative-decoding path: model upload,
// run state, the forward passes (capture / batch capture / verify), the MTP
// draft step and prefill, the greedy and temperature rounds, and the C ABI
// of include/llama98_hip.h.  All arithmetic runs in the kernels of
// l98_kernels.hip; this file only schedules them on one HIP stream.
//
// Reference call structure (paths into the reference tree):
//   forward_chunk          src/forward.c:1210-1617
//   lz_forward_verify      src/forward.c:1774-1808
//   lz_mtp_draft_step      src/forward_mtp.c:32-144
//   lz_mtp_prefill/catchup src/forward_mtp.c:561-642
//   lz_spec_round(_temp)   src/generate.c:694-994, 1234-1377

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <memory>
#include <mutex>
#include <numeric>
#include <vector>

#include "../../include/llama98_hip.h"
#include "l98_dev.h"
#include "mathf.h"

#include "l98_launch.h"

#define CK(x)                                                                   \
    do {                                                                        \
        int _e = (int)(x);                                                      \
        if (_e != 0) {                                                          \
            fprintf(stderr, "l98: %s failed (%d) at %s:%d\n", #x, _e, __FILE__, \
                    __LINE__);                                                  \
            return 1;                                                           \
        }                                                                       \
    } while (0)

static void set_err(char *buf, int len, const char *fmt, ...) {
    if (!buf || len <= 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, (size_t)len, fmt, ap);
    va_end(ap);
}

// ------------------------------------------------------ data symbols ---
// The reference's exported data (llama98.def:117-157; definitions
// src/forward.c:29-448, src/generate.c:226).  The counters are updated by
// the entry points below as the reference's are; the knobs hold the one
// configuration this path implements, and an entry point refuses to run if
// a caller has set another (knobs_ok).

extern "C" {
long long lz_debug_us_draft = 0, lz_debug_us_verify = 0, lz_debug_us_capture = 0, lz_debug_us_catchup = 0;
long long lz_debug_n_capture = 0, lz_debug_n_catchup = 0, lz_debug_n_ring_rollback = 0;
long long lz_debug_n_chunks = 0, lz_debug_n_lmhead = 0, lz_debug_n_kv_rot = 0, lz_debug_attn_skip = 0;
long long lz_debug_mtp_attn_rows = 0;
float lz_debug_mtp_attn_scale = 1.0f;
int lz_debug_mtp_attn_window = 0;
int lz_kv_kfmt = LZ_KVF_Q8, lz_kv_vfmt = LZ_KVF_Q8;
int lz_kv_rot_enable = 0, lz_attn_sink = 0, lz_attn_window = 0;
int lz_moe_topk = 0;
float lz_moe_tau = 1.0f;
int lz_prof_enable = 0;
float lz_prof_us[LZ_PROF_N];
}

static long long us_since(const timespec &t0) {
    timespec t1;
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (long long)(t1.tv_sec - t0.tv_sec) * 1000000LL + (t1.tv_nsec - t0.tv_nsec) / 1000;
}
static timespec now_ts() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t;
}

// 1 when the process-global knobs select what this path computes: Q8 K and
// V caches, no KV rotation, no attention sink or window, the model's own
// routed top-k at temperature 1, and no MTP attention probes.
static int knobs_ok(int model_topk, char *errbuf, int errlen) {
    const char *bad = nullptr;
    if (lz_kv_kfmt != LZ_KVF_Q8 || lz_kv_vfmt != LZ_KVF_Q8) bad = "lz_kv_kfmt / lz_kv_vfmt other than Q8";
    else if (lz_kv_rot_enable) bad = "lz_kv_rot_enable";
    else if (lz_attn_sink || lz_attn_window) bad = "an attention sink or window";
    else if (lz_moe_topk != 0 && lz_moe_topk != model_topk) bad = "lz_moe_topk other than the model's top-k";
    else if (lz_moe_tau != 1.0f) bad = "lz_moe_tau other than 1";
    else if (lz_debug_mtp_attn_scale != 1.0f || lz_debug_mtp_attn_window) bad = "the MTP attention probes";
    if (!bad) return 1;
    if (errbuf && errlen > 0) snprintf(errbuf, (size_t)errlen, "%s: not on this path", bad);
    return 0;
}

// ------------------------------------------------------------- model ---

struct DMat {
    int8_t *q = nullptr;
    float *s = nullptr;       // [rows][cols/gs] scales
    int rows = 0, cols = 0;
    int gs = 0;               // scale group (== cols: one per row)
};

struct DLayer {
    int type = 0;
    float *in_norm = nullptr, *post_norm = nullptr;
    DMat q, k, v, o;
    float *q_norm = nullptr, *k_norm = nullptr;
    DMat kq, kk, kv, fa, fb, kb, kg, ko;
    float *conv = nullptr, *a_log = nullptr, *dt_bias = nullptr, *o_norm = nullptr;
    DMat router, down, up, sg, su, sd;
    float *bias = nullptr;
    ExpertBank w1{}, w2{}, w3{};
    // SubLN per-projection input norms (use_subn): attention q/k/v/o, KDA
    // q/k/v/g/o, MoE router / routed down / routed up / shared gate / up /
    // down; the MTP block's dense FFN gate / up / down
    float *sn_q = nullptr, *sn_k = nullptr, *sn_v = nullptr, *sn_o = nullptr;
    float *kn_q = nullptr, *kn_k = nullptr, *kn_v = nullptr, *kn_g = nullptr, *kn_o = nullptr;
    float *mn_gate = nullptr, *mn_down = nullptr, *mn_up = nullptr, *mn_sg = nullptr, *mn_su = nullptr,
          *mn_sd = nullptr;
    float *fn_gate = nullptr, *fn_up = nullptr, *fn_down = nullptr;
};

struct DModel {
    LZModelConfig c{};
    char *arena = nullptr;
    size_t arena_size = 0, arena_used = 0;
    DMat embed;
    float *final_norm = nullptr;
    std::vector<DLayer> L;
    DLayer mtp;
    DMat mtp_gate, mtp_up, mtp_down, mtp_fc;
    float *mtp_norm = nullptr, *mtp_pre_h = nullptr, *mtp_pre_e = nullptr;
    // a DSpark head (mtp_n_draft > 1) in place of fc: main_proj [d][3d],
    // depth_embed rows [n_draft][d] and mask_embed [d] as f32
    int n_draft = 1;
    DMat mtp_main;
    float *mtp_depth = nullptr, *mtp_mask = nullptr;
    float *rope_cs = nullptr;
    int lin_index[128], full_index[128];
    struct DWide *wide = nullptr;       // scratch of the many-row forwards (first use)
    int version = 5;                    // model.bin version word
    bool has_mtp = true;                // a version-4 file carries no MTP head
    bool grouped = false;               // some matrix has more than one scale per row
};

namespace {

// Sequential reader over the mmapped model.bin.
struct Bin {
    const unsigned char *p = nullptr;
    size_t n = 0, off = 0;
    bool bad = false;
    const void *take(size_t b) {
        if (bad || off + b > n) { bad = true; return nullptr; }
        const void *r = p + off;
        off += b;
        return r;
    }
    int32_t i32() { const void *q = take(4); int32_t v = 0; if (q) memcpy(&v, q, 4); return v; }
    float f32() { const void *q = take(4); float v = 0; if (q) memcpy(&v, q, 4); return v; }
};

// A tensor of the file: codes point into the mapped file; the f32 values
// (Q8 scales, or the data of an F32 tensor) into the file when stored as
// f32, else into `own`, widened at load.
struct HostTensor {
    const int8_t *q = nullptr;
    const float *s = nullptr;     // Q8 scales [rows][cols/gs] or F32 data
    int rows = 0, cols = 0, gs = 0;
    bool is_q8 = false;
    std::shared_ptr<std::vector<float>> own;
};

// lz_f16_to_f32 (src/compat.c:283-312): binary16 widened exactly.
float f16_to_f32(unsigned h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    if (e == 0) {
        if (m == 0) u = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            u = sign | ((uint32_t)(127 - 14 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 0x1Fu) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 127u - 15u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}
// lz_scale_u8_decode (src/compat.c:340-345): base * (u / 255), the quotient
// and the product each rounded to float.
float scale_u8_decode(float base, float u) {
    volatile float levels = 255.0f;
    volatile float q = u / levels;
    volatile float p = base * q;
    return p;
}

// A Q8_0 tensor (visit_read_bin, src/model.c:3567-3812): u32 gs (a multiple
// of 32 dividing the row here), the codes, and the scale plane in the
// file's layout (read_scale_plane, src/model.c:3510-3554): 0 f32 per
// group; 1 binary16 per group; 2 a binary16 base per row, then a u8 per
// group decoded as base * (u / 255).  The device holds f32 scales.
HostTensor rd_q8(Bin &b, int rows, int cols, int layout) {
    HostTensor t;
    const unsigned char *dt = (const unsigned char *)b.take(1);
    uint32_t n = (uint32_t)b.i32(), gs = (uint32_t)b.i32();
    if (!dt || *dt != 1 || n != (uint32_t)rows * (uint32_t)cols || gs == 0 || (gs & 31) || (uint32_t)cols % gs) {
        b.bad = true;
        return t;
    }
    t.q = (const int8_t *)b.take((size_t)rows * cols);
    const size_t ng = (size_t)rows * (cols / gs);
    if (layout == 0) {
        t.s = (const float *)b.take(sizeof(float) * ng);
    } else {
        t.own = std::make_shared<std::vector<float>>(ng);
        if (layout == 1) {
            const uint16_t *h = (const uint16_t *)b.take(2 * ng);
            if (h)
                for (size_t i = 0; i < ng; i++) (*t.own)[i] = f16_to_f32(h[i]);
        } else {
            const uint16_t *base = (const uint16_t *)b.take(2 * (size_t)rows);
            const uint8_t *u = (const uint8_t *)b.take(ng);
            const size_t gpr = ng / (size_t)rows;
            if (base && u)
                for (size_t i = 0; i < ng; i++) (*t.own)[i] = scale_u8_decode(f16_to_f32(base[i / gpr]), (float)u[i]);
        }
        t.s = t.own->data();
    }
    t.rows = rows; t.cols = cols; t.gs = (int)gs; t.is_q8 = true;
    return t;
}

// An F32 tensor of n elements, stored as f32 or as BF16 (dtype 6, widened
// by <<16 as lz_t_f32 does, src/ops_epi.c:1210-1223).
HostTensor rd_f32(Bin &b, int n) {
    HostTensor t;
    const unsigned char *dt = (const unsigned char *)b.take(1);
    uint32_t cnt = (uint32_t)b.i32();
    if (!dt || (*dt != 0 && *dt != 6) || cnt != (uint32_t)n) { b.bad = true; return t; }
    if (*dt == 0) {
        t.s = (const float *)b.take(sizeof(float) * (size_t)n);
    } else {
        const uint16_t *h = (const uint16_t *)b.take(2 * (size_t)n);
        t.own = std::make_shared<std::vector<float>>((size_t)n);
        if (h)
            for (int i = 0; i < n; i++) {
                const uint32_t u = (uint32_t)h[i] << 16;
                memcpy(&(*t.own)[i], &u, 4);
            }
        t.s = t.own->data();
    }
    t.rows = 1; t.cols = n;
    return t;
}

// A table read as lz_t_row_f32 reads its rows (src/ops_epi.c:1260-1290): a
// Q8_0 row is its codes times their group's scale, an F32 / BF16 row its
// values; rows * cols f32 in `own`.
HostTensor rd_rows_f32(Bin &b, int rows, int cols, int layout) {
    HostTensor t;
    if (b.off < b.n && b.p[b.off] == 1) {
        HostTensor q = rd_q8(b, rows, cols, layout);
        if (b.bad) return t;
        t.own = std::make_shared<std::vector<float>>((size_t)rows * cols);
        for (size_t i = 0; i < (size_t)rows * cols; i++) (*t.own)[i] = (float)q.q[i] * q.s[i / (size_t)q.gs];
    } else {
        HostTensor f = rd_f32(b, rows * cols);
        if (b.bad) return t;
        t.own = std::make_shared<std::vector<float>>(f.s, f.s + (size_t)rows * cols);
    }
    t.s = t.own->data();
    t.rows = 1; t.cols = rows * cols;
    return t;
}

void *arena_take(DModel *m, size_t bytes) {
    size_t a = (m->arena_used + 255) & ~(size_t)255;
    if (a + bytes > m->arena_size) return nullptr;
    m->arena_used = a + bytes;
    return m->arena + a;
}

// Uploads go through the arena; on a counting pass (arena == null) they only
// size it.
struct Uploader {
    DModel *m;
    bool count;
    size_t need = 0;
    bool fail = false;
    void *put(const void *src, size_t bytes) {
        if (count) { need = ((need + 255) & ~(size_t)255) + bytes; return nullptr; }
        void *d = arena_take(m, bytes);
        if (!d || !src) { fail = true; return nullptr; }
        if (hipMemcpy(d, src, bytes, hipMemcpyHostToDevice) != hipSuccess) fail = true;
        return d;
    }
    DMat mat(const HostTensor &t) {
        DMat d;
        d.rows = t.rows; d.cols = t.cols; d.gs = t.gs;
        d.q = (int8_t *)put(t.q, (size_t)t.rows * t.cols);
        d.s = (float *)put(t.s, sizeof(float) * (size_t)t.rows * (t.cols / t.gs));
        if (t.gs != t.cols) m->grouped = true;
        return d;
    }
    float *vec(const HostTensor &t) { return (float *)put(t.s, sizeof(float) * (size_t)t.cols); }
    // Stacks per-expert matrices of one projection into a bank.
    ExpertBank bank(const std::vector<HostTensor> &ex) {
        ExpertBank b{};
        size_t rows = ex[0].rows, cols = ex[0].cols, E = ex.size();
        const int gs = ex[0].gs;
        for (const HostTensor &t : ex)
            if (t.gs != gs) fail = true;          // one group size per bank
        const size_t nws = cols / (size_t)(gs > 0 ? gs : (int)cols);
        b.gs = gs == (int)cols ? 0 : gs;
        if (b.gs) m->grouped = true;
        if (count) {
            put(nullptr, E * rows * cols);
            put(nullptr, sizeof(float) * E * rows * nws);
            return b;
        }
        int8_t *q = (int8_t *)arena_take(m, E * rows * cols);
        float *s = (float *)arena_take(m, sizeof(float) * E * rows * nws);
        if (!q || !s) { fail = true; return b; }
        for (size_t e = 0; e < E; e++) {
            if (hipMemcpy(q + e * rows * cols, ex[e].q, rows * cols, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(s + e * rows * nws, ex[e].s, sizeof(float) * rows * nws, hipMemcpyHostToDevice) != hipSuccess)
                fail = true;
        }
        b.q = q; b.s = s;
        return b;
    }
};

struct HostLayer {
    int type = 0;
    HostTensor in_norm, post_norm, q, k, v, o, q_norm, k_norm;
    HostTensor kq, kk, kv, convq, convk, convv, a_log, fa, fb, dt_bias, kb, kg, o_norm, ko;
    HostTensor router, bias, down, up, sg, su, sd;
    std::vector<HostTensor> w1, w2, w3;
    HostTensor sn_q, sn_k, sn_v, sn_o, kn_q, kn_k, kn_v, kn_g, kn_o;
    HostTensor mn_gate, mn_down, mn_up, mn_sg, mn_su, mn_sd, fn_gate, fn_up, fn_down;
    HostTensor ds_main, ds_depth, ds_mask;     // the MTP holder's DSpark tensors
};

// Parses the version-5 model.bin (reference loader order: header
// src/model.c:3993-4200, tensors model_walk src/model.c:2240-2625).
int parse_model(Bin &b, LZModelConfig &c, HostTensor &embed, HostTensor &fnorm,
                std::vector<HostLayer> &L, HostLayer &mtp, HostTensor &mg, HostTensor &mu,
                HostTensor &md, HostTensor &fc, HostTensor &mn, HostTensor &mph, HostTensor &mpe,
                char *err, int errlen, int &ver_out, int &layout_out) {
    const void *magic = b.take(4);
    if (!magic || memcmp(magic, "L98Z", 4) != 0) { set_err(err, errlen, "bad magic"); return LZ_ERR_BIN_MAGIC; }
    const int ver = b.i32();
    ver_out = ver;
    if (ver < 4 || ver > 9) { set_err(err, errlen, "unsupported model.bin version %d", ver); return LZ_ERR_BIN_VERSION; }
    c.vocab_size = b.i32(); c.hidden_size = b.i32(); c.n_layers = b.i32(); c.seq_len = b.i32();
    c.n_heads = b.i32(); c.n_kv_heads = b.i32(); c.head_dim = b.i32();
    const int inter_word = b.i32();                 // intermediate_size (no dense body layer here)
    c.lin_n_k_heads = b.i32(); c.lin_n_v_heads = b.i32(); c.lin_k_head_dim = b.i32();
    c.lin_v_head_dim = b.i32(); c.conv_kernel = b.i32(); c.n_linear_layers = b.i32();
    c.n_full_layers = b.i32(); (void)b.i32(); (void)b.i32(); (void)b.i32();
    c.rms_norm_eps = b.f32(); c.rope_theta = b.f32(); (void)b.f32();
    c.attn_q_dim = b.i32(); c.attn_qgate_dim = b.i32(); c.attn_kv_dim = b.i32();
    c.lin_key_dim = b.i32(); c.lin_value_dim = b.i32(); c.lin_conv_dim = b.i32();
    c.rotary_dim = b.i32();
    for (int i = 0; i < 128; i++) c.layer_types[i] = b.i32();
    c.kda_gate_rank = b.i32();
    c.kda_has_gate_lower_bound = b.i32() != 0; c.kda_gate_lower_bound = b.f32();
    c.num_experts = b.i32(); c.num_experts_per_token = b.i32(); int n_shared = b.i32();
    c.moe_intermediate_size = b.i32(); c.moe_latent_dim = b.i32();
    int first_dense = b.i32(), renorm = b.i32(), sig = b.i32(), lat_norm = b.i32();
    c.moe_shared_width = b.i32();
    // The version ladder of lz_open_bin (src/model.c:3925-3989, 4105-4460):
    // v4 stops after the 13-word tail (no MTP head; the fields after it keep
    // their "off" defaults, the hadamard blocks -1 = derived); v5 carries the
    // rest of the tail and the 522 appended words; v6 the application table,
    // mtp_n_draft, the rotated-vocabulary words and the scale layout; v7, v8,
    // v9 one word each.  This path takes the identity schedule, no rotated
    // vocabulary and none of the v7-v9 mechanisms; mtp_n_draft > 1 (at most
    // LZ_SPEC_K_MAX, alloc_mtp src/model.c:2905-2909) is a DSpark head.
    int rope_type = 0, mla_q = 0, mla_o = 0, kv_share = 0, sink = 0, gr = 0, ced_split = 0, ced_kv = 0;
    bool csa2 = false;
    c.mtp_n_layers = 0;
    c.mtp_n_draft = 1;
    c.mtp_markov_rank = 0;          // config.json only (src/model.c:539); a model.bin has none
    c.hadamard_o = c.hadamard_down = -1;
    if (ver >= 5) {
        c.mtp_n_layers = b.i32(); c.mtp_intermediate_size = b.i32();
        rope_type = b.i32();
        for (int i = 0; i < 4; i++) (void)b.i32();
        c.use_subn = b.i32();
        c.hadamard_o = b.i32();
        c.hadamard_down = b.i32();
        mla_q = b.i32(); mla_o = b.i32(); kv_share = b.i32();
        sink = b.i32(); gr = b.i32(); ced_split = b.i32(); ced_kv = b.i32();
        for (int i = 0; i < 128; i++) csa2 |= b.i32() != 0;      // csa2_on
        for (int i = 0; i < 128 * 2 + 6 + 128; i++) (void)b.i32();
    }
    bool schedule_ok = true, draft_ok = true, rot_ok = true, mix_ok = true;
    layout_out = 0;
    if (ver >= 6) {
        schedule_ok = b.i32() == c.n_layers;                                      // exec_len
        for (int i = 0; i < 128; i++) schedule_ok &= b.i32() == (i < c.n_layers ? i : 0);   // app_layer
        for (int i = 0; i < 128; i++) schedule_ok &= b.i32() == 0;               // app_loop
        c.mtp_n_draft = b.i32();                                                 // mtp_n_draft
        if (c.mtp_n_draft < 1) c.mtp_n_draft = 1;
        draft_ok = c.mtp_n_draft <= LZ_SPEC_K_MAX;
        rot_ok = b.i32() == 0;                                                   // embed_hadamard
        (void)b.i32();                                                           // embed_signs_seed
        layout_out = b.i32();                                                    // scale_layout
        if (ver >= 7) mix_ok &= b.i32() == 0;                                    // loop_input_mix
        if (ver >= 8) mix_ok &= b.i32() == 0;                                    // ced_local
        if (ver >= 9) (void)b.i32();                                             // loop_input_mix_from
    }
    if (b.bad) { set_err(err, errlen, "truncated header"); return LZ_ERR_BIN_OPEN; }
    if (c.mtp_n_draft > 1 && c.mtp_n_layers != 1) draft_ok = false;
    if (!schedule_ok || !draft_ok || !rot_ok || !mix_ok || layout_out < 0 || layout_out > 2 || mla_q || mla_o ||
        kv_share || sink || gr || ced_split || ced_kv || csa2) {
        set_err(err, errlen, "model.bin v%d: a mechanism outside the implemented spec path "
                "(looped schedule, draft slots, rotated vocabulary, input mixing, MLA, KV sharing, sinks, GR, CED "
                "or CSA2)", ver);
        return LZ_ERR_BIN_VERSION;
    }
    // resolve_hadamard (src/model.c:139-182): -1 derives the block from the
    // widths; an explicit block is 0 (off) or a power of two dividing its
    // width (lin_value_dim for hadamard_o, intermediate_size and the MTP
    // width for hadamard_down).
    {
        auto pow2_div = [](int blk, int dim) { return blk == 0 || (blk > 0 && !(blk & (blk - 1)) && dim > 0 && dim % blk == 0); };
        if (c.hadamard_o == -1) {
            int oblk = c.num_experts == 0 ? c.lin_value_dim : 0;
            c.hadamard_o = (oblk >= 2 && !(oblk & (oblk - 1))) ? oblk : 0;
        }
        if (c.hadamard_down == -1) {
            int dblk = 512;
            while (dblk > 1 && inter_word % dblk) dblk >>= 1;
            c.hadamard_down = dblk == 1 ? 0 : dblk;
        }
        if (!pow2_div(c.hadamard_o, c.lin_value_dim) || !pow2_div(c.hadamard_down, inter_word) ||
            (c.use_subn && c.hadamard_down > 1 && c.mtp_intermediate_size % c.hadamard_down)) {
            set_err(err, errlen, "hadamard block does not divide its width");
            return LZ_ERR_BIN_VERSION;
        }
    }
    // The variant this path implements (the synthetic configs): KDA + gated
    // full attention, sigmoid latent MoE with a shared expert, one MTP layer;
    // SubLN (use_subn) on that MoE variant, whose scales are per 32 elements
    // (the default subn scale on a model with experts).
    if (n_shared != 1 || first_dense != 0 || !renorm || !sig || lat_norm ||
        (c.use_subn != 0 && c.use_subn != 1) ||
        (c.use_subn && (c.num_experts < 1 || c.hidden_size > 2048 || c.lin_value_dim > 2048 ||
                        c.attn_q_dim > 2048 || c.mtp_intermediate_size > 2048 || c.moe_shared_width > 2048 ||
                        c.moe_latent_dim > 2048)) ||
        rope_type != 0 || c.mtp_n_layers > 1 || c.mtp_n_layers < 0 || c.num_experts > MAX_EXPERTS ||
        c.num_experts_per_token > MAX_TOPK || c.lin_n_k_heads != c.lin_n_v_heads ||
        c.rotary_dim != c.head_dim || c.hidden_size % 32 || c.n_layers > 128 ||
        (c.mtp_n_draft > 1 && (3 * c.hidden_size > 4096 || c.attn_kv_dim > 2048))) {
        set_err(err, errlen, "model variant outside the implemented spec path");
        return LZ_ERR_BIN_VERSION;
    }
    const int d = c.hidden_size;
    embed = rd_q8(b, c.vocab_size, d, layout_out);
    fnorm = rd_f32(b, d);
    L.resize(c.n_layers);
    for (int l = 0; l < c.n_layers && !b.bad; l++) {
        HostLayer &h = L[l];
        h.type = c.layer_types[l];
        h.in_norm = rd_f32(b, d);
        h.post_norm = rd_f32(b, d);
        if (h.type == 1) {
            h.q = rd_q8(b, c.attn_qgate_dim, d, layout_out);
            h.k = rd_q8(b, c.attn_kv_dim, d, layout_out);
            h.v = rd_q8(b, c.attn_kv_dim, d, layout_out);
            h.o = rd_q8(b, d, c.attn_q_dim, layout_out);
            h.q_norm = rd_f32(b, c.head_dim);
            h.k_norm = rd_f32(b, c.head_dim);
            if (c.use_subn) {
                h.sn_q = rd_f32(b, d); h.sn_k = rd_f32(b, d); h.sn_v = rd_f32(b, d);
                h.sn_o = rd_f32(b, c.attn_q_dim);
            }
        } else if (h.type == 2) {
            int key = c.lin_key_dim, value = c.lin_value_dim, K = c.conv_kernel;
            int nvk = c.lin_n_v_heads * c.lin_k_head_dim;
            h.kq = rd_q8(b, key, d, layout_out);
            h.kk = rd_q8(b, key, d, layout_out);
            h.kv = rd_q8(b, value, d, layout_out);
            h.convq = rd_f32(b, key * K);
            h.convk = rd_f32(b, key * K);
            h.convv = rd_f32(b, value * K);
            h.a_log = rd_f32(b, c.lin_n_v_heads);
            h.fa = rd_q8(b, c.kda_gate_rank, d, layout_out);
            h.fb = rd_q8(b, nvk, c.kda_gate_rank, layout_out);
            h.dt_bias = rd_f32(b, nvk);
            h.kb = rd_q8(b, c.lin_n_v_heads, d, layout_out);
            h.kg = rd_q8(b, value, d, layout_out);
            h.o_norm = rd_f32(b, c.lin_v_head_dim);
            h.ko = rd_q8(b, d, value, layout_out);
            if (c.use_subn) {
                h.kn_q = rd_f32(b, d); h.kn_k = rd_f32(b, d); h.kn_v = rd_f32(b, d); h.kn_g = rd_f32(b, d);
                h.kn_o = rd_f32(b, value);
            }
        } else {
            set_err(err, errlen, "layer %d: unsupported layer type %d", l, h.type);
            return LZ_ERR_BIN_VERSION;
        }
        h.router = rd_q8(b, c.num_experts, d, layout_out);
        h.bias = rd_f32(b, c.num_experts);
        h.down = rd_q8(b, c.moe_latent_dim, d, layout_out);
        h.up = rd_q8(b, d, c.moe_latent_dim, layout_out);
        h.sg = rd_q8(b, c.moe_shared_width, d, layout_out);
        h.su = rd_q8(b, c.moe_shared_width, d, layout_out);
        h.sd = rd_q8(b, d, c.moe_shared_width, layout_out);
        if (c.use_subn) {
            h.mn_gate = rd_f32(b, d); h.mn_down = rd_f32(b, d); h.mn_up = rd_f32(b, c.moe_latent_dim);
            h.mn_sg = rd_f32(b, d); h.mn_su = rd_f32(b, d); h.mn_sd = rd_f32(b, c.moe_shared_width);
        }
        for (int e = 0; e < c.num_experts; e++) {
            h.w1.push_back(rd_q8(b, c.moe_intermediate_size, c.moe_latent_dim, layout_out));
            h.w2.push_back(rd_q8(b, c.moe_latent_dim, c.moe_intermediate_size, layout_out));
            h.w3.push_back(rd_q8(b, c.moe_intermediate_size, c.moe_latent_dim, layout_out));
        }
    }
    mtp.type = 1;
    if (c.mtp_n_layers == 0) {      // no MTP head (a version-4 file)
        if (b.bad || b.off != b.n) { set_err(err, errlen, "model.bin layout mismatch"); return LZ_ERR_BIN_OPEN; }
        return 0;
    }
    mtp.in_norm = rd_f32(b, d);
    mtp.post_norm = rd_f32(b, d);
    if (c.use_subn) { mtp.fn_gate = rd_f32(b, d); mtp.fn_up = rd_f32(b, d); }
    mtp.q = rd_q8(b, c.attn_qgate_dim, d, layout_out);
    mtp.k = rd_q8(b, c.attn_kv_dim, d, layout_out);
    mtp.v = rd_q8(b, c.attn_kv_dim, d, layout_out);
    mtp.o = rd_q8(b, d, c.attn_q_dim, layout_out);
    mtp.q_norm = rd_f32(b, c.head_dim);
    mtp.k_norm = rd_f32(b, c.head_dim);
    if (c.use_subn) {
        mtp.sn_q = rd_f32(b, d); mtp.sn_k = rd_f32(b, d); mtp.sn_v = rd_f32(b, d);
        mtp.sn_o = rd_f32(b, c.attn_q_dim);
    }
    mg = rd_q8(b, c.mtp_intermediate_size, d, layout_out);
    mu = rd_q8(b, c.mtp_intermediate_size, d, layout_out);
    md = rd_q8(b, d, c.mtp_intermediate_size, layout_out);
    if (c.use_subn) mtp.fn_down = rd_f32(b, c.mtp_intermediate_size);
    // MTP_SPECS (src/model.c:2529-2552): fc for one draft slot; a DSpark
    // head's main_proj, depth_embed, mask_embed and the two Markov tensors
    // after the three norms.  A model.bin names no Markov rank, so those
    // are [vocab][0]: empty.
    const bool dspark = c.mtp_n_draft > 1;
    if (!dspark) fc = rd_q8(b, d, 2 * d, layout_out);
    mn = rd_f32(b, d);
    mph = rd_f32(b, d);
    mpe = rd_f32(b, d);
    if (dspark) {
        mtp.ds_main = rd_q8(b, d, 3 * d, layout_out);
        mtp.ds_depth = rd_rows_f32(b, c.mtp_n_draft, d, layout_out);
        mtp.ds_mask = rd_f32(b, d);
        (void)rd_f32(b, 0);                 // markov_embed
        (void)rd_f32(b, 0);                 // markov_proj
    }
    if (b.bad || b.off != b.n) { set_err(err, errlen, "model.bin layout mismatch"); return LZ_ERR_BIN_OPEN; }
    return 0;
}

void upload_all(Uploader &u, DModel *m, const HostTensor &embed, const HostTensor &fnorm,
                const std::vector<HostLayer> &HL, const HostLayer &hm, const HostTensor &mg,
                const HostTensor &mu, const HostTensor &md, const HostTensor &fc,
                const HostTensor &mn, const HostTensor &mph, const HostTensor &mpe) {
    const LZModelConfig &c = m->c;
    m->embed = u.mat(embed);
    m->final_norm = u.vec(fnorm);
    m->L.assign(c.n_layers, DLayer());
    std::vector<float> conv;
    for (int l = 0; l < c.n_layers; l++) {
        const HostLayer &h = HL[l];
        DLayer &D = m->L[l];
        D.type = h.type;
        D.in_norm = u.vec(h.in_norm);
        D.post_norm = u.vec(h.post_norm);
        if (h.type == 1) {
            D.q = u.mat(h.q); D.k = u.mat(h.k); D.v = u.mat(h.v); D.o = u.mat(h.o);
            D.q_norm = u.vec(h.q_norm); D.k_norm = u.vec(h.k_norm);
        } else {
            D.kq = u.mat(h.kq); D.kk = u.mat(h.kk); D.kv = u.mat(h.kv);
            // conv taps of the [q | k | v] channels, one row of K per channel
            conv.clear();
            conv.insert(conv.end(), h.convq.s, h.convq.s + h.convq.cols);
            conv.insert(conv.end(), h.convk.s, h.convk.s + h.convk.cols);
            conv.insert(conv.end(), h.convv.s, h.convv.s + h.convv.cols);
            D.conv = (float *)u.put(conv.data(), sizeof(float) * conv.size());
            D.a_log = u.vec(h.a_log);
            D.fa = u.mat(h.fa); D.fb = u.mat(h.fb);
            D.dt_bias = u.vec(h.dt_bias);
            D.kb = u.mat(h.kb); D.kg = u.mat(h.kg);
            D.o_norm = u.vec(h.o_norm);
            D.ko = u.mat(h.ko);
        }
        D.router = u.mat(h.router);
        D.bias = u.vec(h.bias);
        D.down = u.mat(h.down); D.up = u.mat(h.up);
        D.sg = u.mat(h.sg); D.su = u.mat(h.su); D.sd = u.mat(h.sd);
        D.w1 = u.bank(h.w1); D.w2 = u.bank(h.w2); D.w3 = u.bank(h.w3);
        if (c.use_subn) {
            if (h.type == 1) {
                D.sn_q = u.vec(h.sn_q); D.sn_k = u.vec(h.sn_k); D.sn_v = u.vec(h.sn_v); D.sn_o = u.vec(h.sn_o);
            } else {
                D.kn_q = u.vec(h.kn_q); D.kn_k = u.vec(h.kn_k); D.kn_v = u.vec(h.kn_v); D.kn_g = u.vec(h.kn_g);
                D.kn_o = u.vec(h.kn_o);
            }
            D.mn_gate = u.vec(h.mn_gate); D.mn_down = u.vec(h.mn_down); D.mn_up = u.vec(h.mn_up);
            D.mn_sg = u.vec(h.mn_sg); D.mn_su = u.vec(h.mn_su); D.mn_sd = u.vec(h.mn_sd);
        }
    }
    DLayer &M = m->mtp;
    M.type = 1;
    if (c.mtp_n_layers > 0) {
    M.in_norm = u.vec(hm.in_norm); M.post_norm = u.vec(hm.post_norm);
    M.q = u.mat(hm.q); M.k = u.mat(hm.k); M.v = u.mat(hm.v); M.o = u.mat(hm.o);
    M.q_norm = u.vec(hm.q_norm); M.k_norm = u.vec(hm.k_norm);
    if (c.use_subn) {
        M.sn_q = u.vec(hm.sn_q); M.sn_k = u.vec(hm.sn_k); M.sn_v = u.vec(hm.sn_v); M.sn_o = u.vec(hm.sn_o);
        M.fn_gate = u.vec(hm.fn_gate); M.fn_up = u.vec(hm.fn_up); M.fn_down = u.vec(hm.fn_down);
    }
    m->mtp_gate = u.mat(mg); m->mtp_up = u.mat(mu); m->mtp_down = u.mat(md);
    if (c.mtp_n_draft > 1) {
        m->mtp_main = u.mat(hm.ds_main);
        m->mtp_depth = u.vec(hm.ds_depth);
        m->mtp_mask = u.vec(hm.ds_mask);
    } else {
        m->mtp_fc = u.mat(fc);
    }
    m->mtp_norm = u.vec(mn); m->mtp_pre_h = u.vec(mph); m->mtp_pre_e = u.vec(mpe);
    }
    {
        std::vector<float> cs((size_t)c.seq_len * c.rotary_dim);
        l98_rope_table(cs.data(), c.seq_len, c.rotary_dim, c.rope_theta);
        m->rope_cs = (float *)u.put(cs.data(), sizeof(float) * cs.size());
    }
}

bool g_tables_ready = false;
int ensure_tables() {
    if (g_tables_ready) return 0;
    float tab[32];
    for (int i = 0; i < 32; i++) tab[i] = (float)exp2((double)i / 32.0);   // 2^(i/32), src/ops_quant.c:244
    if (l98k_upload_exp_table(tab) != 0) return 1;
    g_tables_ready = true;
    return 0;
}

}  // namespace

extern "C" int lz_open(LZModel *m, const char *dir, char *errbuf, int errlen) {
    if (!m || !dir) { set_err(errbuf, errlen, "null argument"); return 1; }
    memset(m, 0, sizeof(*m));
    if (errbuf && errlen > 0) errbuf[0] = 0;
    char path[1024];
    snprintf(path, sizeof path, "%s/model.bin", dir);
    int fd = open(path, O_RDONLY);
    if (fd < 0) { set_err(errbuf, errlen, "cannot open %s", path); return 1; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 8) { close(fd); set_err(errbuf, errlen, "empty %s", path); return 1; }
    void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { set_err(errbuf, errlen, "mmap %s failed", path); return 1; }
    Bin b;
    b.p = (const unsigned char *)map;
    b.n = (size_t)st.st_size;
    DModel *dm = new DModel();
    HostTensor embed, fnorm, mg, mu, md, fc, mn, mph, mpe;
    std::vector<HostLayer> HL;
    HostLayer hm;
    int ver = 5, layout = 0;
    int rc = parse_model(b, dm->c, embed, fnorm, HL, hm, mg, mu, md, fc, mn, mph, mpe, errbuf, errlen, ver, layout);
    dm->version = ver;
    dm->has_mtp = dm->c.mtp_n_layers > 0;
    dm->n_draft = dm->c.mtp_n_draft;
    if (rc == 0 && ensure_tables() != 0) { set_err(errbuf, errlen, "HIP device not usable"); rc = 1; }
    if (rc == 0) {
        Uploader cnt{dm, true};
        upload_all(cnt, dm, embed, fnorm, HL, hm, mg, mu, md, fc, mn, mph, mpe);
        dm->arena_size = cnt.need + 4096;
        if (hipMalloc((void **)&dm->arena, dm->arena_size) != hipSuccess) {
            set_err(errbuf, errlen, "hipMalloc of %zu weight bytes failed", dm->arena_size);
            rc = 1;
        } else {
            Uploader up{dm, false};
            upload_all(up, dm, embed, fnorm, HL, hm, mg, mu, md, fc, mn, mph, mpe);
            if (up.fail) { set_err(errbuf, errlen, "weight upload failed"); rc = 1; }
        }
    }
    munmap(map, (size_t)st.st_size);
    if (rc != 0) {
        if (dm->arena) (void)hipFree(dm->arena);
        delete dm;
        return 1;
    }
    int li = 0, fi = 0;
    for (int l = 0; l < dm->c.n_layers; l++) {
        if (dm->c.layer_types[l] == 1) { dm->full_index[l] = fi++; dm->lin_index[l] = -1; }
        else { dm->lin_index[l] = li++; dm->full_index[l] = -1; }
    }
    m->config = dm->c;
    m->bytes_device = (long long)dm->arena_used;
    m->impl = dm;
    return 0;
}

namespace {
void wide_free(DModel *m);
}

extern "C" void lz_free(LZModel *m) {
    if (!m || !m->impl) return;
    DModel *dm = (DModel *)m->impl;
    (void)hipDeviceSynchronize();
    wide_free(dm);
    if (dm->arena) (void)hipFree(dm->arena);
    delete dm;
    m->impl = nullptr;
}

// lz_read_weights (src/model.c:4887-4901): a model.bin is read whole by
// lz_open (src/model.c:3264-3266), so this only reports whether it is open.
extern "C" int lz_read_weights(LZModel *m, char *errbuf, int errlen) {
    if (!m || !m->impl) { set_err(errbuf, errlen, "model not open"); return 1; }
    return 0;
}

// lz_load_config (src/model.h:1327): the configuration of a model without
// loading it.  This path reads model.bin only, so `path` names a model.bin
// or a directory holding one; its header fills *c after the same checks
// lz_open makes.
extern "C" int lz_load_config(LZModelConfig *c, const char *path, char *errbuf, int errlen) {
    if (!c || !path) { set_err(errbuf, errlen, "null argument"); return 1; }
    if (errbuf && errlen > 0) errbuf[0] = 0;
    char file[1024];
    struct stat st;
    if (stat(path, &st) == 0 && S_ISDIR(st.st_mode)) snprintf(file, sizeof file, "%s/model.bin", path);
    else snprintf(file, sizeof file, "%s", path);
    int fd = open(file, O_RDONLY);
    if (fd < 0) { set_err(errbuf, errlen, "cannot open %s", file); return 1; }
    if (fstat(fd, &st) != 0 || st.st_size < 8) { close(fd); set_err(errbuf, errlen, "empty %s", file); return 1; }
    void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) { set_err(errbuf, errlen, "mmap %s failed", file); return 1; }
    Bin b;
    b.p = (const unsigned char *)map;
    b.n = (size_t)st.st_size;
    LZModelConfig cfg{};
    HostTensor embed, fnorm, mg, mu, md, fc, mn, mph, mpe;
    std::vector<HostLayer> HL;
    HostLayer hm;
    int ver = 5, layout = 0;
    int rc = parse_model(b, cfg, embed, fnorm, HL, hm, mg, mu, md, fc, mn, mph, mpe, errbuf, errlen, ver, layout);
    munmap(map, (size_t)st.st_size);
    if (rc != 0) return 1;
    *c = cfg;
    return 0;
}

// ------------------------------------------------------------- state ---

struct DState {
    const DModel *m = nullptr;
    hipStream_t st = nullptr;
    int seq_len = 0, depth = 1, planes = 0;
    size_t kda_slot = 0, conv_slot = 0;     // floats per ring slot
    char *arena = nullptr;
    size_t arena_size = 0, arena_used = 0;
    float *kda = nullptr, *conv = nullptr;
    int8_t *kq = nullptr, *vq = nullptr;
    float *ks = nullptr, *vs = nullptr;
    // activations
    float *x, *x2, *mtp_x, *mtp_x2, *chain, *blk, *up_out, *sd_out;
    float *qg, *kp, *vp, *qh, *att;
    float *pq, *pk, *pv, *pfa, *pb, *pg;
    float *rl, *latx, *sgo, *suo, *h1, *h3, *h2, *hb, *hb2, *ffn_out;
    float *vhidden, *mtp_logits, *logits, *draft_logits, *hcap;
    int8_t *xq, *xq2, *xq3, *xq4;
    float *xqs, *xqs2, *xqs3, *xqs4;
    float *sub_a = nullptr, *sub_b = nullptr;   // SubLN float rows before their norm / transform
    int *sel_idx;
    float *sel_w;
    MoeGroups *grp;
    DevCtl *ctl;
    int *tokbuf;
    // the lm_head GEMV's argmax epilogue: per-tile candidates;
    // amax_tok / amax_mode: the next lm_head's argmax target (taken and
    // cleared by lm_head_gemv)
    unsigned long long *amax_part = nullptr;
    int amax_cap = 0;
    int *amax_tok = nullptr;
    int amax_mode = 0;
    DevCtl *ctl_pinned = nullptr;
    int cap_rows = 0;                       // rows of hcap / tokbuf
    RoundRec *hist = nullptr;               // device round records
    int hist_cap = 0;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    hipEvent_t ph[4] = {};                  // phase marks of a host-driven round (draft / verify / catch-up)
    hipGraphExec_t round_graph[L98_SPEC_K_GPU + 1] = {};
    hipGraphExec_t temp_graph[L98_SPEC_K_GPU + 1] = {};   // device temperature rounds, per k
    float temp_graph_t[L98_SPEC_K_GPU + 1] = {}, temp_graph_p[L98_SPEC_K_GPU + 1] = {};   // their T and top-p
    LZSampler session_samp{};               // the sampler of the current session (l98_session_start)
    bool session_greedy = true;
    // temperature sampling scratch (allocated on first use)
    char *smp_arena = nullptr;
    float *smp_q = nullptr;                 // [L98_SPEC_K_GPU][V] draft distributions of a round
    float *smp_p = nullptr, *smp_probs = nullptr;
    uint32_t *smp_keys = nullptr, *smp_skeys = nullptr;
    int *smp_svals = nullptr;
    void *smp_tmp = nullptr;
    size_t smp_tmp_bytes = 0;
    unsigned long long *smp_rng = nullptr;
    int *smp_out = nullptr;                 // [16] small results
    float *smp_outf = nullptr;              // [16]
};

namespace {

void *st_take(DState *s, size_t bytes) {
    size_t a = (s->arena_used + 255) & ~(size_t)255;
    if (s->arena && a + bytes > s->arena_size) return nullptr;
    s->arena_used = a + bytes;
    return s->arena ? s->arena + a : nullptr;
}

// Two passes: size, then carve.
bool carve(DState *s) {
    const LZModelConfig &c = s->m->c;
    const int d = c.hidden_size, B = MAX_CHUNK;
    int wide = d;
    int dims[] = {2 * d, c.attn_qgate_dim, c.lin_conv_dim, c.moe_shared_width, c.mtp_intermediate_size,
                  c.lin_n_v_heads * c.lin_k_head_dim, c.moe_intermediate_size, c.lin_value_dim,
                  c.attn_q_dim, c.moe_latent_dim, c.mtp_n_draft > 1 ? 3 * d : 0};
    for (int v : dims) wide = v > wide ? v : wide;
    const int pairs = B * c.num_experts_per_token;
    auto F = [&](size_t n) { return (float *)st_take(s, n * sizeof(float)); };
    auto I8 = [&](size_t n) { return (int8_t *)st_take(s, n); };
    s->kda = F(s->kda_slot * s->depth);
    s->conv = F(s->conv_slot * s->depth);
    size_t kv = (size_t)s->planes * s->seq_len * c.attn_kv_dim;
    s->kq = I8(kv); s->vq = I8(kv);
    s->ks = F(kv / 32); s->vs = F(kv / 32);
    s->x = F((size_t)B * d); s->x2 = F((size_t)B * d);
    s->mtp_x = F((size_t)B * d); s->mtp_x2 = F((size_t)B * d); s->chain = F(d); s->blk = F((size_t)B * d);
    s->up_out = F((size_t)B * d); s->sd_out = F((size_t)B * d);
    s->qg = F((size_t)B * c.attn_qgate_dim); s->kp = F((size_t)B * c.attn_kv_dim);
    s->vp = F((size_t)B * c.attn_kv_dim); s->qh = F((size_t)B * c.attn_q_dim);
    s->att = F((size_t)B * c.n_heads * (size_t)((s->seq_len + 3) & ~3));
    s->pq = F((size_t)B * c.lin_key_dim); s->pk = F((size_t)B * c.lin_key_dim);
    s->pv = F((size_t)B * c.lin_value_dim); s->pfa = F((size_t)B * c.kda_gate_rank);
    s->pb = F((size_t)B * c.lin_n_v_heads); s->pg = F((size_t)B * c.lin_value_dim);
    s->rl = F((size_t)B * c.num_experts); s->latx = F((size_t)B * c.moe_latent_dim);
    s->sgo = F((size_t)B * c.moe_shared_width); s->suo = F((size_t)B * c.moe_shared_width);
    s->h1 = F((size_t)pairs * c.moe_intermediate_size); s->h3 = F((size_t)pairs * c.moe_intermediate_size);
    s->h2 = F((size_t)pairs * c.moe_latent_dim);
    s->hb = F((size_t)B * c.mtp_intermediate_size); s->hb2 = F((size_t)B * c.mtp_intermediate_size);
    s->ffn_out = F((size_t)B * d);
    s->vhidden = F((size_t)(L98_SPEC_K_GPU + 1) * d);
    s->mtp_logits = F((size_t)(L98_SPEC_K_GPU + 1) * c.vocab_size);
    s->logits = F(c.vocab_size);
    s->draft_logits = F((size_t)L98_SPEC_K_GPU * c.vocab_size);
    s->hcap = F((size_t)s->cap_rows * d);
    s->xq = I8((size_t)pairs * wide); s->xqs = F((size_t)pairs * wide / 32);
    s->xq2 = I8((size_t)pairs * wide); s->xqs2 = F((size_t)pairs * wide / 32);
    s->xq3 = I8((size_t)pairs * wide); s->xqs3 = F((size_t)pairs * wide / 32);
    s->xq4 = I8((size_t)B * wide); s->xqs4 = F((size_t)B * wide / 32);
    if (c.use_subn) { s->sub_a = F((size_t)B * wide); s->sub_b = F((size_t)B * wide); }
    s->sel_idx = (int *)st_take(s, sizeof(int) * pairs);
    s->sel_w = F(pairs);
    s->grp = (MoeGroups *)st_take(s, sizeof(MoeGroups));
    s->ctl = (DevCtl *)st_take(s, sizeof(DevCtl));
    s->tokbuf = (int *)st_take(s, sizeof(int) * (size_t)s->cap_rows);
    s->amax_cap = 0;
    for (int m = 1; m <= MAX_CHUNK; m++) {
        const int need = l98k_gemv_tiles(c.vocab_size, d, m) * m;
        s->amax_cap = need > s->amax_cap ? need : s->amax_cap;
    }
    s->amax_part = (unsigned long long *)st_take(s, sizeof(unsigned long long) * (size_t)s->amax_cap);
    s->hist_cap = s->seq_len;
    s->hist = (RoundRec *)st_take(s, sizeof(RoundRec) * (size_t)s->hist_cap);
    return true;
}

DState *S(LZRunState *s) { return (DState *)s->impl; }
const DModel *Mo(const LZModel *m) { return (const DModel *)m->impl; }

// A fused GEMV launch.  Jobs with pre-quantized input and no activations
// of their own read the state's xq / xqs.
int gemv(DState *s, std::initializer_list<GemvJob> jobs, int mtok) {
    GemvBatch b{};
    b.n = 0;
    for (const GemvJob &j : jobs) {
        GemvJob &o = b.job[b.n++];
        o = j;
        if (o.pro.mode == PRO_XQ && !o.xq) { o.xq = s->xq; o.xqs = s->xqs; }
    }
    return l98k_gemv(&b, mtok, s->st);
}

// Clears the pending argmax target when the function that set it returns,
// so an error path between setting it and the lm_head leaves nothing behind
// for an unrelated later lm_head GEMV.
struct AmaxScope {
    DState *s;
    AmaxScope(DState *st, int *tok, int mode) : s(st) { s->amax_tok = tok; s->amax_mode = mode; }
    ~AmaxScope() { s->amax_tok = nullptr; }
    AmaxScope(const AmaxScope &) = delete;
    AmaxScope &operator=(const AmaxScope &) = delete;
};

// The tied lm_head GEMV of job j over mtok rows.  When s->amax_tok is set
// (then cleared), the rows' argmaxes (mode s->amax_mode) go there: the GEMV
// keeps each tile's candidates and l98k_argmax_part reduces those, so the
// argmax reads 8 bytes per tile and row instead of the logits.
int lm_head_gemv(DState *s, const GemvJob &j, int mtok) {
    GemvBatch b{};
    b.n = 1;
    b.job[0] = j;
    int *tok = s->amax_tok;
    s->amax_tok = nullptr;
    if (tok) {
        b.amax_mode = s->amax_mode;
        b.amax_part = s->amax_part;
        b.amax_cap = s->amax_cap;
    }
    CK(l98k_gemv(&b, mtok, s->st));
    if (tok)
        CK(l98k_argmax_part(s->amax_part, b.job[0].tiles, j.out, j.out_stride, mtok, s->amax_mode, tok, s->st));
    return 0;
}

// GEMV job prologues (how a tile builds its int8 activation rows).
Prologue PX() {
    Prologue p{};
    p.mode = PRO_XQ;
    return p;
}
Prologue PQ(const float *src, int stride) {
    Prologue p{};
    p.mode = PRO_QUANT; p.src = src; p.src_stride = stride;
    return p;
}
Prologue PS(const float *src, const float *src2, int stride) {
    Prologue p{};
    p.mode = PRO_SILU; p.src = src; p.src2 = src2; p.src_stride = stride;
    return p;
}
// RMSNorm(1+w) of x (+ a (+ b)); x_out receives the folded residual and
// o_out the normed rows (both optional, written once per launch).
Prologue PN(const float *x, int stride, const float *a, const float *b, const float *w, float eps, float *x_out,
            float *o_out, int o_stride) {
    Prologue p{};
    p.mode = PRO_NORM; p.src = x; p.src_stride = stride; p.a = a; p.b = b; p.w = w; p.eps = eps;
    p.x_out = x_out; p.o_out = o_out; p.o_stride = o_stride;
    return p;
}
Prologue PC(const float *h2, const int *sel_idx, const float *sel_w, int topk) {
    Prologue p{};
    p.mode = PRO_COMBINE; p.src = h2; p.sel_idx = sel_idx; p.sel_w = sel_w; p.topk = topk;
    return p;
}

// A norm prologue with the projection's own weight: under SubLN every
// projection normalizes the raw residual itself (w == nullptr quantizes the
// folded rows without a norm: the KDA f_a / b inputs).
Prologue PW(const Prologue &in, const float *w) {
    Prologue p = in;
    p.w = w;
    if (!w) p.mode = PRO_FOLD;
    return p;
}

// One GEMV job: w (rows x cols) whose activations the prologue builds.
GemvJob J(const DMat &w, float *out, int out_stride, const Prologue &pro) {
    GemvJob j{};
    j.w = w.q; j.ws = w.s; j.out = out; j.rows = w.rows; j.in_dim = w.cols; j.out_stride = out_stride;
    j.gs = w.gs == w.cols ? 0 : w.gs;
    j.pro = pro;
    return j;
}
// The same over pre-quantized activations.
GemvJob JX(const DMat &w, float *out, int out_stride, const int8_t *xq, const float *xqs) {
    GemvJob j = J(w, out, out_stride, PX());
    j.xq = xq; j.xqs = xqs;
    return j;
}

ExpertJob EJ(const ExpertBank &bank, float *out, int by_pair, const Prologue &pro) {
    ExpertJob j{};
    j.q = bank.q; j.s = bank.s; j.out = out; j.xq_by_pair = by_pair; j.pro = pro; j.gs = bank.gs;
    return j;
}

// Writes host values into the device control block (pageable source: the
// copy is staged at call time, so the host struct may change right after).
int ctl_put(DState *s, const DevCtl &h) {
    CK(hipMemcpyAsync(s->ctl, &h, sizeof(DevCtl), hipMemcpyHostToDevice, s->st));
    return 0;
}
// The host-API entry points that read mtp_chain take the caller's copy:
// as in the reference, the struct field is the state a caller may set.
int chain_put(DState *d, const LZRunState *s) {
    CK(hipMemcpyAsync(d->chain, s->mtp_chain, sizeof(float) * d->m->c.hidden_size, hipMemcpyHostToDevice, d->st));
    return 0;
}
int ctl_get(DState *s, DevCtl *h) {
    CK(hipMemcpyAsync(s->ctl_pinned, s->ctl, sizeof(DevCtl), hipMemcpyDeviceToHost, s->st));
    CK(hipStreamSynchronize(s->st));
    *h = *s->ctl_pinned;
    return 0;
}

// ---------------------------------------------------------- layers ---

// Attention block: the projections' input rows come from `in` (rows nt);
// output xb2 -> s->blk.
int attn_block(DState *s, const DLayer &L, const Prologue &in, int plane, const int *ctl_pos, int pos_off, int nt,
               int max_pos, bool kv_only) {
    const LZModelConfig &c = s->m->c;
    const int d = c.hidden_size;
    const bool sub = c.use_subn != 0;      // q/k/v/o own norms (src/forward_attn.c:787-822, 1015-1024)
    const Prologue pk = sub ? PW(in, L.sn_k) : in, pv = sub ? PW(in, L.sn_v) : in, pq = sub ? PW(in, L.sn_q) : in;
    if (kv_only)
        CK(gemv(s, {J(L.k, s->kp, c.attn_kv_dim, pk), J(L.v, s->vp, c.attn_kv_dim, pv)}, nt));
    else
        CK(gemv(s, {J(L.k, s->kp, c.attn_kv_dim, pk), J(L.v, s->vp, c.attn_kv_dim, pv),
                    J(L.q, s->qg, c.attn_qgate_dim, pq)}, nt));
    AttnArgs a{};
    a.qg = s->qg; a.kp = s->kp; a.vp = s->vp;
    a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.rope_cs = s->m->rope_cs;
    a.qh = s->qh;
    size_t off = (size_t)plane * s->seq_len * c.attn_kv_dim;
    a.kcache = s->kq + off; a.vcache = s->vq + off;
    a.kscale = s->ks + off / 32; a.vscale = s->vs + off / 32;
    a.out = sub ? s->sub_a : nullptr;
    a.oq = s->xq2; a.oqs = s->xqs2;
    a.ctl_pos = ctl_pos; a.pos_off = pos_off;
    a.nh = c.n_heads; a.nkv = c.n_kv_heads; a.hd = c.head_dim; a.rot = c.rotary_dim;
    a.q_dim = c.attn_q_dim; a.qg_dim = c.attn_qgate_dim; a.kv_dim = c.attn_kv_dim;
    a.kv_only = kv_only ? 1 : 0;
    a.eps = c.rms_norm_eps;
    // attn_scale = lz_rsqrt(head_dim) (src/forward_state.c:1408), float body
    {
        float x = (float)c.head_dim, h = 0.5f * x, y;
        uint32_t u;
        memcpy(&u, &x, 4);
        u = 0x5f375a86u - (u >> 1);
        memcpy(&y, &u, 4);
        y = y * (1.5f - h * y * y);
        y = y * (1.5f - h * y * y);
        a.attn_scale = y;
    }
    if (kv_only) {
        CK(l98k_attn_prep(&a, nt, s->st));
        return 0;
    }
    CK(l98k_attn(&a, nt, max_pos + 1, s->att, s->st));
    if (sub)
        CK(l98k_rmsnorm_ex(s->sub_a, c.attn_q_dim, nullptr, nullptr, L.sn_o, c.attn_q_dim, c.rms_norm_eps, nt,
                           nullptr, 0, s->xq2, s->xqs2, 0, s->st));
    CK(gemv(s, {JX(L.o, s->blk, d, s->xq2, s->xqs2)}, nt));
    return 0;
}

float ssm_scale(int kd) {   // lz_rsqrt(lin_k_head_dim), src/forward_state.c:1409
    float x = (float)kd, h = 0.5f * x, y;
    uint32_t u;
    memcpy(&u, &x, 4);
    u = 0x5f375a86u - (u >> 1);
    memcpy(&y, &u, 4);
    y = y * (1.5f - h * y * y);
    y = y * (1.5f - h * y * y);
    return y;
}

// KDA block: the projections' input rows come from `in`; output -> s->blk.
int kda_block(DState *s, const DLayer &L, const Prologue &in, int li, int nt, int advance) {
    const LZModelConfig &c = s->m->c;
    const int d = c.hidden_size, key = c.lin_key_dim, value = c.lin_value_dim;
    const int nv = c.lin_n_v_heads, kd = c.lin_k_head_dim, vd = c.lin_v_head_dim;
    // SubLN: q/k/v/g normalize the raw residual with their own weights, f_a
    // and b quantize it without a norm (src/forward_kda.c:559-612)
    const bool sub = c.use_subn != 0;
    auto P = [&](const float *w) { return sub ? PW(in, w) : in; };
    CK(gemv(s, {J(L.kq, s->pq, key, P(L.kn_q)), J(L.kk, s->pk, key, P(L.kn_k)), J(L.kv, s->pv, value, P(L.kn_v)),
                J(L.fa, s->pfa, c.kda_gate_rank, P(nullptr)), J(L.kb, s->pb, nv, P(nullptr)),
                J(L.kg, s->pg, value, P(L.kn_g))}, nt));
    const int hist = c.conv_kernel - 1;
    KdaStepArgs a{};
    a.pq = s->pq; a.pk = s->pk; a.pv = s->pv; a.pfa = s->pfa;
    a.fb_q = L.fb.q; a.fb_s = L.fb.s; a.fb_gs = L.fb.gs == L.fb.cols ? 0 : L.fb.gs;
    a.conv_w = L.conv;
    a.conv_ring = s->conv + (size_t)li * c.lin_conv_dim * hist;
    a.conv_slot_stride = s->conv_slot;
    a.bvec = s->pb; a.gz = s->pg;
    a.a_log = L.a_log; a.dt_bias = L.dt_bias; a.o_norm = L.o_norm;
    a.state = s->kda + (size_t)li * nv * kd * vd;
    a.slot_stride = s->kda_slot;
    a.ctl_slot = &s->ctl->slot_base;
    a.xq = s->xq2; a.xqs = s->xqs2;
    a.normed_out = sub ? s->sub_a : nullptr;
    a.nv = nv; a.key = key; a.value = value; a.rank = c.kda_gate_rank;
    a.has_lb = c.kda_has_gate_lower_bound; a.gate_lb = c.kda_gate_lower_bound;
    a.depth = s->depth; a.advance = advance; a.nt = nt;
    a.scale = ssm_scale(kd); a.eps = c.rms_norm_eps;
    CK(l98k_kda_step(&a, kd, c.conv_kernel, s->st));
    if (sub) {
        // o_proj's own norm over the value row, then the block-Hadamard
        // quantization (src/forward_kda.c:954-996); per-32 scales
        const bool had = c.hadamard_o > 1;
        CK(l98k_rmsnorm_ex(s->sub_a, value, nullptr, nullptr, L.kn_o, value, c.rms_norm_eps, nt,
                           had ? s->sub_b : nullptr, value, had ? nullptr : s->xq2, s->xqs2, 0, s->st));
        if (had) CK(l98k_subn_quant(s->sub_b, nt, value, c.hadamard_o, 32, s->xq2, s->xqs2, s->st));
    }
    CK(gemv(s, {JX(L.ko, s->blk, d, s->xq2, s->xqs2)}, nt));
    return 0;
}

// MoE block: the router / latent-down / shared gate-up inputs come from
// `in`; outputs up_out and sd_out (the caller's next norm folds
// x += up_out + sd_out).
int moe_block(DState *s, const DLayer &L, const Prologue &in, int nt) {
    const LZModelConfig &c = s->m->c;
    const int d = c.hidden_size, E = c.num_experts, topk = c.num_experts_per_token;
    const int lat = c.moe_latent_dim, inter = c.moe_intermediate_size, sw = c.moe_shared_width;
    const bool sub = c.use_subn != 0;      // own norms (src/forward_moe.c:349-389, 418-430, 455-525)
    auto P = [&](const float *w) { return sub ? PW(in, w) : in; };
    CK(gemv(s, {J(L.router, s->rl, E, P(L.mn_gate)), J(L.down, s->latx, lat, P(L.mn_down)),
                J(L.sg, s->sgo, sw, P(L.mn_sg)), J(L.su, s->suo, sw, P(L.mn_su))}, nt));
    const int max_groups = nt * topk < E ? nt * topk : E;
    const ExpertJob up2[2] = {EJ(L.w1, s->h1, 0, PQ(s->latx, lat)), EJ(L.w3, s->h3, 0, PQ(s->latx, lat))};
    CK(l98k_moe_up(up2, 2, s->rl, L.bias, E, topk, nt, s->sel_idx, s->sel_w, s->grp, &s->ctl->expert_tally, lat,
                   inter, s->st));
    const ExpertJob down1[1] = {EJ(L.w2, s->h2, 1, PS(s->h1, s->h3, inter))};
    CK(l98k_expert_gemv(down1, 1, s->grp, max_groups, inter, lat, nt, s->st));
    if (sub) {
        // the routed combine and the shared SwiGLU, each normalized with its
        // own weight before its quantization
        const float eps = c.rms_norm_eps;
        CK(l98k_wide_pro_f(2, s->h2, nullptr, 0, s->sel_idx, s->sel_w, topk, lat, nt, s->sub_a, s->st));
        CK(l98k_rmsnorm_ex(s->sub_a, lat, nullptr, nullptr, L.mn_up, lat, eps, nt, nullptr, 0, s->xq3, s->xqs3, 0,
                           s->st));
        CK(l98k_wide_pro_f(1, s->sgo, s->suo, sw, nullptr, nullptr, 0, sw, nt, s->sub_b, s->st));
        CK(l98k_rmsnorm_ex(s->sub_b, sw, nullptr, nullptr, L.mn_sd, sw, eps, nt, nullptr, 0, s->xq4, s->xqs4, 0,
                           s->st));
        CK(gemv(s, {JX(L.up, s->up_out, d, s->xq3, s->xqs3), JX(L.sd, s->sd_out, d, s->xq4, s->xqs4)}, nt));
        return 0;
    }
    CK(gemv(s, {J(L.up, s->up_out, d, PC(s->h2, s->sel_idx, s->sel_w, topk)),
                J(L.sd, s->sd_out, d, PS(s->sgo, s->suo, sw))}, nt));
    return 0;
}

// forward_chunk (src/forward.c:1210-1617) for nt <= MAX_CHUNK tokens whose
// ids are in device memory at toks, positions *ctl_pos + pos_off + t.
//   capture:    device rows [nt][d] of the final-normed hidden, or null
//   logits_out: device [nt][V] when all_logits, else the last row's logits
//               go to s->logits unless skip_logits
int forward_chunk(DState *s, const int *toks, int nt, const int *ctl_pos, int pos_off, int max_pos,
                  float *capture, bool all_logits, float *logits_out, bool skip_logits) {
    const DModel *m = s->m;
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size;
    const float eps = c.rms_norm_eps;
    // The residual stream alternates between two buffers: a norm fused into
    // its consumer GEMV reads one and writes the folded residual to the
    // other, since every block of that launch reads the input.
    float *xb[2] = {s->x, s->x2};
    int cur = 0;
    // Every block of a fused launch normalizes all nt rows itself (reading
    // the rows and their addends), so for several rows of d = 2048, or more
    // than 4096 row elements, a norm kernel that quantizes the rows once,
    // then GEMVs of pre-quantized rows, is faster (measured on the d = 2048
    // verify: 4.25 -> 3.82 ms at 4 rows).  SubLN's per-projection norms only
    // run fused.
    const bool fused = l98k_gemv_norm_fits(d, nt) != 0 &&
                       (c.use_subn || ((size_t)nt * d <= 4096 && (d <= 1024 || nt == 1)));
    if (c.use_subn && !fused) return -1;      // SubLN's per-projection norms run in the GEMV prologues
    CK(l98k_embed(m->embed.q, m->embed.s, toks, d, m->embed.gs, nt, xb[cur], s->st));
    const float *ra = nullptr, *rb = nullptr;     // pending residual of the previous block
    // Input rows of a block: the fused norm prologue, or a norm kernel that
    // folds the residual in place and quantizes into xq.
    auto norm_in = [&](const float *a, const float *b, const float *w, Prologue &P) -> int {
        if (fused) {
            P = PN(xb[cur], d, a, b, w, eps, a ? xb[cur ^ 1] : nullptr, nullptr, 0);
            if (a) cur ^= 1;
            return 0;
        }
        CK(l98k_rmsnorm(xb[cur], d, a, b, w, d, eps, nt, nullptr, 0, s->xq, s->xqs, s->st));
        P = PX();
        return 0;
    };
    for (int l = 0; l < c.n_layers; l++) {
        const DLayer &L = m->L[l];
        Prologue P;
        CK(norm_in(ra, rb, L.in_norm, P));
        if (L.type == 1) CK(attn_block(s, L, P, m->full_index[l], ctl_pos, pos_off, nt, max_pos, false));
        else CK(kda_block(s, L, P, m->lin_index[l], nt, all_logits ? 1 : 0));
        CK(norm_in(s->blk, nullptr, L.post_norm, P));
        CK(moe_block(s, L, P, nt));
        ra = s->up_out;
        rb = s->sd_out;
    }
    // The lm_head's grid is far larger than the chip, so its norm runs once,
    // in its own kernel, rather than in every tile.
    const bool want_logits = all_logits || !skip_logits;
    CK(l98k_rmsnorm(xb[cur], d, ra, rb, m->final_norm, d, eps, nt, capture, d,
                    want_logits ? s->xq : nullptr, s->xqs, s->st));
    if (all_logits) {
        CK(lm_head_gemv(s, JX(m->embed, logits_out, c.vocab_size, s->xq, s->xqs), nt));
    } else if (!skip_logits) {
        CK(gemv(s, {JX(m->embed, s->logits, c.vocab_size, s->xq + (size_t)(nt - 1) * d,
                       s->xqs + (size_t)(nt - 1) * (d / 32))}, 1));
    }
    return 0;
}

// The MTP block's dense FFN and head for nt rows: the attention output
// s->blk is added to the residual rows s->mtp_x, then the FFN
// (dense_ffn_step, src/forward_kda.c:1102-1240), the exit norm (its rows ->
// chain_out when given) and the tied lm_head (logits rows -> out_logits).
int mtp_ffn_head(DState *s, int nt, float *chain_out, float *out_logits) {
    const DModel *m = s->m;
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size, I = c.mtp_intermediate_size;
    const float eps = c.rms_norm_eps;
    float *mx = s->mtp_x2;
    if (c.use_subn) {
        // SubLN: the residual folds in place; gate / up normalize it with
        // their own weights, one scale per row; the SwiGLU output takes
        // down's own norm, then the block-Hadamard quantization
        const float *fnw = m->mtp.fn_down;
        const bool had = c.hadamard_down > 1;
        mx = s->mtp_x;
        CK(l98k_rmsnorm_ex(mx, d, s->blk, nullptr, m->mtp.fn_gate, d, eps, nt, nullptr, 0, s->xq, s->xqs, 1, s->st));
        CK(l98k_rmsnorm_ex(mx, d, nullptr, nullptr, m->mtp.fn_up, d, eps, nt, nullptr, 0, s->xq3, s->xqs3, 1, s->st));
        CK(gemv(s, {JX(m->mtp_gate, s->hb, I, s->xq, s->xqs), JX(m->mtp_up, s->hb2, I, s->xq3, s->xqs3)}, nt));
        CK(l98k_wide_pro_f(1, s->hb, s->hb2, I, nullptr, nullptr, 0, I, nt, s->sub_a, s->st));
        CK(l98k_rmsnorm_ex(s->sub_a, I, nullptr, nullptr, fnw, I, eps, nt, had ? s->sub_b : nullptr, I,
                           had ? nullptr : s->xq, s->xqs, 0, s->st));
        if (had) CK(l98k_subn_quant(s->sub_b, nt, I, c.hadamard_down, 32, s->xq, s->xqs, s->st));
        CK(gemv(s, {JX(m->mtp_down, s->ffn_out, d, s->xq, s->xqs)}, nt));
    } else {
        const Prologue post = PN(s->mtp_x, d, s->blk, nullptr, m->mtp.post_norm, eps, s->mtp_x2, nullptr, 0);
        CK(gemv(s, {J(m->mtp_gate, s->hb, I, post), J(m->mtp_up, s->hb2, I, post)}, nt));
        CK(gemv(s, {J(m->mtp_down, s->ffn_out, d, PS(s->hb, s->hb2, I))}, nt));
    }
    CK(l98k_rmsnorm(mx, d, s->ffn_out, nullptr, m->mtp_norm, d, eps, nt, chain_out, d, s->xq, s->xqs, s->st));
    CK(lm_head_gemv(s, JX(m->embed, out_logits, c.vocab_size, s->xq, s->xqs), nt));
    return 0;
}

// lz_mtp_draft_step on device: input token at toks[0], position
// *ctl_pos + pos_off; logits -> out_logits; argmax (lz_argmax_p1 order) ->
// out_tok (device) when given.
int draft_step(DState *s, const int *toks, const int *ctl_pos, int pos_off, int max_pos,
               float *out_logits, int *out_tok) {
    const DModel *m = s->m;
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size;
    const float eps = c.rms_norm_eps;
    CK(l98k_mtp_pre(m->embed.q, m->embed.s, m->embed.gs, toks, s->chain, d, m->mtp_pre_e, m->mtp_pre_h, eps, 1, s->xq,
                    s->xqs, s->st));
    CK(gemv(s, {JX(m->mtp_fc, s->mtp_x, d, s->xq, s->xqs)}, 1));
    CK(attn_block(s, m->mtp, PN(s->mtp_x, d, nullptr, nullptr, m->mtp.in_norm, eps, nullptr, nullptr, 0),
                  s->planes - 1, ctl_pos, pos_off, 1, max_pos, false));
    AmaxScope amax(s, out_tok, 1);   // argmax in the lm_head's epilogue
    CK(mtp_ffn_head(s, 1, s->chain, out_logits));
    return 0;
}

// lz_mtp_draft_batch on device (src/forward_mtp.c:385-505): the k DSpark
// slots as k rows of one pass.  Row r's main_proj input is [norm(chain) |
// norm(emb(toks[0]) for r = 0, else mask) | depth row r]; the MTP block
// runs at position 0 with no history (mtp_attn_t1), then the FFN, exit norm
// and lm_head.  logits rows -> out_logits; their lz_argmax_p1 indices ->
// out_tok[0..k) when given.  The chain is read, not written.
int dspark_draft(DState *s, const int *toks, int k, float *out_logits, int *out_tok) {
    const DModel *m = s->m;
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size;
    const float eps = c.rms_norm_eps;
    const DLayer &L = m->mtp;
    const bool sub = c.use_subn != 0;
    CK(l98k_dspark_pre(m->embed.q, m->embed.s, m->embed.gs, toks, s->chain, m->mtp_mask, m->mtp_depth, d,
                       m->mtp_pre_e, m->mtp_pre_h, eps, k, s->xq, s->xqs, s->st));
    CK(gemv(s, {JX(m->mtp_main, s->mtp_x, d, s->xq, s->xqs)}, k));
    // q (its gate half is all the T=1 attention reads) and v, sharing the
    // input norm, or SubLN's own norm each (src/forward_mtp.c:226-240)
    const Prologue in = PN(s->mtp_x, d, nullptr, nullptr, L.in_norm, eps, nullptr, nullptr, 0);
    CK(gemv(s, {J(L.q, s->qg, c.attn_qgate_dim, sub ? PW(in, L.sn_q) : in),
                J(L.v, s->vp, c.attn_kv_dim, sub ? PW(in, L.sn_v) : in)}, k));
    const size_t off = (size_t)(s->planes - 1) * s->seq_len * c.attn_kv_dim;      // the MTP plane, row 0
    CK(l98k_attn_t1(s->qg, c.attn_qgate_dim, s->vp, c.attn_kv_dim, c.n_heads, c.n_kv_heads, c.head_dim,
                    c.attn_q_dim, k, s->vq + off, s->vs + off / 32, sub ? s->sub_a : nullptr, s->xq2, s->xqs2,
                    s->st));
    if (sub)
        CK(l98k_rmsnorm_ex(s->sub_a, c.attn_q_dim, nullptr, nullptr, L.sn_o, c.attn_q_dim, eps, k, nullptr, 0,
                           s->xq2, s->xqs2, 0, s->st));
    CK(gemv(s, {JX(L.o, s->blk, d, s->xq2, s->xqs2)}, k));
    AmaxScope amax(s, out_tok, 1);   // argmax in the lm_head's epilogue
    CK(mtp_ffn_head(s, k, nullptr, out_logits));
    return 0;
}

// MTP prefill/catch-up: K/V rows of the MTP plane from (hidden, next token)
// pairs, chunked by MAX_CHUNK.  h: device rows [n][d]; toks: device ids;
// positions *ctl_pos + pos_off + j.
int mtp_prefill_chunked(DState *s, const float *h, const int *toks, int n, const int *ctl_pos, int pos_off) {
    const DModel *m = s->m;
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size;
    const float eps = c.rms_norm_eps;
    for (int done = 0; done < n;) {
        int k = n - done < MAX_CHUNK ? n - done : MAX_CHUNK;
        CK(l98k_mtp_pre(m->embed.q, m->embed.s, m->embed.gs, toks + done, h + (size_t)done * d, d, m->mtp_pre_e,
                        m->mtp_pre_h, eps, k, s->xq, s->xqs, s->st));
        CK(gemv(s, {JX(m->mtp_fc, s->mtp_x, d, s->xq, s->xqs)}, k));
        CK(attn_block(s, m->mtp, PN(s->mtp_x, d, nullptr, nullptr, m->mtp.in_norm, eps, nullptr, nullptr, 0),
                      s->planes - 1, ctl_pos, pos_off + done, k, 0, true));
        done += k;
    }
    return 0;
}

// ------------------------------------------------------- wide forward ---
//
// Many token rows through the trunk at once: a prefill chunk of one session
// (consecutive positions) or the verify rows of several sessions (each its
// own ring, KV planes and positions).  Every projection is one matrix-core
// GEMM over all rows (l98_k_mfma.hip); the routed experts are grouped GEMMs
// over the (token, slot) pairs that chose each expert; the KDA recurrence
// and attention run per session in 8-row sub-chunks with the chunked
// path's kernels.  Each row gets exactly the arithmetic of the chunked path
// (forward_chunk above), so results are bit-identical for any grouping of
// rows.

struct WideItem {
    DState *d;                // the session
    int row0, n, pos0;        // its rows [row0, row0 + n) at positions pos0 ..
};

}  // namespace

struct DWide {
    int cap = 0;              // rows
    char *arena = nullptr;
    float *x, *blk, *up_out, *sd_out, *hcap;
    int8_t *xq, *xq2, *latq, *hq, *cq, *shq;
    float *xqs, *xqs2, *latqs, *hqs, *cqs, *shqs;
    float *pq, *pk, *pv, *pfa, *pb, *pg, *qg, *kp, *vp, *qh;
    float *rl, *latx, *sgo, *suo, *h1, *h3, *h2;
    int *sel_idx;
    float *sel_w;
    int *ng, *gexp, *goff, *gcnt, *list, *pair_token;
    int *toks;
    float *att;
    float *kda_rec, *kda_o;   // split KDA prefill: token records [R][nv][5*kd + 4], recurrence outputs [R][value]
    int8_t *mq;               // MTP prefill: main_proj input rows [R][2d] quantized
    float *mqs;
    float *logits = nullptr;  // rows x vocab, sized on demand
    int logits_rows = 0;
    KdaItem *kitems;          // per-session tables of the item launches [WIDE_MAX]
    AttnItem *aitems;
    float *att_items = nullptr;   // attention scratch of an item launch, sized on demand
    size_t att_items_floats = 0;
    // a session batch's control blocks and their destinations, staged in
    // pinned memory and copied with one transfer (sized on demand)
    char *ctl_host = nullptr, *ctl_dev = nullptr;
    int ctl_cap = 0;
    // the later parts of a split prefill chunk (see batch_capture_dev): each
    // its own scratch and stream, and per part one event per layer plus two
    std::vector<DWide *> peer;
    std::vector<hipStream_t> pst;
    std::vector<hipEvent_t> ev;
};

namespace {

#define WIDE_MAX 512          // rows of one wide forward
#define WIDE_MIN 16           // prefills shorter than this take the chunked path
#define WIDE_SPLIT 64         // wide prefill chunks of at least this many rows run in parts
#define WIDE_PARTS 3          // parts of a split chunk, each on its own stream (measured: 2 parts
                              // 10.1 ms, 3 parts 9.7 ms, 4 parts 15.0 ms for a 512-row prefill; four
                              // streams oversubscribe the process's four hardware queues)
// Each part of a split chunk must exceed MAX_CHUNK rows: a part's rows run as
// prefill items (wide_forward refuses a split part of MAX_CHUNK rows or
// fewer), and the split is taken only when the last part also exceeds it.
static_assert(((WIDE_SPLIT / WIDE_PARTS + MAX_CHUNK - 1) & ~(MAX_CHUNK - 1)) > MAX_CHUNK,
              "the parts of the smallest split chunk must exceed MAX_CHUNK rows");

// nullptr (the callers take the chunked path) for a SubLN model, whose
// per-projection norms this many-row forward does not carry, and for a
// model with grouped weight scales (its matrix-core epilogue takes one
// scale per row).
DWide *wide_alloc(const DModel *m) {
    const LZModelConfig &c = m->c;
    const size_t R = WIDE_MAX, d = c.hidden_size, pairs = R * c.num_experts_per_token;
    size_t wide = d;
    for (int v : {c.attn_qgate_dim, c.lin_value_dim, c.attn_q_dim, c.moe_shared_width, c.moe_latent_dim})
        wide = (size_t)v > wide ? (size_t)v : wide;
    DWide *w = new DWide();
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t o = off; off = (off + bytes + 255) & ~(size_t)255; return o; };
    const size_t ox = take(4 * R * d), oblk = take(4 * R * d), oup = take(4 * R * d), osd = take(4 * R * d),
                 ohc = take(4 * R * d), oxq = take(R * d), oxqs = take(4 * R * d / 32), oxq2 = take(R * wide),
                 oxqs2 = take(4 * R * wide / 32), olq = take(R * c.moe_latent_dim),
                 olqs = take(4 * R * c.moe_latent_dim / 32), ohq = take(pairs * c.moe_intermediate_size),
                 ohqs = take(4 * pairs * c.moe_intermediate_size / 32), ocq = take(R * c.moe_latent_dim),
                 ocqs = take(4 * R * c.moe_latent_dim / 32), oshq = take(R * c.moe_shared_width),
                 oshqs = take(4 * R * c.moe_shared_width / 32), opq = take(4 * R * c.lin_key_dim),
                 opk = take(4 * R * c.lin_key_dim), opv = take(4 * R * c.lin_value_dim),
                 opfa = take(4 * R * c.kda_gate_rank), opb = take(4 * R * c.lin_n_v_heads),
                 opg = take(4 * R * c.lin_value_dim), oqg = take(4 * R * c.attn_qgate_dim),
                 okp = take(4 * R * c.attn_kv_dim), ovp = take(4 * R * c.attn_kv_dim), oqh = take(4 * R * c.attn_q_dim),
                 orl = take(4 * R * c.num_experts), olx = take(4 * R * c.moe_latent_dim),
                 osg = take(4 * R * c.moe_shared_width), osu = take(4 * R * c.moe_shared_width),
                 oh1 = take(4 * pairs * c.moe_intermediate_size), oh3 = take(4 * pairs * c.moe_intermediate_size),
                 oh2 = take(4 * pairs * c.moe_latent_dim), osi = take(4 * pairs), osw = take(4 * pairs),
                 ong = take(4), oge = take(4 * MAX_EXPERTS), ogo = take(4 * MAX_EXPERTS), ogc = take(4 * MAX_EXPERTS),
                 oli = take(4 * pairs), opt = take(4 * pairs), otk = take(4 * R),
                 oki = take(sizeof(KdaItem) * R), oai = take(sizeof(AttnItem) * R),
                 oat = take(4 * (size_t)MAX_CHUNK * c.n_heads * (size_t)((c.seq_len + 3) & ~3)),
                 okr = take(4 * R * c.lin_n_v_heads * (size_t)(5 * c.lin_k_head_dim + 4)),
                 oko = take(4 * R * c.lin_value_dim), omq = take(R * 2 * d), omqs = take(4 * R * 2 * d / 32);
    if (hipMalloc((void **)&w->arena, off) != hipSuccess) { delete w; return nullptr; }
    char *a = w->arena;
    w->cap = WIDE_MAX;
    w->x = (float *)(a + ox); w->blk = (float *)(a + oblk); w->up_out = (float *)(a + oup); w->sd_out = (float *)(a + osd);
    w->hcap = (float *)(a + ohc);
    w->xq = (int8_t *)(a + oxq); w->xqs = (float *)(a + oxqs); w->xq2 = (int8_t *)(a + oxq2); w->xqs2 = (float *)(a + oxqs2);
    w->latq = (int8_t *)(a + olq); w->latqs = (float *)(a + olqs); w->hq = (int8_t *)(a + ohq); w->hqs = (float *)(a + ohqs);
    w->cq = (int8_t *)(a + ocq); w->cqs = (float *)(a + ocqs); w->shq = (int8_t *)(a + oshq); w->shqs = (float *)(a + oshqs);
    w->pq = (float *)(a + opq); w->pk = (float *)(a + opk); w->pv = (float *)(a + opv); w->pfa = (float *)(a + opfa);
    w->pb = (float *)(a + opb); w->pg = (float *)(a + opg); w->qg = (float *)(a + oqg); w->kp = (float *)(a + okp);
    w->vp = (float *)(a + ovp); w->qh = (float *)(a + oqh);
    w->rl = (float *)(a + orl); w->latx = (float *)(a + olx); w->sgo = (float *)(a + osg); w->suo = (float *)(a + osu);
    w->h1 = (float *)(a + oh1); w->h3 = (float *)(a + oh3); w->h2 = (float *)(a + oh2);
    w->sel_idx = (int *)(a + osi); w->sel_w = (float *)(a + osw);
    w->ng = (int *)(a + ong); w->gexp = (int *)(a + oge); w->goff = (int *)(a + ogo); w->gcnt = (int *)(a + ogc);
    w->list = (int *)(a + oli); w->pair_token = (int *)(a + opt); w->toks = (int *)(a + otk);
    w->att = (float *)(a + oat);
    w->kda_rec = (float *)(a + okr); w->kda_o = (float *)(a + oko);
    w->mq = (int8_t *)(a + omq); w->mqs = (float *)(a + omqs);
    w->kitems = (KdaItem *)(a + oki);
    w->aitems = (AttnItem *)(a + oai);
    return w;
}

void wide_release(DWide *w) {
    if (!w) return;
    if (w->arena) (void)hipFree(w->arena);
    if (w->logits) (void)hipFree(w->logits);
    if (w->att_items) (void)hipFree(w->att_items);
    if (w->ctl_host) (void)hipHostFree(w->ctl_host);
    if (w->ctl_dev) (void)hipFree(w->ctl_dev);
    delete w;
}

DWide *wide_get(const DModel *cm) {
    DModel *m = const_cast<DModel *>(cm);
    if (m->c.use_subn || m->grouped) return nullptr;
    if (!m->wide) m->wide = wide_alloc(m);
    return m->wide;
}

// The parts of a split prefill chunk: WIDE_PARTS - 1 peer scratches and
// streams (default priority) and WIDE_PARTS x (n_layers + 2) events; false
// when any of it cannot be made.
bool wide_parts(DModel *m, DWide *w) {
    if (!w->peer.empty()) return true;
    std::vector<DWide *> peer;
    std::vector<hipStream_t> pst;
    std::vector<hipEvent_t> ev((size_t)WIDE_PARTS * (m->c.n_layers + 2), nullptr);
    bool ok = true;
    for (int p = 1; p < WIDE_PARTS && ok; p++) {
        DWide *q = wide_alloc(m);
        hipStream_t sq = nullptr;
        ok = q && hipStreamCreateWithFlags(&sq, hipStreamNonBlocking) == hipSuccess;
        if (q) peer.push_back(q);
        if (sq) pst.push_back(sq);
    }
    for (auto &e : ev) ok = ok && hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        for (auto &e : ev)
            if (e) (void)hipEventDestroy(e);
        for (auto sq : pst) (void)hipStreamDestroy(sq);
        for (auto q : peer) wide_release(q);
        return false;
    }
    w->peer = peer;
    w->pst = pst;
    w->ev = ev;
    return true;
}

void wide_free(DModel *m) {
    DWide *w = m->wide;
    if (!w) return;
    for (auto sq : w->pst) (void)hipStreamSynchronize(sq);
    for (auto &e : w->ev) (void)hipEventDestroy(e);
    for (auto sq : w->pst) (void)hipStreamDestroy(sq);
    for (auto q : w->peer) wide_release(q);
    wide_release(w);
    m->wide = nullptr;
}

// Dense MFMA GEMM of a weight matrix over the rows' quantized activations.
int mf(const DMat &W, const int8_t *xq, const float *xqs, int R, float *out, int out_stride, hipStream_t st) {
    return l98k_mfma_gemm(W.q, W.s, W.rows, W.cols, xq, xqs, R, out, out_stride, st);
}

// Several weight matrices over the same rows, one launch: each job's input
// (xq, xqs) defaults to the call's.
struct MfOut {
    const DMat *W;
    float *out;
    int out_stride;
    const int8_t *xq = nullptr;
    const float *xqs = nullptr;
};
int mf_multi(std::initializer_list<MfOut> jobs, const int8_t *xq, const float *xqs, int R, hipStream_t st) {
    const int8_t *W[6], *X[6];
    const float *ws[6], *Xs[6];
    float *out[6];
    int N[6], os[6], K[6], n = 0;
    for (const MfOut &j : jobs) {
        if (n == 6) return 1;
        W[n] = j.W->q; ws[n] = j.W->s; N[n] = j.W->rows; K[n] = j.W->cols; out[n] = j.out; os[n] = j.out_stride;
        X[n] = j.xq ? j.xq : xq;
        Xs[n] = j.xq ? j.xqs : xqs;
        n++;
    }
    return l98k_mfma_gemm_multi(n, W, ws, N, out, os, K, X, Xs, R, st);
}

// Orders an attention item launch (any order is correct: each item names
// its rows and planes): the longer half of the items by span, longest first,
// then the rest shortest first, so that blocks y and y + n/2 of the launch -
// which share a CU when the grid fills two blocks per CU - pair a long item
// with a short one instead of two long ones.
static void pair_long_short(std::vector<AttnItem> &ai, const std::vector<int> &len) {
    const int n = (int)ai.size();
    if (n < 3) return;
    std::vector<int> idx((size_t)n);
    std::iota(idx.begin(), idx.end(), 0);
    std::stable_sort(idx.begin(), idx.end(), [&](int x, int y) { return len[(size_t)x] > len[(size_t)y]; });
    std::vector<AttnItem> out((size_t)n);
    const int h2 = (n + 1) / 2;
    for (int y = 0; y < n; y++) out[(size_t)y] = ai[(size_t)idx[(size_t)(y < h2 ? y : n - 1 - (y - h2))]];
    ai.swap(out);
}

// The trunk over R rows of w->toks (device ids), grouped into sessions by
// items (row order).  advance: KDA ring advance per token (verify) or not
// (prefill).  capture: device rows [R][d] of the final-normed hidden, or
// null; logits: device rows [R][V] of the tied lm_head, or null.  Every
// launch goes on stream st; the sessions' control blocks must hold their
// slot bases and positions (pos_scratch = the item's pos0) before.
int wide_forward(const DModel *m, DWide *w, const WideItem *items, int n_items, int R, bool advance, float *capture,
                 float *logits, hipStream_t st, int pos_base = 0, hipEvent_t *wait_ev = nullptr,
                 hipEvent_t *rec_ev = nullptr, int l0 = 0, int l1 = -1) {
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size, E = c.num_experts, topk = c.num_experts_per_token;
    const int lat = c.moe_latent_dim, inter = c.moe_intermediate_size, sw = c.moe_shared_width;
    const float eps = c.rms_norm_eps;
    if (l1 < 0) l1 = c.n_layers;
    if (R < 1 || R > w->cap || n_items < 1 || n_items > w->cap || l0 < 0 || l0 >= l1 || l1 > c.n_layers) return 1;
    // Layers [l0, l1) only (a split prefill enqueues its parts layer by layer,
    // in turn): the tables, the attention scratch and the embedding come with
    // layer 0, the final norm with the last layer.
    // the sessions' tables for the item launches
    // Attention runs as one item launch per kernel: over the sessions'
    // verify rows, or over one session's prefill rows cut into MAX_CHUNK-row
    // items (prefill_items: their K and V rows go to the cache first, in one
    // launch), else chunk by chunk.
    bool attn_items = n_items > 1;
    const bool prefill_items = n_items == 1 && items[0].n > MAX_CHUNK && !advance;
    if ((pos_base || wait_ev || rec_ev) && !prefill_items) return 1;   // only a prefill chunk is split
    int n_attn = n_items;
    int max_len = 1, max_rows = 1;          // the attention items' longest row span and most rows
    int kda_max_n = 1;                      // the KDA items' most rows
    {
        std::vector<KdaItem> ki((size_t)n_items);
        std::vector<AttnItem> ai;
        std::vector<int> alen;                  // each attention item's last position + 1
        for (int i = 0; i < n_items; i++) {
            const WideItem &I = items[i];
            DState *s = I.d;
            if (advance && I.n > MAX_CHUNK) return 1;       // one ring advance per verify chunk
            attn_items = attn_items && I.n <= MAX_CHUNK;
            max_len = I.pos0 + I.n > max_len ? I.pos0 + I.n : max_len;
            ki[i] = KdaItem{s->kda, s->conv, &s->ctl->slot_base, s->kda_slot, s->conv_slot, I.row0, I.n, s->depth, 0};
            kda_max_n = I.n > kda_max_n ? I.n : kda_max_n;
            if (prefill_items) {
                for (int c0 = 0; c0 < I.n; c0 += MAX_CHUNK) {
                    const int nr = I.n - c0 < MAX_CHUNK ? I.n - c0 : MAX_CHUNK;
                    ai.push_back(AttnItem{s->kq, s->vq, s->ks, s->vs, &s->ctl->pos_scratch, I.row0 + c0, nr,
                                          s->seq_len, pos_base + c0});
                    alen.push_back(I.pos0 + pos_base + c0 + nr);
                }
            } else {
                ai.push_back(AttnItem{s->kq, s->vq, s->ks, s->vs, &s->ctl->pos_scratch, I.row0, I.n, s->seq_len, 0});
                alen.push_back(I.pos0 + I.n);
            }
        }
        pair_long_short(ai, alen);
        if (prefill_items) {
            attn_items = true;
            n_attn = (int)ai.size();
        }
        for (const AttnItem &x : ai) max_rows = x.n > max_rows ? x.n : max_rows;
        if (l0 == 0) {
            CK(hipMemcpyAsync(w->kitems, ki.data(), sizeof(KdaItem) * ki.size(), hipMemcpyHostToDevice, st));
            CK(hipMemcpyAsync(w->aitems, ai.data(), sizeof(AttnItem) * ai.size(), hipMemcpyHostToDevice, st));
        }
    }
    const size_t att_item = (size_t)MAX_CHUNK * c.n_heads * (size_t)((max_len + 3) & ~3);
    if (l0 == 0 && attn_items && w->att_items_floats < att_item * n_attn) {
        CK(hipStreamSynchronize(st));
        if (w->att_items) (void)hipFree(w->att_items);
        w->att_items = nullptr;
        w->att_items_floats = 0;
        CK(hipMalloc((void **)&w->att_items, sizeof(float) * att_item * n_attn));
        w->att_items_floats = att_item * n_attn;
    }
    if (l0 == 0) CK(l98k_embed(m->embed.q, m->embed.s, w->toks, d, m->embed.gs, R, w->x, st));
    // every layer leaves its two residual addends in up_out and sd_out
    const float *ra = l0 ? w->up_out : nullptr, *rb = l0 ? w->sd_out : nullptr;
    for (int l = l0; l < l1; l++) {
        const DLayer &L = m->L[l];
        CK(l98k_rmsnorm(w->x, d, ra, rb, L.in_norm, d, eps, R, nullptr, 0, w->xq, w->xqs, st));
        if (L.type == 1) {
            const int qgd = c.attn_qgate_dim, kvd = c.attn_kv_dim, qd = c.attn_q_dim;
            CK(mf_multi({{&L.q, w->qg, qgd}, {&L.k, w->kp, kvd}, {&L.v, w->vp, kvd}}, w->xq, w->xqs, R, st));
            const int plane = m->full_index[l];
            if (attn_items) {
                // every session's rows in one launch per kernel
                AttnArgs a{};
                a.qg = w->qg; a.kp = w->kp; a.vp = w->vp;
                a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.rope_cs = m->rope_cs;
                a.qh = w->qh;
                a.out = nullptr;
                a.oq = w->xq2; a.oqs = w->xqs2;
                a.nh = c.n_heads; a.nkv = c.n_kv_heads; a.hd = c.head_dim; a.rot = c.rotary_dim;
                a.q_dim = qd; a.qg_dim = qgd; a.kv_dim = kvd;
                a.kv_only = 0;
                a.eps = eps;
                a.attn_scale = ssm_scale(c.head_dim);
                if (prefill_items) {
                    // every prefill row's K and V into the cache, so each item
                    // finds the earlier items' rows there
                    const WideItem &I = items[0];
                    const DState *s = I.d;
                    AttnArgs p = a;
                    p.kv_only = 1;
                    p.kp = w->kp + (size_t)I.row0 * kvd; p.vp = w->vp + (size_t)I.row0 * kvd;
                    const size_t off = (size_t)plane * s->seq_len * kvd;
                    p.kcache = s->kq + off; p.vcache = s->vq + off;
                    p.kscale = s->ks + off / 32; p.vscale = s->vs + off / 32;
                    p.ctl_pos = &s->ctl->pos_scratch; p.pos_off = pos_base;
                    CK(l98k_attn_prep(&p, I.n, st));
                }
                // (a split chunk's second half reads the first half's K and V rows)
                if (wait_ev) CK(hipStreamWaitEvent(st, wait_ev[l], 0));
                CK(l98k_attn_items(&a, w->aitems, n_attn, plane, max_len, max_rows, w->att_items, att_item,
                                   prefill_items ? 1 : 0, st));
                if (rec_ev) CK(hipEventRecord(rec_ev[l], st));
            }
            for (int it = 0; it < n_items && !attn_items; it++) {
                const WideItem &I = items[it];
                DState *s = I.d;
                for (int c0 = 0; c0 < I.n; c0 += MAX_CHUNK) {
                    const int k = I.n - c0 < MAX_CHUNK ? I.n - c0 : MAX_CHUNK;
                    const int r = I.row0 + c0;
                    AttnArgs a{};
                    a.qg = w->qg + (size_t)r * qgd; a.kp = w->kp + (size_t)r * kvd; a.vp = w->vp + (size_t)r * kvd;
                    a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.rope_cs = m->rope_cs;
                    a.qh = w->qh + (size_t)r * qd;
                    const size_t off = (size_t)plane * s->seq_len * kvd;
                    a.kcache = s->kq + off; a.vcache = s->vq + off;
                    a.kscale = s->ks + off / 32; a.vscale = s->vs + off / 32;
                    a.out = nullptr;
                    a.oq = w->xq2 + (size_t)r * qd; a.oqs = w->xqs2 + (size_t)r * (qd / 32);
                    a.ctl_pos = &s->ctl->pos_scratch; a.pos_off = c0;
                    a.nh = c.n_heads; a.nkv = c.n_kv_heads; a.hd = c.head_dim; a.rot = c.rotary_dim;
                    a.q_dim = qd; a.qg_dim = qgd; a.kv_dim = kvd;
                    a.kv_only = 0;
                    a.eps = eps;
                    a.attn_scale = ssm_scale(c.head_dim);
                    CK(l98k_attn(&a, k, I.pos0 + c0 + k, w->att, st));
                }
            }
            CK(mf(L.o, w->xq2, w->xqs2, R, w->blk, d, st));
        } else {
            const int key = c.lin_key_dim, value = c.lin_value_dim, nv = c.lin_n_v_heads, kd = c.lin_k_head_dim;
            const int rank = c.kda_gate_rank, hist = c.conv_kernel - 1;
            CK(mf_multi({{&L.kq, w->pq, key}, {&L.kk, w->pk, key}, {&L.kv, w->pv, value}, {&L.fa, w->pfa, rank},
                         {&L.kb, w->pb, nv}, {&L.kg, w->pg, value}},
                        w->xq, w->xqs, R, st));
            const int li = m->lin_index[l];
            // every session's rows in one launch (a prefill's rows in
            // sub-chunks inside its blocks)
            KdaStepArgs a{};
            a.pq = w->pq; a.pk = w->pk; a.pv = w->pv; a.pfa = w->pfa;
            a.fb_q = L.fb.q; a.fb_s = L.fb.s; a.fb_gs = L.fb.gs == L.fb.cols ? 0 : L.fb.gs;
            a.conv_w = L.conv;
            a.bvec = w->pb; a.gz = w->pg;
            a.a_log = L.a_log; a.dt_bias = L.dt_bias; a.o_norm = L.o_norm;
            a.xq = w->xq2; a.xqs = w->xqs2;
            a.nv = nv; a.key = key; a.value = value; a.rank = rank;
            a.has_lb = c.kda_has_gate_lower_bound; a.gate_lb = c.kda_gate_lower_bound;
            a.advance = advance ? 1 : 0;
            a.scale = ssm_scale(kd); a.eps = eps;
            if (n_items == 1 && items[0].n > MAX_CHUNK && !advance) {
                // one session's prefill: the state-free work of every row at
                // once, the recurrence, then the gated norm of every row
                const DState *s = items[0].d;
                a.state = s->kda + (size_t)li * nv * kd * c.lin_v_head_dim;
                a.conv_ring = s->conv + (size_t)li * c.lin_conv_dim * hist;
                a.ctl_slot = &s->ctl->slot_base;
                a.slot_stride = s->kda_slot;
                a.conv_slot_stride = s->conv_slot;
                a.depth = s->depth;
                const size_t r0 = (size_t)items[0].row0;
                a.pq += r0 * key; a.pk += r0 * key; a.pv += r0 * value; a.pfa += r0 * rank;
                a.bvec += r0 * nv; a.gz += r0 * value;
                a.xq += r0 * value; a.xqs += r0 * (value / 32);
                a.rec = w->kda_rec;
                a.orow = w->kda_o;
                // (a split chunk's second half starts from the state and conv
                // history the first half leaves)
                if (wait_ev) CK(hipStreamWaitEvent(st, wait_ev[l], 0));
                CK(l98k_kda_split(&a, items[0].n, kd, c.conv_kernel, st));
                if (rec_ev) CK(hipEventRecord(rec_ev[l], st));
            } else {
                CK(l98k_kda_items(&a, w->kitems, n_items, kda_max_n, (size_t)li * nv * kd * c.lin_v_head_dim,
                                  (size_t)li * c.lin_conv_dim * hist, kd, c.conv_kernel, st));
            }
            CK(mf(L.ko, w->xq2, w->xqs2, R, w->blk, d, st));
        }
        CK(l98k_rmsnorm(w->x, d, w->blk, nullptr, L.post_norm, d, eps, R, nullptr, 0, w->xq, w->xqs, st));
        // latent MoE (src/forward_moe.c:220-553) with the shared expert
        CK(mf_multi({{&L.router, w->rl, E}, {&L.down, w->latx, lat}, {&L.sg, w->sgo, sw}, {&L.su, w->suo, sw}},
                    w->xq, w->xqs, R, st));
        const int pairs = R * topk;
        // routing, and the latent rows quantized for the expert GEMMs, in one launch
        CK(l98k_moe_route_wide(w->rl, L.bias, E, topk, R, w->sel_idx, w->sel_w, w->latx, lat, w->latq, w->latqs, st));
        CK(l98k_moe_group(w->sel_idx, pairs, topk, E, w->ng, w->gexp, w->goff, w->gcnt, w->list, w->pair_token, st));
        const int maxg = pairs < E ? pairs : E;
        const int mean_cols = (pairs + maxg - 1) / maxg;
        CK(l98k_mfma_gemm_grouped2(L.w1.q, L.w1.s, w->h1, L.w3.q, L.w3.s, w->h3, inter, lat, w->latq, w->latqs, w->ng,
                                   maxg, w->gexp, w->goff, w->gcnt, w->list, w->pair_token, R, mean_cols, inter, st));
        CK(l98k_wide_pro(1, w->h1, w->h3, inter, nullptr, nullptr, 0, inter, pairs, w->hq, w->hqs, st));
        CK(l98k_mfma_gemm_grouped(L.w2.q, L.w2.s, lat, inter, w->hq, w->hqs, w->ng, maxg, w->gexp, w->goff, w->gcnt,
                                  w->list, nullptr, R, mean_cols, w->h2, lat, st));
        // the shared expert's SiLU-mul rows and the routed experts' combine, one launch
        CK(l98k_wide_pro2(1, w->sgo, w->suo, sw, sw, R, w->shq, w->shqs, 2, w->h2, nullptr, lat, w->sel_idx, w->sel_w,
                          topk, lat, R, w->cq, w->cqs, st));
        CK(mf_multi({{&L.up, w->up_out, d, w->cq, w->cqs}, {&L.sd, w->sd_out, d, w->shq, w->shqs}}, nullptr, nullptr,
                    R, st));
        ra = w->up_out;
        rb = w->sd_out;
    }
    if (l1 < c.n_layers) return 0;
    CK(l98k_rmsnorm(w->x, d, ra, rb, m->final_norm, d, eps, R, capture, d, logits ? w->xq : nullptr, w->xqs, st));
    if (logits) CK(mf(m->embed, w->xq, w->xqs, R, logits, c.vocab_size, st));
    return 0;
}

// The MTP prefill over many rows (lz_mtp_prefill, src/forward_mtp.c:561-627)
// with mtp_prefill_chunked's arithmetic: the main_proj input rows, fc, the
// MTP block's input norm and K / V projections as matrix-core GEMMs, then
// the K / V rows into the MTP plane, WIDE_MAX rows per pass.
int mtp_prefill_wide(DState *s, DWide *w, const float *h, const int *toks, int n, const int *ctl_pos, int pos_off) {
    const DModel *m = s->m;
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size, kvd = c.attn_kv_dim;
    const float eps = c.rms_norm_eps;
    hipStream_t st = s->st;
    for (int done = 0; done < n;) {
        const int R = n - done < w->cap ? n - done : w->cap;
        CK(l98k_mtp_pre(m->embed.q, m->embed.s, m->embed.gs, toks + done, h + (size_t)done * d, d, m->mtp_pre_e,
                        m->mtp_pre_h, eps, R, w->mq, w->mqs, st));
        CK(mf(m->mtp_fc, w->mq, w->mqs, R, w->blk, d, st));
        CK(l98k_rmsnorm(w->blk, d, nullptr, nullptr, m->mtp.in_norm, d, eps, R, nullptr, 0, w->xq, w->xqs, st));
        CK(mf_multi({{&m->mtp.k, w->kp, kvd}, {&m->mtp.v, w->vp, kvd}}, w->xq, w->xqs, R, st));
        AttnArgs a{};
        a.kp = w->kp; a.vp = w->vp;
        a.k_norm = m->mtp.k_norm; a.rope_cs = m->rope_cs;
        const size_t off = (size_t)(s->planes - 1) * s->seq_len * kvd;
        a.kcache = s->kq + off; a.vcache = s->vq + off;
        a.kscale = s->ks + off / 32; a.vscale = s->vs + off / 32;
        a.ctl_pos = ctl_pos; a.pos_off = pos_off + done;
        a.nh = c.n_heads; a.nkv = c.n_kv_heads; a.hd = c.head_dim; a.rot = c.rotary_dim;
        a.q_dim = c.attn_q_dim; a.qg_dim = c.attn_qgate_dim; a.kv_dim = kvd;
        a.kv_only = 1;
        a.eps = eps;
        CK(l98k_attn_prep(&a, R, st));
        done += R;
    }
    return 0;
}

// The MTP prefill / catch-up of n rows: the many-row form for a prefill (n
// >= WIDE_MIN, a model the many-row forward carries), else MAX_CHUNK rows at
// a time.
int mtp_prefill_dev(DState *s, const float *h, const int *toks, int n, const int *ctl_pos, int pos_off) {
    DWide *w = n >= WIDE_MIN ? wide_get(s->m) : nullptr;
    if (w) return mtp_prefill_wide(s, w, h, toks, n, ctl_pos, pos_off);
    return mtp_prefill_chunked(s, h, toks, n, ctl_pos, pos_off);
}

}  // namespace

extern "C" int lz_state_alloc(LZRunState *s, const LZModel *mm, int seq_len, int spec_k_max,
                              char *errbuf, int errlen) {
    if (!s || !mm || !mm->impl) { set_err(errbuf, errlen, "null argument"); return 1; }
    memset(s, 0, sizeof(*s));
    const DModel *m = Mo(mm);
    const LZModelConfig &c = m->c;
    if (!knobs_ok(c.num_experts_per_token, errbuf, errlen)) return 1;
    DState *d = new DState();
    d->m = m;
    d->seq_len = seq_len > 0 ? seq_len : c.seq_len;
    if (d->seq_len > c.seq_len) d->seq_len = c.seq_len;   // the rope table covers the model's seq_len
    d->depth = spec_k_max > 0 ? (spec_k_max > L98_SPEC_K_GPU ? L98_SPEC_K_GPU : spec_k_max) + 1 : 1;
    d->planes = c.n_full_layers + 1;
    d->kda_slot = (size_t)c.n_linear_layers * c.lin_n_v_heads * c.lin_k_head_dim * c.lin_v_head_dim;
    d->conv_slot = (size_t)c.n_linear_layers * c.lin_conv_dim * (c.conv_kernel - 1);
    d->cap_rows = d->seq_len;
    carve(d);                                   // sizing pass
    d->arena_size = d->arena_used + 4096;
    d->arena_used = 0;
    if (hipMalloc((void **)&d->arena, d->arena_size) != hipSuccess) {
        set_err(errbuf, errlen, "hipMalloc of %zu state bytes failed", d->arena_size);
        delete d;
        return 1;
    }
    carve(d);
    if (hipStreamCreateWithFlags(&d->st, hipStreamNonBlocking) != hipSuccess ||
        hipHostMalloc((void **)&d->ctl_pinned, sizeof(DevCtl), hipHostMallocDefault) != hipSuccess ||
        hipEventCreate(&d->ev0) != hipSuccess || hipEventCreate(&d->ev1) != hipSuccess ||
        hipEventCreate(&d->ph[0]) != hipSuccess || hipEventCreate(&d->ph[1]) != hipSuccess ||
        hipEventCreate(&d->ph[2]) != hipSuccess || hipEventCreate(&d->ph[3]) != hipSuccess) {
        set_err(errbuf, errlen, "HIP stream/event setup failed");
        (void)hipFree(d->arena);
        delete d;
        return 1;
    }
    s->impl = d;
    s->seq_len = d->seq_len;
    s->ssm_ring_depth = d->depth;
    s->nt_cap = 4;
    s->bytes_device = (long long)d->arena_size;
    s->logits = (float *)calloc((size_t)c.vocab_size, sizeof(float));
    s->mtp_logits = (float *)calloc((size_t)(L98_SPEC_K_GPU + 1) * c.vocab_size, sizeof(float));
    s->mtp_verify_hidden = (float *)calloc((size_t)(L98_SPEC_K_GPU + 1) * c.hidden_size, sizeof(float));
    s->mtp_chain = (float *)calloc((size_t)c.hidden_size, sizeof(float));
    s->mtp_draft_logits = (float *)calloc((size_t)c.vocab_size, sizeof(float));
    s->mtp_kdraft_logits = c.mtp_n_draft > 1 ? (float *)calloc((size_t)LZ_SPEC_K_MAX * c.vocab_size, sizeof(float))
                                             : nullptr;
    lz_state_reset(s, mm);
    return 0;
}

extern "C" void lz_state_free(LZRunState *s) {
    if (!s) return;
    DState *d = S(s);
    if (d) {
        if (d->st) (void)hipStreamSynchronize(d->st);
        if (d->arena) (void)hipFree(d->arena);
        if (d->smp_arena) (void)hipFree(d->smp_arena);
        if (d->ctl_pinned) (void)hipHostFree(d->ctl_pinned);
        if (d->ev0) (void)hipEventDestroy(d->ev0);
        if (d->ev1) (void)hipEventDestroy(d->ev1);
        for (hipEvent_t e : d->ph)
            if (e) (void)hipEventDestroy(e);
        for (auto &g : d->round_graph)
            if (g) (void)hipGraphExecDestroy(g);
        for (auto &g : d->temp_graph)
            if (g) (void)hipGraphExecDestroy(g);
        if (d->st) (void)hipStreamDestroy(d->st);
        delete d;
    }
    free(s->logits); free(s->mtp_logits); free(s->mtp_verify_hidden);
    free(s->mtp_chain); free(s->mtp_draft_logits); free(s->mtp_kdraft_logits);
    memset(s, 0, sizeof(*s));
}

// lz_state_reset (src/forward.c:654-775): zero every state plane, slot 0,
// mtp_pos 0.
extern "C" void lz_state_reset(LZRunState *s, const LZModel *m) {
    (void)m;
    if (!s || !s->impl) return;
    DState *d = S(s);
    (void)hipMemsetAsync(d->arena, 0, d->arena_used, d->st);
    (void)hipStreamSynchronize(d->st);
    s->ssm_slot = 0;
    s->mtp_pos = 0;
    memset(s->mtp_chain, 0, sizeof(float) * (size_t)d->m->c.hidden_size);
}

// ---------------------------------------------------------- forward API ---

namespace {

bool tok_ok(const LZModelConfig &c, const int *t, int n) {
    for (int i = 0; i < n; i++) if (t[i] < 0 || t[i] >= c.vocab_size) return false;
    return true;
}

// Device-resident round state prepared from the host mirrors.
DevCtl ctl_from(LZRunState *s) {
    DevCtl h{};
    h.mtp_pos = s->mtp_pos;
    h.slot_base = s->ssm_slot;
    h.ssm_slot = s->ssm_slot;
    return h;
}

}  // namespace

namespace {
// One token forward (src/forward.c:1623-1632 with capture, forward.h:1937
// without): logits to s->logits; with capture the final-normed hidden also
// becomes mtp_chain.
float *forward_one(const LZModel *mm, LZRunState *s, int token, int pos, bool capture) {
    if (!mm || !s || !s->impl) return nullptr;
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (token < 0 || token >= c.vocab_size || pos < 0 || pos >= d->seq_len) return nullptr;
    if (!knobs_ok(c.num_experts_per_token, nullptr, 0)) return nullptr;
    const timespec t0 = now_ts();
    DevCtl h = ctl_from(s);
    h.pos_scratch = pos;
    h.tok[0] = token;
    if (ctl_put(d, h)) return nullptr;
    if (forward_chunk(d, d->ctl->tok, 1, &d->ctl->pos_scratch, 0, pos, capture ? d->chain : nullptr, false, nullptr,
                      false))
        return nullptr;
    if (hipMemcpyAsync(s->logits, d->logits, sizeof(float) * c.vocab_size, hipMemcpyDeviceToHost, d->st) ||
        (capture &&
         hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st)) ||
        hipStreamSynchronize(d->st))
        return nullptr;
    lz_debug_n_chunks++;
    lz_debug_n_lmhead++;
    if (capture) {
        lz_debug_us_capture += us_since(t0);
        lz_debug_n_capture++;
    }
    return s->logits;
}
}  // namespace

extern "C" float *lz_forward_capture(const LZModel *mm, LZRunState *s, int token, int pos) {
    return forward_one(mm, s, token, pos, true);
}

extern "C" float *lz_forward(const LZModel *mm, LZRunState *s, int token, int pos) {
    return forward_one(mm, s, token, pos, false);
}

namespace {
int batch_capture_dev(DState *d, LZRunState *s, const int *tokens, int n, int pos0) {
    const LZModelConfig &c = d->m->c;
    if (!knobs_ok(c.num_experts_per_token, nullptr, 0)) return 1;
    DevCtl h = ctl_from(s);
    h.pos_scratch = pos0;
    CK(ctl_put(d, h));
    CK(hipMemcpyAsync(d->tokbuf, tokens, sizeof(int) * (size_t)n, hipMemcpyHostToDevice, d->st));
    DWide *w = n >= WIDE_MIN ? wide_get(d->m) : nullptr;
    if (w) {
        // wide chunks of up to WIDE_MAX rows: each one's positions start at
        // pos_scratch, which the chunk's own control write moves along.  A
        // chunk of at least WIDE_SPLIT rows runs as WIDE_PARTS parts, each on
        // its own stream with its own scratch: part p's layer l waits, before
        // its KDA recurrence or attention, for part p - 1's (the state, conv
        // history and K/V rows of the rows before it), so each part's serial
        // recurrence overlaps the other parts' remaining work.
        DModel *dm = const_cast<DModel *>(d->m);
        for (int done = 0; done < n;) {
            const int k = n - done < w->cap ? n - done : w->cap;
            h.pos_scratch = pos0 + done;
            CK(ctl_put(d, h));
            const int kp = ((k + WIDE_PARTS - 1) / WIDE_PARTS + MAX_CHUNK - 1) & ~(MAX_CHUNK - 1);
            if (k >= WIDE_SPLIT && k - (WIDE_PARTS - 1) * kp > MAX_CHUNK && wide_parts(dm, w)) {
                const int L = c.n_layers, E = L + 2;
                hipEvent_t *ev = w->ev.data();             // part p: ev[p * E + l], start E - 2, end E - 1
                CK(hipEventRecord(ev[E - 2], d->st));      // the other streams start after the control write
                // the parts' layers are enqueued in turn (layer 0 of every
                // part, then layer 1, ...), so every stream has work from the
                // start and each wait follows the record it waits for
                for (int l = 0; l < L; l++) {
                    for (int p = 0; p < WIDE_PARTS; p++) {
                        DWide *wp = p ? w->peer[p - 1] : w;
                        hipStream_t sp = p ? w->pst[p - 1] : d->st;
                        const int r0 = p * kp, kr = p + 1 < WIDE_PARTS ? kp : k - r0;
                        if (l == 0) {
                            if (p) CK(hipStreamWaitEvent(sp, ev[E - 2], 0));
                            CK(hipMemcpyAsync(wp->toks, d->tokbuf + done + r0, sizeof(int) * (size_t)kr,
                                              hipMemcpyDeviceToDevice, sp));
                        }
                        const WideItem item{d, 0, kr, pos0 + done + r0};
                        CK(wide_forward(d->m, wp, &item, 1, kr, false,
                                        d->hcap + (size_t)(done + r0) * c.hidden_size, nullptr, sp, r0,
                                        p ? ev + (size_t)(p - 1) * E : nullptr,
                                        p + 1 < WIDE_PARTS ? ev + (size_t)p * E : nullptr, l, l + 1));
                        if (p && l == L - 1) CK(hipEventRecord(ev[(size_t)p * E + E - 1], sp));
                    }
                }
                for (int p = 1; p < WIDE_PARTS; p++) CK(hipStreamWaitEvent(d->st, ev[(size_t)p * E + E - 1], 0));
            } else {
                CK(hipMemcpyAsync(w->toks, d->tokbuf + done, sizeof(int) * (size_t)k, hipMemcpyDeviceToDevice, d->st));
                const WideItem item{d, 0, k, pos0 + done};
                CK(wide_forward(d->m, w, &item, 1, k, false, d->hcap + (size_t)done * c.hidden_size, nullptr, d->st));
            }
            done += k;
            lz_debug_n_chunks++;
        }
        return 0;
    }
    for (int done = 0; done < n;) {
        int k = n - done < MAX_CHUNK ? n - done : MAX_CHUNK;
        CK(forward_chunk(d, d->tokbuf + done, k, &d->ctl->pos_scratch, done, pos0 + done + k - 1,
                         d->hcap + (size_t)done * c.hidden_size, false, nullptr, true));
        done += k;
        lz_debug_n_chunks++;
    }
    return 0;
}
}  // namespace

extern "C" float *lz_forward_batch_capture(const LZModel *mm, LZRunState *s, const int *tokens, int n,
                                           int pos0, float *hidden_out) {
    if (!mm || !s || !s->impl || !tokens || n < 1 || !hidden_out) return nullptr;
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (!tok_ok(c, tokens, n) || pos0 < 0 || pos0 + n > d->seq_len) return nullptr;
    if (batch_capture_dev(d, s, tokens, n, pos0)) return nullptr;
    if (hipMemcpyAsync(hidden_out, d->hcap, sizeof(float) * (size_t)n * c.hidden_size,
                       hipMemcpyDeviceToHost, d->st) || hipStreamSynchronize(d->st))
        return nullptr;
    return s->logits;
}

extern "C" int lz_forward_verify(const LZModel *mm, LZRunState *s, const int *tokens, int n, int pos0) {
    if (!mm || !s || !s->impl || !tokens || n < 1 || n > LZ_BATCH_MAX) return 1;
    if (!Mo(mm)->has_mtp) return 1;               // the verify needs the MTP head (src/forward.c:1780)
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (!tok_ok(c, tokens, n) || pos0 < 0 || pos0 + n > d->seq_len) return 1;
    if (!knobs_ok(c.num_experts_per_token, nullptr, 0)) return 1;
    const timespec t0 = now_ts();
    DevCtl h = ctl_from(s);
    h.pos_scratch = pos0;
    for (int i = 0; i < n; i++) h.tok[i] = tokens[i];
    if (ctl_put(d, h)) return 1;
    if (forward_chunk(d, d->ctl->tok, n, &d->ctl->pos_scratch, 0, pos0 + n - 1, d->vhidden, true,
                      d->mtp_logits, false))
        return 1;
    s->ssm_slot = (s->ssm_slot + n) % d->depth;
    if (hipMemcpyAsync(s->mtp_logits, d->mtp_logits, sizeof(float) * (size_t)n * c.vocab_size,
                       hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_verify_hidden, d->vhidden, sizeof(float) * (size_t)n * c.hidden_size,
                       hipMemcpyDeviceToHost, d->st) ||
        hipStreamSynchronize(d->st))
        return 1;
    lz_debug_n_chunks++;
    lz_debug_n_lmhead++;
    lz_debug_us_verify += us_since(t0);
    return 0;
}

// A DSpark head (mtp_n_draft > 1) binds no mtp.fc (src/model.c:2531-2532):
// lz_mtp_draft_step, lz_mtp_prefill and lz_mtp_catchup refuse it.
extern "C" float *lz_mtp_draft_step(const LZModel *mm, LZRunState *s, int next_token, int pos) {
    if (!mm || !s || !s->impl || !Mo(mm)->has_mtp || Mo(mm)->n_draft > 1) return nullptr;
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (next_token < 0 || next_token >= c.vocab_size || pos < 0 || pos >= d->seq_len) return nullptr;
    if (!knobs_ok(c.num_experts_per_token, nullptr, 0)) return nullptr;
    const timespec t0 = now_ts();
    DevCtl h = ctl_from(s);
    h.pos_scratch = pos;
    h.tok[0] = next_token;
    if (ctl_put(d, h) || chain_put(d, s)) return nullptr;
    if (draft_step(d, d->ctl->tok, &d->ctl->pos_scratch, 0, pos, d->draft_logits, nullptr)) return nullptr;
    if (hipMemcpyAsync(s->mtp_draft_logits, d->draft_logits, sizeof(float) * c.vocab_size,
                       hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st) ||
        hipStreamSynchronize(d->st))
        return nullptr;
    lz_debug_us_draft += us_since(t0);
    return s->mtp_draft_logits;
}

// lz_mtp_draft_batch (src/forward_mtp.c:385-505): the k DSpark slots'
// base logits from s->mtp_chain, into s->mtp_kdraft_logits.
extern "C" float *lz_mtp_draft_batch(const LZModel *mm, LZRunState *s, int next_token, int k) {
    if (!mm || !s || !s->impl || !Mo(mm)->has_mtp || Mo(mm)->n_draft <= 1 || !s->mtp_kdraft_logits) return nullptr;
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (next_token < 0 || next_token >= c.vocab_size || k <= 0 || k > c.mtp_n_draft) return nullptr;
    if (!knobs_ok(c.num_experts_per_token, nullptr, 0)) return nullptr;
    const timespec t0 = now_ts();
    DevCtl h = ctl_from(s);
    h.tok[0] = next_token;
    if (ctl_put(d, h) || chain_put(d, s) || dspark_draft(d, d->ctl->tok, k, d->draft_logits, nullptr) ||
        hipMemcpyAsync(s->mtp_kdraft_logits, d->draft_logits, sizeof(float) * (size_t)k * c.vocab_size,
                       hipMemcpyDeviceToHost, d->st) ||
        hipStreamSynchronize(d->st))
        return nullptr;
    lz_debug_us_draft += us_since(t0);
    return s->mtp_kdraft_logits;
}

// lz_mtp_markov_correct (src/forward_mtp.c:510-531): logits +=
// markov_proj(markov_embed[x_prev]).  A model.bin head's Markov rank is 0
// (its two tensors are [vocab][0]), so the projection is a row of zeros and
// the update adds +0 to each entry, as the reference's lz_matmul over no
// inputs does.
extern "C" void lz_mtp_markov_correct(const LZModel *mm, LZRunState *s, int x_prev, float *logits) {
    (void)s;
    if (!mm || !mm->impl || !Mo(mm)->has_mtp || Mo(mm)->n_draft <= 1 || !logits) return;
    const LZModelConfig &c = Mo(mm)->c;
    if (x_prev < 0 || x_prev >= c.vocab_size) return;
    for (int v = 0; v < c.vocab_size; v++) logits[v] += 0.0f;
}

extern "C" int lz_mtp_prefill(const LZModel *mm, LZRunState *s, const float *h_body_all,
                              const int *next_tokens, int n, int pos0) {
    if (!mm || !s || !s->impl || !h_body_all || !next_tokens || n < 1 || !Mo(mm)->has_mtp || Mo(mm)->n_draft > 1)
        return 1;
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (!tok_ok(c, next_tokens, n) || pos0 < 0 || pos0 + n > d->seq_len || n > d->cap_rows) return 1;
    DevCtl h = ctl_from(s);
    h.pos_scratch = pos0;
    if (ctl_put(d, h)) return 1;
    if (hipMemcpyAsync(d->hcap, h_body_all, sizeof(float) * (size_t)n * c.hidden_size,
                       hipMemcpyHostToDevice, d->st) ||
        hipMemcpyAsync(d->tokbuf, next_tokens, sizeof(int) * (size_t)n, hipMemcpyHostToDevice, d->st))
        return 1;
    if (mtp_prefill_dev(d, d->hcap, d->tokbuf, n, &d->ctl->pos_scratch, 0)) return 1;
    return hipStreamSynchronize(d->st) != hipSuccess;
}

extern "C" int lz_mtp_catchup(const LZModel *m, LZRunState *s, const float *h_body_all,
                              const int *next_tokens, int n, int pos0) {
    const timespec t0 = now_ts();          // src/forward_mtp.c:635-642
    int rc = lz_mtp_prefill(m, s, h_body_all, next_tokens, n, pos0);
    lz_debug_us_catchup += us_since(t0);
    lz_debug_n_catchup++;
    return rc;
}

// ------------------------------------------------- sampling (host side) ---

static uint32_t rng_u32(lz_u64 *st) {          // xorshift64*, src/sampler.c:112-117
    *st ^= *st >> 12;
    *st ^= *st << 25;
    *st ^= *st >> 27;
    return (uint32_t)((*st * 0x2545F4914F6CDD1DULL) >> 32);
}
extern "C" float lz_random_f32(lz_u64 *state) {  // src/sampler.c:118-120
    return (float)(rng_u32(state) >> 8) / 16777216.0f;
}
static uint32_t fkey_h(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
extern "C" int lz_sample_argmax(const float *p, int n) {   // src/sampler.c:121-137
    int bi = 0;
    uint32_t best = fkey_h(p[0]);
    for (int i = 1; i < n; i++) {
        uint32_t k = fkey_h(p[i]);
        if (k > best) { bi = i; best = k; }
    }
    return bi;
}

namespace {
// Host copies of the float-tier exp for the sampler (same body as d_exp).
float h_exp(float x) {
    static float tab[32];
    static bool ready = false;
    if (!ready) { for (int i = 0; i < 32; i++) tab[i] = (float)exp2((double)i / 32.0); ready = true; }
    const float C2 = 0.242844437f, C1 = 0.207425515f, C0 = 0.549730133f;
    const float LOG2E32 = 1.44269504f * 32.0f;
    if (x > 88.0f) return 3.40282347e+38f;
    if (x < -87.3f) return 0.0f;
    float y32 = x * LOG2E32;
    volatile float m = (y32 - 0.5f) + 12582912.0f;
    float mm = m;
    uint32_t u;
    memcpy(&u, &mm, 4);
    int32_t t = (int32_t)(u & 0x007FFFFFu) - 0x00400000;
    int32_t n = t >> 5, idx = t & 31;
    float r = y32 - (float)t;
    float w = 1.0f + r * 0.03125f;
    uint32_t pb = (uint32_t)(n + 127) << 23;
    float p2n;
    memcpy(&p2n, &pb, 4);
    float c = (C2 * w + C1) * w + C0;
    return p2n * (tab[idx] * c);
}
bool topp_active(float topp) { return topp > 0.0f && topp < 1.0f; }
bool penalties_on(const LZSampler *samp) {
    if (!samp) return false;
    const LZSampleParams &p = samp->p;
    if (p.repeat_last_n == 0) return false;
    return p.repetition_penalty != 1.0f || p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f;
}
bool unsupported_sampler(const LZSampler *samp) {
    if (!samp) return false;
    const LZSampleParams &p = samp->p;
    return penalties_on(samp) || (p.topk > 0 && p.topk < samp->vocab_size) || p.minp > 0.0f ||
           p.think_temp_enabled;
}
}  // namespace

extern "C" int lz_argmax_p1(const float *logits, int n, float *out_p) {   // src/sampler.c:139-155
    int bi = 0;
    float bv = logits[0], l = 1.0f;
    for (int i = 1; i < n; i++) {
        float v = logits[i];
        if (v > bv) { l = l * h_exp(bv - v) + 1.0f; bv = v; bi = i; }
        else l += h_exp(v - bv);
    }
    if (out_p) *out_p = (l > 0.0f) ? 1.0f / l : 1.0f;
    return bi;
}

extern "C" void lz_sample_defaults(LZSampleParams *p) {   // src/sampler.c:8-20
    p->temperature = 0.6f; p->temp_think = 0.3f; p->think_temp_enabled = 0;
    p->topp = 0.8f; p->minp = 0.05f; p->minp_llamacpp = 1; p->topk = 20;
    p->presence_penalty = 1.5f; p->frequency_penalty = 0.0f;
    p->repetition_penalty = 1.1f; p->repeat_last_n = 64;
}
extern "C" int lz_sampler_init(LZSampler *s, int vocab_size, const LZSampleParams *p, lz_u64 seed) {
    if (!s || !p || vocab_size <= 0) return 1;
    s->vocab_size = vocab_size;
    s->p = *p;
    s->rng_state = seed ? seed : 1ULL;
    return 0;
}
extern "C" void lz_sampler_free(LZSampler *s) { (void)s; }

// ------------------------------------------------------- acceptance ---

extern "C" int lz_spec_accept(const int *draft, const int *targ, int n_draft, int bonus, int *out) {
    if (!draft || !targ || !out || n_draft < 0) return 0;      // src/generate.c:232-243
    for (int i = 0; i < n_draft; i++) {
        out[i] = targ[i];
        if (draft[i] != targ[i]) return i;
    }
    out[n_draft] = bonus;
    return n_draft;
}

extern "C" int lz_spec_accept_temp(const float *p, const float *q, int x, int vocab, float u,
                                   lz_u64 *rng, int *out_accepted) {
    if (!p || !q || !rng || vocab <= 0 || x < 0 || x >= vocab) {   // src/generate.c:283-346
        if (out_accepted) *out_accepted = 0;
        return -1;
    }
    // the host rows go to the device and through the round's acceptance
    // kernel (with this u); the generator state comes back.  The staging
    // (both rows, the generator state, the result) persists per device and
    // grows only when a larger vocabulary arrives, so a call allocates
    // nothing once a vocabulary has been seen (the reference's function is
    // not reentrant either; the lock keeps concurrent callers apart).
    static std::mutex mu;
    static char *stage[64] = {};
    static size_t cap[64] = {};
    std::lock_guard<std::mutex> lock(mu);
    int dev = 0, res[2] = {-1, 0}, rc = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) rc = 1;
    const size_t need = 2 * sizeof(float) * (size_t)vocab + 256;
    if (!rc && cap[dev] < need) {
        if (stage[dev]) (void)hipFree(stage[dev]);
        stage[dev] = nullptr;
        cap[dev] = 0;
        if (hipMalloc(&stage[dev], need) != hipSuccess) rc = 1;
        else cap[dev] = need;
    }
    float *dp = rc ? nullptr : reinterpret_cast<float *>(stage[dev]), *dq = dp ? dp + vocab : nullptr;
    unsigned long long *drng = dq ? reinterpret_cast<unsigned long long *>(dq + vocab) : nullptr;
    int *dout = drng ? reinterpret_cast<int *>(drng + 1) : nullptr;
    if (!rc && (hipMemcpy(dp, p, sizeof(float) * (size_t)vocab, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(dq, q, sizeof(float) * (size_t)vocab, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(drng, rng, sizeof(*drng), hipMemcpyHostToDevice) != hipSuccess))
        rc = 1;
    if (!rc && l98k_smp_accept(dp, dq, vocab, x, &u, drng, dout, nullptr)) rc = 1;
    if (!rc && (hipMemcpy(res, dout, sizeof(res), hipMemcpyDeviceToHost) != hipSuccess ||
                hipMemcpy(rng, drng, sizeof(*drng), hipMemcpyDeviceToHost) != hipSuccess))
        rc = 1;
    if (rc) {
        if (out_accepted) *out_accepted = 0;
        return -1;
    }
    if (out_accepted) *out_accepted = res[1];
    return res[0];
}

// ------------------------------------------- no-allocation acceptance ---
// l98_spec_accept_temp_noalloc: lz_spec_accept_temp on host rows with its
// device staging (the two rows, the generator state and the result) in a
// file-scope device array instead of hipMalloc'd buffers, for callers that
// cannot allocate.  Each GPU holds its own copy of the array until the
// process ends; its address on a device is taken once, with that device
// current (the array's name is only a host-side stand-in).  Every call on a
// device shares the array, so calls that overlap on one device race.

#define NOALLOC_MAX_VOCAB L98_NOALLOC_MAX_VOCAB
#define NOALLOC_MAX_DEVICES 64
static __device__ __align__(256) unsigned char scratch[2 * sizeof(float) * NOALLOC_MAX_VOCAB + 256];
static char *g_scratch_ptr[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

// The array's address on the current device (taken on the first call there).
static char *scratch_on_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_ptr[dev] = (char *)ptr;
    }
    return g_scratch_ptr[dev];
}

extern "C" int l98_spec_accept_temp_noalloc(const float *p, const float *q, int x, int vocab, float u, lz_u64 *rng,
                                            int *out_accepted) {
    if (out_accepted) *out_accepted = 0;
    if (!p || !q || !rng || vocab <= 0 || x < 0 || x >= vocab) return -1;   // as src/generate.c:283-346
    if (vocab > NOALLOC_MAX_VOCAB) {
        fprintf(stderr, "l98_spec_accept_temp_noalloc: vocab %d exceeds the static staging of %d\n", vocab,
                NOALLOC_MAX_VOCAB);
        return -2;
    }
    char *base = scratch_on_current_device();
    if (!base) return -3;
    float *dp = (float *)base, *dq = dp + NOALLOC_MAX_VOCAB;
    unsigned long long *drng = (unsigned long long *)(dq + NOALLOC_MAX_VOCAB);
    int *dout = (int *)(drng + 2);
    int res[2] = {-1, 0};
    // the kernel reads rows [0, vocab) only and writes both result words on
    // every path, so nothing in the array needs clearing
    if (hipMemcpy(dp, p, sizeof(float) * (size_t)vocab, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dq, q, sizeof(float) * (size_t)vocab, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(drng, rng, sizeof(*drng), hipMemcpyHostToDevice) != hipSuccess ||
        l98k_smp_accept(dp, dq, vocab, x, &u, drng, dout, nullptr) != 0 ||
        hipMemcpy(res, dout, sizeof(res), hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(rng, drng, sizeof(*drng), hipMemcpyDeviceToHost) != hipSuccess)
        return -3;
    if (out_accepted) *out_accepted = res[1];
    return res[0];
}

// ------------------------------------------------------------- rounds ---

namespace {

// Enqueues one greedy round on the device: k draft steps (argmax into
// ctl->tok), the (k+1)-token verify, the per-row argmaxes, acceptance with
// ring rollback and chain reseed, the MTP catch-up of the accepted drafts
// (always k-1 rows, see k_accept), then the round record and the advance to
// the next round.  Reads nothing back; every scalar lives in ctl, so the
// sequence is graph-capturable.
int enqueue_verify_accept(DState *d, int k_eff, int max_pos, int brk, bool catchup, hipEvent_t mark = nullptr) {
    const LZModelConfig &c = d->m->c;
    const bool dspark = d->m->n_draft > 1;     // no catch-up, mtp_pos kept (src/generate.c:1117-1133)
    {
        AmaxScope amax(d, d->ctl->targ, 0);   // the verify rows' argmaxes in the lm_head's epilogue
        CK(forward_chunk(d, d->ctl->tok, k_eff + 1, &d->ctl->anchor_pos, 1, max_pos, d->vhidden, true,
                         d->mtp_logits, false));
    }
    CK(l98k_accept(d->ctl, d->vhidden, c.hidden_size, d->chain, d->depth, (brk ? 1 : 0) | (dspark ? 2 : 0), d->st));
    if (dspark) catchup = false;
    if (mark) CK(hipEventRecord(mark, d->st));
    if (catchup && k_eff > 1)
        CK(mtp_prefill_dev(d, d->vhidden, d->ctl->catch_tok, k_eff - 1, &d->ctl->catch_pos, 0));
    CK(l98k_set_tokens(d->ctl, 1, d->hist, d->hist_cap, d->st));
    return 0;
}

int enqueue_greedy_round(DState *d, int k, int max_pos, int brk, bool catchup) {
    const LZModelConfig &c = d->m->c;
    if (d->m->n_draft > 1) {      // lz_spec_round_dspark: one draft batch of k slots
        CK(dspark_draft(d, d->ctl->tok, k, d->draft_logits, d->ctl->tok + 1));
        return enqueue_verify_accept(d, k, max_pos, brk, false);
    }
    for (int i = 0; i < k; i++)
        CK(draft_step(d, d->ctl->tok + i, &d->ctl->mtp_pos, i, max_pos, d->draft_logits + (size_t)i * c.vocab_size,
                      d->ctl->tok + 1 + i));
    return enqueue_verify_accept(d, k, max_pos, brk, catchup);
}

int errset(char *errbuf, int errlen, int code, const char *msg) {
    set_err(errbuf, errlen, "%s", msg);
    return -code;
}

}  // namespace

extern "C" int lz_spec_round(const LZModel *mm, LZRunState *s, int anchor, int anchor_pos, int k,
                             float p_min, int n_min, const LZSampler *samp, int brk, int skipc,
                             int *out, int *out_n_accept, int *out_new_pos, int *out_k_eff,
                             char *errbuf, int errlen) {
    if (!mm || !s || !out || !out_n_accept || !out_new_pos || !out_k_eff || !s->impl)
        return errset(errbuf, errlen, LZ_ERR_NULL_ARG, "null argument");
    if (!Mo(mm)->has_mtp) return errset(errbuf, errlen, LZ_ERR_SPEC_NO_HEAD, "model has no MTP head");
    if (Mo(mm)->n_draft > 1)
        return errset(errbuf, errlen, LZ_ERR_FORWARD, "a DSpark head (mtp_n_draft > 1) runs lz_spec_round_dspark");
    if (k < 1 || k > LZ_SPEC_K_MAX || k > s->ssm_ring_depth - 1) {
        set_err(errbuf, errlen, "spec_k %d out of range 1..%d", k,
                k > LZ_SPEC_K_MAX ? LZ_SPEC_K_MAX : s->ssm_ring_depth - 1);
        return -LZ_ERR_SPEC_K_RANGE;
    }
    if (penalties_on(samp)) return errset(errbuf, errlen, LZ_ERR_NULL_ARG, "sampler penalties are not on this path");
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (!knobs_ok(c.num_experts_per_token, errbuf, errlen)) return -LZ_ERR_FORWARD;
    if (anchor < 0 || anchor >= c.vocab_size || anchor_pos + 1 + k >= d->seq_len ||
        s->mtp_pos + k > d->seq_len)
        return errset(errbuf, errlen, LZ_ERR_FORWARD, "forward failed (token/position out of range)");
    const int max_pos = d->seq_len - 1;
    DevCtl h = ctl_from(s);
    h.anchor = anchor;
    h.anchor_pos = anchor_pos;
    h.tok[0] = anchor;
    h.k_eff = k;
    if (ctl_put(d, h) || chain_put(d, s)) return -LZ_ERR_FORWARD;
    // phase marks for the reference's draft / verify / catch-up timers
    if (hipEventRecord(d->ph[0], d->st)) return -LZ_ERR_FORWARD;
    int k_eff = k;
    if (p_min > 0.0f || k_eff < n_min) {
        // The draft loop decides k_eff on the host: p_min needs each step's
        // top-1 probability before the next step (lz_argmax_p1's online
        // softmax, run on the host copy of the logits).
        std::vector<float> lg(c.vocab_size);
        k_eff = 0;
        for (int i = 0; i < k; i++) {
            if (draft_step(d, d->ctl->tok + i, &d->ctl->mtp_pos, i, max_pos, d->draft_logits,
                           d->ctl->tok + 1 + i))
                return -LZ_ERR_FORWARD;
            if (p_min > 0.0f) {
                if (hipMemcpyAsync(lg.data(), d->draft_logits, sizeof(float) * c.vocab_size,
                                   hipMemcpyDeviceToHost, d->st) || hipStreamSynchronize(d->st))
                    return -LZ_ERR_FORWARD;
                float p1;
                (void)lz_argmax_p1(lg.data(), c.vocab_size, &p1);
                if (p1 < p_min) break;
            }
            k_eff = i + 1;
        }
        if (k_eff < n_min) {
            // discard: the draft steps ran and overwrote the chain, which
            // the reference leaves in s->mtp_chain
            if (hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost,
                               d->st) ||
                hipMemcpyAsync(s->mtp_draft_logits, d->draft_logits, sizeof(float) * c.vocab_size,
                               hipMemcpyDeviceToHost, d->st) ||
                hipStreamSynchronize(d->st))
                return -LZ_ERR_FORWARD;
            out[0] = anchor; *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
            return 0;
        }
        int ke = k_eff;
        if (hipEventRecord(d->ph[1], d->st) ||
            hipMemcpyAsync(&d->ctl->k_eff, &ke, sizeof(int), hipMemcpyHostToDevice, d->st) ||
            enqueue_verify_accept(d, k_eff, max_pos, brk, !skipc, d->ph[2]))
            return -LZ_ERR_FORWARD;
    } else {
        for (int i = 0; i < k; i++)
            if (draft_step(d, d->ctl->tok + i, &d->ctl->mtp_pos, i, max_pos, d->draft_logits + (size_t)i * c.vocab_size,
                           d->ctl->tok + 1 + i))
                return -LZ_ERR_FORWARD;
        if (hipEventRecord(d->ph[1], d->st) || enqueue_verify_accept(d, k, max_pos, brk, !skipc, d->ph[2]))
            return -LZ_ERR_FORWARD;
    }
    if (hipEventRecord(d->ph[3], d->st)) return -LZ_ERR_FORWARD;
    // the fields the reference's round leaves for its caller (the reseeded
    // mtp_chain, the verify logits and hidden rows, the last draft step's
    // logits) ride on the same sync as ctl
    const float *last_draft = (p_min > 0.0f || k < n_min) ? d->draft_logits
                                                          : d->draft_logits + (size_t)(k - 1) * c.vocab_size;
    if (hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_logits, d->mtp_logits, sizeof(float) * (size_t)(k_eff + 1) * c.vocab_size,
                       hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_verify_hidden, d->vhidden, sizeof(float) * (size_t)(k_eff + 1) * c.hidden_size,
                       hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_draft_logits, last_draft, sizeof(float) * c.vocab_size, hipMemcpyDeviceToHost,
                       d->st))
        return -LZ_ERR_FORWARD;
    if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
    int n_accept = h.n_accept;
    for (int i = 0; i <= n_accept; i++) out[i] = h.out[i];
    s->ssm_slot = h.ssm_slot;
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    s->mtp_pos += n_accept;
    // the reference's counters (src/generate.c:826, src/forward_mtp.c:639-640,
    // src/forward.c:86-88): device time between the phase marks
    {
        float ms[3] = {0, 0, 0};
        for (int i = 0; i < 3; i++) (void)hipEventElapsedTime(&ms[i], d->ph[i], d->ph[i + 1]);
        lz_debug_us_draft += (long long)(ms[0] * 1000.0f);
        lz_debug_us_verify += (long long)(ms[1] * 1000.0f);
        lz_debug_n_chunks++;
        lz_debug_n_lmhead++;
        if (n_accept < k_eff) lz_debug_n_ring_rollback++;
        if (n_accept > 1 && !skipc) {
            lz_debug_us_catchup += (long long)(ms[2] * 1000.0f);
            lz_debug_n_catchup++;
        }
    }
    return n_accept + 1;
}

namespace {

// The temperature sampling scratch of a state, carved from one allocation
// on first use: the round's draft distributions, a target distribution, the
// softmax and the top-p candidate keys/indices (sorted copies too), the
// sort's scratch, the generator state and small results.
bool smp_ensure(DState *d) {
    if (d->smp_arena) return true;
    const size_t V = (size_t)d->m->c.vocab_size;
    const size_t tmp = l98k_smp_sort_tmp_bytes((int)V);
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t a = off; off = (off + bytes + 255) & ~(size_t)255; return a; };
    const size_t oq = take(sizeof(float) * V * L98_SPEC_K_GPU), op = take(sizeof(float) * V),
                 opr = take(sizeof(float) * V), ok = take(4 * V), osk = take(4 * V),
                 osv = take(4 * V), ot = take(tmp), orng = take(8), oo = take(64), oof = take(64);
    char *a = nullptr;
    if (hipMalloc(&a, off) != hipSuccess) return false;
    d->smp_arena = a;
    d->smp_q = (float *)(a + oq);
    d->smp_p = (float *)(a + op);
    d->smp_probs = (float *)(a + opr);
    d->smp_keys = (uint32_t *)(a + ok);
    d->smp_skeys = (uint32_t *)(a + osk);
    d->smp_svals = (int *)(a + osv);
    d->smp_tmp = a + ot;
    d->smp_tmp_bytes = tmp;
    d->smp_rng = (unsigned long long *)(a + orng);
    d->smp_out = (int *)(a + oo);
    d->smp_outf = (float *)(a + oof);
    return true;
}

// lz_target_dist (top-k and min-p off, src/sampler.c:682-730) of a device
// logits row into d->smp_p: softmax(row / T), then with top-p the
// candidates >= (1 - top_p) / (V - 1) sorted by probability (stable), the
// prefix up to the first cumulative mass >= top_p renormalized.
// skip: a device flag (null: never) that turns every launch into a no-op.
int dev_target_dist(DState *d, const float *row, int V, float temp, float topp, const int *skip = nullptr) {
    const float inv = 1.0f / temp;
    if (!topp_active(topp)) return l98k_smp_softmax(row, V, inv, d->smp_p, 0.0f, nullptr, nullptr, skip, d->st);
    const float cutoff = (V > 1) ? (1.0f - topp) / (float)(V - 1) : 0.0f;
    if (l98k_smp_softmax(row, V, inv, d->smp_probs, cutoff, d->smp_keys, d->smp_out + 8, skip, d->st) ||
        l98k_smp_sort_desc(d->smp_keys, d->smp_skeys, d->smp_svals, V, d->smp_tmp, skip, d->st))
        return 1;
    return l98k_smp_topp_dist(d->smp_probs, V, d->smp_skeys, d->smp_svals, d->smp_out + 8, topp, d->smp_p, skip,
                              d->st);
}

// lz_sample_ex for temperature > 0 (src/sampler.c:794-840) on a device
// logits row; the generator state round-trips through the device.
int dev_sample_ex(DState *d, const float *row, int V, float temp, float topp, lz_u64 *rng, int *tok) {
    if (!smp_ensure(d)) return 1;
    const float inv = 1.0f / temp;
    if (hipMemcpyAsync(d->smp_rng, rng, sizeof(lz_u64), hipMemcpyHostToDevice, d->st)) return 1;
    if (!topp_active(topp)) {
        if (l98k_smp_softmax(row, V, inv, d->smp_probs, 0.0f, nullptr, nullptr, nullptr, d->st) ||
            l98k_smp_draw(d->smp_probs, V, d->smp_rng, d->smp_out, nullptr, nullptr, nullptr, d->st))
            return 1;
    } else {
        const float cutoff = (V > 1) ? (1.0f - topp) / (float)(V - 1) : 0.0f;
        if (l98k_smp_softmax(row, V, inv, d->smp_probs, cutoff, d->smp_keys, d->smp_out + 8, nullptr, d->st) ||
            l98k_smp_sort_desc(d->smp_keys, d->smp_skeys, d->smp_svals, V, d->smp_tmp, nullptr, d->st) ||
            l98k_smp_sample_topp(d->smp_probs, V, d->smp_skeys, d->smp_svals, d->smp_out + 8, topp, d->smp_rng,
                                 d->smp_out, d->st))
            return 1;
    }
    if (hipMemcpyAsync(tok, d->smp_out, sizeof(int), hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(rng, d->smp_rng, sizeof(lz_u64), hipMemcpyDeviceToHost, d->st) || hipStreamSynchronize(d->st))
        return 1;
    return 0;
}

// One temperature round on the device: lz_spec_round_temp with p_min = 0,
// n_min = 0 and the one-slot head (src/generate.c:1234-1377).  k chained
// draft steps, each q_i = softmax(logits/T) and a draw into ctl->tok[1+i]
// (lz_sample_temp_q, src/sampler.c:736-747); the (k+1)-row verify; per
// row i the target distribution (lz_target_dist) and the acceptance test
// with residual resampling, which on a rejection records n_accept = i and
// sets ctl->smp_done, after which every sampling launch of the round does
// nothing (the reference's loop stops there, drawing nothing more); the
// bonus draw from row k when no row rejected; then the ring rollback, chain
// reseed, catch-up and round record of the greedy round.  Every scalar
// lives in ctl and the generator state in device memory, so the sequence
// is graph-capturable.
int enqueue_temp_round(DState *d, int k, int max_pos, float temp, float topp) {
    const LZModelConfig &c = d->m->c;
    const int V = c.vocab_size;
    const float inv = 1.0f / temp;
    for (int i = 0; i < k; i++) {
        float *qi = d->smp_q + (size_t)i * V;
        CK(draft_step(d, d->ctl->tok + i, &d->ctl->mtp_pos, i, max_pos, d->draft_logits, nullptr));
        CK(l98k_smp_softmax(d->draft_logits, V, inv, qi, 0.0f, nullptr, nullptr, nullptr, d->st));
        CK(l98k_smp_draw(qi, V, d->smp_rng, d->smp_out, d->smp_outf, d->ctl->tok + 1 + i, nullptr, d->st));
    }
    CK(forward_chunk(d, d->ctl->tok, k + 1, &d->ctl->anchor_pos, 1, max_pos, d->vhidden, true, d->mtp_logits,
                     false));
    CK(l98k_set_tokens(d->ctl, 2, nullptr, 0, d->st));
    const int *done = &d->ctl->smp_done;
    for (int i = 0; i < k; i++) {
        CK(dev_target_dist(d, d->mtp_logits + (size_t)i * V, V, temp, topp, done));
        CK(l98k_smp_accept_row(d->smp_p, d->smp_q + (size_t)i * V, V, d->ctl->tok + 1 + i, d->smp_rng,
                               d->ctl->out + i, &d->ctl->n_accept, &d->ctl->smp_done, i, d->st));
    }
    CK(dev_target_dist(d, d->mtp_logits + (size_t)k * V, V, temp, topp, done));
    CK(l98k_smp_draw(d->smp_p, V, d->smp_rng, d->smp_out, nullptr, d->ctl->out + k, done, d->st));
    CK(l98k_accept(d->ctl, d->vhidden, c.hidden_size, d->chain, d->depth, 4, d->st));
    if (k > 1) CK(mtp_prefill_dev(d, d->vhidden, d->ctl->catch_tok, k - 1, &d->ctl->catch_pos, 0));
    CK(l98k_set_tokens(d->ctl, 1, d->hist, d->hist_cap, d->st));
    return 0;
}

}  // namespace

// lz_spec_round_dspark (greedy, penalties off), src/generate.c:1000-1133:
// one draft batch of k slots, each slot's Markov correction (a zero row)
// and lz_argmax_p1 in slot order with the p_min cut, the verify, acceptance,
// ring rollback and the chain reseed.  No catch-up, mtp_pos unchanged.  With
// p_min = 0 and n_min <= k the round stays on the device as one sequence.
extern "C" int lz_spec_round_dspark(const LZModel *mm, LZRunState *s, int anchor, int anchor_pos, int k,
                                    float p_min, int n_min, const LZSampler *samp, int brk, int *out,
                                    int *out_n_accept, int *out_new_pos, int *out_k_eff, char *errbuf,
                                    int errlen) {
    if (!mm || !s || !out || !out_n_accept || !out_new_pos || !out_k_eff || !s->impl)
        return errset(errbuf, errlen, LZ_ERR_NULL_ARG, "null argument");
    if (!Mo(mm)->has_mtp) return errset(errbuf, errlen, LZ_ERR_SPEC_NO_HEAD, "model has no MTP head");
    const int nd = Mo(mm)->n_draft;
    if (k < 1 || k > LZ_SPEC_K_MAX || k > s->ssm_ring_depth - 1 || k > nd) {
        const int lim = k > LZ_SPEC_K_MAX ? LZ_SPEC_K_MAX : k > s->ssm_ring_depth - 1 ? s->ssm_ring_depth - 1 : nd;
        set_err(errbuf, errlen, "spec_k %d out of range 1..%d", k, lim);
        return -LZ_ERR_SPEC_K_RANGE;
    }
    if (nd <= 1 || !s->mtp_kdraft_logits) return errset(errbuf, errlen, LZ_ERR_FORWARD, "not a DSpark head");
    if (penalties_on(samp)) return errset(errbuf, errlen, LZ_ERR_NULL_ARG, "sampler penalties are not on this path");
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    const int V = c.vocab_size;
    if (!knobs_ok(c.num_experts_per_token, errbuf, errlen)) return -LZ_ERR_FORWARD;
    if (anchor < 0 || anchor >= V || anchor_pos + 1 + k >= d->seq_len)
        return errset(errbuf, errlen, LZ_ERR_FORWARD, "forward failed (token/position out of range)");
    const int max_pos = d->seq_len - 1;
    DevCtl h = ctl_from(s);
    h.anchor = anchor;
    h.anchor_pos = anchor_pos;
    h.tok[0] = anchor;
    h.k_eff = k;
    if (ctl_put(d, h) || chain_put(d, s) || hipEventRecord(d->ph[0], d->st)) return -LZ_ERR_FORWARD;
    if (dspark_draft(d, d->ctl->tok, k, d->draft_logits, d->ctl->tok + 1)) return -LZ_ERR_FORWARD;
    int k_eff = k;
    if (p_min > 0.0f || k < n_min) {
        // the cut needs each slot's top-1 probability (lz_argmax_p1's online
        // softmax) on the host copy of the rows
        if (hipMemcpyAsync(s->mtp_kdraft_logits, d->draft_logits, sizeof(float) * (size_t)k * V,
                           hipMemcpyDeviceToHost, d->st) || hipStreamSynchronize(d->st))
            return -LZ_ERR_FORWARD;
        k_eff = 0;
        int prev = anchor;
        for (int i = 0; i < k; i++) {
            float *row = s->mtp_kdraft_logits + (size_t)i * V, p1;
            lz_mtp_markov_correct(mm, s, prev, row);
            prev = lz_argmax_p1(row, V, &p1);
            if (p1 < p_min) break;
            k_eff = i + 1;
        }
        if (k_eff < n_min) {     // discard; the draft batch left the chain as it was
            out[0] = anchor; *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
            return 0;
        }
        const int ke = k_eff;
        if (hipMemcpyAsync(&d->ctl->k_eff, &ke, sizeof(int), hipMemcpyHostToDevice, d->st)) return -LZ_ERR_FORWARD;
    }
    if (hipEventRecord(d->ph[1], d->st) || enqueue_verify_accept(d, k_eff, max_pos, brk, false) ||
        hipEventRecord(d->ph[2], d->st))
        return -LZ_ERR_FORWARD;
    if (hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_logits, d->mtp_logits, sizeof(float) * (size_t)(k_eff + 1) * V,
                       hipMemcpyDeviceToHost, d->st) ||
        hipMemcpyAsync(s->mtp_verify_hidden, d->vhidden, sizeof(float) * (size_t)(k_eff + 1) * c.hidden_size,
                       hipMemcpyDeviceToHost, d->st) ||
        (p_min <= 0.0f && k >= n_min &&
         hipMemcpyAsync(s->mtp_kdraft_logits, d->draft_logits, sizeof(float) * (size_t)k * V, hipMemcpyDeviceToHost,
                        d->st)))
        return -LZ_ERR_FORWARD;
    if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
    const int n_accept = h.n_accept;
    for (int i = 0; i <= n_accept; i++) out[i] = h.out[i];
    s->ssm_slot = h.ssm_slot;
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    {
        float ms[2] = {0, 0};
        for (int i = 0; i < 2; i++) (void)hipEventElapsedTime(&ms[i], d->ph[i], d->ph[i + 1]);
        lz_debug_us_draft += (long long)(ms[0] * 1000.0f);
        lz_debug_us_verify += (long long)(ms[1] * 1000.0f);
        lz_debug_n_chunks++;
        lz_debug_n_lmhead++;
        if (n_accept < k_eff) lz_debug_n_ring_rollback++;
    }
    return n_accept + 1;
}

namespace {
// lz_spec_round_temp with the draft width bounded by k_cap: LZ_SPEC_K_MAX
// for the reference entry point, L98_SPEC_K_GPU for this library's own
// generation loop.  A DSpark head (mtp_n_draft > 1) takes
// lz_spec_round_dspark_temp's form (src/generate.c:1382-1505): one draft
// batch of k <= mtp_n_draft slots, each slot's corrected row sampled in
// turn, no catch-up and no mtp_pos advance.
int spec_round_temp(const LZModel *mm, LZRunState *s, int anchor, int anchor_pos, int k, float p_min, int n_min,
                    LZSampler *samp, int brk, int skipc, int *out, int *out_n_accept, int *out_new_pos,
                    int *out_k_eff, char *errbuf, int errlen, int k_cap) {
    if (!mm || !s || !samp || !out || !out_n_accept || !out_new_pos || !out_k_eff || !s->impl)
        return errset(errbuf, errlen, LZ_ERR_NULL_ARG, "null argument");
    if (!Mo(mm)->has_mtp) return errset(errbuf, errlen, LZ_ERR_SPEC_NO_HEAD, "model has no MTP head");
    const bool ds = Mo(mm)->n_draft > 1;
    if (ds && Mo(mm)->n_draft < k_cap) k_cap = Mo(mm)->n_draft;
    if (k < 1 || k > k_cap || k > s->ssm_ring_depth - 1) {
        set_err(errbuf, errlen, "spec_k %d out of range 1..%d", k, k > k_cap ? k_cap : s->ssm_ring_depth - 1);
        return -LZ_ERR_SPEC_K_RANGE;
    }
    if (unsupported_sampler(samp))
        return errset(errbuf, errlen, LZ_ERR_NULL_ARG, "sampler option not on this path");
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    const int V = c.vocab_size;
    if (!knobs_ok(c.num_experts_per_token, errbuf, errlen)) return -LZ_ERR_FORWARD;
    timespec t0 = now_ts();
    if (anchor < 0 || anchor >= V || anchor_pos + 1 + k >= d->seq_len || (!ds && s->mtp_pos + k > d->seq_len))
        return errset(errbuf, errlen, LZ_ERR_FORWARD, "forward failed (token/position out of range)");
    const float temp = samp->p.temperature, topp = samp->p.topp;
    DevCtl h = ctl_from(s);
    h.anchor = anchor; h.anchor_pos = anchor_pos; h.tok[0] = anchor;
    if (ctl_put(d, h) || chain_put(d, s)) return -LZ_ERR_FORWARD;
    if (!smp_ensure(d) ||
        hipMemcpyAsync(d->smp_rng, &samp->rng_state, sizeof(lz_u64), hipMemcpyHostToDevice, d->st))
        return -LZ_ERR_FORWARD;
    int draft[L98_SPEC_K_GPU], k_eff = 0;
    const float inv = 1.0f / temp;
    // the DSpark rows' Markov correction adds a zero row: nothing to apply
    if (ds && dspark_draft(d, d->ctl->tok, k, d->draft_logits, nullptr)) return -LZ_ERR_FORWARD;
    for (int i = 0; i < k; i++) {
        if (!ds && draft_step(d, d->ctl->tok + i, &d->ctl->mtp_pos, i, s->mtp_pos + k, d->draft_logits, nullptr))
            return -LZ_ERR_FORWARD;
        const float *row = d->draft_logits + (ds ? (size_t)i * V : 0);
        // lz_sample_temp_q (src/sampler.c:736-747): q = softmax(logits/T),
        // then the multinomial draw; the draw also becomes the next draft
        // step's input token
        float *qi = d->smp_q + (size_t)i * V;
        int idx = 0;
        float qidx = 0.0f;
        if (l98k_smp_softmax(row, V, inv, qi, 0.0f, nullptr, nullptr, nullptr, d->st) ||
            l98k_smp_draw(qi, V, d->smp_rng, d->smp_out, d->smp_outf, d->ctl->tok + 1 + i, nullptr, d->st) ||
            hipMemcpyAsync(&idx, d->smp_out, sizeof(int), hipMemcpyDeviceToHost, d->st) ||
            hipMemcpyAsync(&qidx, d->smp_outf, sizeof(float), hipMemcpyDeviceToHost, d->st) ||
            hipStreamSynchronize(d->st))
            return -LZ_ERR_FORWARD;
        if (qidx < p_min) break;
        draft[i] = idx;
        h.tok[1 + i] = idx;
        k_eff = i + 1;
    }
    if (k_eff < n_min) {
        if (hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st) ||
            hipStreamSynchronize(d->st))
            return -LZ_ERR_FORWARD;
        out[0] = anchor; *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
        return 0;
    }
    lz_debug_us_draft += us_since(t0);
    t0 = now_ts();
    int base = s->ssm_slot;
    if (forward_chunk(d, d->ctl->tok, k_eff + 1, &d->ctl->anchor_pos, 1, anchor_pos + k_eff + 1,
                      d->vhidden, true, d->mtp_logits, false))
        return -LZ_ERR_FORWARD;
    lz_debug_n_chunks++;
    lz_debug_n_lmhead++;
    // acceptance on the device (lz_spec_accept_temp, src/generate.c:283-346):
    // the target distribution of each verify row, then u, then the residual
    // draw on a rejection; the bonus draw when every draft is accepted
    int n_accept = k_eff;
    for (int i = 0; i < k_eff; i++) {
        int res[2] = {0, 0};
        if (dev_target_dist(d, d->mtp_logits + (size_t)i * V, V, temp, topp) ||
            l98k_smp_accept(d->smp_p, d->smp_q + (size_t)i * V, V, draft[i], nullptr, d->smp_rng, d->smp_out, d->st) ||
            hipMemcpyAsync(res, d->smp_out, sizeof(res), hipMemcpyDeviceToHost, d->st) || hipStreamSynchronize(d->st))
            return -LZ_ERR_FORWARD;
        out[i] = res[0];
        if (!res[1]) { n_accept = i; break; }
    }
    if (n_accept == k_eff) {
        if (dev_target_dist(d, d->mtp_logits + (size_t)k_eff * V, V, temp, topp) ||
            l98k_smp_draw(d->smp_p, V, d->smp_rng, d->smp_out, nullptr, nullptr, nullptr, d->st) ||
            hipMemcpyAsync(out + k_eff, d->smp_out, sizeof(int), hipMemcpyDeviceToHost, d->st))
            return -LZ_ERR_FORWARD;
    }
    if (hipMemcpyAsync(&samp->rng_state, d->smp_rng, sizeof(lz_u64), hipMemcpyDeviceToHost, d->st) ||
        hipStreamSynchronize(d->st))
        return -LZ_ERR_FORWARD;
    lz_debug_us_verify += us_since(t0);
    s->ssm_slot = (base + k_eff + 1) % d->depth;
    if (n_accept < k_eff) lz_debug_n_ring_rollback++;
    if (n_accept < k_eff && !brk) s->ssm_slot = (base + n_accept + 1) % d->depth;
    // reseed the chain from the accepted row; catch-up
    if (hipMemcpyAsync(d->chain, d->vhidden + (size_t)n_accept * c.hidden_size, sizeof(float) * c.hidden_size,
                       hipMemcpyDeviceToDevice, d->st))
        return -LZ_ERR_FORWARD;
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    if (ds) {
        if (hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st) ||
            hipStreamSynchronize(d->st))
            return -LZ_ERR_FORWARD;
        return n_accept + 1;
    }
    if (n_accept > 1 && !skipc) {
        t0 = now_ts();
        DevCtl h2 = h;
        h2.pos_scratch = s->mtp_pos + 1;
        for (int i = 0; i <= n_accept; i++) h2.out[i] = out[i];
        if (ctl_put(d, h2) ||
            mtp_prefill_dev(d, d->vhidden, d->ctl->out, n_accept - 1, &d->ctl->pos_scratch, 0) ||
            hipStreamSynchronize(d->st))
            return -LZ_ERR_FORWARD;
        lz_debug_us_catchup += us_since(t0);
        lz_debug_n_catchup++;
    }
    if (hipMemcpyAsync(s->mtp_chain, d->chain, sizeof(float) * c.hidden_size, hipMemcpyDeviceToHost, d->st) ||
        hipStreamSynchronize(d->st))
        return -LZ_ERR_FORWARD;
    s->mtp_pos += n_accept;
    return n_accept + 1;
}
}  // namespace

extern "C" int lz_spec_round_temp(const LZModel *mm, LZRunState *s, int anchor, int anchor_pos, int k,
                                  float p_min, int n_min, LZSampler *samp, int brk, int skipc,
                                  int *out, int *out_n_accept, int *out_new_pos, int *out_k_eff,
                                  char *errbuf, int errlen) {
    if (mm && mm->impl && Mo(mm)->n_draft > 1)
        return errset(errbuf, errlen, LZ_ERR_FORWARD, "a DSpark head (mtp_n_draft > 1) runs lz_spec_round_dspark_temp");
    return spec_round_temp(mm, s, anchor, anchor_pos, k, p_min, n_min, samp, brk, skipc, out, out_n_accept,
                           out_new_pos, out_k_eff, errbuf, errlen, LZ_SPEC_K_MAX);
}

// lz_spec_round_dspark_temp (penalties off), src/generate.c:1382-1505.
extern "C" int lz_spec_round_dspark_temp(const LZModel *mm, LZRunState *s, int anchor, int anchor_pos, int k,
                                         float p_min, int n_min, LZSampler *samp, int brk, int *out,
                                         int *out_n_accept, int *out_new_pos, int *out_k_eff, char *errbuf,
                                         int errlen) {
    if (mm && mm->impl && Mo(mm)->has_mtp && Mo(mm)->n_draft <= 1)
        return errset(errbuf, errlen, LZ_ERR_FORWARD, "not a DSpark head");
    if (mm && mm->impl && Mo(mm)->n_draft > 1 && k > Mo(mm)->n_draft && k <= LZ_SPEC_K_MAX) {
        set_err(errbuf, errlen, "spec_k %d out of range 1..%d", k, Mo(mm)->n_draft);
        return -LZ_ERR_SPEC_K_RANGE;
    }
    return spec_round_temp(mm, s, anchor, anchor_pos, k, p_min, n_min, samp, brk, 1, out, out_n_accept,
                           out_new_pos, out_k_eff, errbuf, errlen, LZ_SPEC_K_MAX);
}

// --------------------------------------------------------- generation ---

static double g_last_loop_s = 0.0;
extern "C" double l98_last_loop_seconds(void) { return g_last_loop_s; }

extern "C" int l98_row_sums(const float *x, int rows, int n, float *out) {
    if (!x || !out || rows < 1 || n < 1 || n > 2048) return 1;
    float *dx = nullptr, *dout = nullptr;
    int rc = 0;
    if (hipMalloc(&dx, sizeof(float) * (size_t)rows * n) != hipSuccess ||
        hipMalloc(&dout, sizeof(float) * (size_t)rows) != hipSuccess)
        rc = 1;
    if (!rc && hipMemcpy(dx, x, sizeof(float) * (size_t)rows * n, hipMemcpyHostToDevice) != hipSuccess) rc = 1;
    if (!rc && l98k_row_sums(dx, rows, n, dout, nullptr)) rc = 1;
    if (!rc && hipMemcpy(out, dout, sizeof(float) * (size_t)rows, hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
    if (dx) (void)hipFree(dx);
    if (dout) (void)hipFree(dout);
    return rc;
}

// Host arrays in, host arrays out: device copies, one launch, copies back.
namespace {
struct DevBuf {
    void *p = nullptr;
    ~DevBuf() { if (p) (void)hipFree(p); }
    bool get(const void *src, size_t bytes) {
        if (hipMalloc(&p, bytes) != hipSuccess) { p = nullptr; return false; }
        return !src || hipMemcpy(p, src, bytes, hipMemcpyHostToDevice) == hipSuccess;
    }
    bool put(void *dst, size_t bytes) const { return hipMemcpy(dst, p, bytes, hipMemcpyDeviceToHost) == hipSuccess; }
};
bool fwht_args_ok(int rows, int n, int blk) {
    return rows >= 1 && n >= 1 && n <= 8192 && blk >= 1 && blk <= n && (blk & (blk - 1)) == 0 && n % blk == 0;
}
}  // namespace

extern "C" int l98_fwht_i32(const int32_t *x, int32_t *y, int rows, int n, int blk) {
    if (!x || !y || !fwht_args_ok(rows, n, blk)) return 1;
    const size_t b = sizeof(int32_t) * (size_t)rows * n;
    DevBuf dx, dy;
    if (!dx.get(x, b) || !dy.get(nullptr, b)) return 1;
    if (l98k_fwht_i32((const int32_t *)dx.p, (int32_t *)dy.p, rows, n, blk, nullptr)) return 1;
    return dy.put(y, b) ? 0 : 1;
}

extern "C" int l98_fwht_f32(float *v, int rows, int n, int blk, int rot) {
    if (!v || !fwht_args_ok(rows, n, blk)) return 1;
    const size_t b = sizeof(float) * (size_t)rows * n;
    DevBuf dv;
    if (!dv.get(v, b)) return 1;
    if (l98k_fwht_f32((float *)dv.p, rows, n, blk, rot, nullptr)) return 1;
    return dv.put(v, b) ? 0 : 1;
}

extern "C" int l98_subn_fwht_quant(const float *x, int rows, int n, int blk, int gw, int8_t *q, float *s) {
    if (!x || !q || !s || !fwht_args_ok(rows, n, blk) || n % 32 != 0) return 1;
    const size_t nx = (size_t)rows * n;
    DevBuf dx, dq, ds;
    if (!dx.get(x, sizeof(float) * nx) || !dq.get(nullptr, nx) || !ds.get(nullptr, sizeof(float) * (nx / 32)))
        return 1;
    if (l98k_subn_quant((const float *)dx.p, rows, n, blk, gw, (int8_t *)dq.p, (float *)ds.p, nullptr)) return 1;
    return dq.put(q, nx) && ds.put(s, sizeof(float) * (nx / 32)) ? 0 : 1;
}

extern "C" int l98_moe_route(const float *logits, const float *bias, int nt, int E, int topk, int *idx, float *w) {
    if (!logits || !idx || !w || nt < 1 || nt > MAX_CHUNK || E < 1 || E > MAX_EXPERTS || topk < 1 || topk > MAX_TOPK)
        return 1;
    if (ensure_tables()) return 1;
    float *dl = nullptr, *db = nullptr, *dw = nullptr;
    int *di = nullptr, rc = 0;
    if (hipMalloc(&dl, sizeof(float) * (size_t)nt * E) != hipSuccess || hipMalloc(&db, sizeof(float) * E) != hipSuccess ||
        hipMalloc(&dw, sizeof(float) * nt * topk) != hipSuccess || hipMalloc(&di, sizeof(int) * nt * topk) != hipSuccess)
        rc = 1;
    if (!rc && hipMemcpy(dl, logits, sizeof(float) * (size_t)nt * E, hipMemcpyHostToDevice) != hipSuccess) rc = 1;
    if (!rc && (bias ? hipMemcpy(db, bias, sizeof(float) * E, hipMemcpyHostToDevice)
                     : hipMemset(db, 0, sizeof(float) * E)) != hipSuccess)
        rc = 1;
    if (!rc && l98k_moe_route(dl, db, E, topk, nt, di, dw, nullptr)) rc = 1;
    if (!rc && (hipMemcpy(idx, di, sizeof(int) * nt * topk, hipMemcpyDeviceToHost) != hipSuccess ||
                hipMemcpy(w, dw, sizeof(float) * nt * topk, hipMemcpyDeviceToHost) != hipSuccess))
        rc = 1;
    if (dl) (void)hipFree(dl);
    if (db) (void)hipFree(db);
    if (dw) (void)hipFree(dw);
    if (di) (void)hipFree(di);
    return rc;
}

extern "C" int l98_gemm_q8(const int8_t *w, const float *ws, int N, int K, const int8_t *xq, const float *xqs, int M,
                           float *out) {
    if (!w || !ws || !xq || !xqs || !out || N < 1 || M < 1 || K < 32 || (K & 31)) return 1;
    DevBuf dw, dws, dx, dxs, dout;
    if (!dw.get(w, (size_t)N * K) || !dws.get(ws, sizeof(float) * N) || !dx.get(xq, (size_t)M * K) ||
        !dxs.get(xqs, sizeof(float) * (size_t)M * (K / 32)) || !dout.get(nullptr, sizeof(float) * (size_t)M * N))
        return 1;
    if (l98k_mfma_gemm((const int8_t *)dw.p, (const float *)dws.p, N, K, (const int8_t *)dx.p, (const float *)dxs.p, M,
                       (float *)dout.p, N, nullptr))
        return 1;
    return dout.put(out, sizeof(float) * (size_t)M * N) ? 0 : 1;
}

extern "C" int l98_sort_desc(const uint32_t *keys, int n, uint32_t *keys_out, int *idx_out) {
    if (!keys || !keys_out || !idx_out || n < 1 || n > (1 << 20)) return 1;
    for (int i = 0; i < n; i++)
        if (keys[i] >= (1u << 30)) return 1;
    DevBuf dk, dko, dio, dt;
    if (!dk.get(keys, sizeof(uint32_t) * (size_t)n) || !dko.get(nullptr, sizeof(uint32_t) * (size_t)n) ||
        !dio.get(nullptr, sizeof(int) * (size_t)n) || !dt.get(nullptr, l98k_smp_sort_tmp_bytes(n)))
        return 1;
    if (l98k_smp_sort_desc((uint32_t *)dk.p, (uint32_t *)dko.p, (int *)dio.p, n, dt.p, nullptr, nullptr)) return 1;
    return dko.put(keys_out, sizeof(uint32_t) * (size_t)n) && dio.put(idx_out, sizeof(int) * (size_t)n) ? 0 : 1;
}

extern "C" int l98_argmax_rows(const float *x, int rows, int n, int mode, int *out) {
    if (!x || !out || rows < 1 || rows > MAX_CHUNK || n < 1 || (mode != 0 && mode != 1)) return 1;
    DevBuf dx, dout;
    if (!dx.get(x, sizeof(float) * (size_t)rows * n) || !dout.get(nullptr, sizeof(int) * rows)) return 1;
    if (l98k_argmax((const float *)dx.p, n, rows, mode, (int *)dout.p, nullptr)) return 1;
    return dout.put(out, sizeof(int) * rows) ? 0 : 1;
}

// The lm_head path's argmax: an int8 GEMV (one scale per weight row, or
// groups of gs) over M
// pre-quantized rows with the argmax epilogue, then l98k_argmax_part;
// logits [M][N] and the rows' argmaxes (mode 0 or 1) come back.
extern "C" int l98_gemv_argmax(const int8_t *w, const float *ws, int N, int K, int gs, const int8_t *xq,
                               const float *xqs, int M, int mode, float *logits, int *out) {
    if (!w || !ws || !xq || !xqs || !logits || !out || N < 1 || K < 32 || (K & 31) || M < 1 || M > MAX_CHUNK ||
        (mode != 0 && mode != 1) || gs < 0 || (gs && ((gs & 31) || K % gs)))
        return 1;
    if (gs == K) gs = 0;
    const size_t nws = gs ? (size_t)(K / gs) : 1;
    int cap = 0;
    for (int m = 1; m <= MAX_CHUNK; m++) {
        const int need = l98k_gemv_tiles(N, K, m) * m;
        cap = need > cap ? need : cap;
    }
    DevBuf dw, dws, dx, dxs, dl, dp, dout;
    if (!dw.get(w, (size_t)N * K) || !dws.get(ws, sizeof(float) * N * nws) || !dx.get(xq, (size_t)M * K) ||
        !dxs.get(xqs, sizeof(float) * (size_t)M * (K / 32)) || !dl.get(nullptr, sizeof(float) * (size_t)M * N) ||
        !dp.get(nullptr, sizeof(unsigned long long) * (size_t)cap) || !dout.get(nullptr, sizeof(int) * M))
        return 1;
    GemvBatch b{};
    b.n = 1;
    GemvJob &j = b.job[0];
    j.w = (const int8_t *)dw.p; j.ws = (const float *)dws.p; j.out = (float *)dl.p;
    j.xq = (const int8_t *)dx.p; j.xqs = (const float *)dxs.p;
    j.rows = N; j.in_dim = K; j.out_stride = N; j.gs = gs;
    j.pro.mode = PRO_XQ;
    b.amax_mode = mode;
    b.amax_part = (unsigned long long *)dp.p;
    b.amax_cap = cap;
    if (l98k_gemv(&b, M, nullptr) ||
        l98k_argmax_part(b.amax_part, j.tiles, j.out, N, M, mode, (int *)dout.p, nullptr))
        return 1;
    return dl.put(logits, sizeof(float) * (size_t)M * N) && dout.put(out, sizeof(int) * M) ? 0 : 1;
}

extern "C" int l98_prefix_query(const float *x, int rows, int n, int mode, const float *c, int *out, float *outv) {
    if (!x || !out || !outv || rows < 1 || n < 1 || mode < 0 || mode > 2 || (mode && !c)) return 1;
    float *dx = nullptr, *dc = nullptr, *dv = nullptr;
    int *dout = nullptr, rc = 0;
    if (hipMalloc(&dx, sizeof(float) * (size_t)rows * n) != hipSuccess || hipMalloc(&dc, sizeof(float) * rows) != hipSuccess ||
        hipMalloc(&dv, sizeof(float) * rows) != hipSuccess || hipMalloc(&dout, sizeof(int) * rows) != hipSuccess)
        rc = 1;
    if (!rc && hipMemcpy(dx, x, sizeof(float) * (size_t)rows * n, hipMemcpyHostToDevice) != hipSuccess) rc = 1;
    if (!rc && mode && hipMemcpy(dc, c, sizeof(float) * rows, hipMemcpyHostToDevice) != hipSuccess) rc = 1;
    if (!rc && l98k_smp_xprefix(dx, rows, n, mode, mode ? dc : nullptr, dout, dv, nullptr)) rc = 1;
    if (!rc && (hipMemcpy(out, dout, sizeof(int) * rows, hipMemcpyDeviceToHost) != hipSuccess ||
                hipMemcpy(outv, dv, sizeof(float) * rows, hipMemcpyDeviceToHost) != hipSuccess))
        rc = 1;
    for (void *q : {(void *)dx, (void *)dc, (void *)dv, (void *)dout})
        if (q) (void)hipFree(q);
    return rc;
}

extern "C" const char *l98_device_name(void) {
    static char name[256];
    hipDeviceProp_t p;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) return "none";
    snprintf(name, sizeof name, "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
    return name;
}

extern "C" int l98_session_start(const LZModel *mm, LZRunState *s, const int *prompt, int n_prompt,
                                 const LZSampler *samp) {
    if (!mm || !s || !s->impl || !prompt || n_prompt < 2) return -LZ_ERR_NULL_ARG;
    if (!Mo(mm)->has_mtp) return -LZ_ERR_SPEC_NO_HEAD;
    DState *d = S(s);
    const LZModelConfig &c = d->m->c;
    if (!tok_ok(c, prompt, n_prompt) || n_prompt >= d->seq_len) return -LZ_ERR_FORWARD;
    d->session_greedy = !samp || !(samp->p.temperature > 0.0f);
    if (samp) d->session_samp = *samp;
    // prefill + MTP prefill (src/generate.c:2806-2960)
    lz_state_reset(s, mm);
    if (batch_capture_dev(d, s, prompt, n_prompt - 1, 0)) return -LZ_ERR_FORWARD;
    // A DSpark head has no fc for the MTP prefill to project through, and
    // none of its steps reads the MTP KV rows: its session is the body
    // prefill alone (the driver's MTP-prefill skip, src/generate.c:2817-2830).
    if (d->m->n_draft <= 1) {
        DevCtl h = ctl_from(s);
        h.pos_scratch = 0;
        if (ctl_put(d, h) ||
            hipMemcpyAsync(d->tokbuf, prompt + 1, sizeof(int) * (size_t)(n_prompt - 1), hipMemcpyHostToDevice, d->st) ||
            mtp_prefill_dev(d, d->hcap, d->tokbuf, n_prompt - 1, &d->ctl->pos_scratch, 0))
            return -LZ_ERR_FORWARD;
        s->mtp_pos = n_prompt - 1;
    }
    // first anchor from a capture forward
    float *lg = lz_forward_capture(mm, s, prompt[n_prompt - 1], n_prompt - 1);
    if (!lg) return -LZ_ERR_FORWARD;
    int anchor = 0;
    if (d->session_greedy) anchor = lz_sample_argmax(lg, c.vocab_size);
    else if (dev_sample_ex(d, d->logits, c.vocab_size, d->session_samp.p.temperature, d->session_samp.p.topp,
                           &d->session_samp.rng_state, &anchor))
        return -LZ_ERR_FORWARD;
    DevCtl h = ctl_from(s);
    h.anchor = anchor;
    h.anchor_pos = n_prompt - 1;
    h.tok[0] = anchor;
    if (ctl_put(d, h) || hipStreamSynchronize(d->st)) return -LZ_ERR_FORWARD;
    return anchor;
}

extern "C" int l98_session_sampler(const LZRunState *s, LZSampler *out) {
    if (!s || !s->impl || !out) return 1;
    *out = S(const_cast<LZRunState *>(s))->session_samp;
    return 0;
}

// Rounds that stay inside the state whatever they accept: a round's verify
// writes positions up to anchor_pos + k + 1 and advances the anchor by at
// most k + 1; its drafts and catch-up write MTP rows up to mtp_pos + k - 1
// and advance mtp_pos by at most k.
static int rounds_that_fit(const DState *d, const DevCtl &h, int k) {
    long a = ((long)d->seq_len - 2 - h.anchor_pos - k) / (k + 1) + 1;
    long b = ((long)d->seq_len - h.mtp_pos - k) / k + 1;
    long r = a < b ? a : b;
    return r < 0 ? 0 : (int)r;
}

extern "C" int l98_greedy_rounds(const LZModel *mm, LZRunState *s, int k, int n_rounds, int use_graph,
                                 int *tokens, int cap, int *n_accept_out, float *device_ms) {
    return l98_greedy_rounds_ex(mm, s, k, n_rounds, use_graph, tokens, cap, n_accept_out, nullptr, nullptr,
                                device_ms);
}

extern "C" int l98_greedy_rounds_ex(const LZModel *mm, LZRunState *s, int k, int n_rounds, int use_graph,
                                    int *tokens, int cap, int *n_accept_out, int *experts_out,
                                    int *new_pos_out, float *device_ms) {
    if (!mm || !s || !s->impl || n_rounds < 1) return -LZ_ERR_NULL_ARG;
    if (!Mo(mm)->has_mtp) return -LZ_ERR_SPEC_NO_HEAD;
    if (k < 1 || k > L98_SPEC_K_GPU || k > s->ssm_ring_depth - 1) return -LZ_ERR_SPEC_K_RANGE;
    if (Mo(mm)->n_draft > 1 && k > Mo(mm)->n_draft) return -LZ_ERR_SPEC_K_RANGE;     // DSpark: k <= mtp_n_draft
    DState *d = S(s);
    if (n_rounds > d->hist_cap) return -LZ_ERR_NULL_ARG;
    const int max_pos = d->seq_len - 1;
    // ctl.round = 0 (records restart at hist[0]); k_eff = k
    {
        DevCtl h;
        if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
        if (n_rounds > rounds_that_fit(d, h, k)) return -LZ_ERR_FORWARD;
        h.round = 0;
        h.expert_tally = 0;
        h.k_eff = k;
        if (ctl_put(d, h)) return -LZ_ERR_FORWARD;
    }
    if (use_graph && !d->round_graph[k]) {
        hipGraph_t g = nullptr;
        if (hipStreamBeginCapture(d->st, hipStreamCaptureModeThreadLocal) != hipSuccess) return -LZ_ERR_FORWARD;
        int rc = enqueue_greedy_round(d, k, max_pos, 0, true);
        if (hipStreamEndCapture(d->st, &g) != hipSuccess || rc) return -LZ_ERR_FORWARD;
        if (hipGraphInstantiate(&d->round_graph[k], g, nullptr, nullptr, 0) != hipSuccess) {
            (void)hipGraphDestroy(g);
            return -LZ_ERR_FORWARD;
        }
        (void)hipGraphDestroy(g);
    }
    (void)hipEventRecord(d->ev0, d->st);
    for (int r = 0; r < n_rounds; r++) {
        if (use_graph) {
            if (hipGraphLaunch(d->round_graph[k], d->st) != hipSuccess) return -LZ_ERR_FORWARD;
        } else if (enqueue_greedy_round(d, k, max_pos, 0, true)) {
            return -LZ_ERR_FORWARD;
        }
    }
    (void)hipEventRecord(d->ev1, d->st);
    if (hipEventSynchronize(d->ev1) != hipSuccess) return -LZ_ERR_FORWARD;
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, d->ev0, d->ev1);
    if (device_ms) *device_ms = ms;
    g_last_loop_s = ms * 1e-3;
    std::vector<RoundRec> rec((size_t)n_rounds);
    if (hipMemcpy(rec.data(), d->hist, sizeof(RoundRec) * rec.size(), hipMemcpyDeviceToHost) != hipSuccess)
        return -LZ_ERR_FORWARD;
    int n = 0;
    for (int r = 0; r < n_rounds; r++) {
        if (rec[r].n_accept < rec[r].k_eff) lz_debug_n_ring_rollback++;
        if (rec[r].n_accept > 1) lz_debug_n_catchup++;
        lz_debug_n_chunks++;
        lz_debug_n_lmhead++;
        if (n_accept_out) n_accept_out[r] = rec[r].n_accept;
        if (experts_out) experts_out[r] = rec[r].experts;
        if (new_pos_out) new_pos_out[r] = rec[r].new_pos;
        for (int j = 0; j <= rec[r].n_accept; j++) {
            if (tokens && n < cap) tokens[n] = rec[r].out[j];
            n++;
        }
    }
    DevCtl h;
    if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
    s->ssm_slot = h.slot_base;
    s->mtp_pos = h.mtp_pos;
    if (hipMemcpy(s->mtp_chain, d->chain, sizeof(float) * d->m->c.hidden_size, hipMemcpyDeviceToHost) != hipSuccess)
        return -LZ_ERR_FORWARD;
    return n;
}

// ------------------------------------------------------ session batches ---
//
// Several independent sessions (one LZRunState each, as the reference keeps
// one sequence per state) advanced together: each session's work is
// enqueued on its own stream, interleaved, so the device runs them
// concurrently; the host waits once for all of them.

static double now_ms() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e3 + t.tv_nsec * 1e-6;
}

static int batch_ok(const LZModel *mm, LZRunState **states, int n_seq) {
    if (!mm || !mm->impl || !states || n_seq < 1) return 0;
    for (int i = 0; i < n_seq; i++)
        if (!states[i] || !states[i]->impl || S(states[i])->m != Mo(mm)) return 0;
    return 1;
}

extern "C" int l98_verify_batch(const LZModel *mm, LZRunState **states, int n_seq, const int *tokens, int n_tok,
                                const int *pos0, int copy_out, float *wall_ms) {
    if (!batch_ok(mm, states, n_seq) || !tokens || !pos0 || n_tok < 1 || n_tok > LZ_BATCH_MAX) return 1;
    if (!Mo(mm)->has_mtp) return 1;
    const LZModelConfig &c = Mo(mm)->c;
    for (int i = 0; i < n_seq; i++) {
        DState *d = S(states[i]);
        if (!tok_ok(c, tokens + (size_t)i * n_tok, n_tok) || pos0[i] < 0 || pos0[i] + n_tok > d->seq_len) return 1;
        if (hipStreamSynchronize(d->st) != hipSuccess) return 1;
    }
    const int R = n_seq * n_tok;
    DWide *w = R <= WIDE_MAX ? wide_get(Mo(mm)) : nullptr;
    if (w && w->logits_rows < R) {
        if (w->logits) (void)hipFree(w->logits);
        w->logits = nullptr;
        w->logits_rows = 0;
        if (hipMalloc((void **)&w->logits, sizeof(float) * (size_t)R * c.vocab_size) != hipSuccess) return 1;
        w->logits_rows = R;
    }
    if (!knobs_ok(c.num_experts_per_token, nullptr, 0)) return 1;
    const double t0 = now_ms();
    if (w) {
        // every session's rows through one wide forward on the first
        // session's stream: one launch per op over all R rows
        hipStream_t st = S(states[0])->st;
        std::vector<WideItem> items((size_t)n_seq);
        // the control blocks go up as one transfer of [n DevCtl][n
        // destinations][n logits destinations][n hidden destinations] from
        // pinned memory, then one launch puts each in place
        const size_t cbytes = (sizeof(DevCtl) + sizeof(DevCtl *) + 2 * sizeof(float *)) * (size_t)n_seq;
        if (w->ctl_cap < n_seq) {
            if (w->ctl_host) (void)hipHostFree(w->ctl_host);
            if (w->ctl_dev) (void)hipFree(w->ctl_dev);
            w->ctl_host = w->ctl_dev = nullptr;
            w->ctl_cap = 0;
            if (hipHostMalloc((void **)&w->ctl_host, cbytes, hipHostMallocDefault) != hipSuccess ||
                hipMalloc((void **)&w->ctl_dev, cbytes) != hipSuccess)
                return 1;
            w->ctl_cap = n_seq;
        }
        DevCtl *hs = reinterpret_cast<DevCtl *>(w->ctl_host);
        DevCtl **dst = reinterpret_cast<DevCtl **>(w->ctl_host + sizeof(DevCtl) * (size_t)n_seq);
        float **ldst = reinterpret_cast<float **>(dst + n_seq), **hdst = ldst + n_seq;
        for (int i = 0; i < n_seq; i++) {
            DState *d = S(states[i]);
            hs[i] = ctl_from(states[i]);
            hs[i].pos_scratch = pos0[i];
            dst[i] = d->ctl;
            ldst[i] = d->mtp_logits;
            hdst[i] = d->vhidden;
            items[i] = WideItem{d, i * n_tok, n_tok, pos0[i]};
        }
        if (hipMemcpyAsync(w->ctl_dev, w->ctl_host, cbytes, hipMemcpyHostToDevice, st) ||
            l98k_put_ctl(reinterpret_cast<const DevCtl *>(w->ctl_dev),
                         reinterpret_cast<DevCtl *const *>(w->ctl_dev + sizeof(DevCtl) * (size_t)n_seq), n_seq, st))
            return 1;
        if (hipMemcpyAsync(w->toks, tokens, sizeof(int) * (size_t)R, hipMemcpyHostToDevice, st) ||
            wide_forward(Mo(mm), w, items.data(), n_seq, R, true, w->hcap, w->logits, st))
            return 1;
        // every session's verify logits and hidden rows into its own buffers
        float *const *ldev = reinterpret_cast<float *const *>(w->ctl_dev + (sizeof(DevCtl) + sizeof(DevCtl *)) *
                                                                               (size_t)n_seq);
        if (l98k_scatter_rows(w->logits, (size_t)n_tok * c.vocab_size, ldev, n_seq, st) ||
            l98k_scatter_rows(w->hcap, (size_t)n_tok * c.hidden_size, ldev + n_seq, n_seq, st))
            return 1;
        for (int i = 0; i < n_seq; i++) {
            DState *d = S(states[i]);
            states[i]->ssm_slot = (states[i]->ssm_slot + n_tok) % d->depth;
        }
        if (hipStreamSynchronize(st) != hipSuccess) return 1;
        lz_debug_n_chunks++;
        lz_debug_n_lmhead++;
    } else {
        for (int i = 0; i < n_seq; i++) {
            LZRunState *s = states[i];
            DState *d = S(s);
            DevCtl h = ctl_from(s);
            h.pos_scratch = pos0[i];
            for (int j = 0; j < n_tok; j++) h.tok[j] = tokens[(size_t)i * n_tok + j];
            if (ctl_put(d, h)) return 1;
            if (forward_chunk(d, d->ctl->tok, n_tok, &d->ctl->pos_scratch, 0, pos0[i] + n_tok - 1, d->vhidden, true,
                              d->mtp_logits, false))
                return 1;
            s->ssm_slot = (s->ssm_slot + n_tok) % d->depth;
        }
        for (int i = 0; i < n_seq; i++)
            if (hipStreamSynchronize(S(states[i])->st) != hipSuccess) return 1;
    }
    if (wall_ms) *wall_ms = (float)(now_ms() - t0);
    if (copy_out) {
        for (int i = 0; i < n_seq; i++) {
            LZRunState *s = states[i];
            DState *d = S(s);
            if (hipMemcpyAsync(s->mtp_logits, d->mtp_logits, sizeof(float) * (size_t)n_tok * c.vocab_size,
                               hipMemcpyDeviceToHost, d->st) ||
                hipMemcpyAsync(s->mtp_verify_hidden, d->vhidden, sizeof(float) * (size_t)n_tok * c.hidden_size,
                               hipMemcpyDeviceToHost, d->st))
                return 1;
        }
        for (int i = 0; i < n_seq; i++)
            if (hipStreamSynchronize(S(states[i])->st) != hipSuccess) return 1;
    }
    return 0;
}

namespace {

// ----------------------------------------------- batched session rounds ---
//
// n sessions' greedy rounds as many-row passes over their rows, on the first
// session's stream, with draft_step's, enqueue_verify_accept's and
// mtp_prefill_chunked's arithmetic through the many-row kernels (the MFMA
// GEMMs, the RMSNorm rows, the SiLU-mul rows and the item attention give the
// GEMV path's bits):
//   * draft step j: one row per session (its tok[j] and chain), the MTP
//     block at its position mtp_pos + j (one attention item per session), the
//     FFN, the exit norm (the new chain rows) and the tied lm_head, argmax
//     p1 per row into tok[j + 1];
//   * the verify: wide_forward over the sessions' K1 = k + 1 rows each at
//     anchor_pos, argmax per row as targ;
//   * acceptance with ring rollback and the chain reseed per session, the
//     catch-up of k - 1 rows per session (K and V into the MTP plane at
//     catch_pos), the round record and the advance.
struct RoundBatch {
    char *mem = nullptr;             // device tables
    BatchSess *bs = nullptr;
    AttnItem *draft_items = nullptr; // [k][n]: row r, position mtp_pos + j
    AttnItem *catch_items = nullptr; // [n]: rows r*(k-1) .., position catch_pos
    int *am = nullptr;               // argmaxes [n * K1]
    ~RoundBatch() { if (mem) (void)hipFree(mem); }
};

int wide_draft_step(const DModel *m, DWide *w, const RoundBatch &rb, int n, int j, int max_len, hipStream_t st) {
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size, I = c.mtp_intermediate_size, V = c.vocab_size;
    const int qgd = c.attn_qgate_dim, kvd = c.attn_kv_dim, qd = c.attn_q_dim;
    const float eps = c.rms_norm_eps;
    const DLayer &L = m->mtp;
    CK(l98k_batch_round(0, rb.bs, n, j, 1, 0, d, nullptr, nullptr, w->toks, w->hcap, st));
    CK(l98k_mtp_pre(m->embed.q, m->embed.s, m->embed.gs, w->toks, w->hcap, d, m->mtp_pre_e, m->mtp_pre_h, eps, n,
                    w->mq, w->mqs, st));
    CK(mf(m->mtp_fc, w->mq, w->mqs, n, w->x, d, st));
    CK(l98k_rmsnorm(w->x, d, nullptr, nullptr, L.in_norm, d, eps, n, nullptr, 0, w->xq, w->xqs, st));
    CK(mf_multi({{&L.q, w->qg, qgd}, {&L.k, w->kp, kvd}, {&L.v, w->vp, kvd}}, w->xq, w->xqs, n, st));
    AttnArgs a{};
    a.qg = w->qg; a.kp = w->kp; a.vp = w->vp;
    a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.rope_cs = m->rope_cs;
    a.qh = w->qh;
    a.oq = w->xq2; a.oqs = w->xqs2;
    a.nh = c.n_heads; a.nkv = c.n_kv_heads; a.hd = c.head_dim; a.rot = c.rotary_dim;
    a.q_dim = qd; a.qg_dim = qgd; a.kv_dim = kvd;
    a.eps = eps;
    a.attn_scale = ssm_scale(c.head_dim);
    const size_t att_item = (size_t)MAX_CHUNK * c.n_heads * (size_t)((max_len + 3) & ~3);
    CK(l98k_attn_items(&a, rb.draft_items + (size_t)j * n, n, c.n_full_layers, max_len, 1, w->att_items, att_item, 0,
                       st));
    CK(mf(L.o, w->xq2, w->xqs2, n, w->blk, d, st));
    // the FFN (dense_ffn_step): the residual folds in place, post-norm, gate
    // / up, SiLU-mul, down, then the exit norm (the chain rows) and the head
    CK(l98k_rmsnorm(w->x, d, w->blk, nullptr, L.post_norm, d, eps, n, nullptr, 0, w->xq, w->xqs, st));
    CK(mf_multi({{&m->mtp_gate, w->h1, I}, {&m->mtp_up, w->h3, I}}, w->xq, w->xqs, n, st));
    CK(l98k_wide_pro(1, w->h1, w->h3, I, nullptr, nullptr, 0, I, n, w->hq, w->hqs, st));
    CK(mf(m->mtp_down, w->hq, w->hqs, n, w->blk, d, st));
    CK(l98k_rmsnorm(w->x, d, w->blk, nullptr, m->mtp_norm, d, eps, n, w->hcap, d, w->xq, w->xqs, st));
    CK(mf(m->embed, w->xq, w->xqs, n, w->logits, V, st));
    CK(l98k_argmax(w->logits, V, n, 1, rb.am, st));
    return l98k_batch_round(1, rb.bs, n, j, 1, 0, d, rb.am, w->hcap, nullptr, nullptr, st);
}

// The catch-up of k - 1 rows per session after the acceptance: the rows'
// main_proj input from (verify hidden row j, catch_tok[j]), fc, the MTP
// block's input norm and K / V into each session's MTP plane at catch_pos + j.
int wide_catchup(const DModel *m, DWide *w, const RoundBatch &rb, int n, int k, hipStream_t st) {
    const LZModelConfig &c = m->c;
    const int d = c.hidden_size, kvd = c.attn_kv_dim, nc = k - 1, R = n * nc;
    const float eps = c.rms_norm_eps;
    CK(l98k_batch_round(4, rb.bs, n, 0, k + 1, nc, d, nullptr, w->hcap, w->toks, w->blk, st));
    CK(l98k_mtp_pre(m->embed.q, m->embed.s, m->embed.gs, w->toks, w->blk, d, m->mtp_pre_e, m->mtp_pre_h, eps, R,
                    w->mq, w->mqs, st));
    CK(mf(m->mtp_fc, w->mq, w->mqs, R, w->x, d, st));
    CK(l98k_rmsnorm(w->x, d, nullptr, nullptr, m->mtp.in_norm, d, eps, R, nullptr, 0, w->xq, w->xqs, st));
    CK(mf_multi({{&m->mtp.k, w->kp, kvd}, {&m->mtp.v, w->vp, kvd}}, w->xq, w->xqs, R, st));
    AttnArgs a{};
    a.kp = w->kp; a.vp = w->vp;
    a.k_norm = m->mtp.k_norm; a.rope_cs = m->rope_cs;
    a.nh = c.n_heads; a.nkv = c.n_kv_heads; a.hd = c.head_dim; a.rot = c.rotary_dim;
    a.q_dim = c.attn_q_dim; a.qg_dim = c.attn_qgate_dim; a.kv_dim = kvd;
    a.kv_only = 1;
    a.eps = eps;
    return l98k_attn_prep_items(&a, rb.catch_items, n, c.n_full_layers, st);
}

// Whether a batch of sessions can take the batched rounds: the many-row
// forward carries the model (no SubLN, no grouped scales), a one-slot MTP
// head, every row fits one many-row pass, and the FFN rows fit the expert
// buffers they borrow.
bool batched_rounds_ok(const DModel *m, int n_seq, int k) {
    const LZModelConfig &c = m->c;
    if (m->n_draft > 1 || c.use_subn || n_seq < 1 || k < 1) return false;
    if ((size_t)n_seq * (k + 1) > WIDE_MAX || (size_t)n_seq * (k - 1 > 0 ? k - 1 : 1) > WIDE_MAX) return false;
    const size_t pairs = (size_t)WIDE_MAX * c.num_experts_per_token;
    return (size_t)n_seq * c.mtp_intermediate_size <= pairs * c.moe_intermediate_size;
}

int greedy_rounds_batched(const LZModel *mm, LZRunState **states, int n_seq, int k, int n_rounds, float *wall_ms) {
    const DModel *m = Mo(mm);
    const LZModelConfig &c = m->c;
    const int K1 = k + 1, R = n_seq * K1, V = c.vocab_size;
    DWide *w = wide_get(m);
    if (!w || !batched_rounds_ok(m, n_seq, k)) return 1;
    hipStream_t st = S(states[0])->st;
    int max_len = 1;
    for (int i = 0; i < n_seq; i++) max_len = S(states[i])->seq_len > max_len ? S(states[i])->seq_len : max_len;
    // scratch sized once, before the timed loop
    if (w->logits_rows < R) {
        if (w->logits) (void)hipFree(w->logits);
        w->logits = nullptr;
        w->logits_rows = 0;
        if (hipMalloc((void **)&w->logits, sizeof(float) * (size_t)R * V) != hipSuccess) return 1;
        w->logits_rows = R;
    }
    const size_t att_item = (size_t)MAX_CHUNK * c.n_heads * (size_t)((max_len + 3) & ~3);
    if (w->att_items_floats < att_item * n_seq) {
        if (w->att_items) (void)hipFree(w->att_items);
        w->att_items = nullptr;
        w->att_items_floats = 0;
        if (hipMalloc((void **)&w->att_items, sizeof(float) * att_item * n_seq) != hipSuccess) return 1;
        w->att_items_floats = att_item * n_seq;
    }
    RoundBatch rb;
    const size_t o_bs = 0, o_di = (sizeof(BatchSess) * n_seq + 255) & ~(size_t)255,
                 o_ci = o_di + ((sizeof(AttnItem) * (size_t)k * n_seq + 255) & ~(size_t)255),
                 o_am = o_ci + ((sizeof(AttnItem) * n_seq + 255) & ~(size_t)255), bytes = o_am + sizeof(int) * R;
    if (hipMalloc((void **)&rb.mem, bytes) != hipSuccess) return 1;
    rb.bs = (BatchSess *)(rb.mem + o_bs);
    rb.draft_items = (AttnItem *)(rb.mem + o_di);
    rb.catch_items = (AttnItem *)(rb.mem + o_ci);
    rb.am = (int *)(rb.mem + o_am);
    std::vector<BatchSess> hb((size_t)n_seq);
    std::vector<AttnItem> hd((size_t)k * n_seq), hc((size_t)n_seq);
    std::vector<WideItem> items((size_t)n_seq);
    for (int i = 0; i < n_seq; i++) {
        DState *d = S(states[i]);
        hb[i] = BatchSess{d->ctl, d->chain, d->hist, d->hist_cap, d->depth};
        for (int j = 0; j < k; j++)
            hd[(size_t)j * n_seq + i] = AttnItem{d->kq, d->vq, d->ks, d->vs, &d->ctl->mtp_pos, i, 1, d->seq_len, j};
        hc[i] = AttnItem{d->kq, d->vq, d->ks, d->vs, &d->ctl->catch_pos, i * (k - 1), k - 1, d->seq_len, 0};
        // positions come from each control block; pos0 only bounds the rows' reach
        items[i] = WideItem{d, i * K1, K1, d->seq_len - K1};
    }
    if (hipMemcpy(rb.bs, hb.data(), sizeof(BatchSess) * n_seq, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(rb.draft_items, hd.data(), sizeof(AttnItem) * hd.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(rb.catch_items, hc.data(), sizeof(AttnItem) * n_seq, hipMemcpyHostToDevice) != hipSuccess)
        return 1;
    const double t0 = now_ms();
    for (int r = 0; r < n_rounds; r++) {
        for (int j = 0; j < k; j++) CK(wide_draft_step(m, w, rb, n_seq, j, max_len, st));
        CK(l98k_batch_round(2, rb.bs, n_seq, 0, K1, 0, c.hidden_size, nullptr, nullptr, w->toks, nullptr, st));
        CK(wide_forward(m, w, items.data(), n_seq, R, true, w->hcap, w->logits, st));
        CK(l98k_argmax(w->logits, V, R, 0, rb.am, st));
        CK(l98k_batch_round(3, rb.bs, n_seq, 0, K1, 0, c.hidden_size, rb.am, w->hcap, nullptr, nullptr, st));
        if (k > 1) CK(wide_catchup(m, w, rb, n_seq, k, st));
        CK(l98k_batch_round(5, rb.bs, n_seq, 0, K1, 0, c.hidden_size, nullptr, nullptr, nullptr, nullptr, st));
    }
    if (hipStreamSynchronize(st) != hipSuccess) return 1;
    if (wall_ms) *wall_ms = (float)(now_ms() - t0);
    lz_debug_n_chunks += n_rounds;
    lz_debug_n_lmhead += n_rounds;
    return 0;
}

}  // namespace

extern "C" int l98_greedy_rounds_batch_ex(const LZModel *mm, LZRunState **states, int n_seq, int k, int n_rounds,
                                          int *tokens, int cap, int *n_out, float *wall_ms, int mode) {
    if (!batch_ok(mm, states, n_seq) || n_rounds < 1 || !n_out || mode < 0 || mode > 1) return -LZ_ERR_NULL_ARG;
    if (!Mo(mm)->has_mtp) return -LZ_ERR_SPEC_NO_HEAD;
    // mode 0: the batched rounds when the model and the batch allow them;
    // mode 1: each session's own round graph on its own stream
    const bool batched = mode == 0 && batched_rounds_ok(Mo(mm), n_seq, k) && wide_get(Mo(mm)) != nullptr;
    for (int i = 0; i < n_seq; i++) {
        LZRunState *s = states[i];
        DState *d = S(s);
        if (k < 1 || k > L98_SPEC_K_GPU || k > s->ssm_ring_depth - 1) return -LZ_ERR_SPEC_K_RANGE;
        if (Mo(mm)->n_draft > 1 && k > Mo(mm)->n_draft) return -LZ_ERR_SPEC_K_RANGE;
        if (n_rounds > d->hist_cap) return -LZ_ERR_NULL_ARG;
        DevCtl h;
        if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
        if (n_rounds > rounds_that_fit(d, h, k)) return -LZ_ERR_FORWARD;
        h.round = 0;
        h.expert_tally = 0;
        h.k_eff = k;
        if (ctl_put(d, h)) return -LZ_ERR_FORWARD;
        if (!batched && !d->round_graph[k]) {
            hipGraph_t g = nullptr;
            if (hipStreamBeginCapture(d->st, hipStreamCaptureModeThreadLocal) != hipSuccess) return -LZ_ERR_FORWARD;
            int rc = enqueue_greedy_round(d, k, d->seq_len - 1, 0, true);
            if (hipStreamEndCapture(d->st, &g) != hipSuccess || rc) return -LZ_ERR_FORWARD;
            if (hipGraphInstantiate(&d->round_graph[k], g, nullptr, nullptr, 0) != hipSuccess) {
                (void)hipGraphDestroy(g);
                return -LZ_ERR_FORWARD;
            }
            (void)hipGraphDestroy(g);
        }
        if (hipStreamSynchronize(d->st) != hipSuccess) return -LZ_ERR_FORWARD;
    }
    if (batched) {
        if (greedy_rounds_batched(mm, states, n_seq, k, n_rounds, wall_ms)) return -LZ_ERR_FORWARD;
    } else {
        const double t0 = now_ms();
        for (int r = 0; r < n_rounds; r++)
            for (int i = 0; i < n_seq; i++) {
                DState *d = S(states[i]);
                if (hipGraphLaunch(d->round_graph[k], d->st) != hipSuccess) return -LZ_ERR_FORWARD;
            }
        for (int i = 0; i < n_seq; i++)
            if (hipStreamSynchronize(S(states[i])->st) != hipSuccess) return -LZ_ERR_FORWARD;
        if (wall_ms) *wall_ms = (float)(now_ms() - t0);
    }
    int total = 0;
    std::vector<RoundRec> rec((size_t)n_rounds);
    for (int i = 0; i < n_seq; i++) {
        LZRunState *s = states[i];
        DState *d = S(s);
        if (hipMemcpy(rec.data(), d->hist, sizeof(RoundRec) * rec.size(), hipMemcpyDeviceToHost) != hipSuccess)
            return -LZ_ERR_FORWARD;
        int n = 0;
        for (int r = 0; r < n_rounds; r++)
            for (int j = 0; j <= rec[r].n_accept; j++) {
                if (tokens && n < cap) tokens[(size_t)i * cap + n] = rec[r].out[j];
                n++;
            }
        n_out[i] = n;
        total += n;
        DevCtl h;
        if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
        s->ssm_slot = h.slot_base;
        s->mtp_pos = h.mtp_pos;
        if (hipMemcpy(s->mtp_chain, d->chain, sizeof(float) * d->m->c.hidden_size, hipMemcpyDeviceToHost) !=
            hipSuccess)
            return -LZ_ERR_FORWARD;
    }
    return total;
}

extern "C" int l98_batched_rounds_ok(const LZModel *mm, int n_seq, int k) {
    if (!mm || !mm->impl) return 0;
    return batched_rounds_ok(Mo(mm), n_seq, k) && wide_get(Mo(mm)) != nullptr ? 1 : 0;
}

extern "C" void l98_set_attn_path(int mode) { l98k_set_attn_path(mode); }

extern "C" int l98_greedy_rounds_batch(const LZModel *mm, LZRunState **states, int n_seq, int k, int n_rounds,
                                       int *tokens, int cap, int *n_out, float *wall_ms) {
    return l98_greedy_rounds_batch_ex(mm, states, n_seq, k, n_rounds, tokens, cap, n_out, wall_ms, 0);
}

// n temperature rounds on the device, one HIP graph launch each (captured
// per k, and again when T or top-p change), with the generator state in
// device memory from *rng and back into it.  Returns the tokens emitted
// (their ids in tokens[0 .. cap)), or -LZErr; k_eff / n_accept per round.
static int temp_rounds_dev(const LZModel *mm, LZRunState *s, int k, int n_rounds, float temp, float topp,
                           lz_u64 *rng, int *tokens, int cap, int *k_eff_out, int *n_accept_out) {
    DState *d = S(s);
    if (n_rounds < 1 || n_rounds > d->hist_cap || Mo(mm)->n_draft > 1) return -LZ_ERR_NULL_ARG;
    const int max_pos = d->seq_len - 1;
    if (!smp_ensure(d)) return -LZ_ERR_FORWARD;
    {
        DevCtl h;
        if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
        if (n_rounds > rounds_that_fit(d, h, k)) return -LZ_ERR_FORWARD;
        h.round = 0;
        h.expert_tally = 0;
        h.k_eff = k;
        if (ctl_put(d, h)) return -LZ_ERR_FORWARD;
    }
    if (d->temp_graph[k] && (d->temp_graph_t[k] != temp || d->temp_graph_p[k] != topp)) {
        (void)hipGraphExecDestroy(d->temp_graph[k]);
        d->temp_graph[k] = nullptr;
    }
    if (!d->temp_graph[k]) {
        hipGraph_t g = nullptr;
        if (hipStreamBeginCapture(d->st, hipStreamCaptureModeThreadLocal) != hipSuccess) return -LZ_ERR_FORWARD;
        int rc = enqueue_temp_round(d, k, max_pos, temp, topp);
        if (hipStreamEndCapture(d->st, &g) != hipSuccess || rc) return -LZ_ERR_FORWARD;
        if (hipGraphInstantiate(&d->temp_graph[k], g, nullptr, nullptr, 0) != hipSuccess) {
            (void)hipGraphDestroy(g);
            return -LZ_ERR_FORWARD;
        }
        (void)hipGraphDestroy(g);
        d->temp_graph_t[k] = temp;
        d->temp_graph_p[k] = topp;
    }
    if (hipMemcpyAsync(d->smp_rng, rng, sizeof(lz_u64), hipMemcpyHostToDevice, d->st) != hipSuccess)
        return -LZ_ERR_FORWARD;
    (void)hipEventRecord(d->ev0, d->st);
    for (int r = 0; r < n_rounds; r++)
        if (hipGraphLaunch(d->temp_graph[k], d->st) != hipSuccess) return -LZ_ERR_FORWARD;
    (void)hipEventRecord(d->ev1, d->st);
    if (hipMemcpyAsync(rng, d->smp_rng, sizeof(lz_u64), hipMemcpyDeviceToHost, d->st) != hipSuccess ||
        hipStreamSynchronize(d->st) != hipSuccess)
        return -LZ_ERR_FORWARD;
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, d->ev0, d->ev1);
    g_last_loop_s = ms * 1e-3;
    std::vector<RoundRec> rec((size_t)n_rounds);
    if (hipMemcpy(rec.data(), d->hist, sizeof(RoundRec) * rec.size(), hipMemcpyDeviceToHost) != hipSuccess)
        return -LZ_ERR_FORWARD;
    int n = 0;
    for (int r = 0; r < n_rounds; r++) {
        if (rec[r].n_accept < rec[r].k_eff) lz_debug_n_ring_rollback++;
        if (rec[r].n_accept > 1) lz_debug_n_catchup++;
        lz_debug_n_chunks++;
        lz_debug_n_lmhead++;
        if (k_eff_out) k_eff_out[r] = rec[r].k_eff;
        if (n_accept_out) n_accept_out[r] = rec[r].n_accept;
        for (int j = 0; j <= rec[r].n_accept; j++) {
            if (tokens && n < cap) tokens[n] = rec[r].out[j];
            n++;
        }
    }
    DevCtl h;
    if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
    s->ssm_slot = h.slot_base;
    s->mtp_pos = h.mtp_pos;
    if (hipMemcpy(s->mtp_chain, d->chain, sizeof(float) * d->m->c.hidden_size, hipMemcpyDeviceToHost) != hipSuccess)
        return -LZ_ERR_FORWARD;
    return n;
}

extern "C" int l98_generate(const LZModel *mm, LZRunState *s, const int *prompt, int n_prompt, int k,
                            int n_new, LZSampler *samp, int *tokens, int cap, int *k_eff_out,
                            int *n_accept_out, int *n_rounds) {
    if (!mm || !s || !s->impl || !prompt || n_prompt < 2 || !tokens) return -LZ_ERR_NULL_ARG;
    if (k < 1 || k > L98_SPEC_K_GPU || k > s->ssm_ring_depth - 1) return -LZ_ERR_SPEC_K_RANGE;
    if (Mo(mm)->n_draft > 1 && k > Mo(mm)->n_draft) return -LZ_ERR_SPEC_K_RANGE;     // DSpark: k <= mtp_n_draft
    DState *d = S(s);
    if (n_prompt + n_new + 2 * (k + 1) >= d->seq_len) return -LZ_ERR_FORWARD;
    int anchor = l98_session_start(mm, s, prompt, n_prompt, samp);
    if (anchor < 0) return anchor;
    int n = 0, rounds = 0;
    if (n < cap) tokens[n] = anchor;
    n++;
    if (!d->session_greedy && Mo(mm)->n_draft <= 1) {
        // temperature rounds on the device, in batches that cannot pass
        // n_new (as the greedy loop below); the generator state comes back
        // after each batch
        LZSampler &local = d->session_samp;
        std::vector<int> ke((size_t)n_new + 8), nac((size_t)n_new + 8);
        while (n < n_new) {
            int batch = (n_new - n) / (k + 1);
            if (batch < 1) batch = 1;
            if (batch > 64) batch = 64;
            DevCtl h;
            if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
            const int fit = rounds_that_fit(d, h, k);
            if (fit < 1) return -LZ_ERR_FORWARD;
            if (batch > fit) batch = fit;
            std::vector<int> tk((size_t)batch * (k + 1));
            int got = temp_rounds_dev(mm, s, k, batch, local.p.temperature, local.p.topp, &local.rng_state, tk.data(),
                                      (int)tk.size(), ke.data(), nac.data());
            if (got < 0) return got;
            int pos = 0;
            for (int r = 0; r < batch; r++) {
                if (k_eff_out) k_eff_out[rounds] = ke[r];
                if (n_accept_out) n_accept_out[rounds] = nac[r];
                rounds++;
                for (int i = 0; i <= nac[r]; i++, pos++) { if (n < cap) tokens[n] = tk[pos]; n++; }
            }
        }
        if (n_rounds) *n_rounds = rounds;
        if (samp) samp->rng_state = local.rng_state;
        return n;
    }
    if (!d->session_greedy) {
        LZSampler &local = d->session_samp;
        int anchor_pos = n_prompt - 1;
        while (n < n_new) {
            int out[L98_SPEC_K_GPU + 1], na = 0, np = 0, ke = 0;
            int r = spec_round_temp(mm, s, anchor, anchor_pos, k, 0.0f, 0, &local, 0, 0, out, &na, &np, &ke,
                                    nullptr, 0, L98_SPEC_K_GPU);
            if (r <= 0) return r < 0 ? r : -LZ_ERR_FORWARD;
            if (k_eff_out) k_eff_out[rounds] = ke;
            if (n_accept_out) n_accept_out[rounds] = na;
            rounds++;
            for (int i = 0; i <= na; i++) { if (n < cap) tokens[n] = out[i]; n++; }
            anchor = out[na];
            anchor_pos = np;
        }
        if (n_rounds) *n_rounds = rounds;
        if (samp) samp->rng_state = local.rng_state;
        return n;
    }
    // Greedy: a round emits 1..k+1 tokens and the loop stops at the first
    // round that reaches n_new, as the reference's does.  A device batch of
    // want / (k+1) rounds cannot pass n_new, so batches never run a round
    // the reference would not (the state after the call is the reference's).
    std::vector<int> na(n_new + 8);
    while (n < n_new) {
        int want = n_new - n;
        int batch = want / (k + 1);
        if (batch < 1) batch = 1;
        if (batch > 64) batch = 64;
        {
            DevCtl h;
            if (ctl_get(d, &h)) return -LZ_ERR_FORWARD;
            int fit = rounds_that_fit(d, h, k);
            if (fit < 1) return -LZ_ERR_FORWARD;
            if (batch > fit) batch = fit;
        }
        std::vector<int> tk((size_t)batch * (k + 1));
        int got = l98_greedy_rounds(mm, s, k, batch, 1, tk.data(), (int)tk.size(), na.data(), nullptr);
        if (got < 0) return got;
        int pos = 0;
        for (int r = 0; r < batch && n < n_new; r++) {
            if (k_eff_out) k_eff_out[rounds] = k;
            if (n_accept_out) n_accept_out[rounds] = na[r];
            rounds++;
            for (int j = 0; j <= na[r]; j++) { if (n < cap) tokens[n] = tk[pos + j]; n++; }
            pos += na[r] + 1;
        }
    }
    if (n_rounds) *n_rounds = rounds;
    return n;
}

// Times `iters` launches of one kernel of the round with HIP events on the
// state's stream; returns 0 and the mean per launch.  which:
//   0  tied lm_head GEMV (vocab rows, hidden input) with mrows token rows,
//      back to back;
//   1  the verify forward of mrows tokens (ctl->tok at ctl->anchor_pos + 1..).
//      It reads the ring state at ctl->slot_base and writes the slots after
//      it and KV rows the next verify rewrites, so repeated launches read
//      identical inputs and leave the session's state usable;
//   2  a device-to-device copy of the lm_head's vocab x hidden int8 bytes
//      (the calibration kernel for the HBM byte counters);
//   3  the lm_head GEMV as in 0, each launch after a 512 MiB copy that
//      evicts the device's last-level cache (only the GEMV is timed);
//   4  the RMSNorm-prologue GEMV of the KDA layers' inputs (q, k, v, f_a,
//      b, g projections) over mrows rows, every KDA layer in order, back to
//      back (the mean is per launch);
//   5  the same for the attention layers' inputs (k, v, q);
//   6  the same for every layer's MoE input (router, latent down, shared
//      gate and up).  4-6 read the state's residual rows and write only
//      scratch rows, so the session stays usable.
// Streaming probe: 16 dependent launches of `blocks` blocks of `threads`
// threads, each block streaming its own kb_per_block KiB with all loads of a
// pass in flight, each launch on a fresh region of a 1 GiB buffer (beyond
// the last-level cache); *us_per_launch is the mean per launch.
extern "C" int l98_time_stream(LZRunState *s, int blocks, int threads, int kb_per_block, int iters,
                               float *us_per_launch) {
    if (!s || !s->impl || blocks < 1 || kb_per_block < 1 || iters < 1 || !us_per_launch) return 1;
    DState *d = S(s);
    const size_t per = (size_t)kb_per_block << 10, span = per * (size_t)blocks, total = (size_t)1 << 30;
    if (span > total / 16) return 1;
    char *buf = nullptr;
    if (hipMalloc(&buf, total + 4096) != hipSuccess) return 1;
    int rc = hipMemsetAsync(buf, 1, total, d->st) != hipSuccess;
    int *out = reinterpret_cast<int *>(buf + total);
    float ms = 0.0f;
    if (!rc) rc = l98k_stream(buf, blocks, threads, (int)(per / 16), out, d->st);
    if (!rc) {
        (void)hipEventRecord(d->ev0, d->st);
        for (int it = 0; it < iters && !rc; it++)
            for (int i = 0; i < 16 && !rc; i++)
                rc = l98k_stream(buf + (size_t)i * (total / 16), blocks, threads, (int)(per / 16), out, d->st);
        (void)hipEventRecord(d->ev1, d->st);
        if (!rc && hipEventSynchronize(d->ev1) != hipSuccess) rc = 1;
        if (!rc) (void)hipEventElapsedTime(&ms, d->ev0, d->ev1);
    }
    (void)hipStreamSynchronize(d->st);
    (void)hipFree(buf);
    if (rc) return 1;
    *us_per_launch = ms * 1e3f / (float)(16 * iters);
    return 0;
}

extern "C" int l98_time_kernel(const LZModel *mm, LZRunState *s, int which, int mrows, int iters,
                               float *avg_ms) {
    if (!mm || !s || !s->impl || iters < 1 || mrows < 1 || mrows > MAX_CHUNK || !avg_ms) return 1;
    DState *d = S(s);
    const DModel *m = d->m;
    const LZModelConfig &c = m->c;
    if (which >= 7 && which <= 11) {
        // launch floor: a chain of CHAIN dependent launches (7: empty
        // kernel, 1 block; 8: empty, 256 blocks; 9: 256 blocks each reading
        // the mrows x hidden floats the previous launch wrote; 11: mode 9
        // plus a last-block reduction per 8 blocks (release, counter,
        // acquire, the group's partials read back); all captured once as a
        // HIP graph and replayed; 10: mode 8 launched on the stream without
        // a graph); avg_ms is per launch
        const int CHAIN = 64, n = mrows * c.hidden_size;
        const int grid = which == 7 ? 1 : 256, kind = which == 9 ? 1 : which == 11 ? 2 : 0;
        if (n < 256 || n > 8192) return 1;
        float *buf = nullptr;
        // two n-float buffers, then (mode 11) grid x 256 partials and the counters
        const size_t nbuf = 2 * (size_t)n + (size_t)grid * 256 + grid;
        if (hipMalloc(&buf, nbuf * sizeof(float)) != hipSuccess) return 1;
        int rc = hipMemsetAsync(buf, 0, nbuf * sizeof(float), d->st) != hipSuccess;
        hipGraph_t g = nullptr;
        hipGraphExec_t ge = nullptr;
        auto chain = [&]() { return l98k_launch_chain(kind, CHAIN, grid, buf, buf + n, n, d->st); };
        if (!rc && which != 10) {
            if (hipStreamBeginCapture(d->st, hipStreamCaptureModeThreadLocal) != hipSuccess) rc = 1;
            else {
                const int crc = chain();
                if (hipStreamEndCapture(d->st, &g) != hipSuccess || crc) rc = 1;
                else if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) rc = 1;
            }
        }
        auto once = [&]() { return which == 10 ? chain() : (int)(hipGraphLaunch(ge, d->st) != hipSuccess); };
        float ms = 0.0f;
        if (!rc) rc = once();
        if (!rc) {
            (void)hipEventRecord(d->ev0, d->st);
            for (int i = 0; i < iters && !rc; i++) rc = once();
            (void)hipEventRecord(d->ev1, d->st);
            if (!rc && hipEventSynchronize(d->ev1) != hipSuccess) rc = 1;
            if (!rc) (void)hipEventElapsedTime(&ms, d->ev0, d->ev1);
        }
        (void)hipStreamSynchronize(d->st);
        if (ge) (void)hipGraphExecDestroy(ge);
        if (g) (void)hipGraphDestroy(g);
        (void)hipFree(buf);
        if (rc) return 1;
        *avg_ms = ms / (float)iters / (float)CHAIN;
        return 0;
    }
    if (which < 0 || which > 6) return 1;
    std::vector<int> layers;                    // the layers modes 4-6 run, in order
    for (int l = 0; l < c.n_layers; l++)
        if ((which == 4 && m->L[l].type == 2) || (which == 5 && m->L[l].type == 1) || which == 6) layers.push_back(l);
    if (which >= 4 && layers.empty()) return 1;
    const int per_iter = which >= 4 ? (int)layers.size() : 1;
    const size_t wbytes = (size_t)c.vocab_size * c.hidden_size;
    const size_t flush_bytes = (size_t)512 << 20;
    const bool cold = which == 3;
    void *scratch = nullptr;
    if (which >= 2 && hipMalloc(&scratch, which == 2 ? wbytes : 2 * flush_bytes) != hipSuccess) return 1;
    const int d_ = c.hidden_size;
    const float eps = c.rms_norm_eps;
    auto once = [&]() -> int {
        if (which == 0 || which == 3)
            return gemv(d, {JX(m->embed, d->mtp_logits, c.vocab_size, d->xq, d->xqs)}, mrows);
        if (which == 2)
            return hipMemcpyAsync(scratch, m->embed.q, wbytes, hipMemcpyDeviceToDevice, d->st) != hipSuccess;
        for (int l : layers) {
            const DLayer &L = m->L[l];
            int rc = 0;
            if (which == 4) {
                const Prologue P = PN(d->x, d_, d->up_out, d->sd_out, L.in_norm, eps, d->x2, nullptr, 0);
                rc = gemv(d, {J(L.kq, d->pq, c.lin_key_dim, P), J(L.kk, d->pk, c.lin_key_dim, P),
                              J(L.kv, d->pv, c.lin_value_dim, P), J(L.fa, d->pfa, c.kda_gate_rank, P),
                              J(L.kb, d->pb, c.lin_n_v_heads, P), J(L.kg, d->pg, c.lin_value_dim, P)}, mrows);
            } else if (which == 5) {
                const Prologue P = PN(d->x, d_, d->up_out, d->sd_out, L.in_norm, eps, d->x2, nullptr, 0);
                rc = gemv(d, {J(L.k, d->kp, c.attn_kv_dim, P), J(L.v, d->vp, c.attn_kv_dim, P),
                              J(L.q, d->qg, c.attn_qgate_dim, P)}, mrows);
            } else {
                const Prologue P = PN(d->x, d_, d->blk, nullptr, L.post_norm, eps, d->x2, nullptr, 0);
                rc = gemv(d, {J(L.router, d->rl, c.num_experts, P), J(L.down, d->latx, c.moe_latent_dim, P),
                              J(L.sg, d->sgo, c.moe_shared_width, P), J(L.su, d->suo, c.moe_shared_width, P)},
                          mrows);
            }
            if (rc) return rc;
        }
        if (which >= 4) return 0;
        return forward_chunk(d, d->ctl->tok, mrows, &d->ctl->anchor_pos, 1, d->seq_len - 1, d->vhidden, true,
                             d->mtp_logits, false);
    };
    int rc = 0;
    float ms = 0.0f;
    if (once()) rc = 1;
    if (!rc && !cold) {
        (void)hipEventRecord(d->ev0, d->st);
        for (int i = 0; i < iters && !rc; i++) rc = once();
        (void)hipEventRecord(d->ev1, d->st);
        if (!rc && hipEventSynchronize(d->ev1) != hipSuccess) rc = 1;
        if (!rc) (void)hipEventElapsedTime(&ms, d->ev0, d->ev1);
    } else if (!rc) {
        char *fl = (char *)scratch;
        for (int i = 0; i < iters && !rc; i++) {
            if (hipMemcpyAsync(fl + flush_bytes, fl, flush_bytes, hipMemcpyDeviceToDevice, d->st) != hipSuccess) rc = 1;
            (void)hipEventRecord(d->ev0, d->st);
            if (!rc) rc = once();
            (void)hipEventRecord(d->ev1, d->st);
            float one = 0.0f;
            if (!rc && hipEventSynchronize(d->ev1) != hipSuccess) rc = 1;
            if (!rc) (void)hipEventElapsedTime(&one, d->ev0, d->ev1);
            ms += one;
        }
    }
    if (scratch) (void)hipFree(scratch);
    if (rc) return 1;
    *avg_ms = ms / (float)iters / (float)per_iter;
    return 0;
}

// Attention kernels against the Q8 KV cache
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_devmath.h"

// ------------------------------------------------------------ attention ---

// One 64-lane block per (token, head): RMSNorm(1+w) of a q head (read from
// the interleaved [q | gate] projection) or a k head, NeoX rotary on the
// first rot dims, then q to qh or k quantized per 32 into the KV plane at
// slot pos; the last nkv blocks of a token quantize v heads.
// (attn_impl src/forward_attn.c:878-960; lz_rope src/ops_rope.c:21-67.)
__device__ __forceinline__ void attn_prep_body(const AttnArgs &a, int t, int hh) {
    __shared__ __align__(16) float sh[256], sq[256];
    __shared__ float s_inv;
    const int nq = a.kv_only ? 0 : a.nh;
    const int lane = threadIdx.x;
    const int hd = a.hd, half = a.rot >> 1;
    const int pos = *a.ctl_pos + a.pos_off + t;
    if (hh >= nq + a.nkv) {                       // v head: quantize the projection
        const int h = hh - nq - a.nkv;
        for (int base = 0; base < hd; base += 64) {
            int i = base + lane;
            if (base + (lane & ~31) < hd) {
                int col = h * hd + i;
                float v = a.vp[(size_t)t * a.kv_dim + col];
                d_quant_group32(v, a.vcache + (size_t)pos * a.kv_dim + col,
                                a.vscale + (size_t)pos * (a.kv_dim >> 5) + (col >> 5));
            }
        }
        return;
    }
    const bool isq = hh < nq;
    const int h = isq ? hh : hh - nq;
    const float *src = isq ? a.qg + (size_t)t * a.qg_dim + (size_t)h * 2 * hd
                           : a.kp + (size_t)t * a.kv_dim + (size_t)h * hd;
    const float *nw = isq ? a.q_norm : a.k_norm;
    const float *cs = a.rope_cs + (size_t)pos * half * 2;
    float v[4], w[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int ic = imin(lane + 64 * u, hd - 1);
        v[u] = src[ic];
        w[u] = nw[ic];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int i = lane + 64 * u;
        if (i < hd) { sh[i] = v[u]; sq[i] = v[u] * v[u]; }
    }
    __syncthreads();
    if (lane == 0) s_inv = d_rsqrt(d_ss_over_n(serial_sum(sq, hd), hd) + a.eps);
    __syncthreads();
    const float inv = s_inv;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int i = lane + 64 * u;
        if (i < hd) sh[i] = v[u] * inv * (1.0f + w[u]);
    }
    __syncthreads();
    for (int i = lane; i < half; i += 64) {
        float c = cs[i * 2], s = cs[i * 2 + 1];
        float x0 = sh[i], x1 = sh[i + half];
        sh[i] = x0 * c - x1 * s;
        sh[i + half] = x1 * c + x0 * s;
    }
    __syncthreads();
    if (isq) {
        for (int i = lane; i < hd; i += 64) a.qh[(size_t)t * a.q_dim + (size_t)h * hd + i] = sh[i];
    } else {
        for (int base = 0; base < hd; base += 64) {
            int i = base + lane;
            if (base + (lane & ~31) < hd) {
                int col = h * hd + i;
                d_quant_group32(sh[i], a.kcache + (size_t)pos * a.kv_dim + col,
                                a.kscale + (size_t)pos * (a.kv_dim >> 5) + (col >> 5));
            }
        }
    }
}

__global__ __launch_bounds__(64) void k_attn_prep(AttnArgs a) {
    const int per_tok = (a.kv_only ? 0 : a.nh) + 2 * a.nkv;
    const int t = blockIdx.x / per_tok;
    attn_prep_body(a, t, blockIdx.x - t * per_tok);
}

// Attention of the chunk's tokens against the Q8 KV cache (attn_score_loop
// Q8 branch, src/forward_attn.c:206-660; score_q8_row :30-41; lz_softmax
// src/ops_norm.c:903-990; wsum_q8_row :17-21).  A session's chunk (<= 8
// rows) runs as one launch, k_attn_fused: block (q head, token) computes its
// own scores (see attn_av_body), then the softmax and value sum.  The
// many-item launch (the session batch's verify rows, a prefill's rows) has
// two kernels:
//
// k_attn_scores_items: one block per (64-position slice, kv head, token).
// The block prepares what it needs itself: the kv_mul q heads of the token
// (RMSNorm(1+w), NeoX rotary: src/forward_attn.c:878-960, src/ops_rope.c:
// 21-67) and, for positions of the chunk's own tokens, the K rows from the
// K projection (norm, rotary, per-32 quantization); every other K row comes
// from the cache.  The block of token t' whose slice holds t''s position
// writes t''s K and V rows to the cache, so each new row is written once.
// One thread per (q head, position) computes the score: each 32-group
// product sum serial, then the groups serial (score_q8_row order), times
// attn_scale.  Scores go to att [token][head][position].
#define ATT_SLICE 64
#define ATT_MAX_HD 128
#define ATT_MAX_VEC 24                  // kv_mul q heads + up to MAX_CHUNK new K rows

// NV: the vectors the block prepares at most (kv_mul + MAX_CHUNK); the
// kernels take 12 when kv_mul <= 4, so more blocks share a CU's LDS.
template <int NV = ATT_MAX_VEC>
__device__ __forceinline__ void attn_scores_body(const AttnArgs &a, float *__restrict__ att, int att_stride, int slice,
                                                 int kvh, int t) {
    __shared__ __align__(16) float s_x[NV * ATT_MAX_HD];     // vectors being prepared
    __shared__ __align__(16) float s_sq[NV * (ATT_MAX_HD + 4)];
    __shared__ float s_inv[NV];
    __shared__ __align__(16) int8_t s_k[ATT_SLICE * (ATT_MAX_HD + 16)];   // K rows, padded
    __shared__ float s_ks[ATT_SLICE * (ATT_MAX_HD / 32)];
    const int tid = threadIdx.x;
    const int hd = a.hd, half = a.rot >> 1, kv_mul = a.nh / a.nkv, nb = hd >> 5;
    const int kstride = hd + 16;
    const int pos0 = *a.ctl_pos + a.pos_off;
    const int pos_t = pos0 + t, L = pos_t + 1;
    const int p_lo = slice * ATT_SLICE;
    if (p_lo >= L) return;
    const int n_here = imin(ATT_SLICE, L - p_lo);
    // new rows of this slice: chunk tokens t' <= t with position in the slice
    const int nr_lo = imin(imin(t + 1, imax(0, p_lo - pos0)), t + 1);
    const int nr_hi = imin(t + 1, imax(0, p_lo + n_here - pos0));
    const int n_new = nr_hi - nr_lo;
    const int nvec = kv_mul + n_new;
    const int h0 = kvh * kv_mul;
    // 1. loads: cached K rows of the slice (p < pos0), the vectors to prepare
    const int cpr = hd >> 4;
    const int n_cached = imax(0, imin(n_here, pos0 - p_lo));
    for (int base = 0; base < ATT_SLICE * cpr; base += 256) {
        const int idx = base + tid;
        const int r = idx / cpr, c = idx - r * cpr;
        if (r < n_cached)
            *reinterpret_cast<int4 *>(s_k + r * kstride + c * 16) =
                *reinterpret_cast<const int4 *>(a.kcache + (size_t)(p_lo + r) * a.kv_dim + kvh * hd + c * 16);
    }
    for (int idx = tid; idx < n_cached * nb; idx += 256) {
        const int r = idx / nb, g = idx - r * nb;
        s_ks[r * nb + g] = a.kscale[(size_t)(p_lo + r) * (a.kv_dim >> 5) + kvh * nb + g];
    }
    for (int f = tid; f < nvec * hd; f += 256) {
        const int v = f / hd, i = f - v * hd;
        const float x = v < kv_mul ? a.qg[(size_t)t * a.qg_dim + (size_t)(h0 + v) * 2 * hd + i]
                                   : a.kp[(size_t)(nr_lo + v - kv_mul) * a.kv_dim + kvh * hd + i];
        s_x[v * hd + i] = x;
        s_sq[v * (hd + 4) + i] = x * x;
    }
    __syncthreads();
    // 2. RMSNorm sums, one lane per vector (serial, index order)
    if (tid < nvec) s_inv[tid] = d_rsqrt(d_ss_over_n(serial_sum(s_sq + tid * (hd + 4), hd), hd) + a.eps);
    __syncthreads();
    for (int f = tid; f < nvec * hd; f += 256) {
        const int v = f / hd, i = f - v * hd;
        const float w = v < kv_mul ? a.q_norm[i] : a.k_norm[i];
        s_x[v * hd + i] = s_x[v * hd + i] * s_inv[v] * (1.0f + w);
    }
    __syncthreads();
    // 3. rotary on the first rot dims (pairs i, i + half)
    for (int f = tid; f < nvec * half; f += 256) {
        const int v = f / half, i = f - v * half;
        const int pos = v < kv_mul ? pos_t : pos0 + nr_lo + v - kv_mul;
        const float c = a.rope_cs[((size_t)pos * half + i) * 2], s = a.rope_cs[((size_t)pos * half + i) * 2 + 1];
        const float x0 = s_x[v * hd + i], x1 = s_x[v * hd + i + half];
        s_x[v * hd + i] = x0 * c - x1 * s;
        s_x[v * hd + i + half] = x1 * c + x0 * s;
    }
    __syncthreads();
    // 4. new K rows: per-32 quantization into the slice (and the cache, by the
    //    token's own block); its V row goes to the cache too.  Groups are 32
    //    consecutive lanes (hd % 32 == 0, 256 % hd == 0 or hd % 256 == 0).
    for (int base = 0; base < NV * ATT_MAX_HD; base += 256) {
        const int f = base + tid;
        const int nk = n_new * hd;
        if (base >= nk) break;                       // uniform over the block
        const int fc = imin(f, nk - 1);
        const int r = fc / hd, i = fc - r * hd;
        const int tt = nr_lo + r, p = pos0 + tt;
        const float y = s_x[(kv_mul + r) * hd + i];
        int8_t q;
        float sg;
        d_quant_group32(y, &q, &sg);
        if (f < nk) {
            s_k[(p - p_lo) * kstride + i] = q;
            if ((i & 31) == 0) s_ks[(p - p_lo) * nb + (i >> 5)] = sg;
            if (tt == t) {
                a.kcache[(size_t)p * a.kv_dim + kvh * hd + i] = q;
                if ((i & 31) == 0) a.kscale[(size_t)p * (a.kv_dim >> 5) + kvh * nb + (i >> 5)] = sg;
            }
        }
        const float vv = a.vp[(size_t)tt * a.kv_dim + kvh * hd + i];
        int8_t qv;
        float sv;
        d_quant_group32(vv, &qv, &sv);
        if (f < nk && tt == t) {
            a.vcache[(size_t)p * a.kv_dim + kvh * hd + i] = qv;
            if ((i & 31) == 0) a.vscale[(size_t)p * (a.kv_dim >> 5) + kvh * nb + (i >> 5)] = sv;
        }
    }
    __syncthreads();
    // 5. scores: item = (q head g, position) ; a wave shares g
    const float scale = a.attn_scale;
    for (int item = tid; item < kv_mul * ATT_SLICE; item += 256) {
        const int g = item / ATT_SLICE, pl = item - g * ATT_SLICE;
        if (pl >= n_here) continue;
        const int8_t *kr = s_k + pl * kstride;
        const float *ks = s_ks + pl * nb;
        const float *qq = s_x + g * hd;
        float sum = 0.0f;
        for (int dd = 0; dd < hd; dd += 32) {
            const int4 k0 = *reinterpret_cast<const int4 *>(kr + dd);
            const int4 k1 = *reinterpret_cast<const int4 *>(kr + dd + 16);
            const int8_t *kb0 = reinterpret_cast<const int8_t *>(&k0);
            const int8_t *kb1 = reinterpret_cast<const int8_t *>(&k1);
            float acc = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; e++) acc += qq[dd + e] * (float)kb0[e];
#pragma unroll
            for (int e = 0; e < 16; e++) acc += qq[dd + 16 + e] * (float)kb1[e];
            sum += acc * ks[dd >> 5];
        }
        att[((size_t)t * a.nh + h0 + g) * att_stride + p_lo + pl] = sum * scale;
    }
}

// One launch over several sessions' rows (the session batch's verify), or
// over one session's prefill rows cut into MAX_CHUNK-row items whose K and V
// rows are all in the cache before the launch: item i is rows [row0, row0 +
// n) (n <= MAX_CHUNK) against its KV plane, positions *ctl_pos + pos_off +
// t; the launch's AttnArgs carry the layer's weights and the row buffers at
// row 0.  Block z = (item, token).
__device__ __forceinline__ AttnArgs attn_item_args(const AttnArgs &b, const AttnItem &it, int plane) {
    AttnArgs a = b;
    const size_t off = (size_t)plane * it.seq_len * b.kv_dim;
    a.qg = b.qg + (size_t)it.row0 * b.qg_dim;
    a.kp = b.kp + (size_t)it.row0 * b.kv_dim;
    a.vp = b.vp + (size_t)it.row0 * b.kv_dim;
    a.qh = b.qh + (size_t)it.row0 * b.q_dim;
    a.kcache = it.kq + off;
    a.vcache = it.vq + off;
    a.kscale = it.ks + off / 32;
    a.vscale = it.vs + off / 32;
    a.out = b.out ? b.out + (size_t)it.row0 * b.q_dim : nullptr;
    a.oq = b.oq + (size_t)it.row0 * b.q_dim;
    a.oqs = b.oqs + (size_t)it.row0 * (b.q_dim >> 5);
    a.ctl_pos = it.ctl_pos;
    a.pos_off = it.pos_off;
    return a;
}

__global__ __launch_bounds__(256) void k_attn_scores_items(AttnArgs b, const AttnItem *__restrict__ items, int plane,
                                                           float *__restrict__ att, int att_stride,
                                                           size_t att_item) {
    const int item = blockIdx.z / MAX_CHUNK, t = blockIdx.z - item * MAX_CHUNK;
    const AttnItem it = items[item];
    if (t >= it.n) return;
    const AttnArgs a = attn_item_args(b, it, plane);
    attn_scores_body(a, att + (size_t)item * att_item, att_stride, blockIdx.x, blockIdx.y, t);
}

// k_attn_av_items: one block of 8 waves per (q head, token).  Softmax over the
// token's scores (max, exp, the serial loop's sum - taken by the exact wave
// sum up to 2048 positions -, scale), then the value sum
// out[d] = sum_p a[p] * v[p][d] * vs[p][d/32] walked in position order by
// one lane per d.  The V rows of up to `sc` positions are staged in LDS
// with every load in flight; the products (a*v)*vs of 64 positions at a
// time are formed by the producer waves into a double buffer [d][64] while
// the consumer lanes (hd/64 waves) add the previous 64 in order, so the
// consumer's loop is one LDS read per four adds.  Then the sigmoid output
// gate and the per-32 quantization of the head's output (the o_proj input).
// CH: positions per product chunk (128 where the block's LDS holds the
// larger double buffer, else 64); a d row of the buffer is CH + 4 floats
// (bank spread)
#define AV_ESUM_FLOATS (64 * (32 + 4))  // padded exp row of the exact wave sum (L <= 2048)

// Stages V rows [p0, p0 + n) of kv head kvh (hd int8 + hd/32 scales each)
// into LDS with every load of the block in flight before the first store
// (n * hd / 16 <= AV_THREADS * AV_STAGE_MAX).
#define AV_THREADS 512
#define AV_STAGE_MAX 16
// STEP: cpr = hd/16 and nb = hd/32 divide AV_THREADS, so item
// u * AV_THREADS + tid is tid's (row, column) plus u * (AV_THREADS / cpr)
// rows, with no division per round.  Every round's load is issued (rounds
// past the end read the last item again) before the first store: the empty
// asm takes every loaded register, so the compiler can neither sink a load
// into its store's branch nor copy it out of one, either of which would wait
// out the loads' latency one after another.
// With a score row (arow, L <= AV_SCORE_MAX * AV_THREADS), its loads join
// the same batch and it is stored to s_a.
#define AV_SCORE_MAX 4
template <bool STEP>
__device__ __forceinline__ void av_stage(const int8_t *__restrict__ vc, const float *__restrict__ vs, int kv_dim,
                                         int kvh, int hd, int p0, int n, int8_t *s_v, float *s_vs,
                                         const float *__restrict__ arow, int L, float *s_a) {
    const int tid = threadIdx.x, cpr = hd >> 4, nb = hd >> 5;
    const int total = n * cpr, stotal = n * nb;
    const int8_t *vbase = vc + (size_t)p0 * kv_dim + kvh * hd;
    const float *sbase = vs + (size_t)p0 * (kv_dim >> 5) + kvh * nb;
    const int rstep = AV_THREADS / cpr, sstep = AV_THREADS / nb;
    const int r0 = tid / cpr, c0 = tid - r0 * cpr, rl = (total - 1) / cpr, cl = total - 1 - rl * cpr;
    const int q0 = tid / nb, g0 = tid - q0 * nb, ql = (stotal - 1) / nb, gl = stotal - 1 - ql * nb;
    int4 r[AV_STAGE_MAX];
    float q[AV_STAGE_MAX / 2], sa[AV_SCORE_MAX];
#pragma unroll
    for (int k = 0; k < AV_SCORE_MAX; k++) sa[k] = arow ? arow[imin(k * AV_THREADS + tid, L - 1)] : 0.0f;
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX; u++) {
        const int idx = u * AV_THREADS + tid;
        int row, c;
        if (STEP) {
            const bool in = idx < total;
            row = in ? u * rstep + r0 : rl;
            c = in ? c0 : cl;
        } else {
            const int ic = imin(idx, total - 1);
            row = ic / cpr;
            c = ic - row * cpr;
        }
        r[u] = *reinterpret_cast<const int4 *>(vbase + (size_t)row * kv_dim + c * 16);
    }
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX / 2; u++) {
        const int sidx = u * AV_THREADS + tid;
        int srow, g;
        if (STEP) {
            const bool in = sidx < stotal;
            srow = in ? u * sstep + q0 : ql;
            g = in ? g0 : gl;
        } else {
            const int ic = imin(sidx, stotal - 1);
            srow = ic / nb;
            g = ic - srow * nb;
        }
        q[u] = sbase[(size_t)srow * (kv_dim >> 5) + g];
    }
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX; u++) asm volatile("" : "+v"(r[u].x), "+v"(r[u].y), "+v"(r[u].z), "+v"(r[u].w));
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX / 2; u++) asm volatile("" : "+v"(q[u]));
#pragma unroll
    for (int k = 0; k < AV_SCORE_MAX; k++) asm volatile("" : "+v"(sa[k]));
    if (arow) {
#pragma unroll
        for (int k = 0; k < AV_SCORE_MAX; k++)
            if (k * AV_THREADS + tid < L) s_a[k * AV_THREADS + tid] = sa[k];
    }
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX; u++)
        if (u * AV_THREADS < total) reinterpret_cast<int4 *>(s_v)[imin(u * AV_THREADS + tid, total - 1)] = r[u];
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX / 2; u++)
        if (u * AV_THREADS < stotal) s_vs[imin(u * AV_THREADS + tid, stotal - 1)] = q[u];
}
__device__ __forceinline__ void av_stage_any(const int8_t *__restrict__ vc, const float *__restrict__ vs, int kv_dim,
                                             int kvh, int hd, int p0, int n, int8_t *s_v, float *s_vs,
                                             const float *__restrict__ arow, int L, float *s_a) {
    if (AV_THREADS % (hd >> 4) == 0 && AV_THREADS % (hd >> 5) == 0)
        av_stage<true>(vc, vs, kv_dim, kvh, hd, p0, n, s_v, s_vs, arow, L, s_a);
    else
        av_stage<false>(vc, vs, kv_dim, kvh, hd, p0, n, s_v, s_vs, arow, L, s_a);
}

// FUSED (the chunk path of one session, k_attn_fused): the block first does
// the scores kernel's work for its own (q head, token) over every position,
// into LDS: its q head and the chunk's new K rows 0..t of its kv head
// (RMSNorm(1+w), NeoX rotary, K quantized per 32) and those rows' V
// quantized per 32; positions before the chunk read K from the cache, the
// chunk's positions the block's own rows; token t's K and V rows go to the
// cache from the kv head's first q head's block.  The staged V rows of the
// chunk's positions are then replaced by the block's own (the cache rows may
// still be in flight from other blocks of the launch).
template <int CH, bool FUSED = false>
__device__ __forceinline__ void attn_av_body(const AttnArgs &a, const float *__restrict__ att, int att_stride, int sc,
                                             int h, int t) {
    EXP_TAB_LOAD(tab);
    extern __shared__ __align__(16) char smem[];
    __shared__ uint32_t s_red[AV_THREADS / 64];
    __shared__ float s_inv;
    __shared__ PsRec s_rec[128];
    constexpr int NEWR = FUSED ? MAX_CHUNK : 1;
    __shared__ __align__(16) int8_t s_knew[NEWR * ATT_MAX_HD], s_vnew[NEWR * ATT_MAX_HD];
    __shared__ float s_ksn[NEWR * (ATT_MAX_HD / 32)], s_vsn[NEWR * (ATT_MAX_HD / 32)], s_vin[NEWR + 1];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int hd = a.hd, nb = hd >> 5, kv_mul = a.nh / a.nkv, kvh = h / kv_mul;
    const int pos0 = *a.ctl_pos + a.pos_off, pos_t = pos0 + t, L = pos_t + 1;
    const int Lp = (att_stride + 3) & ~3;
    float *s_a = reinterpret_cast<float *>(smem);                                   // [Lp]
    constexpr int AV_CH = CH, AV_PAD = CH + 4;
    float *prod = s_a + Lp;                                                          // [2][hd][AV_PAD]
    int8_t *s_v = reinterpret_cast<int8_t *>(prod + 2 * hd * AV_PAD);               // [sc][hd]
    float *s_vs = reinterpret_cast<float *>(s_v + (size_t)sc * hd);                  // [sc][nb]
    float *s_e = s_vs + (size_t)sc * nb;                                             // [AV_ESUM_FLOATS]
    const float *arow = FUSED ? nullptr : att + ((size_t)t * a.nh + h) * att_stride;
    const int cpr = hd >> 4;
    // the chunk's rows among V positions [sp0, sp0 + nsc): the block's own
    // quantized rows replace the staged ones
    auto patch_new = [&](int sp0, int nsc) {
        const int lo = imax(pos0, sp0), hi = imin(L, sp0 + nsc);
        for (int f = tid; f < (hi - lo) * hd; f += AV_THREADS) {
            const int r = f / hd, i = f - r * hd;
            s_v[(size_t)(lo + r - sp0) * hd + i] = s_vnew[(lo + r - pos0) * hd + i];
        }
        for (int f = tid; f < (hi - lo) * nb; f += AV_THREADS) {
            const int r = f / nb, g = f - r * nb;
            s_vs[(size_t)(lo + r - sp0) * nb + g] = s_vsn[(lo + r - pos0) * nb + g];
        }
    };
    if constexpr (FUSED) {
        // vectors: 0 = the q head, 1 + r = the chunk's K row r (r <= t);
        // prepared in the product buffer, which the value pass uses later
        float *s_x = prod, *s_sq = prod + (1 + MAX_CHUNK) * ATT_MAX_HD;
        const int nvec = 2 + t, half = a.rot >> 1;
        for (int f = tid; f < nvec * hd; f += AV_THREADS) {
            const int v = f / hd, i = f - v * hd;
            const float x = v == 0 ? a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * hd + i]
                                   : a.kp[(size_t)(v - 1) * a.kv_dim + kvh * hd + i];
            s_x[v * hd + i] = x;
            s_sq[v * (hd + 4) + i] = x * x;
        }
        __syncthreads();
        if (tid < nvec) s_vin[tid] = d_rsqrt(d_ss_over_n(serial_sum(s_sq + tid * (hd + 4), hd), hd) + a.eps);
        __syncthreads();
        for (int f = tid; f < nvec * hd; f += AV_THREADS) {
            const int v = f / hd, i = f - v * hd;
            const float w = v == 0 ? a.q_norm[i] : a.k_norm[i];
            s_x[v * hd + i] = s_x[v * hd + i] * s_vin[v] * (1.0f + w);
        }
        __syncthreads();
        for (int f = tid; f < nvec * half; f += AV_THREADS) {
            const int v = f / half, i = f - v * half;
            const int pos = v == 0 ? pos_t : pos0 + v - 1;
            const float c = a.rope_cs[((size_t)pos * half + i) * 2], sn = a.rope_cs[((size_t)pos * half + i) * 2 + 1];
            const float x0 = s_x[v * hd + i], x1 = s_x[v * hd + i + half];
            s_x[v * hd + i] = x0 * c - x1 * sn;
            s_x[v * hd + i + half] = x1 * c + x0 * sn;
        }
        __syncthreads();
        // K rows 0..t and their V rows per 32 (32-lane groups: hd % 32 == 0)
        const bool writer = h == kvh * kv_mul;
        for (int base = 0; base < (t + 1) * hd; base += AV_THREADS) {
            const int nk = (t + 1) * hd, f = base + tid;
            const int fc = imin(f, nk - 1), r = fc / hd, i = fc - r * hd;
            int8_t qk, qv;
            float sk, sv;
            d_quant_group32(s_x[(1 + r) * hd + i], &qk, &sk);
            d_quant_group32(a.vp[(size_t)r * a.kv_dim + kvh * hd + i], &qv, &sv);
            if (f < nk) {
                s_knew[r * hd + i] = qk;
                s_vnew[r * hd + i] = qv;
                if ((i & 31) == 0) { s_ksn[r * nb + (i >> 5)] = sk; s_vsn[r * nb + (i >> 5)] = sv; }
                if (writer && r == t) {
                    const size_t row = (size_t)pos_t * a.kv_dim + kvh * hd + i;
                    a.kcache[row] = qk;
                    a.vcache[row] = qv;
                    if ((i & 31) == 0) {
                        const size_t srow = (size_t)pos_t * (a.kv_dim >> 5) + kvh * nb + (i >> 5);
                        a.kscale[srow] = sk;
                        a.vscale[srow] = sv;
                    }
                }
            }
        }
        __syncthreads();
        // scores: each 32-group's products summed in order, then the groups,
        // times attn_scale (score_q8_row)
        const float scale = a.attn_scale;
        auto score = [&](const int8_t *kr, const float *ks) {
            float sum = 0.0f;
            for (int dd = 0; dd < hd; dd += 32) {
                const int4 k0 = *reinterpret_cast<const int4 *>(kr + dd);
                const int4 k1 = *reinterpret_cast<const int4 *>(kr + dd + 16);
                const int8_t *kb0 = reinterpret_cast<const int8_t *>(&k0);
                const int8_t *kb1 = reinterpret_cast<const int8_t *>(&k1);
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) acc += s_x[dd + e] * (float)kb0[e];
#pragma unroll
                for (int e = 0; e < 16; e++) acc += s_x[dd + 16 + e] * (float)kb1[e];
                sum += acc * ks[dd >> 5];
            }
            return sum * scale;
        };
        for (int p = tid; p < L; p += AV_THREADS) {
            if (p < pos0)
                s_a[p] = score(a.kcache + (size_t)p * a.kv_dim + kvh * hd,
                               a.kscale + (size_t)p * (a.kv_dim >> 5) + kvh * nb);
            else
                s_a[p] = score(s_knew + (p - pos0) * hd, s_ksn + (p - pos0) * nb);
        }
    }
    // scores and the first V stage -> LDS, their loads in one batch (score
    // rows past AV_SCORE_MAX * AV_THREADS positions: the rest after)
    av_stage_any(a.vcache, a.vscale, a.kv_dim, kvh, hd, 0, imin(sc, L), s_v, s_vs, arow, L, s_a);
    if constexpr (!FUSED)
        for (int p = AV_SCORE_MAX * AV_THREADS + tid; p < L; p += AV_THREADS) s_a[p] = arow[p];
    EXP_TAB_PUT(tab);
    __syncthreads();
    if constexpr (FUSED) patch_new(0, imin(sc, L));    // (the softmax's barriers come before any read)
    // softmax: max (order-preserving key), exp, serial sum, scale
    uint32_t best = 0;
    for (int p = tid; p < L; p += AV_THREADS) best = umax(best, d_fkey(s_a[p]));
    for (int o = 32; o > 0; o >>= 1) best = umax(best, (uint32_t)__shfl_xor((int)best, o));
    if (lane == 0) s_red[wave] = best;
    __syncthreads();
    uint32_t bk = s_red[0];
#pragma unroll
    for (int w = 1; w < AV_THREADS / 64; w++) bk = umax(bk, s_red[w]);
    const float mx = d_unkey(bk);
    // the exps also go to the padded row layout of the exact wave sum
    // (lane chunks of 8, 16 or 32 for L up to 512, 1024, 2048)
    const int esh = L <= 512 ? 3 : L <= 1024 ? 4 : 5, ech = 1 << esh;
    for (int p = tid; p < L; p += AV_THREADS) {
        const float e = d_exp(s_a[p] - mx, tab);
        s_a[p] = e;
        s_e[(p >> esh) * (ech + 4) + (p & (ech - 1))] = e;
    }
    __syncthreads();
    if (wave == 0) {                     // the serial loop's sum, bit for bit
        float sum;
        if (L > 2048)
            sum = serial_sum(s_a, L);
        else if (esh == 3)
            sum = wave_sum_nonneg<8>(s_e, L, s_rec);
        else if (esh == 4)
            sum = wave_sum_nonneg<16>(s_e, L, s_rec);
        else
            sum = wave_sum_nonneg<32>(s_e, L, s_rec);
        if (lane == 0) s_inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = s_inv;
    for (int p = tid; p < L; p += AV_THREADS) s_a[p] *= inv;
    __syncthreads();
    // value sum
    const int ncons = (hd + 63) >> 6;              // consumer waves
    const bool cons = wave < ncons;
    const int d = wave * 64 + lane;
    const int nprod = AV_THREADS - ncons * 64, ptid = tid - ncons * 64;
    float o = 0.0f;
    // products of chunk positions [q0, q0 + AV_CH) of the staged range starting at sp0
    auto produce = [&](int q0, int sp0, int nsc, int buf) {
        float *pb = prod + (size_t)buf * hd * AV_PAD;
        for (int u = ptid; u < AV_CH * cpr; u += nprod) {
            const int pl = u / cpr, seg = u - pl * cpr;
            const int p = q0 + pl;                   // absolute position
            const int ls = p - sp0;                  // row in the stage
            // rows past the staged range use row 0 with a = 0: the product
            // is +-0, and adding +-0 leaves the sum unchanged
            const bool live = ls < nsc;
            const int4 v4 = reinterpret_cast<const int4 *>(s_v)[(live ? ls : 0) * cpr + seg];
            const float ap = live ? s_a[p] : 0.0f, vsc = s_vs[(live ? ls : 0) * nb + (seg >> 1)];
            const int vw[4] = {v4.x, v4.y, v4.z, v4.w};
            float pr[16];
#pragma unroll
            for (int i = 0; i < 16; i++) pr[i] = ap * (float)(int8_t)((vw[i >> 2] >> (8 * (i & 3))) & 0xFF) * vsc;
#pragma unroll
            for (int i = 0; i < 16; i++) pb[(seg * 16 + i) * AV_PAD + pl] = pr[i];
        }
    };
    for (int sp0 = 0; sp0 < L; sp0 += sc) {
        const int nsc = imin(sc, L - sp0);
        if (sp0 > 0) {
            __syncthreads();
            av_stage_any(a.vcache, a.vscale, a.kv_dim, kvh, hd, sp0, nsc, s_v, s_vs, nullptr, 0, nullptr);
            __syncthreads();
            if constexpr (FUSED) {
                patch_new(sp0, nsc);
                __syncthreads();
            }
        }
        const int nch = (nsc + AV_CH - 1) / AV_CH;
        if (!cons) produce(sp0, sp0, nsc, 0);
        __syncthreads();
        for (int c = 0; c < nch; c++) {
            if (cons) {
                if (d < hd) {
                    // all of the chunk's reads in flight before the first add
                    const float *pr = prod + (size_t)(c & 1) * hd * AV_PAD + (size_t)d * AV_PAD;
                    float4 q[AV_CH / 4];
#pragma unroll
                    for (int i = 0; i < AV_CH / 4; i++) q[i] = *reinterpret_cast<const float4 *>(pr + 4 * i);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < AV_CH / 4; i++) { o += q[i].x; o += q[i].y; o += q[i].z; o += q[i].w; }
                }
            } else if (c + 1 < nch) {
                produce(sp0 + (c + 1) * AV_CH, sp0, nsc, (c + 1) & 1);
            }
            __syncthreads();
        }
    }
    if (cons) {
        const int dc = d < hd ? d : hd - 1;
        const float gate = a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * hd + hd + dc];
        o *= d_sigmoid(gate, tab);
        const int col = h * hd + dc;
        if (a.out && d < hd) a.out[(size_t)t * a.q_dim + col] = o;
        int8_t q;
        float sg;
        d_quant_group32(o, &q, &sg);
        if (d < hd) {
            a.oq[(size_t)t * a.q_dim + col] = q;
            if ((dc & 31) == 0) a.oqs[(size_t)t * (a.q_dim >> 5) + (col >> 5)] = sg;
        }
    }
}

// The chunk path of one session in one launch: block (q head, token) does
// its own scores (see attn_av_body, FUSED), then the softmax and value sum.
template <int CH>
__global__ __launch_bounds__(AV_THREADS) void k_attn_fused(AttnArgs a, int att_stride, int sc) {
    attn_av_body<CH, true>(a, nullptr, att_stride, sc, blockIdx.x, blockIdx.y);
}

template <int CH>
__global__ __launch_bounds__(AV_THREADS) void k_attn_av_items(AttnArgs b, const AttnItem *__restrict__ items,
                                                       int plane, const float *__restrict__ att, int att_stride,
                                                       size_t att_item, int sc) {
    const int item = blockIdx.y / MAX_CHUNK, t = blockIdx.y - item * MAX_CHUNK;
    const AttnItem it = items[item];
    if (t >= it.n) return;
    const AttnArgs a = attn_item_args(b, it, plane);
    attn_av_body<CH>(a, att + (size_t)item * att_item, att_stride, sc, blockIdx.x, t);
}

// The chunk path of one session at long contexts, in two launches instead
// of k_attn_fused's single block per (q head, token), which walks every
// position's score, the softmax's serial sum and the value chains on one CU:
//   k_attn_scores_chunk: one block per (64-position slice, kv head, token),
//     attn_scores_body: the kv_mul q heads and the slice's new K rows
//     prepared in the block, the scores into att, the new K and V rows into
//     the cache by their own token's block;
//   k_attn_avg<HD>: one block per (q head, token, 32-wide output group):
//     the token's score row, the softmax (max by order-preserving key, exp,
//     the serial loop's sum by the exact wave sum over segments of AG_SEG
//     values, each segment's sum entering the next as its first element,
//     scale), then the group's 32 value chains in position order: four
//     producer waves form (a * v) * vs for AG_CH positions at a time into a
//     double buffer while lanes 0-31 of wave 0 add the previous AG_CH, the
//     producers' V loads running AG_NPF chunks ahead (the first ones issued
//     before the softmax); then the gate and the group's quantization.
// The arithmetic is attn_av_body's, so the bits are k_attn_fused's.
#define AG_CH 128
#define AG_PAD (AG_CH + 4)
#define AG_NPF 4
#define AG_THREADS 320
#define AG_SEG 2047
template <int NV>
__global__ __launch_bounds__(256) void k_attn_scores_chunk(AttnArgs a, float *att, int att_stride) {
    attn_scores_body<NV>(a, att, att_stride, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Dynamic LDS of k_attn_avg: the product double buffer, then the score
// row in the exact sum's segment layout (segment k: slot 0 the carried sum,
// then positions k * AG_SEG ..; the scores, the exps and the weights in
// turn occupy the same slots).
__host__ __device__ inline int ag_segments(int att_stride) { return (att_stride + AG_SEG - 1) / AG_SEG; }
__host__ __device__ inline size_t ag_lds_bytes(int att_stride) {
    return (2 * 32 * AG_PAD + (size_t)ag_segments(att_stride) * ps_row_floats<32>()) * sizeof(float);
}
__device__ __forceinline__ int ag_slot(int p) {
    const int k = p / AG_SEG;
    return k * ps_row_floats<32>() + ps_slot<32>(p - k * AG_SEG + 1);
}

template <int HD>
__global__ __launch_bounds__(AG_THREADS) void k_attn_avg(AttnArgs a, const float *__restrict__ att, int att_stride) {
    EXP_TAB_LOAD(tab);
    extern __shared__ __align__(16) char smem[];
    __shared__ uint32_t s_red[AG_THREADS / 64];
    __shared__ float s_inv;
    __shared__ PsRec s_rec[128];
    constexpr int NB = HD / 32, PSR = ps_row_floats<32>();
    const int h = blockIdx.x, t = blockIdx.y, g = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = h / (a.nh / a.nkv);
    const int L = *a.ctl_pos + a.pos_off + t + 1;
    const int nch = (L + AG_CH - 1) / AG_CH, nseg = (L + AG_SEG - 1) / AG_SEG;
    float *prod = reinterpret_cast<float *>(smem);                       // [2][32][AG_PAD]
    float *s_ps = prod + 2 * 32 * AG_PAD;                                 // [segments][PSR]
    // producers: thread ptid takes position ptid / 2 of each chunk, bytes
    // 16 (ptid % 2) .. +16 of the group
    const bool prodw = wave >= 1;
    const int ptid = tid - 64, pp = ptid >> 1, ph = ptid & 1;
    const int8_t *vb = a.vcache + kvh * HD + 32 * g + 16 * ph;
    const float *vsb = a.vscale + kvh * NB + g;
    const size_t vst = (size_t)a.kv_dim, sst = (size_t)(a.kv_dim >> 5);
    int4 r[AG_NPF];
    float rs[AG_NPF];
    // chunk c's piece into ring slot J (a constant after unrolling);
    // positions past the row re-read its last one
#define AG_LOAD(c_, J)                                                         \
    do {                                                                       \
        const int p_ = imin((c_) * AG_CH + pp, L - 1);                         \
        r[J] = *reinterpret_cast<const int4 *>(vb + (size_t)p_ * vst);         \
        rs[J] = vsb[(size_t)p_ * sst];                                         \
    } while (0)
    if (prodw) {
#pragma unroll
        for (int j = 0; j < AG_NPF; j++) AG_LOAD(j, j);
    }
    // the score row, its max by order-preserving key
    const float *arow = att + ((size_t)t * a.nh + h) * att_stride;
    uint32_t best = 0;
    // (16 loads per thread in flight at once: one batch up to 5,120 positions)
    for (int p0 = 0; p0 < L; p0 += 16 * AG_THREADS) {
        float x[16];
#pragma unroll
        for (int u = 0; u < 16; u++) x[u] = arow[imin(p0 + u * AG_THREADS + tid, L - 1)];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int p = p0 + u * AG_THREADS + tid;
            if (p < L) {
                s_ps[ag_slot(p)] = x[u];
                best = umax(best, d_fkey(x[u]));
            }
        }
    }
    EXP_TAB_PUT(tab);
    for (int o = 32; o > 0; o >>= 1) best = umax(best, (uint32_t)__shfl_xor((int)best, o));
    if (lane == 0) s_red[wave] = best;
    __syncthreads();
    uint32_t bk = s_red[0];
#pragma unroll
    for (int w = 1; w < AG_THREADS / 64; w++) bk = umax(bk, s_red[w]);
    const float mx = d_unkey(bk);
    // exps in place
    for (int p = tid; p < L; p += AG_THREADS) {
        float *e = s_ps + ag_slot(p);
        *e = d_exp(*e - mx, tab);
    }
    __syncthreads();
    if (wave == 0) {                     // the serial loop's sum, bit for bit
        float carry = 0.0f;
        for (int k = 0; k < nseg; k++) {
            float *row = s_ps + k * PSR;
            if (lane == 0) row[0] = carry;
            __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            carry = wave_sum_nonneg<32>(row, imin(AG_SEG, L - k * AG_SEG) + 1, s_rec);
        }
        if (lane == 0) s_inv = (carry > 0.0f) ? 1.0f / carry : 0.0f;
    }
    __syncthreads();
    const float inv = s_inv;
    for (int p = tid; p < L; p += AG_THREADS) s_ps[ag_slot(p)] *= inv;
    __syncthreads();
    // value chains
    auto produce = [&](int c, int buf, int4 v4, float vsc) {
        const int p = c * AG_CH + pp;
        // past the row: a = 0, a product of +-0, which leaves the sum as it is
        const float ap = p < L ? s_ps[ag_slot(p)] : 0.0f;
        float *pb = prod + buf * 32 * AG_PAD + 16 * ph * AG_PAD + pp;
        const int w4[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int i = 0; i < 16; i++) pb[i * AG_PAD] = ap * (float)(int8_t)((w4[i >> 2] >> (8 * (i & 3))) & 0xFF) * vsc;
    };
    const int d = lane & 31;
    float o = 0.0f;
    if (prodw) {
        produce(0, 0, r[0], rs[0]);
        AG_LOAD(AG_NPF, 0);
    }
    __syncthreads();
#pragma unroll 1
    for (int c0 = 0; c0 < nch; c0 += AG_NPF) {
#pragma unroll
        for (int j = 0; j < AG_NPF; j++) {
            const int c = c0 + j;
            if (c >= nch) break;                      // uniform
            if (!prodw) {
                // the chunk in quarters, each quarter's reads issued before
                // the previous quarter's adds
                const float4 *pr = reinterpret_cast<const float4 *>(prod + (c & 1) * 32 * AG_PAD + d * AG_PAD);
                constexpr int QN = AG_CH / 16;
                float4 q0[QN], q1[QN];
#pragma unroll
                for (int i = 0; i < QN; i++) q0[i] = pr[i];
#pragma unroll
                for (int qr = 0; qr < 4; qr += 2) {
#pragma unroll
                    for (int i = 0; i < QN; i++) q1[i] = pr[(qr + 1) * QN + i];
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < QN; i++) { o += q0[i].x; o += q0[i].y; o += q0[i].z; o += q0[i].w; }
                    if (qr + 2 < 4) {
#pragma unroll
                        for (int i = 0; i < QN; i++) q0[i] = pr[(qr + 2) * QN + i];
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < QN; i++) { o += q1[i].x; o += q1[i].y; o += q1[i].z; o += q1[i].w; }
                }
            } else if (c + 1 < nch) {
                const int jn = (j + 1) % AG_NPF;
                produce(c + 1, (c + 1) & 1, r[jn], rs[jn]);
                AG_LOAD(c + 1 + AG_NPF, jn);
            }
            __syncthreads();
        }
    }
#undef AG_LOAD
    if (prodw) return;
    // gate, the group's quantization (lanes 32-63 repeat lanes 0-31 and store nothing)
    const int dd = 32 * g + d;
    const float gate = a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * HD + HD + dd];
    o *= d_sigmoid(gate, tab);
    const int col = h * HD + dd;
    if (a.out && lane < 32) a.out[(size_t)t * a.q_dim + col] = o;
    int8_t q;
    float sg;
    d_quant_group32(o, &q, &sg);
    if (lane < 32) {
        a.oq[(size_t)t * a.q_dim + col] = q;
        if (lane == 0) a.oqs[(size_t)t * (a.q_dim >> 5) + (col >> 5)] = sg;
    }
}

// k_attn_av_rows: the softmax and value sums of an item launch whose rows
// all lie below position 512, for 64-wide heads: one block per (q head,
// item), wave t = the item's token t, lane = output element d.  The item's
// V rows are staged once for its eight tokens, transposed ([d][position],
// and the scales [group][position]), so a lane reads four positions' bytes
// in one access; each wave takes its token's softmax (max, exp, the exact
// wave sum of the serial loop, scale), then lane d adds (a[p] * v[p][d]) *
// vs[p][d/32] over positions p = 0 .. pos in order - the arithmetic of
// attn_av_body, per token.  Then the gate and the per-32 quantization.
#define AVR_L 512
#define AVR_HD 64
__global__ __launch_bounds__(512) void k_attn_av_rows(AttnArgs b, const AttnItem *__restrict__ items, int plane,
                                                      const float *__restrict__ att, int att_stride, size_t att_item,
                                                      int own_scores) {
    EXP_TAB_LOAD(tab);
    __shared__ __align__(16) int8_t s_vt[AVR_HD][AVR_L];          // V transposed
    __shared__ __align__(16) float s_vst[AVR_HD / 32][AVR_L];     // its scales, transposed
    __shared__ __align__(16) float s_a[MAX_CHUNK][AVR_L];         // scores, then probabilities
    __shared__ __align__(16) float s_e[MAX_CHUNK][64 * (8 + 4)];  // exps in the exact sum's layout (8 per lane)
    __shared__ PsRec s_rec[MAX_CHUNK][128];
    __shared__ __align__(16) float s_q[MAX_CHUNK][AVR_HD];        // own_scores: the prepared q heads
    const int h = blockIdx.x, item = blockIdx.y;
    const AttnItem it = items[item];
    const AttnArgs a = attn_item_args(b, it, plane);
    const float *arows = att + (size_t)item * att_item;
    const int tid = threadIdx.x, t = tid >> 6, lane = tid & 63;
    const int kv_mul = a.nh / a.nkv, kvh = h / kv_mul, nb = AVR_HD / 32;
    const int pos0 = *a.ctl_pos + a.pos_off, n = it.n, Lmax = pos0 + n;
    const bool live = t < n;
    const int L = pos0 + imin(t, n - 1) + 1;
    // stage: V rows [0, Lmax) of the kv head (4 int4 per row), their scales,
    // and each wave's score row
    for (int f = tid; f < Lmax * 4; f += 512) {
        const int p = f >> 2, c = f & 3;
        const int4 v4 = *reinterpret_cast<const int4 *>(a.vcache + (size_t)p * a.kv_dim + kvh * AVR_HD + 16 * c);
        const int w4[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int k = 0; k < 16; k++) s_vt[16 * c + k][p] = (int8_t)((w4[k >> 2] >> (8 * (k & 3))) & 0xFF);
    }
    for (int f = tid; f < Lmax * nb; f += 512) {
        const int p = f / nb, g = f - p * nb;
        s_vst[g][p] = a.vscale[(size_t)p * (a.kv_dim >> 5) + kvh * nb + g];
    }
    if (live && !own_scores)
        for (int p = lane; p < L; p += 64) s_a[t][p] = arows[((size_t)t * a.nh + h) * att_stride + p];
    if (live && own_scores) {
        // every K row is in the cache: the wave prepares its token's q head
        // (RMSNorm(1+w) with the serial sum, NeoX rotary) and computes the
        // scores itself, as k_attn_scores_items does
        const int pos_t = L - 1, half = a.rot >> 1;
        const float x = a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * AVR_HD + lane];
        s_e[t][lane] = x * x;
        __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0): the squares are in LDS
        __builtin_amdgcn_wave_barrier();
        const float inv = d_rsqrt(d_ss_over_n(serial_sum(s_e[t], AVR_HD), AVR_HD) + a.eps);
        const float y = x * inv * (1.0f + a.q_norm[lane]);
        const float yo = __shfl(y, lane < half ? lane + half : lane - half);     // the rotary partner
        float r = y;
        if (lane < half) {
            const float c = a.rope_cs[((size_t)pos_t * half + lane) * 2], sn = a.rope_cs[((size_t)pos_t * half + lane) * 2 + 1];
            r = y * c - yo * sn;
        } else if (lane < 2 * half) {
            const int i = lane - half;
            const float c = a.rope_cs[((size_t)pos_t * half + i) * 2], sn = a.rope_cs[((size_t)pos_t * half + i) * 2 + 1];
            r = y * c + yo * sn;
        }
        s_q[t][lane] = r;
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        const float scale = a.attn_scale;
        for (int p = lane; p < L; p += 64) {
            const int8_t *kr = a.kcache + (size_t)p * a.kv_dim + kvh * AVR_HD;
            const float *ks = a.kscale + (size_t)p * (a.kv_dim >> 5) + kvh * nb;
            float sum = 0.0f;
#pragma unroll
            for (int dd = 0; dd < AVR_HD; dd += 32) {
                const int4 k0 = *reinterpret_cast<const int4 *>(kr + dd);
                const int4 k1 = *reinterpret_cast<const int4 *>(kr + dd + 16);
                const int8_t *kb0 = reinterpret_cast<const int8_t *>(&k0);
                const int8_t *kb1 = reinterpret_cast<const int8_t *>(&k1);
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) acc += s_q[t][dd + e] * (float)kb0[e];
#pragma unroll
                for (int e = 0; e < 16; e++) acc += s_q[t][dd + 16 + e] * (float)kb1[e];
                sum += acc * ks[dd >> 5];
            }
            s_a[t][p] = sum * scale;
        }
    }
    EXP_TAB_PUT(tab);
    __syncthreads();
    // softmax of the wave's token: max (order-preserving key), exp, the
    // serial loop's sum, scale
    if (live) {
        uint32_t best = 0;
        for (int p = lane; p < L; p += 64) best = umax(best, d_fkey(s_a[t][p]));
        for (int o = 32; o > 0; o >>= 1) best = umax(best, (uint32_t)__shfl_xor((int)best, o));
        const float mx = d_unkey(best);
        for (int p = lane; p < L; p += 64) {
            const float e = d_exp(s_a[t][p] - mx, tab);
            s_a[t][p] = e;
            s_e[t][(p >> 3) * 12 + (p & 7)] = e;
        }
        // positions L .. of the padded row read as 0 inside the exact sum
        __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0): the wave's exps are in LDS
        __builtin_amdgcn_wave_barrier();
        const float sum = wave_sum_nonneg<8>(s_e[t], L, s_rec[t]);
        const float inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
        for (int p = lane; p < L; p += 64) s_a[t][p] *= inv;
    }
    __syncthreads();
    if (!live) return;
    // value sum, four positions per step (the adds stay in position order)
    const int d = lane, g = d >> 5;
    float o = 0.0f;
    const int L4 = L & ~3;
    for (int p = 0; p < L4; p += 4) {
        const float4 ap = *reinterpret_cast<const float4 *>(&s_a[t][p]);
        const uint32_t vb = *reinterpret_cast<const uint32_t *>(&s_vt[d][p]);
        const float4 vs = *reinterpret_cast<const float4 *>(&s_vst[g][p]);
        const float p0 = ap.x * (float)(int8_t)(vb & 0xFF) * vs.x;
        const float p1 = ap.y * (float)(int8_t)((vb >> 8) & 0xFF) * vs.y;
        const float p2 = ap.z * (float)(int8_t)((vb >> 16) & 0xFF) * vs.z;
        const float p3 = ap.w * (float)(int8_t)(vb >> 24) * vs.w;
        o += p0;
        o += p1;
        o += p2;
        o += p3;
    }
    for (int p = L4; p < L; p++) o += s_a[t][p] * (float)s_vt[d][p] * s_vst[g][p];
    const float gate = a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * AVR_HD + AVR_HD + d];
    o *= d_sigmoid(gate, tab);
    const int col = h * AVR_HD + d;
    if (a.out) a.out[(size_t)t * a.q_dim + col] = o;
    int8_t q;
    float sg;
    d_quant_group32(o, &q, &sg);
    a.oq[(size_t)t * a.q_dim + col] = q;
    if ((d & 31) == 0) a.oqs[(size_t)t * (a.q_dim >> 5) + (col >> 5)] = sg;
}

// k_attn_rows<HD, WPT>: the softmax and value sums of an item launch whose
// K and V rows are all in the cache, 64- or 128-wide heads, positions up to
// what the block's LDS holds (the launch checks): one block of 8 waves per
// (q head, item) holding TPB = 8 / WPT tokens (WPT = 2 when every item has
// at most 4 rows).
//   1. each token's first wave prepares its q head (RMSNorm(1+w) with the
//      serial sum, NeoX rotary), as attn_prep_body does;
//   2. scores, chunk by chunk of SCH = 512 / (HD/32) K rows: lane (position,
//      32-group g) converts its 32 int8 of the row once and runs the group's
//      product chain (the 32 products in order from 0) for every token of
//      the block, times the group's scale; then lane (token, position) adds
//      the groups in order from 0 and applies attn_scale: the additions of
//      attn_scores_body, each in its own order, so the bits are its bits;
//   3. each token's first wave takes the softmax (max by order-preserving
//      key, exp, the serial loop's sum, scale);
//   4. value sums, chunk by chunk of VCH = 8192 / HD V rows staged once as
//      fp32 (row-major, scales [group][position]): a lane takes one element
//      d of two consecutive tokens and adds (a[p] * v[p][d]) * vs[p][d/32]
//      to each token's sum over the positions in order, four per step (one
//      read of v for both; the LDS reads, not the VALU, bound this phase);
//   5. the sigmoid output gate and the per-32 quantization.
// Every chunk's global loads are issued into registers before the previous
// chunk is computed (the first K chunk's before step 1, the first V chunk's
// with the last K chunk), and stored to LDS after it.
// LDS: the staging area (STAGE bytes), then the score rows [TPB][lp] floats
// (dynamic).
#define AR_STATIC_MARGIN (5 * 1024)     // the kernel's static LDS (q heads, exp table) and slack
#define AR_THREADS (MAX_CHUNK * 64)
#define GLOBAL __attribute__((address_space(1)))     // the cache planes: global loads, not flat
typedef int v4i_a __attribute__((ext_vector_type(4)));
typedef float v4f_a __attribute__((ext_vector_type(4)));
template <int HD>
struct ArPlan {
    static constexpr int NDP = HD / 64, NB = HD / 32, CPR = HD / 16, KS = HD + 16;
    static constexpr int WPG = 8 / NB, SCH = WPG * 64;          // scores: waves per group, positions per chunk
    static constexpr int VCH = AR_THREADS * 16 / HD, VS = HD + 4; // values: positions per chunk, floats per row
    static constexpr int K_BYTES = SCH * KS + SCH * NB * 4 + MAX_CHUNK * NB * SCH * 4;
    static constexpr int V_BYTES = VCH * VS * 4 + NB * VCH * 4;
    static constexpr int Q_BYTES = MAX_CHUNK * HD * 4;
    static constexpr int m2(int x, int y) { return x > y ? x : y; }
    static constexpr int STAGE = (m2(m2(K_BYTES, V_BYTES), Q_BYTES) + 15) & ~15;
    static_assert(SCH * CPR == 2 * AR_THREADS && SCH * NB == AR_THREADS && VCH * HD / 4 == 4 * AR_THREADS &&
                      NB * VCH <= AR_THREADS && (SCH * KS) % 16 == 0 && (VCH * VS * 4) % 16 == 0,
                  "chunk staging layout");
};

template <int HD, int WPT>
__global__ __launch_bounds__(AR_THREADS) void k_attn_rows(AttnArgs b, const AttnItem *__restrict__ items,
                                                          int plane, int lp) {
    using P = ArPlan<HD>;
    constexpr int NDP = P::NDP, NB = P::NB, CPR = P::CPR, KS = P::KS, VS = P::VS, NTHR = AR_THREADS;
    constexpr int SCH = P::SCH, VCH = P::VCH, WPG = P::WPG;
    constexpr int TPB = MAX_CHUNK / WPT;                          // tokens per block
    EXP_TAB_LOAD(tab);
    extern __shared__ __align__(16) char smem[];
    __shared__ __align__(16) float s_q[TPB][HD];                 // the prepared q heads
    char *stage = smem;
    float *s_a = reinterpret_cast<float *>(smem + P::STAGE);      // [TPB][lp]
    // block -> (q head, item): blocks go to the 8 XCDs in turn by linear
    // index L, and L and L + B/2 share a CU; when the grid allows, XCD x
    // takes the (item, head) pairs [x B/16, (x+1) B/16) of each half, so the
    // q heads of a kv head (and an item's kv heads) share one L2, and the
    // halves keep the host's long/short item pairing on each CU
    int h = blockIdx.x, item = blockIdx.y;
    {
        const int B = gridDim.x * gridDim.y, hb = B >> 1;
        if ((B & 15) == 0 && (B >> 4) % (b.nh / b.nkv) == 0) {
            const int L = blockIdx.y * gridDim.x + blockIdx.x, hf = L >= hb ? 1 : 0, r = L - hf * hb;
            const int lam = hf * hb + (r & 7) * (B >> 4) + (r >> 3);
            item = lam / gridDim.x;
            h = lam - item * gridDim.x;
        }
    }
    const AttnItem it = items[item];
    const AttnArgs a = attn_item_args(b, it, plane);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, t = wave / WPT, part = wave - t * WPT;
    const int kv_mul = a.nh / a.nkv, kvh = h / kv_mul;
    const int pos0 = __builtin_amdgcn_readfirstlane(*a.ctl_pos + a.pos_off), n = it.n, Lmax = pos0 + n;
    const bool live = t < n, lead = live && part == 0;
    const int L = pos0 + imin(t, n - 1) + 1;
    float *arow = s_a + (size_t)t * lp;
    const int8_t *kbase = a.kcache + kvh * HD;
    const float *ksbase = a.kscale + kvh * NB;
    const int8_t *vbase = a.vcache + kvh * HD;
    const float *vsbase = a.vscale + kvh * NB;
    const size_t rst = (size_t)a.kv_dim, sst = (size_t)(a.kv_dim >> 5);
    // the thread's share of a K chunk (two 16-byte pieces and one scale) and
    // of a V chunk (four 4-byte pieces f = u * NTHR + tid, row f / DPR - so a
    // wave's pieces are whole rows, and its fp32 stores contiguous runs -
    // and one scale for tid < VCH * NB); a piece past the chunk's end reads
    // the chunk's last row
    constexpr int DPR = HD / 4;
    v4i_a kr[2];
    int vr[4];
    float ksv, vsv = 0.0f;
#define AR_LOAD_K(c0)                                                                                   \
    {                                                                                                   \
        const int nc_ = imin(SCH, Lmax - (c0));                                                         \
        _Pragma("unroll") for (int u = 0; u < 2; u++) {                                                 \
            const int f = u * NTHR + tid, p = imin(f / CPR, nc_ - 1), c = f % CPR;                      \
            kr[u] = *(const GLOBAL v4i_a *)(kbase + (size_t)((c0) + p) * rst + c * 16);                 \
        }                                                                                               \
        ksv = ((const GLOBAL float *)ksbase)[(size_t)((c0) + imin(tid / NB, nc_ - 1)) * sst + tid % NB]; \
    }
#define AR_LOAD_V(c0)                                                                                   \
    {                                                                                                   \
        const int nc_ = imin(VCH, Lmax - (c0));                                                         \
        _Pragma("unroll") for (int u = 0; u < 4; u++) {                                                 \
            const int f = u * NTHR + tid;                                                               \
            vr[u] = *(const GLOBAL int *)(vbase + (size_t)((c0) + imin(f / DPR, nc_ - 1)) * rst + (f % DPR) * 4); \
        }                                                                                               \
        if (tid < VCH * NB)                                                                             \
            vsv = ((const GLOBAL float *)vsbase)[(size_t)((c0) + imin(tid / NB, nc_ - 1)) * sst + tid % NB]; \
    }
    AR_LOAD_K(0);
    // 1. q heads: squares in the staging area, the serial sum, RMSNorm(1+w),
    //    rotary (partners through s_q)
    if (lead) {
        float *sq = reinterpret_cast<float *>(stage) + t * HD;
        const int half = a.rot >> 1, pos_t = L - 1;
        float x[NDP], y[NDP];
#pragma unroll
        for (int u = 0; u < NDP; u++) {
            x[u] = a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * HD + u * 64 + lane];
            sq[u * 64 + lane] = x[u] * x[u];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0): the squares are in LDS
        __builtin_amdgcn_wave_barrier();
        const float inv = d_rsqrt(d_ss_over_n(serial_sum(sq, HD), HD) + a.eps);
#pragma unroll
        for (int u = 0; u < NDP; u++) {
            y[u] = x[u] * inv * (1.0f + a.q_norm[u * 64 + lane]);
            s_q[t][u * 64 + lane] = y[u];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        float r[NDP];
#pragma unroll
        for (int u = 0; u < NDP; u++) {
            const int i = u * 64 + lane;
            r[u] = y[u];
            if (i < half) {
                const float c = a.rope_cs[((size_t)pos_t * half + i) * 2], sn = a.rope_cs[((size_t)pos_t * half + i) * 2 + 1];
                r[u] = y[u] * c - s_q[t][i + half] * sn;
            } else if (i < 2 * half) {
                const int j = i - half;
                const float c = a.rope_cs[((size_t)pos_t * half + j) * 2], sn = a.rope_cs[((size_t)pos_t * half + j) * 2 + 1];
                r[u] = y[u] * c + s_q[t][j] * sn;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < NDP; u++) s_q[t][u * 64 + lane] = r[u];
    }
    EXP_TAB_PUT(tab);
    __syncthreads();
    // 2. scores, chunk by chunk of K rows
    {
        int8_t *s_k = reinterpret_cast<int8_t *>(stage);                              // [SCH][KS]
        float *s_ks = reinterpret_cast<float *>(stage + SCH * KS);                     // [SCH][NB]
        float *s_part = s_ks + SCH * NB;                                               // [TPB][NB][SCH]
        const float scale = a.attn_scale;
        const int g = wave / WPG, pl = (wave - g * WPG) * 64 + lane;
        for (int c0 = 0; c0 < Lmax; c0 += SCH) {
            const int nc = imin(SCH, Lmax - c0);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int f = u * NTHR + tid, p = f / CPR, c = f % CPR;
                if (p < nc) *reinterpret_cast<v4i_a *>(s_k + p * KS + c * 16) = kr[u];
            }
            if (tid < nc * NB) s_ks[tid] = ksv;
            __syncthreads();
            if (c0 + SCH < Lmax) AR_LOAD_K(c0 + SCH) else AR_LOAD_V(0);
            // lane (pl, g): the group's chains for every token; a position
            // past the chunk's end computes on row 0 and is never added
            {
                const int pc = pl < nc ? pl : 0;
                const v4i_a k0 = *reinterpret_cast<const v4i_a *>(s_k + pc * KS + g * 32);
                const v4i_a k1 = *reinterpret_cast<const v4i_a *>(s_k + pc * KS + g * 32 + 16);
                float acc[TPB];
#pragma unroll
                for (int j = 0; j < TPB; j++) acc[j] = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; e++) {
                    const int w = e < 16 ? k0[e >> 2] : k1[(e - 16) >> 2];
                    const float kf = (float)(int8_t)((w >> (8 * (e & 3))) & 0xFF);
#pragma unroll
                    for (int j = 0; j < TPB; j++) acc[j] += s_q[j][g * 32 + e] * kf;
                }
                const float ks = s_ks[pc * NB + g];
#pragma unroll
                for (int j = 0; j < TPB; j++) s_part[(j * NB + g) * SCH + pl] = acc[j] * ks;
            }
            __syncthreads();
            // lane (token, position): the groups in order
#pragma unroll
            for (int r = 0; r < TPB * SCH / NTHR; r++) {
                const int idx = r * NTHR + tid, j = idx / SCH, p = idx % SCH;
                if (j < n && c0 + p < pos0 + j + 1 && p < nc) {
                    float sum = 0.0f;
#pragma unroll
                    for (int gg = 0; gg < NB; gg++) sum += s_part[(j * NB + gg) * SCH + p];
                    s_a[(size_t)j * lp + c0 + p] = sum * scale;
                }
            }
        }
    }
    // the last K chunk's registers are taken here, so that no later write of
    // a register a K prefetch could still own (on a path the compiler cannot
    // exclude) waits for the V chunk loads in flight
    asm volatile("" ::"v"(kr[0]), "v"(kr[1]), "v"(ksv));
    __syncthreads();
    // 3. softmax of each token, by its first wave: max by order-preserving
    //    key, exp, the serial loop's sum over the score row, scale (every
    //    token at once; the exact wave sum's tables would take the
    //    registers that let two blocks share a CU)
    if (lead) {
        uint32_t best = 0;
        for (int p = lane; p < L; p += 64) best = umax(best, d_fkey(arow[p]));
        for (int o = 32; o > 0; o >>= 1) best = umax(best, (uint32_t)__shfl_xor((int)best, o));
        const float mx = d_unkey(best);
        for (int p = lane; p < L; p += 64) arow[p] = d_exp(arow[p] - mx, tab);
        __builtin_amdgcn_s_waitcnt(0xC07F);           // lgkmcnt(0): the wave's exps are in LDS
        __builtin_amdgcn_wave_barrier();
        const float sum = serial_sum(arow, L);
        const float inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
        for (int p = lane; p < L; p += 64) arow[p] *= inv;
    }
    // 4. value sums, chunk by chunk of V rows (fp32): lane l of wave w takes
    //    element d = (w % NDH) * 64 + l of tokens t0 = 2 (w / NDH) and t0 + 1,
    //    so each V element read feeds two chains; t0 + 1 has one position more
    constexpr int NDH = HD / 64;                                   // waves per token pair
    const int tp = wave / NDH, dv = (wave - tp * NDH) * 64 + lane, t0 = 2 * tp;
    const bool vwork = tp < TPB / 2 && t0 < n, vboth = t0 + 1 < n;
    const int La = pos0 + t0 + 1, Lb = vboth ? La + 1 : La;
    float o0 = 0.0f, o1 = 0.0f;
    {
        float *s_vf = reinterpret_cast<float *>(stage);                                // [VCH][VS]
        float *s_vst = s_vf + VCH * VS;                                                // [NB][VCH]
        for (int c0 = 0; c0 < Lmax; c0 += VCH) {
            const int nc = imin(VCH, Lmax - c0);
            __syncthreads();                          // the stage's previous readers are done
            {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int f = u * NTHR + tid, p = f / DPR, c = f % DPR;
                    if (p < nc) {
                        v4f_a f4;
#pragma unroll
                        for (int k = 0; k < 4; k++) f4[k] = (float)(int8_t)((vr[u] >> (8 * k)) & 0xFF);
                        *reinterpret_cast<v4f_a *>(s_vf + p * VS + c * 4) = f4;
                    }
                }
                if (tid < nc * NB) s_vst[(tid % NB) * VCH + tid / NB] = vsv;
            }
            __syncthreads();
            if (c0 + VCH < Lmax) AR_LOAD_V(c0 + VCH);
            // this chunk's positions of t0 (pa) and of t0 + 1 (pb = pa or pa + 1)
            const int pa = __builtin_amdgcn_readfirstlane(imax(0, imin(nc, La - c0)));
            const int pb = __builtin_amdgcn_readfirstlane(imax(0, imin(nc, Lb - c0)));
            if (vwork && pb > 0) {
                const int pa4 = pa & ~3;
                const float *a0 = s_a + (size_t)t0 * lp + c0, *a1 = a0 + lp;
                const float *vsr = s_vst + (dv >> 5) * VCH, *vc = s_vf + dv;
                // four positions a step, in two register sets: the next
                // step's reads are issued before this step's products (past
                // the end they read the last step again); the scheduling
                // barrier keeps them above the products, and the empty asm
                // after the products takes their registers, so they neither
                // wait before the products nor fold into the next step
#define AR_V_READ(S, q)                                                                     \
    S##x0 = *reinterpret_cast<const v4f_a *>(a0 + (q));                                     \
    S##x1 = *reinterpret_cast<const v4f_a *>(a1 + (q));                                     \
    S##s = *reinterpret_cast<const v4f_a *>(vsr + (q));                                     \
    S##v0 = vc[(q) * VS];                                                                   \
    S##v1 = vc[((q) + 1) * VS];                                                             \
    S##v2 = vc[((q) + 2) * VS];                                                             \
    S##v3 = vc[((q) + 3) * VS]
#define AR_V_STEP(S)                                                                        \
    {                                                                                       \
        const float q0 = S##x0[0] * S##v0 * S##s[0], q1 = S##x0[1] * S##v1 * S##s[1];       \
        const float q2 = S##x0[2] * S##v2 * S##s[2], q3 = S##x0[3] * S##v3 * S##s[3];       \
        const float r0 = S##x1[0] * S##v0 * S##s[0], r1 = S##x1[1] * S##v1 * S##s[1];       \
        const float r2 = S##x1[2] * S##v2 * S##s[2], r3 = S##x1[3] * S##v3 * S##s[3];       \
        o0 += q0;                                                                           \
        o1 += r0;                                                                           \
        o0 += q1;                                                                           \
        o1 += r1;                                                                           \
        o0 += q2;                                                                           \
        o1 += r2;                                                                           \
        o0 += q3;                                                                           \
        o1 += r3;                                                                           \
    }
#define AR_V_HOLD(S)                                                                        \
    asm volatile("" : "+v"(o0), "+v"(o1), "+v"(S##x0), "+v"(S##x1), "+v"(S##s), "+v"(S##v0), \
                 "+v"(S##v1), "+v"(S##v2), "+v"(S##v3))
                if (pa4 > 0) {
                    v4f_a Ax0, Ax1, As, Bx0, Bx1, Bs;
                    float Av0, Av1, Av2, Av3, Bv0, Bv1, Bv2, Bv3;
                    AR_V_READ(A, 0);
                    for (int p = 0;; p += 8) {
                        AR_V_READ(B, imin(p + 4, pa4 - 4));
                        __builtin_amdgcn_sched_barrier(0);
                        AR_V_STEP(A);
                        AR_V_HOLD(B);
                        if (p + 4 >= pa4) break;
                        AR_V_READ(A, imin(p + 8, pa4 - 4));
                        __builtin_amdgcn_sched_barrier(0);
                        AR_V_STEP(B);
                        AR_V_HOLD(A);
                        if (p + 8 >= pa4) break;
                    }
                }
#undef AR_V_READ
#undef AR_V_STEP
#undef AR_V_HOLD
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int p = pa4 + j;
                    if (p >= pb) break;
                    const float v = vc[p * VS], s = vsr[p];
                    if (p < pa) o0 += a0[p] * v * s;
                    o1 += a1[p] * v * s;
                }
            }
        }
    }
#undef AR_LOAD_K
#undef AR_LOAD_V
    if (!vwork) return;
    // 5. gate, quantization (t0, then t0 + 1 when it is a row of the item)
#pragma unroll
    for (int i = 0; i < 2; i++) {
        if (i == 1 && !vboth) break;
        const int tt = t0 + i;
        const float gate = a.qg[(size_t)tt * a.qg_dim + (size_t)h * 2 * HD + HD + dv];
        const float y = (i ? o1 : o0) * d_sigmoid(gate, tab);
        const int col = h * HD + dv;
        if (a.out) a.out[(size_t)tt * a.q_dim + col] = y;
        int8_t q;
        float sg;
        d_quant_group32(y, &q, &sg);
        a.oq[(size_t)tt * a.q_dim + col] = q;
        if ((dv & 31) == 0) a.oqs[(size_t)tt * (a.q_dim >> 5) + (col >> 5)] = sg;
    }
}

// k_attn_prep_items: every item's new K and V rows quantized into its
// cache plane (attn_prep_body without the q heads), one 64-lane block per
// (k or v head, token, item); tokens past an item's n return.
__global__ __launch_bounds__(64) void k_attn_prep_items(AttnArgs b, const AttnItem *__restrict__ items, int plane) {
    const AttnItem it = items[blockIdx.z];
    if ((int)blockIdx.y >= it.n) return;
    AttnArgs a = attn_item_args(b, it, plane);
    a.kv_only = 1;
    attn_prep_body(a, blockIdx.y, blockIdx.x);
}

// mtp_attn_t1 (src/forward_mtp.c:191-376, Q8 KV float arm): attention of
// a DSpark slot at position 0 of the MTP plane with no history, one block
// per slot row r.  The softmax over the single score is exactly 1, so K,
// Q, RoPE and the scores never enter: V is quantized per 32 (the plane's
// row 0 keeps the last slot's, as the reference's slots overwrite it in
// turn), each output element is 0 + (1 * q) * scale (wsum_q8_row,
// src/forward_attn.c:17-21, with weight 1), times sigmoid of its gate, then
// the o_proj input: the float row (out, SubLN's own norm follows) or its
// per-32 quantization (oq, oqs).
__global__ __launch_bounds__(256) void k_attn_t1(const float *__restrict__ qg, int qg_dim,
                                                 const float *__restrict__ vp, int kv_dim, int nh, int nkv, int hd,
                                                 int q_dim, int rows, int8_t *__restrict__ vc0,
                                                 float *__restrict__ vs0, float *__restrict__ out,
                                                 int8_t *__restrict__ oq, float *__restrict__ oqs) {
    EXP_TAB_LOAD(tab);
    __shared__ int8_t s_vq[2048];
    __shared__ float s_vs[64];
    const int r = blockIdx.x, tid = threadIdx.x, kv_mul = nh / nkv;
    const bool last = r == rows - 1;
    for (int b = 0; b < kv_dim; b += 256) {
        const int i = b + tid;
        const float x = vp[(size_t)r * kv_dim + (i < kv_dim ? i : kv_dim - 1)];
        int8_t q;
        float sg = 0.0f;
        d_quant_group32(x, &q, &sg);
        if (i < kv_dim) {
            s_vq[i] = q;
            if (last) vc0[i] = q;
            if ((i & 31) == 0) {
                s_vs[i >> 5] = sg;
                if (last) vs0[i >> 5] = sg;
            }
        }
    }
    EXP_TAB_PUT(tab);
    __syncthreads();
    for (int b = 0; b < q_dim; b += 256) {
        const int j = b + tid, jc = j < q_dim ? j : q_dim - 1;
        const int h = jc / hd, e = jc - h * hd, src = (h / kv_mul) * hd + e;
        float o = 0.0f + (1.0f * (float)s_vq[src]) * s_vs[src >> 5];
        o *= d_sigmoid(qg[(size_t)r * qg_dim + (size_t)h * 2 * hd + hd + e], tab);
        if (out) {
            if (j < q_dim) out[(size_t)r * q_dim + j] = o;
            continue;
        }
        int8_t q;
        float sg = 0.0f;
        d_quant_group32(o, &q, &sg);
        if (j < q_dim) {
            oq[(size_t)r * q_dim + j] = q;
            if ((j & 31) == 0) oqs[(size_t)r * (q_dim >> 5) + (j >> 5)] = sg;
        }
    }
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_attn(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

extern "C" int l98k_attn_t1(const float *qg, int qg_dim, const float *vp, int kv_dim, int nh, int nkv, int hd,
                            int q_dim, int rows, int8_t *vc0, float *vs0, float *out, int8_t *oq, float *oqs,
                            hipStream_t st) {
    if (rows < 1 || kv_dim > 2048 || (kv_dim & 31) || (q_dim & 31) || (hd & 31) || nkv < 1 || nh % nkv ||
        q_dim != nh * hd || kv_dim != nkv * hd || qg_dim != 2 * q_dim || (!out && (!oq || !oqs)))
        return -1;
    hipLaunchKernelGGL(k_attn_t1, dim3(rows), dim3(256), 0, st, qg, qg_dim, vp, kv_dim, nh, nkv, hd, q_dim, rows,
                       vc0, vs0, out, oq, oqs);
    return (int)hipGetLastError();
}

extern "C" int l98k_attn_prep(const AttnArgs *a, int nt, hipStream_t st) {
    if (a->hd > 256 || (a->hd & 31) || a->rot > a->hd || nt < 1) return -1;
    const int per_tok = (a->kv_only ? 0 : a->nh) + 2 * a->nkv;
    hipLaunchKernelGGL(k_attn_prep, dim3(nt * per_tok), dim3(64), 0, st, *a);
    return (int)hipGetLastError();
}

// Largest dynamic LDS a block may use on this device (queried once).
static int lds_limit() {
    static int lim = 0;
    if (!lim) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        lim = v;
    }
    return lim;
}

// The value-sum launch's LDS plan for scores rows of att_stride floats:
// the CH = 128 instance when its double buffer fits, else 64; sc staged V
// positions.  Returns false when neither fits.
static bool av_plan(int hd, int max_len, int att_stride, int *ch_out, int *sc_out, size_t *lds_out) {
    const size_t per_pos = (size_t)hd + (size_t)(hd >> 5) * sizeof(float);
    const int lim = lds_limit() - 4096;
    for (int ch : {128, 64}) {
        const size_t fixed = ((size_t)att_stride + 2 * (size_t)hd * (ch + 4) + AV_ESUM_FLOATS) * sizeof(float);
        if (fixed + (size_t)ch * per_pos > (size_t)lim) continue;
        int sc = (int)(((size_t)lim - fixed) / per_pos) & ~(ch - 1);
        const int need = (max_len + ch - 1) & ~(ch - 1);
        if (sc > need) sc = need;
        const int sc_regs = (AV_THREADS * AV_STAGE_MAX / (hd >> 4)) & ~(ch - 1);
        if (sc > sc_regs) sc = sc_regs;
        *ch_out = ch;
        *sc_out = sc;
        *lds_out = fixed + (size_t)sc * per_pos;
        return true;
    }
    return false;
}

static void av_allow_lds() {
    static bool attr_set = false;
    if (attr_set) return;
    const int lim = lds_limit() - 4096;
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_av_items<128>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_av_items<64>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    attr_set = true;
}

// Attention of several sessions' rows in one launch per kernel: items
// (device) give each session's rows [row0, row0 + n) (n <= MAX_CHUNK), KV
// plane bases and position; base carries the layer's weights and the row
// buffers at row 0.  max_len: the longest item's last position + 1; att:
// n_items scratch blocks of att_item floats.
extern "C" int l98k_attn_items(const AttnArgs *a, const AttnItem *items, int n_items, int plane, int max_len,
                               int nmax, float *att, size_t att_item, int kv_cached, hipStream_t st) {
    if (a->nkv < 1 || a->nh % a->nkv || (a->hd & 31) || 256 % a->hd || a->hd > ATT_MAX_HD || a->rot > a->hd ||
        (a->rot & 1) || n_items < 1 || max_len < 1 || !a->oq || !a->oqs || !att || a->kv_only)
        return -1;
    if (a->nh / a->nkv + MAX_CHUNK > ATT_MAX_VEC) return -1;
    const int att_stride = (max_len + 3) & ~3;
    if ((size_t)MAX_CHUNK * a->nh * att_stride > att_item) return -1;
    const bool rows = a->hd == AVR_HD && max_len <= AVR_L;
    if (rows && kv_cached) {
        // every row's K is in the cache: the value-sum blocks take their scores
        hipLaunchKernelGGL(k_attn_av_rows, dim3(a->nh, n_items), dim3(512), 0, st, *a, items, plane, att, att_stride,
                           att_item, 1);
        return (int)hipGetLastError();
    }
    // 64- or 128-wide heads past the rows kernel's reach: the new K and V
    // rows into the caches first (unless they are there), then one block per
    // (q head, item) with the score rows in LDS, two waves per token when
    // every item has at most half a chunk of rows
    const int wpt = nmax <= MAX_CHUNK / 2 ? 2 : 1;
    const size_t ar_lds = (size_t)(a->hd == 128 ? ArPlan<128>::STAGE : ArPlan<64>::STAGE) +
                          (size_t)(MAX_CHUNK / wpt) * att_stride * sizeof(float);
    if (!rows && (a->hd == 64 || a->hd == 128) && nmax >= 1 && nmax <= MAX_CHUNK &&
        ar_lds <= (size_t)(lds_limit() - AR_STATIC_MARGIN)) {
        if (!kv_cached) {
            hipLaunchKernelGGL(k_attn_prep_items, dim3(2 * a->nkv, MAX_CHUNK, n_items), dim3(64), 0, st, *a, items,
                               plane);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return (int)e;
        }
        static bool ar_attr = false;
        if (!ar_attr) {
            const int lim = lds_limit() - AR_STATIC_MARGIN;
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_rows<128, 1>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lim);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_rows<128, 2>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lim);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_rows<64, 1>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lim);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_rows<64, 2>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lim);
            ar_attr = true;
        }
        const dim3 grid(a->nh, n_items), blk(AR_THREADS);
        if (a->hd == 128 && wpt == 2)
            hipLaunchKernelGGL((k_attn_rows<128, 2>), grid, blk, ar_lds, st, *a, items, plane, att_stride);
        else if (a->hd == 128)
            hipLaunchKernelGGL((k_attn_rows<128, 1>), grid, blk, ar_lds, st, *a, items, plane, att_stride);
        else if (wpt == 2)
            hipLaunchKernelGGL((k_attn_rows<64, 2>), grid, blk, ar_lds, st, *a, items, plane, att_stride);
        else
            hipLaunchKernelGGL((k_attn_rows<64, 1>), grid, blk, ar_lds, st, *a, items, plane, att_stride);
        return (int)hipGetLastError();
    }
    const int slices = (max_len + ATT_SLICE - 1) / ATT_SLICE;
    hipLaunchKernelGGL(k_attn_scores_items, dim3(slices, a->nkv, n_items * MAX_CHUNK), dim3(256), 0, st, *a, items,
                       plane, att, att_stride, att_item);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    if (rows) {
        hipLaunchKernelGGL(k_attn_av_rows, dim3(a->nh, n_items), dim3(512), 0, st, *a, items, plane, att, att_stride,
                           att_item, 0);
        return (int)hipGetLastError();
    }
    av_allow_lds();
    int ch = 0, sc = 0;
    size_t lds = 0;
    if (!av_plan(a->hd, max_len, att_stride, &ch, &sc, &lds)) return -1;
    if (ch == 128)
        hipLaunchKernelGGL(k_attn_av_items<128>, dim3(a->nh, n_items * MAX_CHUNK), dim3(AV_THREADS), lds, st, *a, items,
                           plane, att, att_stride, att_item, sc);
    else
        hipLaunchKernelGGL(k_attn_av_items<64>, dim3(a->nh, n_items * MAX_CHUNK), dim3(AV_THREADS), lds, st, *a, items,
                           plane, att, att_stride, att_item, sc);
    return (int)hipGetLastError();
}

// The K and V rows of every item's tokens into its session's cache plane
// (a batch of sessions' MTP catch-up rows).
extern "C" int l98k_attn_prep_items(const AttnArgs *a, const AttnItem *items, int n_items, int plane, hipStream_t st) {
    if (a->hd > 256 || (a->hd & 31) || a->rot > a->hd || n_items < 1 || n_items > 65535) return -1;
    hipLaunchKernelGGL(k_attn_prep_items, dim3(2 * a->nkv, MAX_CHUNK, n_items), dim3(64), 0, st, *a, items, plane);
    return (int)hipGetLastError();
}

// Which chunk path l98k_attn takes: 0 by the session's capacity (the two
// launches past AG_AUTO_LEN positions), 1 always the one launch, 2 the two
// launches wherever their LDS fits.
#define AG_AUTO_LEN 2048
static int g_attn_path = 0;
extern "C" void l98k_set_attn_path(int mode) { g_attn_path = mode; }

extern "C" int l98k_attn(const AttnArgs *a, int nt, int max_len, float *att, hipStream_t st) {
    // hd divides 256: the new K rows' quantization takes 32-lane groups of
    // a 256-thread block
    if (a->nkv < 1 || a->nh % a->nkv || (a->hd & 31) || 256 % a->hd || a->hd > ATT_MAX_HD || a->rot > a->hd || (a->rot & 1) ||
        nt < 1 || nt > MAX_CHUNK || max_len < 1 || !a->oq || !a->oqs || !att)
        return -1;
    const int kv_mul = a->nh / a->nkv;
    if (kv_mul + MAX_CHUNK > ATT_MAX_VEC) return -1;
    const int att_stride = (max_len + 3) & ~3;
    // two launches: the scores of every (slice, kv head, token), then the
    // softmax and value chains of every (q head, token, output group)
    const size_t ag_lds = ag_lds_bytes(att_stride);
    const bool ag_fits = (a->hd == 64 || a->hd == 128) && ag_lds <= (size_t)(lds_limit() - 8192);
    if (ag_fits && (g_attn_path == 2 || (g_attn_path == 0 && max_len > AG_AUTO_LEN))) {
        static bool ag_attr = false;
        if (!ag_attr) {
            const int lim = lds_limit() - 8192;
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_avg<128>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lim);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_avg<64>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, lim);
            ag_attr = true;
        }
        const int slices = (max_len + ATT_SLICE - 1) / ATT_SLICE;
        if (kv_mul + MAX_CHUNK <= 12)
            hipLaunchKernelGGL(k_attn_scores_chunk<12>, dim3(slices, a->nkv, nt), dim3(256), 0, st, *a, att, att_stride);
        else
            hipLaunchKernelGGL(k_attn_scores_chunk<ATT_MAX_VEC>, dim3(slices, a->nkv, nt), dim3(256), 0, st, *a, att,
                               att_stride);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        if (a->hd == 128)
            hipLaunchKernelGGL(k_attn_avg<128>, dim3(a->nh, nt, 4), dim3(AG_THREADS), ag_lds, st, *a, att, att_stride);
        else
            hipLaunchKernelGGL(k_attn_avg<64>, dim3(a->nh, nt, 2), dim3(AG_THREADS), ag_lds, st, *a, att, att_stride);
        return (int)hipGetLastError();
    }
    // one launch: each (q head, token) block does its own scores, then the
    // softmax and the value sum (scores row, the product double buffer, then
    // as many staged V positions, a multiple of the chunk, as the LDS limit
    // leaves beside the kernel's static LDS; 128-position chunks when a whole
    // chunk of V still fits)
    const int hd = a->hd;
    const size_t per_pos = (size_t)hd + (size_t)(hd >> 5) * sizeof(float);
    const int lim = lds_limit() - 8192;
    auto plan = [&](int ch, int *sc_out, size_t *lds_out) {
        const size_t fixed = ((size_t)att_stride + 2 * (size_t)hd * (ch + 4) + AV_ESUM_FLOATS) * sizeof(float);
        if (fixed + (size_t)ch * per_pos > (size_t)lim) return false;
        int sc = (int)(((size_t)lim - fixed) / per_pos) & ~(ch - 1);
        const int need = (max_len + ch - 1) & ~(ch - 1);
        if (sc > need) sc = need;
        const int sc_regs = (AV_THREADS * AV_STAGE_MAX / (hd >> 4)) & ~(ch - 1);   // one register-staged pass
        if (sc > sc_regs) sc = sc_regs;
        *sc_out = sc;
        *lds_out = fixed + (size_t)sc * per_pos;
        return true;
    };
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_fused<128>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lim);
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_fused<64>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lim);
        attr_set = true;
    }
    int sc = 0;
    size_t lds = 0;
    if (plan(128, &sc, &lds))
        hipLaunchKernelGGL(k_attn_fused<128>, dim3(a->nh, nt), dim3(AV_THREADS), lds, st, *a, att_stride, sc);
    else if (plan(64, &sc, &lds))
        hipLaunchKernelGGL(k_attn_fused<64>, dim3(a->nh, nt), dim3(AV_THREADS), lds, st, *a, att_stride, sc);
    else
        return -1;
    return (int)hipGetLastError();
}


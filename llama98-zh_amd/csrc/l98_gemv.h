// The int8 GEMV tile engine shared by the dense and the grouped-expert
// GEMV kernels, with its host-side shape helpers.
#ifndef L98_GEMV_H
#define L98_GEMV_H
#include "l98_devmath.h"

// ------------------------------------------------------------- GEMV/q8 ---
//
// o[t][row] = 0.0f + (sum_s float(acc[t,row,s]) * xqs[t][s]) * ws[row]
// with acc the exact int32 sum over each 32-element group
// (lz_matmul_xq_nt -> matmul_q8_impl + epi_q8, src/ops_matmul.c:336-466,
// src/ops_epi.c:983-1017).
//
// A 256-lane block streams one tile of R rows (R*in_dim <= 32 KiB): each
// wave issues all of its 16-byte weight loads of its 8 KiB quarter first.
// While they are in flight the block builds the M int8 activation rows in
// LDS (the job's prologue: copy pre-quantized rows, or quantize float rows,
// optionally after the residual fold + RMSNorm, SiLU-mul or MoE slot
// combine that produced them), so the producer's serial work overlaps the
// weight latency and needs no launch of its own.  The 16-element partial
// dot products (v_dot4_i32_i8) of neighbouring lanes add up to the exact
// 32-element group sums (an integer add, order-free), which go to LDS; then
// one lane per (row, token) runs the epilogue serially over the groups, in
// the reference order.  Weights stream once per launch for any M <= 8.

#define GEMV_THREADS 256
#define GEMV_WAVE_BYTES 8192
#define GEMV_TILE_BYTES (GEMV_WAVE_BYTES * (GEMV_THREADS / 64))
#define GEMV_MAXJ (GEMV_WAVE_BYTES / 16 / 64)
#define GEMV_MAX_IN 4096
#define PRO_MAX_IN 2048                 // float prologues: <= 8 float4 per lane per row
// Float prologues keep PJ float4 per lane per row (PJ*256 elements); the
// kernels are instantiated for PJ = 0 (pre-quantized input only), 1, 2, 4, 8.
static inline int pro_pj(int in_dim) {
    const int j = (in_dim + 255) / 256;
    return j <= 1 ? 1 : j <= 2 ? 2 : j <= 4 ? 4 : 8;
}
typedef int v4i __attribute__((ext_vector_type(4)));
// Token slots of the instance that runs m rows: 1, 2, 4, 5, 6 or 8 (the
// verify of k = 4 and 5 drafts has its own instance instead of paying for 8).
static inline int gemv_slots(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 6 ? m : 8; }

// LDS bytes of one tile: staged activations, their scales, and the larger of
// the group sums and the RMSNorm squares (m rows in the exact sum's layout
// for 4 * pj elements per lane, then the four waves' walk tables).
__host__ __device__ inline size_t gemv_lds_bytes(int m, int in_dim, int R, int norm, int pj) {
    const size_t part = (size_t)R * m * ((in_dim >> 5) + 4) * 4;
    const size_t sq = norm ? (size_t)m * 64 * (4 * pj + 4) * 4 + 4 * 128 * sizeof(PsRec) : 0;
    return (size_t)m * in_dim + (size_t)((m * (in_dim >> 5) + 3) & ~3) * 4 + (part > sq ? part : sq);
}

__device__ __forceinline__ float4 f4_silu_mul(float4 p, float4 q, const float *tab) {
    return make_float4(d_silu(p.x, tab) * q.x, d_silu(p.y, tab) * q.y, d_silu(p.z, tab) * q.z,
                       d_silu(p.w, tab) * q.w);
}

// Per-32 quantization of a tile's float rows (wave w holds rows w, w+4 as
// float4 f = lane + 64*j) into sx / sxs.
template <int RW, int PJN>
__device__ __forceinline__ void quant_rows(const float4 (&v)[RW][PJN], int wave, int lane, int nm, int nf, int nb,
                                           int in_dim, int8_t *sx, float *sxs) {
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int t = wave + 4 * r;
#pragma unroll
        for (int j = 0; j < PJN; j++) {
            float sg;
            const uint32_t q = quant_octet(v[r][j], &sg);
            const int f = lane + 64 * j;
            if (t < nm && f < nf) {
                reinterpret_cast<uint32_t *>(sx + (size_t)t * in_dim)[f] = q;
                if (!(f & 7)) sxs[t * nb + (f >> 3)] = sg;
            }
        }
    }
}

// Builds the tile's activation rows in LDS from the job's prologue: sx
// [M][in_dim] int8 and sxs [M][in_dim/32].  Row t of the tile is activation
// row xrow[t]; rows t >= nm are left unused.  The prologue's global loads are
// issued first, then issue_w() (the tile's weight loads), then the
// prologue's arithmetic, so the weight loads are in flight behind it and the
// first use of a prologue value waits only for the prologue's own loads.
// Float prologues: wave w builds rows w and w + 4 (one float4 per lane per
// 256 elements), so the quantization groups are lane octets.  PRO_NORM
// (lz_rmsnorm, src/ops_norm.c:690-747, after the residual fold x += a (+ b)
// of src/forward.c:1449-1557): the squares go to LDS and wave w takes the
// index-order sum of rows w and w + 4 (wave_sum_nonneg); the block with `writer` set
// stores the updated residual and the normed rows.  PRO_SILU:
// lz_ffn_gate_up's silu(g)*u (src/forward_kda.c:1067-1088).  PRO_COMBINE:
// the slot-ordered weighted sum of the experts' outputs
// (src/forward_moe.c:128-200).  Every load is unconditional (rows past nm
// and elements past the row end are clamped to valid addresses and their
// values unused), and each mode is one straight-line block.  Contains block
// barriers: call from every thread.
#define XQ_PER_THREAD 4
// Prologue-mode sets a kernel instance is compiled for (bit 1 << PRO_*);
// every other mode's code is left out of the instance.
#define MB(m) (1 << (m))
#define MODES_X MB(PRO_XQ)
#define MODES_N MB(PRO_NORM)
#define MODES_S MB(PRO_SILU)
#define MODES_Q MB(PRO_QUANT)
#define MODES_CS (MB(PRO_COMBINE) | MB(PRO_SILU))
#define MODES_NF (MB(PRO_NORM) | MB(PRO_FOLD))
// Instance flag: the jobs' weights have grouped scales (more than one per
// row); instances without it keep one scale per row in a register.
#define MG (1 << 7)
// Instance flag: the launch's argmax epilogue (GemvBatch.amax_out).
#define MA (1 << 8)

// The packed argmax candidate of output value v at index i: the float key
// above the complemented index, so the larger value wins and, among equal
// keys, the lower index.  mode 0: sample_argmax's key (src/sampler.c:121);
// 1: lz_argmax_p1's compare (NaN never wins, -0 ties +0).
__device__ __forceinline__ unsigned long long amax_cand(float v, int i, int mode) {
    const uint32_t k = mode == 0 ? d_fkey(v) : (v != v) ? 0u : d_fkey(v == 0.0f ? 0.0f : v);
    return ((unsigned long long)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}
// The activation loads of a prologue go out before the tile's weight loads:
// the empty asm with a memory clobber keeps every earlier load above it
// (no pass may sink one into a later conditional use, behind the weights,
// where its wait would retire the weights too), and sched_barrier keeps the
// scheduler from interleaving them.  The prologue's arithmetic (the norm's
// exact sum) then runs while the weights are in flight.
#define PRO_ISSUE_W()                            \
    do {                                         \
        asm volatile("" ::: "memory");           \
        __builtin_amdgcn_sched_barrier(0);       \
        issue_w();                               \
        __builtin_amdgcn_sched_barrier(0);       \
    } while (0)

template <int M, int PJ, int MODES, typename IssueW>
__device__ __forceinline__ void build_rows(const Prologue &P, const int8_t *xq,
                                           const float *xqs, int in_dim, const int (&xrow)[M], int nm,
                                           bool writer, int8_t *sx, float *sxs, float *sq, float *s_inv,
                                           float *tab, IssueW issue_w) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nb = in_dim >> 5, nf = in_dim >> 2;
    if (PJ == 0 || ((MODES & MB(PRO_XQ)) && P.mode == PRO_XQ)) {
        // int4 chunk idx of the tile's rows: token idx / cpr, chunk idx % cpr;
        // the stores are unconditional (clamped: past the end they rewrite
        // the last chunk with its own value).
        // (no __restrict__ on xq / xqs: the empty asm's memory clobber in
        // PRO_ISSUE_W then keeps these loads above the weights', which a
        // restrict-qualified read-only pointer would let the compiler sink
        // to their LDS stores, each behind a wait for the whole tile)
        const int cpr = in_dim >> 4;
        const int total = M * cpr, stotal = M * nb;
        // loads per thread in the first batch: M rows of up to GEMV_MAX_IN
        constexpr int XU = (M * (GEMV_MAX_IN / 16) + GEMV_THREADS - 1) / GEMV_THREADS < XQ_PER_THREAD
                               ? (M * (GEMV_MAX_IN / 16) + GEMV_THREADS - 1) / GEMV_THREADS
                               : XQ_PER_THREAD;
        v4i r[XU];                       // a vector type: kept in registers (an int4 array went to scratch)
        float sc[XU];
#pragma unroll
        for (int u = 0; u < XU; u++) {
            const int idx = imin(u * GEMV_THREADS + tid, total - 1);
            const int t = idx / cpr, p = idx - t * cpr;
            r[u] = *reinterpret_cast<const v4i *>(xq + (size_t)xrow[t < nm ? t : 0] * in_dim + p * 16);
            const int si = imin(u * GEMV_THREADS + tid, stotal - 1);
            const int ts = si / nb;
            sc[u] = xqs[(size_t)xrow[ts < nm ? ts : 0] * nb + (si - ts * nb)];
        }
        PRO_ISSUE_W();
#pragma unroll
        for (int u = 0; u < XU; u++) {
            reinterpret_cast<v4i *>(sx)[imin(u * GEMV_THREADS + tid, total - 1)] = r[u];
            sxs[imin(u * GEMV_THREADS + tid, stotal - 1)] = sc[u];
        }
        for (int base = XU * GEMV_THREADS; base < total; base += GEMV_THREADS) {
            const int idx = imin(base + tid, total - 1);
            const int t = idx / cpr, p = idx - t * cpr;
            reinterpret_cast<int4 *>(sx)[idx] =
                *reinterpret_cast<const int4 *>(xq + (size_t)xrow[t < nm ? t : 0] * in_dim + p * 16);
        }
        for (int base = XU * GEMV_THREADS; base < stotal; base += GEMV_THREADS) {
            const int si = imin(base + tid, stotal - 1);
            const int ts = si / nb;
            sxs[si] = xqs[(size_t)xrow[ts < nm ? ts : 0] * nb + (si - ts * nb)];
        }
        return;
    }
    constexpr int RW = (M + 3) / 4;
    constexpr int PJN = PJ > 0 ? PJ : 1;
    int xr[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int t = wave + 4 * r;
        xr[r] = xrow[t < nm ? t : 0];
    }
    int fc[PJN];
#pragma unroll
    for (int j = 0; j < PJN; j++) fc[j] = imin(lane + 64 * j, nf - 1);
    float4 v[RW][PJN];
    if ((MODES & MB(PRO_QUANT)) && P.mode == PRO_QUANT) {
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++)
                v[r][j] = reinterpret_cast<const float4 *>(P.src + (size_t)xr[r] * P.src_stride)[fc[j]];
        PRO_ISSUE_W();
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
    } else if ((MODES & MB(PRO_SILU)) && P.mode == PRO_SILU) {
        // the table entry through an opaque global pointer: a plain global
        // load, which the barrier below keeps ahead of the weights (a
        // constant-memory load may be moved after them, and a flat load's
        // wait would retire them too; either way the table's store would
        // wait the weights out)
        const float *tabp = c_exp_tab;
        asm volatile("" : "+s"(tabp));
        const float tabv = ((const __attribute__((address_space(1))) float *)tabp)[lane & 31];
        float4 q[RW][PJN];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                v[r][j] = reinterpret_cast<const float4 *>(P.src + (size_t)xr[r] * P.src_stride)[fc[j]];
                q[r][j] = reinterpret_cast<const float4 *>(P.src2 + (size_t)xr[r] * P.src_stride)[fc[j]];
            }
        PRO_ISSUE_W();
        if (tid < 32) tab[tid] = tabv;
        __syncthreads();
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) v[r][j] = f4_silu_mul(v[r][j], q[r][j], tab);
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
    } else if ((MODES & MB(PRO_COMBINE)) && P.mode == PRO_COMBINE) {
        int sidx[RW][MAX_TOPK];
        float swt[RW][MAX_TOPK];
        float4 h[RW][MAX_TOPK][PJN];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int k = 0; k < MAX_TOPK; k++) {
                const int pair = xr[r] * P.topk + imin(k, P.topk - 1);
                sidx[r][k] = P.sel_idx[pair];
                swt[r][k] = P.sel_w[pair];
#pragma unroll
                for (int j = 0; j < PJN; j++)
                    h[r][k][j] = reinterpret_cast<const float4 *>(P.src + (size_t)pair * in_dim)[fc[j]];
            }
        PRO_ISSUE_W();
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int k = 0; k < MAX_TOPK; k++) {
                    const float wk = swt[r][k];
                    const float4 hk = h[r][k][j];
                    const float4 y2 = make_float4(y.x + wk * hk.x, y.y + wk * hk.y, y.z + wk * hk.z, y.w + wk * hk.w);
                    if (k < P.topk && sidx[r][k] >= 0) y = y2;
                }
                v[r][j] = y;
            }
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
    } else if (MODES & (MB(PRO_NORM) | MB(PRO_FOLD))) {   // PRO_NORM, PRO_FOLD
        // PRO_FOLD: the folded rows are quantized without a norm (only in
        // instances compiled for it; elsewhere do_norm is a constant)
        const bool do_norm = !(MODES & MB(PRO_FOLD)) || P.mode == PRO_NORM;
        const bool has_a = P.a != nullptr, has_b = P.b != nullptr;
        const float *pa = has_a ? P.a : P.src;
        const float *pb = has_b ? P.b : pa;
        const int sa = has_a ? in_dim : P.src_stride, sb = has_b ? in_dim : sa;
        float4 wn[PJN], ad[RW][PJN], bd[RW][PJN];
#pragma unroll
        for (int j = 0; j < PJN; j++) wn[j] = reinterpret_cast<const float4 *>(do_norm ? P.w : P.src)[fc[j]];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                v[r][j] = reinterpret_cast<const float4 *>(P.src + (size_t)xr[r] * P.src_stride)[fc[j]];
                ad[r][j] = reinterpret_cast<const float4 *>(pa + (size_t)xr[r] * sa)[fc[j]];
                bd[r][j] = reinterpret_cast<const float4 *>(pb + (size_t)xr[r] * sb)[fc[j]];
            }
        PRO_ISSUE_W();
        // x + (a + b), x + a, or x
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                float4 a2 = ad[r][j];
                const float4 b2 = bd[r][j];
                const float4 ab = make_float4(a2.x + b2.x, a2.y + b2.y, a2.z + b2.z, a2.w + b2.w);
                if (has_b) a2 = ab;
                const float4 x = v[r][j];
                const float4 xa = make_float4(x.x + a2.x, x.y + a2.y, x.z + a2.z, x.w + a2.w);
                if (has_a) v[r][j] = xa;
            }
        // squares in the layout of the exact wave sum (4 * PJN elements per
        // lane); wave w sums rows w and w + 4
        constexpr int PC = 4 * PJN;
        constexpr int rowf = ps_row_floats<PC>();
        if (do_norm) {
#pragma unroll
            for (int r = 0; r < RW; r++) {
                const int t = wave + 4 * r;
#pragma unroll
                for (int j = 0; j < PJN; j++) {
                    const int f = lane + 64 * j;
                    if (t < nm && f < nf) {
                        const float4 x = v[r][j];
                        *reinterpret_cast<float4 *>(sq + (size_t)t * rowf + ps_slot<PC>(4 * f)) =
                            make_float4(x.x * x.x, x.y * x.y, x.z * x.z, x.w * x.w);
                    }
                }
            }
            __syncthreads();
            PsRec *rec = reinterpret_cast<PsRec *>(sq + (size_t)M * rowf) + wave * 128;
            for (int t = wave; t < nm; t += 4) {
                const float ss = wave_sum_nonneg<PC>(sq + (size_t)t * rowf, in_dim, rec);
                if (lane == 0) s_inv[t] = d_rsqrt(d_ss_over_n(ss, in_dim) + P.eps);
            }
            __syncthreads();
        }
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int t = wave + 4 * r;
            const float inv = do_norm ? s_inv[t < nm ? t : 0] : 1.0f;
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                const int f = lane + 64 * j;
                const float4 x = v[r][j], w = wn[j];
                const float4 o = do_norm ? make_float4(x.x * inv * (1.0f + w.x), x.y * inv * (1.0f + w.y),
                                                       x.z * inv * (1.0f + w.z), x.w * inv * (1.0f + w.w))
                                         : x;
                if (writer && t < nm && f < nf) {
                    if (P.x_out) reinterpret_cast<float4 *>(P.x_out + (size_t)xr[r] * P.src_stride)[f] = x;
                    if (P.o_out) reinterpret_cast<float4 *>(P.o_out + (size_t)xr[r] * P.o_stride)[f] = o;
                }
                v[r][j] = o;
            }
        }
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
    }
}

// Partial dot products of one tile.  Lane chunk j is c0 + 64 j; its (row,
// offset) advance by 64 chunks per step.  When cpr divides 64 every chunk
// of the lane sits at the same in-row offset and its activation chunks are
// read from LDS once.  Neighbouring lanes hold the two 16-byte halves of a
// 32-element group: after the pair sum (DPP) both store the same exact
// int32 group sum to the same slot.  Chunk steps past the tile's R rows are
// skipped (wave-uniform); chunks past the live rows repeat the last chunk's
// weights into rows the epilogue ignores.
template <int M>
__device__ __forceinline__ void tile_dot(const int4 (&wv)[GEMV_MAXJ], const int8_t *sx, int *part, int in_dim, int R) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cpr = in_dim >> 4, pstride = (in_dim >> 5) + 4;
    const int4 *sx4 = reinterpret_cast<const int4 *>(sx);
    const int c0 = wave * (GEMV_WAVE_BYTES / 16) + lane;
    const int q64 = 64 / cpr, m64 = 64 - q64 * cpr;
    const int cmax = R * cpr;
    const bool reuse = m64 == 0;
    int r = c0 / cpr, p = c0 - r * cpr;
    int4 xv[M];
    if (reuse && (cmax & (GEMV_WAVE_BYTES / 16 - 1)) == 0) {
        // every lane's chunks share one in-row offset and this wave's 8 KiB
        // quarter is all live (or all past the tile's rows): straight-line
        // code, the token rows' dot products interleaved
        if (wave * (GEMV_WAVE_BYTES / 16) >= cmax) return;
#pragma unroll
        for (int t = 0; t < M; t++) xv[t] = sx4[t * cpr + p];
#pragma unroll
        for (int j = 0; j < GEMV_MAXJ; j++) {
            int a[M];
#pragma unroll
            for (int t = 0; t < M; t++) a[t] = __builtin_amdgcn_sdot4(wv[j].x, xv[t].x, 0, false);
#pragma unroll
            for (int t = 0; t < M; t++) a[t] = __builtin_amdgcn_sdot4(wv[j].y, xv[t].y, a[t], false);
#pragma unroll
            for (int t = 0; t < M; t++) a[t] = __builtin_amdgcn_sdot4(wv[j].z, xv[t].z, a[t], false);
#pragma unroll
            for (int t = 0; t < M; t++) a[t] = __builtin_amdgcn_sdot4(wv[j].w, xv[t].w, a[t], false);
            int *dst = part + (r + j * q64) * M * pstride + (p >> 1);
#pragma unroll
            for (int t = 0; t < M; t++) {
                a[t] += __builtin_amdgcn_update_dpp(0, a[t], 0xB1, 0xF, 0xF, false);     // lane ^ 1
                dst[t * pstride] = a[t];
            }
        }
        return;
    }
    if (reuse) {
#pragma unroll
        for (int t = 0; t < M; t++) xv[t] = sx4[t * cpr + p];
    }
#pragma unroll
    for (int j = 0; j < GEMV_MAXJ; j++) {
        if (wave * (GEMV_WAVE_BYTES / 16) + 64 * j < cmax) {
            if (!reuse) {
#pragma unroll
                for (int t = 0; t < M; t++) xv[t] = sx4[t * cpr + p];
            }
            int *dst = part + r * M * pstride + (p >> 1);
#pragma unroll
            for (int t = 0; t < M; t++) {
                int a = __builtin_amdgcn_sdot4(wv[j].x, xv[t].x, 0, false);
                a = __builtin_amdgcn_sdot4(wv[j].y, xv[t].y, a, false);
                a = __builtin_amdgcn_sdot4(wv[j].z, xv[t].z, a, false);
                a = __builtin_amdgcn_sdot4(wv[j].w, xv[t].w, a, false);
                a += __builtin_amdgcn_update_dpp(0, a, 0xB1, 0xF, 0xF, false);     // lane ^ 1
                dst[t * pstride] = a;
            }
        }
        r += q64;
        p += m64;
        if (p >= cpr) { p -= cpr; r++; }
    }
}

// Epilogue of a row whose weight scales come in groups of r 32-element
// groups (r = gs/32 < nb), epi_q8 (src/ops_epi.c:983-1022): r > 1, per run
// of r groups dot = sum float(acc)*xqs from 0, sum += dot*ws[run] in run
// order; r == 1, four accumulators take groups g, g+1, g+2, g+3 of each
// whole four (the rest go to the first) as float(acc)*(xqs*ws), then
// (a0 + a2) + (a1 + a3).  wsr: the row's scales (global memory).
__device__ __forceinline__ float tile_epilogue_g(const int *pp, const float *xs, int nb, int r, const float *wsr) {
    float sum = 0.0f;
    if (r > 1) {
        for (int run = 0; run < nb / r; run++) {
            float dot = 0.0f;
            for (int g = 0; g < r; g++) dot += (float)pp[run * r + g] * xs[run * r + g];
            sum += dot * wsr[run];
        }
        return sum;
    }
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int g = 0;
    for (; g + 3 < nb; g += 4) {
        a0 += (float)pp[g] * (xs[g] * wsr[g]);
        a1 += (float)pp[g + 1] * (xs[g + 1] * wsr[g + 1]);
        a2 += (float)pp[g + 2] * (xs[g + 2] * wsr[g + 2]);
        a3 += (float)pp[g + 3] * (xs[g + 3] * wsr[g + 3]);
    }
    for (; g < nb; g++) a0 += (float)pp[g] * (xs[g] * wsr[g]);
    return (a0 + a2) + (a1 + a3);
}

// Epilogue of one (row er, token et) pair: sum_s float(acc[s]) * xqs[s] in
// group order, then times the row scale (src/ops_epi.c:983-1017); a
// one-group row takes epi_one_group.
__device__ __forceinline__ float tile_epilogue(const int *pp, const float *xs, int nb, float wsv) {
    if (nb == 1) return epi_one_group(pp[0], xs[0], wsv);
    float dot = 0.0f;
    if ((nb & 3) == 0) {
        // the LDS reads run up to three groups of four ahead of the
        // dependent adds
        const int4 *pp4 = reinterpret_cast<const int4 *>(pp);
        const float4 *xs4 = reinterpret_cast<const float4 *>(xs);
        const int n4 = nb >> 2;
        int4 q0 = pp4[0], q1 = pp4[imin(1, n4 - 1)], q2 = pp4[imin(2, n4 - 1)];
        float4 x0 = xs4[0], x1 = xs4[imin(1, n4 - 1)], x2 = xs4[imin(2, n4 - 1)];
        for (int g = 0; g < n4; g++) {
            const int4 q3 = pp4[imin(g + 3, n4 - 1)];
            const float4 x3 = xs4[imin(g + 3, n4 - 1)];
            dot += (float)q0.x * x0.x;
            dot += (float)q0.y * x0.y;
            dot += (float)q0.z * x0.z;
            dot += (float)q0.w * x0.w;
            q0 = q1; q1 = q2; q2 = q3;
            x0 = x1; x1 = x2; x2 = x3;
        }
    } else {
        for (int g = 0; g < nb; g++) dot += (float)pp[g] * xs[g];
    }
    float sum = 0.0f;
    sum += dot * wsv;
    return sum;
}

// The tile's weights: one 8 KiB quarter per wave, all loads in flight.
__device__ __forceinline__ void tile_load(int4 (&wv)[GEMV_MAXJ], const int8_t *__restrict__ wt, int nchunk) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const v4i *w4 = reinterpret_cast<const v4i *>(wt);
#pragma unroll
    for (int j = 0; j < GEMV_MAXJ; j++) {
        const int c = imin(wave * (GEMV_WAVE_BYTES / 16) + lane + 64 * j, nchunk - 1);
        const v4i q = __builtin_nontemporal_load(w4 + c);
        wv[j] = make_int4(q.x, q.y, q.z, q.w);
    }
}

// One GEMV tile of rows_here <= R rows.  xrow[t]: activation row of token
// slot t (registers); s_orow[t]: output row of token slot t (LDS, read after
// a barrier); nm: live token slots.  The caller fills the LDS exp table
// first.
template <int M, int PJ, int MODES>
__device__ __forceinline__ void gemv_tile(const int8_t *__restrict__ wt, const float *__restrict__ ws, int rows_here,
                                          int R, int in_dim, const Prologue &P, const int8_t *xq,
                                          const float *xqs, const int (&xrow)[M], const int *s_orow,
                                          int nm, bool writer, float *__restrict__ out, size_t out_stride,
                                          int row0, int32_t *__restrict__ acc_out, int acc_rows, char *smem,
                                          float *s_inv, float *tab, int gs = 0,
                                          unsigned long long *s_am = nullptr, int amax_mode = 0) {
    // scales per row (ws holds [rows][nws]): one unless the instance is
    // compiled for grouped scales
    constexpr bool GROUPED = (MODES & MG) != 0;
    const int nws = (GROUPED && gs > 0 && gs < in_dim) ? in_dim / gs : 1;
    const int tid = threadIdx.x;
    const int cpr = in_dim >> 4, nb = in_dim >> 5, pstride = nb + 4;
    const int nchunk = rows_here * cpr;
    int8_t *sx = reinterpret_cast<int8_t *>(smem);                                   // [M][in_dim]
    float *sxs = reinterpret_cast<float *>(smem + (size_t)M * in_dim);                // [M][nb]
    int *part = reinterpret_cast<int *>(sxs + ((M * nb + 3) & ~3));                   // [R][M][nb+4]
    int4 wv[GEMV_MAXJ];
    const int er = tid / M, et = tid - er * M;
    float wsv = 0.0f;
    auto issue_w = [&]() {
        tile_load(wv, wt, nchunk);
        wsv = ws[(size_t)(row0 + imin(er, rows_here - 1)) * nws];     // the epilogue lane's (first) row scale
    };
    build_rows<M, PJ, MODES>(P, xq, xqs, in_dim, xrow, nm, writer, sx, sxs, reinterpret_cast<float *>(part), s_inv,
                             tab, issue_w);
    __syncthreads();
    tile_dot<M>(wv, sx, part, in_dim, R);
    __syncthreads();
    if (er < rows_here && et < nm) {
        const int *pp = part + (er * M + et) * pstride;
        float o;
        if (GROUPED && nws > 1) o = tile_epilogue_g(pp, sxs + et * nb, nb, gs >> 5, ws + (size_t)(row0 + er) * nws);
        else o = tile_epilogue(pp, sxs + et * nb, nb, wsv);
        out[(size_t)s_orow[et] * out_stride + row0 + er] = o;
        if (MODES & MA) atomicMax(&s_am[et], amax_cand(o, row0 + er, amax_mode));
        if (acc_out)
            for (int g = 0; g < nb; g++) acc_out[((size_t)et * acc_rows + row0 + er) * nb + g] = pp[g];
    }
}

// Dynamic LDS a GEMV block may use: the device's per-block limit (160 KiB
// on gfx950), less room for the kernels' static LDS.  Queried once.
static inline size_t gemv_lds_limit() {
    static size_t lim = 0;
    if (!lim) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        lim = (size_t)v - 12 * 1024;
    }
    return lim;
}

// Lets kernel `k` take dynamic LDS above the default 64 KiB (once per kernel).
#define ALLOW_BIG_LDS(k)                                                                                  \
    do {                                                                                                  \
        static bool done_ = false;                                                                        \
        if (!done_) {                                                                                     \
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k), hipFuncAttributeMaxDynamicSharedMemorySize, \
                                      (int)gemv_lds_limit());                                             \
            done_ = true;                                                                                 \
        }                                                                                                 \
    } while (0)

// Rows per GEMV tile: the tile is at most GEMV_TILE_BYTES of weights and
// R*m (row, token) epilogue pairs fit the block.
static int gemv_rows_per_tile(int in_dim, int m) {
    int r = GEMV_TILE_BYTES / in_dim;
    if (r < 1) r = 1;
    if (r > GEMV_THREADS / m) r = GEMV_THREADS / m;
    return r;
}

static bool prologue_ok(const Prologue &P, int in_dim, const int8_t *xq, const float *xqs) {
    if (P.mode == PRO_XQ) return xq && xqs;
    if (in_dim > PRO_MAX_IN || !P.src) return false;
    if (P.mode == PRO_QUANT) return P.src_stride >= in_dim && !(P.src_stride & 3);
    if (P.mode == PRO_SILU) return P.src2 && P.src_stride >= in_dim && !(P.src_stride & 3);
    if (P.mode == PRO_NORM) return P.w && P.src_stride >= in_dim && !(P.src_stride & 3) && !(P.o_stride & 3);
    if (P.mode == PRO_FOLD) return P.src_stride >= in_dim && !(P.src_stride & 3) && !(P.o_stride & 3);
    if (P.mode == PRO_COMBINE) return P.sel_idx && P.sel_w && P.topk >= 1 && P.topk <= MAX_TOPK;
    return false;
}

#endif

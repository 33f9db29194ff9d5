// Row kernels (embedding, RMSNorm, MTP input), argmax and round control
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_devmath.h"

// -------------------------------------------------------------- embed ---

// lz_t_row_f32 for a Q8_0 per-row table: x = float(q) * scale[row].
// lz_t_row_f32 of a Q8_0 row (src/ops_epi.c:1276-1280): q * its group's
// scale, groups of gs (gs = d: one scale per row).
__global__ void k_embed(const int8_t *__restrict__ q, const float *__restrict__ s,
                        const int *__restrict__ toks, int d, int gs, float *__restrict__ x) {
    int t = blockIdx.y;
    int tok = toks[t];
    const int8_t *row = q + (size_t)tok * d;
    const float *sr = s + (size_t)tok * (d / gs);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        x[(size_t)t * d + i] = (float)row[i] * sr[i / gs];
}

template <int PJ, bool NORM, bool TOK>
__global__ __launch_bounds__(64) void k_rmsnorm(float *__restrict__ x, int x_stride,
                                                const float *__restrict__ a, const float *__restrict__ b,
                                                const float *__restrict__ w, int n, float eps,
                                                float *__restrict__ out, int out_stride,
                                                int8_t *__restrict__ xq, float *__restrict__ xqs) {
    __shared__ __align__(16) float sq[ps_row_floats<4 * PJ>()];
    __shared__ PsRec rec[128];
    __shared__ float s_inv;
    const int row = blockIdx.x, lane = threadIdx.x, nf = n >> 2;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * x_stride);
    float4 v[PJ], wn[PJ];
#pragma unroll
    for (int j = 0; j < PJ; j++) {
        const int fc = imin(lane + 64 * j, nf - 1);
        v[j] = xr[fc];
        wn[j] = reinterpret_cast<const float4 *>(w ? w : x)[fc];
    }
    if (a) {
        float4 av[PJ];
#pragma unroll
        for (int j = 0; j < PJ; j++) av[j] = reinterpret_cast<const float4 *>(a + (size_t)row * n)[imin(lane + 64 * j, nf - 1)];
        if (b) {
#pragma unroll
            for (int j = 0; j < PJ; j++) {
                const float4 bv = reinterpret_cast<const float4 *>(b + (size_t)row * n)[imin(lane + 64 * j, nf - 1)];
                av[j] = make_float4(av[j].x + bv.x, av[j].y + bv.y, av[j].z + bv.z, av[j].w + bv.w);
            }
        }
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            v[j] = make_float4(v[j].x + av[j].x, v[j].y + av[j].y, v[j].z + av[j].z, v[j].w + av[j].w);
            if (lane + 64 * j < nf) xr[lane + 64 * j] = v[j];
        }
    }
    norm_row<PJ, NORM, TOK>(v, wn, n, eps, sq, rec, &s_inv, out ? out + (size_t)row * out_stride : nullptr,
                            xq ? xq + (size_t)row * n : nullptr, xqs ? xqs + (size_t)row * (n >> 5) : nullptr);
}

// The same row operation (one scale per 32) with a 256-thread block per
// row, for rows of more than 512 elements: thread t holds float4 t + 256 j
// of the row, so the loads, the residual fold, the normalization and the
// per-32 quantization (an aligned lane octet per group, as above) spread
// over four waves, and wave 0 takes the index-order sum of the squares with
// the one-wave kernel's exact wave sum (the same layout, so the same bits).
template <int PJ, bool NORM>
__global__ __launch_bounds__(256) void k_rmsnorm_b(float *__restrict__ x, int x_stride,
                                                   const float *__restrict__ a, const float *__restrict__ b,
                                                   const float *__restrict__ w, int n, float eps,
                                                   float *__restrict__ out, int out_stride,
                                                   int8_t *__restrict__ xq, float *__restrict__ xqs) {
    constexpr int PB = PJ / 4, PC = 4 * PJ;           // float4 per thread; the sum's lane chunk
    static_assert(PJ == 4 || PJ == 8, "rows of 513..2048 elements");
    __shared__ __align__(16) float sq[ps_row_floats<PC>()];
    __shared__ PsRec rec[128];
    __shared__ float s_inv;
    const int row = blockIdx.x, tid = threadIdx.x, nf = n >> 2;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * x_stride);
    float4 v[PB], wn[PB];
#pragma unroll
    for (int j = 0; j < PB; j++) {
        const int fc = imin(tid + 256 * j, nf - 1);
        v[j] = xr[fc];
        wn[j] = reinterpret_cast<const float4 *>(w ? w : x)[fc];
    }
    if (a) {
        float4 av[PB];
#pragma unroll
        for (int j = 0; j < PB; j++) av[j] = reinterpret_cast<const float4 *>(a + (size_t)row * n)[imin(tid + 256 * j, nf - 1)];
        if (b) {
#pragma unroll
            for (int j = 0; j < PB; j++) {
                const float4 bv = reinterpret_cast<const float4 *>(b + (size_t)row * n)[imin(tid + 256 * j, nf - 1)];
                av[j] = make_float4(av[j].x + bv.x, av[j].y + bv.y, av[j].z + bv.z, av[j].w + bv.w);
            }
        }
#pragma unroll
        for (int j = 0; j < PB; j++) {
            v[j] = make_float4(v[j].x + av[j].x, v[j].y + av[j].y, v[j].z + av[j].z, v[j].w + av[j].w);
            if (tid + 256 * j < nf) xr[tid + 256 * j] = v[j];
        }
    }
    float inv = 1.0f;
    if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < PB; j++) {
            const int f = tid + 256 * j;
            if (f < nf)
                *reinterpret_cast<float4 *>(sq + ps_slot<PC>(4 * f)) =
                    make_float4(v[j].x * v[j].x, v[j].y * v[j].y, v[j].z * v[j].z, v[j].w * v[j].w);
        }
        __syncthreads();
        if (tid < 64) {
            const float ss = wave_sum_nonneg<PC>(sq, n, rec);
            if (tid == 0) s_inv = d_rsqrt(d_ss_over_n(ss, n) + eps);
        }
        __syncthreads();
        inv = s_inv;
    }
    float *orow = out ? out + (size_t)row * out_stride : nullptr;
    int8_t *qrow = xq ? xq + (size_t)row * n : nullptr;
    float *srow = xq ? xqs + (size_t)row * (n >> 5) : nullptr;
#pragma unroll
    for (int j = 0; j < PB; j++) {
        const int f = tid + 256 * j;
        float4 o = v[j];
        if constexpr (NORM)
            o = make_float4(v[j].x * inv * (1.0f + wn[j].x), v[j].y * inv * (1.0f + wn[j].y),
                            v[j].z * inv * (1.0f + wn[j].z), v[j].w * inv * (1.0f + wn[j].w));
        if (orow && f < nf) reinterpret_cast<float4 *>(orow)[f] = o;
        if (qrow) {
            float sg;
            const uint32_t q = quant_octet(o, &sg);
            if (f < nf) {
                reinterpret_cast<uint32_t *>(qrow)[f] = q;
                if (!(f & 7)) srow[f >> 3] = sg;
            }
        }
    }
}

// MTP input rows (lz_mtp_draft_step / lz_mtp_prefill, src/forward_mtp.c:
// e = embed(tok); concat = [rmsnorm(e, pre_e) | rmsnorm(h, pre_h)], then the
// per-32 quantization of concat for the fc projection).  blockIdx.y = 0: the
// embedding half, 1: the hidden half.  d % 32 == 0, so the halves quantize
// independently.
template <int PJ>
__global__ __launch_bounds__(64) void k_mtp_pre(const int8_t *__restrict__ emb_q, const float *__restrict__ emb_s,
                                                const int *__restrict__ toks, const float *__restrict__ h,
                                                int d, int gs, const float *__restrict__ w_e,
                                                const float *__restrict__ w_h, float eps,
                                                int8_t *__restrict__ xq, float *__restrict__ xqs) {
    __shared__ __align__(16) float sq[ps_row_floats<4 * PJ>()];
    __shared__ PsRec rec[128];
    __shared__ float s_inv;
    const int r = blockIdx.x, half = blockIdx.y, lane = threadIdx.x, nf = d >> 2;
    const float4 *wn4 = reinterpret_cast<const float4 *>(half == 0 ? w_e : w_h);
    float4 v[PJ], wn[PJ];
    if (half == 0) {
        const int tok = toks[r];
        const uint32_t *er = reinterpret_cast<const uint32_t *>(emb_q + (size_t)tok * d);
        const float *sr = emb_s + (size_t)tok * (d / gs);
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const int fe = imin(lane + 64 * j, nf - 1);
            const uint32_t q = er[fe];
            const float sc = sr[4 * fe / gs];      // the four codes share a 32-group
            v[j] = make_float4((float)(int8_t)(q & 0xFF) * sc, (float)(int8_t)((q >> 8) & 0xFF) * sc,
                               (float)(int8_t)((q >> 16) & 0xFF) * sc, (float)(int8_t)(q >> 24) * sc);
        }
    } else {
#pragma unroll
        for (int j = 0; j < PJ; j++) v[j] = reinterpret_cast<const float4 *>(h + (size_t)r * d)[imin(lane + 64 * j, nf - 1)];
    }
#pragma unroll
    for (int j = 0; j < PJ; j++) wn[j] = wn4[imin(lane + 64 * j, nf - 1)];
    norm_row<PJ>(v, wn, d, eps, sq, rec, &s_inv, nullptr, xq + (size_t)r * 2 * d + (size_t)half * d,
                 xqs + (size_t)r * (2 * d >> 5) + (size_t)half * (d >> 5));
}

// The DSpark draft batch's main_proj input (lz_mtp_draft_batch,
// src/forward_mtp.c:404-439): row r (slot r) is [rmsnorm(chain, pre_h) |
// rmsnorm(e_r, pre_e) | depth row r], e_0 the embedding row of the anchor
// token, e_r (r > 0) the shared mask row, then its per-32 quantization.
// blockIdx.y picks the third; d % 32 == 0, so the thirds quantize
// independently.
template <int PJ>
__global__ __launch_bounds__(64) void k_dspark_pre(const int8_t *__restrict__ emb_q, const float *__restrict__ emb_s,
                                                   const int *__restrict__ tok, const float *__restrict__ chain,
                                                   const float *__restrict__ mask, const float *__restrict__ depth,
                                                   int d, int gs, const float *__restrict__ w_e,
                                                   const float *__restrict__ w_h, float eps,
                                                   int8_t *__restrict__ xq, float *__restrict__ xqs) {
    __shared__ __align__(16) float sq[ps_row_floats<4 * PJ>()];
    __shared__ PsRec rec[128];
    __shared__ float s_inv;
    const int r = blockIdx.x, third = blockIdx.y, lane = threadIdx.x, nf = d >> 2;
    float4 v[PJ], wn[PJ];
    const float *src = third == 0 ? chain : third == 2 ? depth + (size_t)r * d : mask;
    if (third == 1 && r == 0) {
        const uint32_t *er = reinterpret_cast<const uint32_t *>(emb_q + (size_t)tok[0] * d);
        const float *sr = emb_s + (size_t)tok[0] * (d / gs);
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const int fe = imin(lane + 64 * j, nf - 1);
            const uint32_t q = er[fe];
            const float sc = sr[4 * fe / gs];
            v[j] = make_float4((float)(int8_t)(q & 0xFF) * sc, (float)(int8_t)((q >> 8) & 0xFF) * sc,
                               (float)(int8_t)((q >> 16) & 0xFF) * sc, (float)(int8_t)(q >> 24) * sc);
        }
    } else {
#pragma unroll
        for (int j = 0; j < PJ; j++) v[j] = reinterpret_cast<const float4 *>(src)[imin(lane + 64 * j, nf - 1)];
    }
    int8_t *q = xq + (size_t)r * 3 * d + (size_t)third * d;
    float *qs = xqs + (size_t)r * (3 * d >> 5) + (size_t)third * (d >> 5);
    if (third == 2) {
        norm_row<PJ, false>(v, wn, d, eps, sq, rec, &s_inv, nullptr, q, qs);
        return;
    }
    const float4 *wn4 = reinterpret_cast<const float4 *>(third == 0 ? w_h : w_e);
#pragma unroll
    for (int j = 0; j < PJ; j++) wn[j] = wn4[imin(lane + 64 * j, nf - 1)];
    norm_row<PJ>(v, wn, d, eps, sq, rec, &s_inv, nullptr, q, qs);
}

// Index-order sums of non-negative rows (wave_sum_nonneg, the sum the
// RMSNorm kernels use), one 64-lane block per row: the library's check of
// that routine on arbitrary inputs.
template <int C>
__global__ __launch_bounds__(64) void k_row_sums(const float *__restrict__ x, int n, float *__restrict__ out) {
    __shared__ __align__(16) float row[ps_row_floats<C>()];
    __shared__ PsRec rec[128];
    const float *xr = x + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += 64) row[ps_slot<C>(i)] = xr[i];
    __syncthreads();
    const float s = wave_sum_nonneg<C>(row, n, rec);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}

extern "C" int l98k_row_sums(const float *x, int rows, int n, float *out, hipStream_t st) {
    if (rows < 1 || n < 1 || n > 2048) return -1;
    if (n <= 256) hipLaunchKernelGGL(k_row_sums<4>, dim3(rows), dim3(64), 0, st, x, n, out);
    else if (n <= 512) hipLaunchKernelGGL(k_row_sums<8>, dim3(rows), dim3(64), 0, st, x, n, out);
    else if (n <= 1024) hipLaunchKernelGGL(k_row_sums<16>, dim3(rows), dim3(64), 0, st, x, n, out);
    else hipLaunchKernelGGL(k_row_sums<32>, dim3(rows), dim3(64), 0, st, x, n, out);
    return (int)hipGetLastError();
}

// -------------------------------------------------------- argmax / ctl ---

#define LZ_ARGMAX_ROWS 8
#define ARGMAX_THREADS 1024

// Per row argmax, one block of 1024 lanes per row: every lane scans a
// strided share of the row with its loads in flight, then a block max of
// the packed (key, ~index) words.  One block per row needs no hand-over
// between blocks (a device-scope fence on this chip writes back and
// invalidates every cache, which costs more than the row's read).  mode 0:
// order-preserving key, first index wins (sample_argmax,
// src/sampler.c:121-137).  mode 1: float '>' compare, first index wins
// (lz_argmax_p1's scan, src/sampler.c:139-155).
__global__ __launch_bounds__(ARGMAX_THREADS) void k_argmax(const float *__restrict__ x, int n, int mode,
                                                           int *__restrict__ out) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *r = x + (size_t)row * n;
    unsigned long long best = 0;
    auto fold = [&](float v, int i) {
        uint32_t k;
        if (mode == 0) k = d_fkey(v);
        else k = (v != v) ? 0u : d_fkey(v == 0.0f ? 0.0f : v);
        const unsigned long long cand = ((unsigned long long)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
        best = cand > best ? cand : best;
    };
    if ((n & 3) == 0 && ((uintptr_t)r & 15) == 0) {
        // float4 f = tid + 1024 * u: eight loads in flight per round
        const float4 *r4 = reinterpret_cast<const float4 *>(r);
        const int n4 = n >> 2;
        for (int base = 0; base < n4; base += 8 * ARGMAX_THREADS) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = r4[imin(base + u * ARGMAX_THREADS + tid, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int f = base + u * ARGMAX_THREADS + tid;
                if (f < n4) {
                    fold(v[u].x, 4 * f);
                    fold(v[u].y, 4 * f + 1);
                    fold(v[u].z, 4 * f + 2);
                    fold(v[u].w, 4 * f + 3);
                }
            }
        }
    } else {
        for (int i = tid; i < n; i += ARGMAX_THREADS) fold(r[i], i);
    }
    best = wave_max_u64(best);
    __shared__ unsigned long long sb[ARGMAX_THREADS / 64];
    if ((tid & 63) == 0) sb[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = 0;
        for (int i = 0; i < ARGMAX_THREADS / 64; i++) b = sb[i] > b ? sb[i] : b;
        int idx = (int)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
        // lz_argmax_p1 starts from element 0 and takes only v > best: a NaN
        // there is never beaten, so the row's answer is 0.
        if (mode == 1) {
            const float r0 = r[0];
            if (r0 != r0) idx = 0;
        }
        out[row] = idx;
    }
}

// The argmax of rows whose GEMV stored per-tile candidates (the lm_head's
// argmax epilogue): row r's candidates part[r * tiles .. + tiles) are the
// packed (key, complemented index) maxima of each tile, so their maximum is
// k_argmax's result over the row (x: the rows, for mode 1's NaN-at-0 rule).
__global__ __launch_bounds__(256) void k_argmax_part(const unsigned long long *__restrict__ part, int tiles,
                                                     const float *__restrict__ x, int n, int mode,
                                                     int *__restrict__ out) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const unsigned long long *p = part + (size_t)row * tiles;
    unsigned long long v[8], best = 0;
    for (int base = 0; base < tiles; base += 8 * 256) {
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = p[imin(base + u * 256 + tid, tiles - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) best = v[u] > best ? v[u] : best;
    }
    best = wave_max_u64(best);
    __shared__ unsigned long long sb[4];
    if ((tid & 63) == 0) sb[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = 0;
        for (int i = 0; i < 4; i++) b = sb[i] > b ? sb[i] : b;
        int idx = (int)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
        if (mode == 1) {
            const float r0 = x[(size_t)row * n];
            if (r0 != r0) idx = 0;
        }
        out[row] = idx;
    }
}

// Acceptance of a greedy round (lz_spec_accept, src/generate.c:232-243) and
// the device-side bookkeeping of lz_spec_round (src/generate.c:802-993):
// ring rollback, mtp_chain reseed from the accepted row, catch-up count,
// next anchor and positions.
// flags: bit 0 debug_break_rollback; bit 1 a DSpark round (no catch-up rows,
// mtp_pos unchanged: src/generate.c:1117-1133).
__device__ __forceinline__ void accept_body(DevCtl *ctl, const float *__restrict__ vhidden, int d,
                                            float *__restrict__ chain, int depth, int flags) {
    // flags: 1 the rollback break, 2 a DSpark round (no catch-up), 4 a
    // temperature round (n_accept and out[] already written by its
    // acceptance launches)
    const bool brk = (flags & 1) != 0, dspark = (flags & 2) != 0, sampled = (flags & 4) != 0;
    __shared__ int s_n;
    if (threadIdx.x == 0) {
        int k_eff = ctl->k_eff;
        int n = k_eff;
        if (sampled) {
            n = ctl->n_accept;
        } else {
            for (int i = 0; i < k_eff; i++) {
                ctl->out[i] = ctl->targ[i];
                if (ctl->tok[1 + i] != ctl->targ[i]) { n = i; break; }
            }
            if (n == k_eff) ctl->out[k_eff] = ctl->targ[k_eff];
        }
        ctl->n_accept = n;
        int base = ctl->slot_base;
        int slot = (base + k_eff + 1) % depth;           // what the verify left
        if (n < k_eff && !brk) slot = (base + n + 1) % depth;
        ctl->ssm_slot = slot;
        ctl->new_pos = ctl->anchor_pos + 1 + n;
        // catch-up pairs (verify_hidden[j], out[j]) j < n-1 at mtp_pos+1+j
        ctl->catch_n = n > 1 && !dspark ? n - 1 : 0;
        ctl->catch_pos = ctl->mtp_pos + 1;
        // Catch-up always runs k-1 rows so a round has a fixed shape; rows
        // j >= catch_n land at MTP positions >= the next round's mtp_pos,
        // which that round's draft steps overwrite before any read.
        for (int j = 0; j < 8; j++) ctl->catch_tok[j] = j < ctl->catch_n ? ctl->out[j] : ctl->out[0];
        ctl->mtp_pos_next = dspark ? ctl->mtp_pos : ctl->mtp_pos + n;
        s_n = n;
    }
    __syncthreads();
    const int n = s_n;
    for (int i = threadIdx.x; i < d; i += blockDim.x) chain[i] = vhidden[(size_t)n * d + i];
}

__global__ void k_accept(DevCtl *ctl, const float *__restrict__ vhidden, int d,
                         float *__restrict__ chain, int depth, int flags) {
    accept_body(ctl, vhidden, d, chain, depth, flags);
}

// The finished round into hist; the next round's anchor (op 1 below).
__device__ __forceinline__ void next_round(DevCtl *ctl, RoundRec *hist, int hist_cap) {
    if (hist && ctl->round < hist_cap) {
        RoundRec *r = hist + ctl->round;
        r->n_accept = ctl->n_accept;
        r->k_eff = ctl->k_eff;
        r->new_pos = ctl->new_pos;
        r->ssm_slot = ctl->ssm_slot;
        r->experts = ctl->expert_tally;
        for (int j = 0; j < 8; j++) r->out[j] = ctl->out[j];
    }
    ctl->expert_tally = 0;
    ctl->round++;
    ctl->anchor = ctl->out[ctl->n_accept];
    ctl->anchor_pos = ctl->new_pos;
    ctl->mtp_pos = ctl->mtp_pos_next;
    ctl->slot_base = ctl->ssm_slot;
    ctl->tok[0] = ctl->anchor;
}

// Round bookkeeping on the device.  op 0: draft input 0 = anchor.  op 1:
// record the finished round in hist and advance to the next one as the
// generation driver does with have_seed (src/generate.c:1850-1866,
// 2096-2104): anchor = out[n_accept] at position new_pos, mtp_pos and the
// ring slot carried over.  op 2: a temperature round's acceptance starts
// (n_accept = k_eff until a row rejects, no row decided).
__global__ void k_set_tokens(DevCtl *ctl, int op, RoundRec *hist, int hist_cap) {
    if (threadIdx.x != 0) return;
    if (op == 0) {
        ctl->tok[0] = ctl->anchor;
    } else if (op == 2) {
        ctl->n_accept = ctl->k_eff;
        ctl->smp_done = 0;
    } else if (op == 1) {
        next_round(ctl, hist, hist_cap);
    }
}

// ------------------------------------------------- session batch rounds ---
//
// A batch of sessions' greedy rounds as many-row passes: block r works for
// session r (its BatchSess entry).  Draft step j reads each session's input
// token tok[j] and chain into rows (k_batch_draft_in) and writes the rows'
// argmaxes and exit-norm rows back (k_batch_draft_out); the verify's token
// rows come from tok[0..K1), at positions anchor_pos + 1 + t (the first of
// them into pos_scratch, k_batch_verify_in); k_batch_accept takes each session's K1 argmaxes as
// targ and runs k_accept's acceptance on its hidden rows; the catch-up rows
// are (hidden row j, catch_tok[j]) for j < k-1 (k_batch_catch_in); then
// each session's round record and advance (k_batch_next).

__global__ __launch_bounds__(256) void k_batch_draft_in(const BatchSess *__restrict__ bs, int j, int d,
                                                        int *__restrict__ toks, float *__restrict__ h) {
    const BatchSess b = bs[blockIdx.x];
    if (threadIdx.x == 0) toks[blockIdx.x] = b.ctl->tok[j];
    for (int i = threadIdx.x; i < d; i += 256) h[(size_t)blockIdx.x * d + i] = b.chain[i];
}

__global__ __launch_bounds__(256) void k_batch_draft_out(const BatchSess *__restrict__ bs, int j, int d,
                                                         const int *__restrict__ am, const float *__restrict__ h) {
    const BatchSess b = bs[blockIdx.x];
    if (threadIdx.x == 0) b.ctl->tok[j + 1] = am[blockIdx.x];
    for (int i = threadIdx.x; i < d; i += 256) b.chain[i] = h[(size_t)blockIdx.x * d + i];
}

__global__ __launch_bounds__(64) void k_batch_verify_in(const BatchSess *__restrict__ bs, int K1,
                                                        int *__restrict__ toks) {
    const BatchSess b = bs[blockIdx.x];
    if ((int)threadIdx.x < K1) toks[blockIdx.x * K1 + threadIdx.x] = b.ctl->tok[threadIdx.x];
    if (threadIdx.x == 0) b.ctl->pos_scratch = b.ctl->anchor_pos + 1;      // the anchor's row follows anchor_pos
}

__global__ __launch_bounds__(256) void k_batch_accept(const BatchSess *__restrict__ bs, int K1, const int *__restrict__ am,
                                                      const float *__restrict__ vh, int d) {
    const BatchSess b = bs[blockIdx.x];
    if ((int)threadIdx.x < K1) b.ctl->targ[threadIdx.x] = am[blockIdx.x * K1 + threadIdx.x];
    __syncthreads();
    accept_body(b.ctl, vh + (size_t)blockIdx.x * K1 * d, d, b.chain, b.depth, 0);
}

__global__ __launch_bounds__(256) void k_batch_catch_in(const BatchSess *__restrict__ bs, int K1, int nc, int d,
                                                        const float *__restrict__ vh, int *__restrict__ toks,
                                                        float *__restrict__ h) {
    const BatchSess b = bs[blockIdx.x];
    if ((int)threadIdx.x < nc) toks[blockIdx.x * nc + threadIdx.x] = b.ctl->catch_tok[threadIdx.x];
    for (int f = threadIdx.x; f < nc * d; f += 256) {
        const int j = f / d, i = f - j * d;
        h[((size_t)blockIdx.x * nc + j) * d + i] = vh[((size_t)blockIdx.x * K1 + j) * d + i];
    }
}

__global__ void k_batch_next(const BatchSess *__restrict__ bs) {
    if (threadIdx.x != 0) return;
    const BatchSess b = bs[blockIdx.x];
    next_round(b.ctl, b.hist, b.hist_cap);
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_misc(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

extern "C" int l98k_upload_exp_table(const float *tab) {
    int e;
    if ((e = l98k_upload_exp_table_misc(tab)) != 0) return e;
    if ((e = l98k_upload_exp_table_gemv(tab)) != 0) return e;
    if ((e = l98k_upload_exp_table_moe(tab)) != 0) return e;
    if ((e = l98k_upload_exp_table_kda(tab)) != 0) return e;
    if ((e = l98k_upload_exp_table_smp(tab)) != 0) return e;
    if ((e = l98k_upload_exp_table_mfma(tab)) != 0) return e;
    return l98k_upload_exp_table_attn(tab);
}

extern "C" int l98k_embed(const int8_t *q, const float *s, const int *toks, int d, int gs, int nt,
                          float *x, hipStream_t st) {
    if (gs <= 0) gs = d;
    if (gs & 31 || d % gs) return -1;
    hipLaunchKernelGGL(k_embed, dim3((d + 255) / 256, nt), dim3(256), 0, st, q, s, toks, d, gs, x);
    return (int)hipGetLastError();
}

#define NORM_CASES(X) X(1) X(2) X(4) X(8)

extern "C" int l98k_rmsnorm_ex(float *x, int x_stride, const float *a, const float *b, const float *w,
                               int n, float eps, int rows, float *out, int out_stride, int8_t *xq,
                               float *xqs, int tok, hipStream_t st) {
    if (n < 32 || n > 256 * 8 || (n & 31) || (x_stride & 3) || (out && (out_stride & 3)) || rows < 1 ||
        (xq && !xqs))
        return -1;
    if (!tok && n > 512) {
        // rows of 513..2048 elements: a 256-thread block per row
        if (n <= 1024 && w)
            hipLaunchKernelGGL((k_rmsnorm_b<4, true>), dim3(rows), dim3(256), 0, st, x, x_stride, a, b, w, n, eps, out,
                               out_stride, xq, xqs);
        else if (n <= 1024)
            hipLaunchKernelGGL((k_rmsnorm_b<4, false>), dim3(rows), dim3(256), 0, st, x, x_stride, a, b, w, n, eps, out,
                               out_stride, xq, xqs);
        else if (w)
            hipLaunchKernelGGL((k_rmsnorm_b<8, true>), dim3(rows), dim3(256), 0, st, x, x_stride, a, b, w, n, eps, out,
                               out_stride, xq, xqs);
        else
            hipLaunchKernelGGL((k_rmsnorm_b<8, false>), dim3(rows), dim3(256), 0, st, x, x_stride, a, b, w, n, eps, out,
                               out_stride, xq, xqs);
        return (int)hipGetLastError();
    }
#define NORM_LAUNCH(PJ)                                                                                   \
    if (n <= 256 * PJ) {                                                                                  \
        if (w && !tok)                                                                                    \
            hipLaunchKernelGGL((k_rmsnorm<PJ, true, false>), dim3(rows), dim3(64), 0, st, x, x_stride, a, b, w, \
                               n, eps, out, out_stride, xq, xqs);                                         \
        else if (w)                                                                                       \
            hipLaunchKernelGGL((k_rmsnorm<PJ, true, true>), dim3(rows), dim3(64), 0, st, x, x_stride, a, b, w, \
                               n, eps, out, out_stride, xq, xqs);                                         \
        else if (!tok)                                                                                    \
            hipLaunchKernelGGL((k_rmsnorm<PJ, false, false>), dim3(rows), dim3(64), 0, st, x, x_stride, a, b, \
                               w, n, eps, out, out_stride, xq, xqs);                                      \
        else                                                                                              \
            hipLaunchKernelGGL((k_rmsnorm<PJ, false, true>), dim3(rows), dim3(64), 0, st, x, x_stride, a, b, \
                               w, n, eps, out, out_stride, xq, xqs);                                      \
        return (int)hipGetLastError();                                                                    \
    }
    NORM_CASES(NORM_LAUNCH)
#undef NORM_LAUNCH
    return -1;
}

extern "C" int l98k_rmsnorm(float *x, int x_stride, const float *a, const float *b, const float *w,
                            int n, float eps, int rows, float *out, int out_stride, int8_t *xq,
                            float *xqs, hipStream_t st) {
    if (!w) return -1;
    return l98k_rmsnorm_ex(x, x_stride, a, b, w, n, eps, rows, out, out_stride, xq, xqs, 0, st);
}

extern "C" int l98k_mtp_pre(const int8_t *emb_q, const float *emb_s, int gs, const int *toks, const float *h,
                            int d, const float *w_e, const float *w_h, float eps, int rows, int8_t *xq, float *xqs,
                            hipStream_t st) {
    if (gs <= 0) gs = d;
    if (d < 32 || d > 256 * 8 || (d & 31) || rows < 1 || (gs & 31) || d % gs) return -1;
#define PRE_LAUNCH(PJ)                                                                                  \
    if (d <= 256 * PJ) {                                                                                \
        hipLaunchKernelGGL(k_mtp_pre<PJ>, dim3(rows, 2), dim3(64), 0, st, emb_q, emb_s, toks, h, d, gs, w_e, \
                           w_h, eps, xq, xqs);                                                          \
        return (int)hipGetLastError();                                                                  \
    }
    NORM_CASES(PRE_LAUNCH)
#undef PRE_LAUNCH
    return -1;
}

extern "C" int l98k_dspark_pre(const int8_t *emb_q, const float *emb_s, int gs, const int *tok, const float *chain,
                               const float *mask, const float *depth, int d, const float *w_e, const float *w_h,
                               float eps, int rows, int8_t *xq, float *xqs, hipStream_t st) {
    if (gs <= 0) gs = d;
    if (d < 32 || d > 256 * 8 || (d & 31) || rows < 1 || (gs & 31) || d % gs) return -1;
#define DSPARK_LAUNCH(PJ)                                                                                 \
    if (d <= 256 * PJ) {                                                                                  \
        hipLaunchKernelGGL(k_dspark_pre<PJ>, dim3(rows, 3), dim3(64), 0, st, emb_q, emb_s, tok, chain, mask, \
                           depth, d, gs, w_e, w_h, eps, xq, xqs);                                         \
        return (int)hipGetLastError();                                                                    \
    }
    NORM_CASES(DSPARK_LAUNCH)
#undef DSPARK_LAUNCH
    return -1;
}

extern "C" int l98k_argmax(const float *x, int n, int rows, int mode, int *out, hipStream_t st) {
    if (rows < 1 || rows > 65535 || n < 1) return -1;
    hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(ARGMAX_THREADS), 0, st, x, n, mode, out);
    return (int)hipGetLastError();
}

extern "C" int l98k_argmax_part(const unsigned long long *part, int tiles, const float *x, int n, int rows, int mode,
                                int *out, hipStream_t st) {
    if (rows < 1 || rows > LZ_ARGMAX_ROWS || tiles < 1 || n < 1) return -1;
    hipLaunchKernelGGL(k_argmax_part, dim3(rows), dim3(256), 0, st, part, tiles, x, n, mode, out);
    return (int)hipGetLastError();
}

extern "C" int l98k_accept(DevCtl *ctl, const float *vhidden, int d, float *chain, int depth,
                           int flags, hipStream_t st) {
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(256), 0, st, ctl, vhidden, d, chain, depth, flags);
    return (int)hipGetLastError();
}

extern "C" int l98k_set_tokens(DevCtl *ctl, int op, RoundRec *hist, int hist_cap, hipStream_t st) {
    hipLaunchKernelGGL(k_set_tokens, dim3(1), dim3(64), 0, st, ctl, op, hist, hist_cap);
    return (int)hipGetLastError();
}


// Launch-floor probes (l98_time_kernel modes 7-10): an empty kernel, and a
// handoff kernel whose every block reads the n floats the previous launch
// wrote (as a GEMV's blocks read the activation rows their producer wrote
// on other XCDs) while block 0 writes the next buffer.
__global__ void k_nop() {}

// n <= 8192: every load of a thread is issued before the first use
// (addresses clamped, no branches).
__global__ __launch_bounds__(256) void k_handoff(const float *__restrict__ in, float *__restrict__ out, int n) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++)
        v[u] = *reinterpret_cast<const float4 *>(in + imin((u * 256 + (int)threadIdx.x) * 4, n - 4));
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; u++) acc += v[u].x + v[u].y + v[u].z + v[u].w;
    if (blockIdx.x == 0)
        for (int i = (int)threadIdx.x; i < n; i += 256) out[i] = in[i] + (acc == 12345.0f ? 1.0f : 0.0f);
}

// The handoff kernel plus a last-block reduction: blocks come in groups of
// 8; each writes 256 floats of partials, then a device-scope release and a
// counter increment; the group's last block (acquire) reads its group's
// 2048 partials and writes one value per thread.
__global__ __launch_bounds__(256) void k_lastblock(const float *__restrict__ in, float *__restrict__ out, int n,
                                                   float *__restrict__ part, unsigned int *__restrict__ cnt) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++)
        v[u] = *reinterpret_cast<const float4 *>(in + imin((u * 256 + (int)threadIdx.x) * 4, n - 4));
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; u++) acc += v[u].x + v[u].y + v[u].z + v[u].w;
    part[blockIdx.x * 256 + threadIdx.x] = acc;
    __shared__ unsigned int s_old;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_old = atomicAdd(&cnt[blockIdx.x >> 3], 1u);
    __syncthreads();
    if ((s_old & 7u) != 7u) return;
    __threadfence();
    const int g0 = (int)(blockIdx.x & ~7u) * 256;
    float r = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) r += part[g0 + b * 256 + threadIdx.x];
    if ((int)threadIdx.x < n) out[(blockIdx.x >> 3) * 256 + threadIdx.x] = in[threadIdx.x] + (r == 12345.0f ? 1.0f : 0.0f);
}

extern "C" int l98k_launch_chain(int kind, int launches, int grid, float *a, float *b, int n, hipStream_t st) {
    if (launches < 1 || grid < 1 || grid > 65536 || (kind >= 1 && (!a || !b || n < 256 || n > 8192 || (n & 3))) ||
        (kind == 2 && (grid & 7)))
        return -1;
    for (int i = 0; i < launches; i++) {
        float *src = (i & 1) ? b : a, *dst = (i & 1) ? a : b;
        if (kind == 0) hipLaunchKernelGGL(k_nop, dim3(grid), dim3(256), 0, st);
        else if (kind == 1) hipLaunchKernelGGL(k_handoff, dim3(grid), dim3(256), 0, st, src, dst, n);
        else
            // partials and counters past the two n-float buffers (the caller
            // sizes the buffer for them)
            hipLaunchKernelGGL(k_lastblock, dim3(grid), dim3(256), 0, st, src, dst, n, b + n,
                               reinterpret_cast<unsigned int *>(b + n + (size_t)grid * 256));
    }
    return (int)hipGetLastError();
}

typedef int v4i_s __attribute__((ext_vector_type(4)));

// Per-CU streaming probe: each block streams `chunks` 16-byte chunks of its
// own region of w with non-temporal loads, J per thread in flight per
// pass, and writes one word (so the loads are live).
template <int J>
__global__ void k_stream(const int4 *__restrict__ w, int chunks, int *__restrict__ out) {
    const int4 *base = w + (size_t)blockIdx.x * chunks;
    int acc = 0;
    for (int c0 = 0; c0 < chunks; c0 += J * (int)blockDim.x) {
        v4i_s q[J];
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int c = imin(c0 + j * (int)blockDim.x + (int)threadIdx.x, chunks - 1);
            q[j] = __builtin_nontemporal_load(reinterpret_cast<const v4i_s *>(base) + c);
        }
#pragma unroll
        for (int j = 0; j < J; j++) acc ^= q[j].x ^ q[j].y ^ q[j].z ^ q[j].w;
    }
    if (acc == 0x12345678) out[blockIdx.x] = acc;
}

extern "C" int l98k_stream(const void *w, int blocks, int threads, int chunks, int *out, hipStream_t st) {
    if (blocks < 1 || (threads != 256 && threads != 512 && threads != 1024) || chunks < 1) return -1;
    hipLaunchKernelGGL(k_stream<16>, dim3(blocks), dim3(threads), 0, st, reinterpret_cast<const int4 *>(w), chunks,
                       out);
    return (int)hipGetLastError();
}

// Control block i of a staging array copied to its session's (block i), so
// a session batch's blocks go up as one host transfer.
__global__ __launch_bounds__(128) void k_put_ctl(const DevCtl *__restrict__ src, DevCtl *const *__restrict__ dst) {
    const int *s = reinterpret_cast<const int *>(src + blockIdx.x);
    int *d = reinterpret_cast<int *>(dst[blockIdx.x]);
    for (int j = threadIdx.x; j < (int)(sizeof(DevCtl) / sizeof(int)); j += 128) d[j] = s[j];
}

extern "C" int l98k_put_ctl(const DevCtl *src, DevCtl *const *dst, int n, hipStream_t st) {
    if (n < 1) return -1;
    hipLaunchKernelGGL(k_put_ctl, dim3(n), dim3(128), 0, st, src, dst);
    return (int)hipGetLastError();
}

// Item i's `per` floats (per % 4 == 0) from src + i * per to dst[i]: a
// session batch's logits and hidden rows into each session's own buffers in
// one launch (grid: (slices, n)).
__global__ __launch_bounds__(256) void k_scatter_rows(const float4 *__restrict__ src, size_t per4,
                                                      float *const *__restrict__ dst) {
    const float4 *s = src + (size_t)blockIdx.y * per4;
    float4 *d = reinterpret_cast<float4 *>(dst[blockIdx.y]);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < per4; i += (size_t)gridDim.x * 256) d[i] = s[i];
}

extern "C" int l98k_scatter_rows(const float *src, size_t per, float *const *dst, int n, hipStream_t st) {
    if (n < 1 || n > 65535 || (per & 3) || per == 0) return -1;
    const size_t per4 = per >> 2;
    size_t slices = (per4 + 4 * 256 - 1) / (4 * 256);
    if (slices > 256) slices = 256;
    hipLaunchKernelGGL(k_scatter_rows, dim3((unsigned)slices, n), dim3(256), 0, st,
                       reinterpret_cast<const float4 *>(src), per4, dst);
    return (int)hipGetLastError();
}

extern "C" int l98k_batch_round(int op, const BatchSess *bs, int n, int j, int K1, int nc, int d, const int *am,
                                const float *rows, int *toks, float *h, hipStream_t st) {
    if (n < 1 || K1 < 1 || K1 > 16 || nc < 0 || nc > 8) return -1;
    switch (op) {
    case 0: hipLaunchKernelGGL(k_batch_draft_in, dim3(n), dim3(256), 0, st, bs, j, d, toks, h); break;
    case 1: hipLaunchKernelGGL(k_batch_draft_out, dim3(n), dim3(256), 0, st, bs, j, d, am, rows); break;
    case 2: hipLaunchKernelGGL(k_batch_verify_in, dim3(n), dim3(64), 0, st, bs, K1, toks); break;
    case 3: hipLaunchKernelGGL(k_batch_accept, dim3(n), dim3(256), 0, st, bs, K1, am, rows, d); break;
    case 4: hipLaunchKernelGGL(k_batch_catch_in, dim3(n), dim3(256), 0, st, bs, K1, nc, d, rows, toks, h); break;
    case 5: hipLaunchKernelGGL(k_batch_next, dim3(n), dim3(64), 0, st, bs); break;
    default: return -1;
    }
    return (int)hipGetLastError();
}

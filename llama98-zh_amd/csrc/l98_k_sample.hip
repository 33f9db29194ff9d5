// Temperature sampling on the device, bit-identical to the reference's
// float sampler: softmax over the vocabulary (src/ops_norm.c:903-990 float
// tier), the draft distribution q = softmax(logits/T) with its multinomial
// draw (lz_sample_temp_q + sample_mult, src/sampler.c:159-167, 736-747),
// the top-p target distribution (lz_target_dist / select_candidates,
// src/sampler.c:563-730), the speculative acceptance with residual
// resampling (lz_spec_accept_temp, src/generate.c:261-346), the draw from a
// distribution (sample_from_dist, src/generate.c:1151-1160), and
// lz_sample_ex with top-p (src/sampler.c:794-840).
//
// Every sum the reference accumulates serially over the vocabulary - the
// softmax denominator, the cdf scans of the draws, the kept top-p mass, the
// residual mass - is the exact serial float result, computed by one block
// with the binade-run method of wave_sum_nonneg (l98_devmath.h) extended to
// prefix queries: after one walk over the special elements, every element's
// exact prefix is s_after(its run's special) + (grid steps since) * ulp, so
// "the first index whose prefix passes the coin" is a parallel minimum.
// The top-p candidates are ordered by a stable descending LSD radix sort of
// this file's own (three passes of 10-bit digits: a candidate key, the bits
// of a probability in [0, 1], is below 2^30).
//
// The kernels a device-resident temperature round runs take `skip`, a
// device flag (the round's "decided" word): when it is set the launch does
// nothing, so the acceptance rows after the first rejection consume no
// random numbers, as the reference's loop stops there.
#include <cstring>

#include "l98_devmath.h"

__device__ __forceinline__ uint32_t umin_u32(uint32_t a, uint32_t b) { return a < b ? a : b; }

#define SMP_THREADS 1024
#define SMP_WAVES (SMP_THREADS / 64)
#define SMP_RMAX 1024                    // special elements the walk's table holds

struct __align__(16) XRec {
    float p;
    uint32_t info;                       // binade guess | (index + 1) << 8
    uint32_t a, b;                       // before the sort: thread, local q prefix; after: q prefix lo, hi
};

struct SmpLds {
    float incl[SMP_THREADS];
    uint32_t cnt_ex[SMP_THREADS];
    unsigned long long q_ex[SMP_THREADS];
    XRec rec[SMP_RMAX + 2];
    float sA[SMP_RMAX + 2], sE[SMP_RMAX + 2];
    float wf[SMP_WAVES];
    uint32_t wu[SMP_WAVES];
    unsigned long long wq[SMP_WAVES];
    int K, fail, result, iv;
    float fres, fv;
    unsigned long long qtot;
};

// ------------------------------------------------------ block helpers ---

__device__ __forceinline__ float blk_incl_f32(float x, SmpLds &L) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float v = wave_scan_f32(x);
    if (lane == 63) L.wf[w] = v;
    __syncthreads();
    if (w == 0) {
        float t = lane < SMP_WAVES ? L.wf[lane] : 0.0f;
        t = wave_scan_f32(t);
        if (lane < SMP_WAVES) L.wf[lane] = t;
    }
    __syncthreads();
    const float r = (w ? L.wf[w - 1] : 0.0f) + v;
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t blk_excl_u32(uint32_t x, SmpLds &L) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t v = wave_scan_u32(x);
    if (lane == 63) L.wu[w] = v;
    __syncthreads();
    if (w == 0) {
        uint32_t t = lane < SMP_WAVES ? L.wu[lane] : 0u;
        t = wave_scan_u32(t);
        if (lane < SMP_WAVES) L.wu[lane] = t;
    }
    __syncthreads();
    const uint32_t r = (w ? L.wu[w - 1] : 0u) + v - x;
    __syncthreads();
    return r;
}

__device__ __forceinline__ unsigned long long blk_excl_u64(unsigned long long x, SmpLds &L, unsigned long long *total) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    unsigned long long v = x;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(v, o);
        if (lane >= o) v += y;
    }
    if (lane == 63) L.wq[w] = v;
    __syncthreads();
    if (tid == 0) {
        unsigned long long a = 0;
        for (int i = 0; i < SMP_WAVES; i++) { a += L.wq[i]; L.wq[i] = a; }
    }
    __syncthreads();
    const unsigned long long r = (w ? L.wq[w - 1] : 0ull) + v - x;
    *total = L.wq[SMP_WAVES - 1];
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t blk_max_u32(uint32_t v, SmpLds &L) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { const uint32_t y = __shfl_xor(v, o); v = y > v ? y : v; }
    if (lane == 0) L.wu[w] = v;
    __syncthreads();
    uint32_t m = L.wu[0];
    for (int i = 1; i < SMP_WAVES; i++) m = L.wu[i] > m ? L.wu[i] : m;
    __syncthreads();
    return m;
}

__device__ __forceinline__ int blk_min_i32(int v, SmpLds &L) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { const int y = __shfl_xor(v, o); v = y < v ? y : v; }
    if (lane == 0) L.wu[w] = (uint32_t)v;
    __syncthreads();
    int m = (int)L.wu[0];
    for (int i = 1; i < SMP_WAVES; i++) m = (int)L.wu[i] < m ? (int)L.wu[i] : m;
    __syncthreads();
    return m;
}

// xorshift64*, then 24 bits to [0, 1) (lz_random_f32, src/sampler.c:112-120)
__device__ __forceinline__ float d_random_f32(unsigned long long *st) {
    unsigned long long s = *st;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *st = s;
    const uint32_t r = (uint32_t)((s * 0x2545F4914F6CDD1DULL) >> 32);
    return (float)(r >> 8) / 16777216.0f;
}

// ----------------------------------------------- exact prefix engine ---

#define XP_TOTAL 0                       // L.fres = the serial sum
#define XP_FIRST_GT 1                    // L.result = first i with c < prefix_i (-1 if none), L.fres = that prefix
#define XP_FIRST_GE 2                    // L.result = first i with prefix_i >= c (-1 if none), L.fres = that prefix
                                         // (the total when there is none)

// An element is also special when the guessed sums around it come within
// 2^-10 of a binade edge: the serial loop's rounding drift (a row of
// probabilities that sums to about 1 ends a few ulps of 1 away from any
// accurate sum) can put its real sum on the other side of the edge, and a
// run the walk adds as one must not cross one.
__device__ __forceinline__ bool xp_near(float A, float An) {
    return f_binade(A * (1.0f - 0x1p-10f)) != f_binade(An * (1.0f + 0x1p-10f));
}

// The serial loop s = 0; s += x[i] over x[0..n) (non-negative values,
// get(i) returns x[i], and 0 for i >= n), answered for `mode` by the whole
// block.  Thread t owns elements [t*CH, (t+1)*CH).  Contains barriers.
// Each pass reads the thread's elements XP_BATCH at a time, every load of a
// batch issued before the first use.
#define XP_BATCH 8
// vec: the row is 16-byte aligned and CH a multiple of 4, so a batch is
// four 16-byte loads per thread (XP_BATCH * 2 elements)
template <class G, class F>
__device__ __forceinline__ void xp_walk(const G &get, int i0, int CH, bool vec, const bool &stop, F f) {
    if (vec) {
        constexpr int B = 2 * XP_BATCH;
        for (int k0 = 0; k0 < CH && !stop; k0 += B) {
            float4 v[B / 4];
#pragma unroll
            for (int u = 0; u < B / 4; u++) v[u] = get.clamped4(i0 + k0 + 4 * u);  // past the chunk: ignored
#pragma unroll
            for (int u = 0; u < B; u++) {
                const float x = (u & 3) == 0 ? v[u >> 2].x : (u & 3) == 1 ? v[u >> 2].y : (u & 3) == 2 ? v[u >> 2].z
                                                                                                    : v[u >> 2].w;
                if (k0 + u < CH && !stop) f(k0 + u, x);
            }
        }
        return;
    }
    for (int k0 = 0; k0 < CH && !stop; k0 += XP_BATCH) {
        float v[XP_BATCH];
#pragma unroll
        for (int u = 0; u < XP_BATCH; u++) v[u] = get.clamped(i0 + k0 + u);     // past the chunk: ignored
#pragma unroll
        for (int u = 0; u < XP_BATCH; u++)
            if (k0 + u < CH && !stop) f(k0 + u, v[u]);
    }
}

template <class G>
__device__ __forceinline__ void xprefix(const G &get, int n, int mode, float c, SmpLds &L) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (n < 1) {                          // an empty row: no index passes, the sum is 0
        if (tid == 0) { L.result = -1; L.fres = 0.0f; }
        __syncthreads();
        return;
    }
    // a multiple of 4 (threads past the row hold zeros, which leave every
    // prefix as it is)
    const int CH = (((n + SMP_THREADS - 1) / SMP_THREADS) + 3) & ~3;
    const int i0 = tid * CH;
    const bool never = false, vec = get.aligned();
    // approximate prefix (the binade guesses)
    float T = 0.0f;
    xp_walk(get, i0, CH, vec, never, [&](int, float x) { T += x; });
    const float incl = blk_incl_f32(T, L);
    L.incl[tid] = incl;
    if (tid == 0) { L.K = 0; L.fail = 0; }
    __syncthreads();
    const float off = tid ? L.incl[tid - 1] : 0.0f;
    if (!(T <= 3.0e38f) || f_binade(incl) >= 254) L.fail = 1;
    // classify; each special element takes a table slot (sorted below)
    uint32_t cnt = 0, qs = 0;
    {
        float A = off;
        int E0 = f_binade(off);
        xp_walk(get, i0, CH, vec, never, [&](int k, float x) {
            const int i = i0 + k;
            const float An = (k == CH - 1) ? incl : A + x;
            const int E1 = f_binade(An);
            uint32_t q;
            const uint32_t plain = ps_classify(x, E0, xp_near(A, An) ? -1 : E1, &q);
            if (!plain) {
                const int slot = atomicAdd(&L.K, 1);
                if (slot < SMP_RMAX) {
                    XRec r;
                    r.p = x;
                    r.info = (uint32_t)E1 | ((uint32_t)(i + 1) << 8);
                    r.a = (uint32_t)tid;
                    r.b = qs;
                    L.rec[1 + slot] = r;
                }
                cnt++;
            }
            qs += q;
            A = An;
            E0 = E1;
        });
    }
    L.cnt_ex[tid] = blk_excl_u32(cnt, L);
    unsigned long long qtot;
    L.q_ex[tid] = blk_excl_u64(qs, L, &qtot);
    __syncthreads();
    const int K = L.K;
    if (K > SMP_RMAX) {
        if (tid == 0) L.fail = 1;
    } else {
        // bitonic sort of the table by element index
        int P = 1;
        while (P < K) P <<= 1;
        if (tid >= K && tid < P) { XRec r; r.p = 0.0f; r.info = 0xFFFFFF00u; r.a = 0; r.b = 0; L.rec[1 + tid] = r; }
        __syncthreads();
        for (int k2 = 2; k2 <= P; k2 <<= 1) {
            for (int j = k2 >> 1; j > 0; j >>= 1) {
                const int ixj = tid ^ j;
                if (tid < P && ixj > tid) {
                    const XRec ra = L.rec[1 + tid], rb = L.rec[1 + ixj];
                    const bool up = (tid & k2) == 0;
                    if (((ra.info >> 8) > (rb.info >> 8)) == up) { L.rec[1 + tid] = rb; L.rec[1 + ixj] = ra; }
                }
                __syncthreads();
            }
        }
        // global q prefix of each special element; the virtual start and the sentinel
        if (tid < K) {
            XRec r = L.rec[1 + tid];
            const unsigned long long ps = L.q_ex[r.a] + r.b;
            r.a = (uint32_t)ps;
            r.b = (uint32_t)(ps >> 32);
            L.rec[1 + tid] = r;
        }
        if (tid == 0) { XRec r; r.p = 0.0f; r.info = 0u; r.a = 0; r.b = 0; L.rec[0] = r; }
        if (tid == 1) {
            XRec r; r.p = 0.0f; r.info = (uint32_t)(n + 1) << 8; r.a = (uint32_t)qtot; r.b = (uint32_t)(qtot >> 32);
            L.rec[K + 1] = r;
        }
        __syncthreads();
        // walk, systolic over 64 records at a time (wave 0): sA = the sum
        // after record j's element, sE = after its run
        if (w == 0) {
            float carry = 0.0f;
            bool bad = false;
            for (int b0 = 0; b0 <= K; b0 += 64) {
                const int j = b0 + lane, jj = j <= K ? j : K;
                const XRec me = L.rec[jj], nx = L.rec[jj + 1];
                const int E = (int)(me.info & 255u), ia = (int)(me.info >> 8), ib = (int)(nx.info >> 8) - 1;
                const int eb = E > 1 ? E : 1;
                const unsigned long long psm = ((unsigned long long)me.b << 32) | me.a;
                const unsigned long long psn = ((unsigned long long)nx.b << 32) | nx.a;
                const unsigned long long Q = psn - psm;
                const float top = __builtin_amdgcn_ldexpf(1.0f, eb - 126);
                const float Qu0 = (float)(Q < 16777216ull ? Q : 16777216ull) * __builtin_amdgcn_ldexpf(1.0f, eb - 150);
                const bool empty = ib <= ia || j > K;
                const float P0 = j > K ? 0.0f : me.p;
                const float lo0 = E ? __builtin_amdgcn_ldexpf(1.0f, E - 127) : 0.0f, hi0 = top - Qu0;
                const bool feasible = Q <= 16777216ull && hi0 >= lo0;
                const float lo = empty ? 0.0f : feasible ? lo0 : -1.0f;
                const float hi = empty ? __builtin_inff() : feasible ? hi0 : -1.0f;
                const float Qu = empty ? 0.0f : Qu0;
                const int steps = (K + 1 - b0) < 64 ? (K + 1 - b0) : 64;
                float s1 = 0.0f, sout = 0.0f;
                for (int st = 0; st < steps; st++) {
                    float sin = wave_shr1_f32(sout);
                    sin = lane == 0 ? carry : sin;
                    s1 = sin + P0;
                    sout = s1 + Qu;
                }
                const bool ok = lane >= steps || __builtin_amdgcn_fmed3f(s1, lo, hi) == s1;
                if (__ballot(!ok) != 0) bad = true;
                if (lane < steps) { L.sA[j] = s1; L.sE[j] = sout; }
                carry = f_rl(sout, steps - 1);
            }
            if (lane == 0 && bad) L.fail = 1;
        }
    }
    __syncthreads();
    if (L.fail) {
        // the serial loop itself (inputs the walk cannot take)
        if (tid == 0) {
            float s = 0.0f;
            int res = -1;
            for (int i = 0; i < n; i++) {
                s += get(i);
                if (mode == XP_FIRST_GT && c < s) { res = i; break; }
                if (mode == XP_FIRST_GE && s >= c) { res = i; break; }
            }
            L.result = res;
            L.fres = s;
        }
        __syncthreads();
        return;
    }
    if (mode == XP_TOTAL) {
        if (tid == 0) { L.fres = L.sE[K]; L.result = -1; }
        __syncthreads();
        return;
    }
    // every element's exact prefix; the first one past c
    int best = 0x7FFFFFFF;
    float bestv = 0.0f;
    {
        float A = off;
        int E0 = f_binade(off);
        uint32_t rk = L.cnt_ex[tid];
        unsigned long long qp = L.q_ex[tid];
        bool found = false;
        xp_walk(get, i0, CH, vec, found, [&](int k, float x) {
            const int i = i0 + k;
            const float An = (k == CH - 1) ? incl : A + x;
            const int E1 = f_binade(An);
            uint32_t q;
            const uint32_t plain = ps_classify(x, E0, xp_near(A, An) ? -1 : E1, &q);
            float pref;
            if (!plain) {
                rk++;
                pref = L.sA[rk];
            } else {
                qp += q;
                const XRec r = L.rec[rk];
                const int E = (int)(r.info & 255u), eb = E > 1 ? E : 1;
                const unsigned long long run = qp - (((unsigned long long)r.b << 32) | r.a);
                pref = L.sA[rk] + (float)run * __builtin_amdgcn_ldexpf(1.0f, eb - 150);
            }
            const bool hit = i < n && (mode == XP_FIRST_GT ? c < pref : pref >= c);
            if (hit) { best = i; bestv = pref; found = true; }
            A = An;
            E0 = E1;
        });
    }
    const int first = blk_min_i32(best, L);
    if (best == first && first != 0x7FFFFFFF) L.fres = bestv;
    if (tid == 0) {
        L.result = first == 0x7FFFFFFF ? -1 : first;
        if (first == 0x7FFFFFFF) L.fres = L.sE[K];
    }
    __syncthreads();
}

// Row accessors: operator() reads element i (0 past n); clamped(i) reads
// it with the index clamped into the row and selects 0 past n, a load with
// no branch, so a thread's loads can all be in flight together.
// clamped4(i), i a multiple of 4: elements i .. i+3 (0 past n), one 16-byte
// load inside the row; aligned(): the row's base allows those loads.
struct GetArr {
    const float *x;
    int n;
    __device__ float operator()(int i) const { return i < n ? x[i] : 0.0f; }
    __device__ float clamped(int i) const {
        const float v = x[imin(i, n - 1)];
        return i < n ? v : 0.0f;
    }
    __device__ float4 clamped4(int i) const {
        if (i + 3 < n) return *reinterpret_cast<const float4 *>(x + i);
        return make_float4(clamped(i), clamped(i + 1), clamped(i + 2), clamped(i + 3));
    }
    __device__ bool aligned() const { return ((uintptr_t)x & 15) == 0; }
};
struct GetResid {                        // max(p - q, 0) (sample_residual's dd > 0 terms)
    const float *p, *q;
    int n;
    __device__ float operator()(int i) const {
        if (i >= n) return 0.0f;
        const float dd = p[i] - q[i];
        return dd > 0.0f ? dd : 0.0f;
    }
    __device__ float clamped(int i) const {
        const int ic = imin(i, n - 1);
        const float dd = p[ic] - q[ic];
        return i < n && dd > 0.0f ? dd : 0.0f;
    }
    __device__ float4 clamped4(int i) const {
        if (i + 3 < n) {
            const float4 a = *reinterpret_cast<const float4 *>(p + i), b = *reinterpret_cast<const float4 *>(q + i);
            const float dx = a.x - b.x, dy = a.y - b.y, dz = a.z - b.z, dw = a.w - b.w;
            return make_float4(dx > 0.0f ? dx : 0.0f, dy > 0.0f ? dy : 0.0f, dz > 0.0f ? dz : 0.0f,
                               dw > 0.0f ? dw : 0.0f);
        }
        return make_float4(clamped(i), clamped(i + 1), clamped(i + 2), clamped(i + 3));
    }
    __device__ bool aligned() const { return (((uintptr_t)p | (uintptr_t)q) & 15) == 0; }
};
struct GetKeys {                         // probabilities from sorted order-preserving keys
    const uint32_t *k;
    int n;
    __device__ float operator()(int i) const { return i < n ? __uint_as_float(k[i]) : 0.0f; }
    __device__ float clamped(int i) const {
        const float v = __uint_as_float(k[imin(i, n - 1)]);
        return i < n ? v : 0.0f;
    }
    __device__ float4 clamped4(int i) const {
        if (i + 3 < n) {
            const uint4 u = *reinterpret_cast<const uint4 *>(k + i);
            return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
        }
        return make_float4(clamped(i), clamped(i + 1), clamped(i + 2), clamped(i + 3));
    }
    __device__ bool aligned() const { return ((uintptr_t)k & 15) == 0; }
};

// first index of the largest value (order-preserving key, strict >)
__device__ __forceinline__ int blk_argmax(const float *x, int n, SmpLds &L) {
    uint32_t best = 0u;
    int bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += SMP_THREADS) {
        const uint32_t k = d_fkey(x[i]);
        if (k > best || bi == 0x7FFFFFFF) { best = k; bi = i; }
    }
    const uint32_t m = blk_max_u32(best, L);
    return blk_min_i32(best == m ? bi : 0x7FFFFFFF, L);
}

// ----------------------------------------------------------- kernels ---

// probs = softmax(logits * inv_t) (the logits scaled in place first, as
// the reference does); with cutoff > 0 also the top-p candidate keys
// (order-preserving bits for probs >= cutoff, 0 otherwise) and indices for
// the descending sort, and their count.
__global__ __launch_bounds__(SMP_THREADS) void k_smp_softmax(const float *__restrict__ logits, int n, float inv_t,
                                                             float *__restrict__ probs, float cutoff,
                                                             uint32_t *__restrict__ keys,
                                                             int *__restrict__ n_cand, const int *__restrict__ skip) {
    __shared__ SmpLds L;
    __shared__ float tab[32];
    if (skip && *skip) return;
    const int tid = threadIdx.x;
    if (tid < 32) tab[tid] = c_exp_tab[tid];
    uint32_t mk = 0u;
#pragma unroll 8
    for (int i = tid; i < n; i += SMP_THREADS) {
        const float s = logits[i] * inv_t;
        probs[i] = s;
        const uint32_t k = d_fkey(s);
        mk = k > mk ? k : mk;
    }
    const float mx = d_unkey(blk_max_u32(mk, L));
#pragma unroll 8
    for (int i = tid; i < n; i += SMP_THREADS) probs[i] = d_exp(probs[i] - mx, tab);
    __syncthreads();
    xprefix(GetArr{probs, n}, n, XP_TOTAL, 0.0f, L);
    const float sum = L.fres;
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    uint32_t cnt = 0;
#pragma unroll 8
    for (int i = tid; i < n; i += SMP_THREADS) {
        const float p = probs[i] * inv;
        probs[i] = p;
        if (keys) {
            // a probability is at most 1 (e <= sum), so a key is below 2^30
            const bool c = p >= cutoff;
            keys[i] = c ? umin_u32(__float_as_uint(p), 0x3F800000u) : 0u;
            cnt += c ? 1u : 0u;
        }
    }
    if (keys) {
        uint32_t tot = blk_excl_u32(cnt, L) + cnt;
        tot = blk_max_u32(tot, L);
        if (tid == 0) *n_cand = (int)tot;
    }
}

// A draw from a distribution: coin = rng, the first i whose cdf passes it
// (sample_mult / sample_from_dist: n - 1 when none does).  Writes the index
// to *out_tok (and to *ctl_tok when given) and p[index] to *out_p.
__global__ __launch_bounds__(SMP_THREADS) void k_smp_draw(const float *__restrict__ p, int n,
                                                          unsigned long long *__restrict__ rng, int *__restrict__ out_tok,
                                                          float *__restrict__ out_p, int *__restrict__ ctl_tok,
                                                          const int *__restrict__ skip) {
    __shared__ SmpLds L;
    if (skip && *skip) return;
    if (threadIdx.x == 0) L.fv = d_random_f32(rng);
    __syncthreads();
    xprefix(GetArr{p, n}, n, XP_FIRST_GT, L.fv, L);
    if (threadIdx.x == 0) {
        const int idx = L.result >= 0 ? L.result : n - 1;
        *out_tok = idx;
        if (out_p) *out_p = p[idx];
        if (ctl_tok) *ctl_tok = idx;
    }
}

// The top-p target distribution from the softmax and the candidates sorted
// by probability, descending (stable: ties keep index order): the kept
// prefix ends at the first cumulative mass >= top_p (or takes every
// candidate), each kept probability is divided by the kept mass, the rest
// are 0; no candidate: one-hot at the argmax.
__global__ __launch_bounds__(SMP_THREADS) void k_smp_topp_dist(const float *__restrict__ probs, int n,
                                                               const uint32_t *__restrict__ skeys,
                                                               const int *__restrict__ svals,
                                                               const int *__restrict__ n_cand, float topp,
                                                               float *__restrict__ p_out, const int *__restrict__ skip) {
    __shared__ SmpLds L;
    if (skip && *skip) return;
    const int tid = threadIdx.x, nc = *n_cand;
    for (int i = tid; i < n; i += SMP_THREADS) p_out[i] = 0.0f;
    if (nc <= 0) {
        const int a = blk_argmax(probs, n, L);
        __syncthreads();
        if (tid == 0) p_out[a] = 1.0f;
        return;
    }
    xprefix(GetKeys{skeys, nc}, nc, XP_FIRST_GE, topp * 1.0f, L);
    const int last = L.result >= 0 ? L.result : nc - 1;
    const float mass = L.fres;
    __syncthreads();
    for (int j = tid; j <= last; j += SMP_THREADS) p_out[svals[j]] = __uint_as_float(skeys[j]) / mass;
}

// lz_spec_accept_temp on device rows: u (given, or drawn); accept x iff u < min(1,
// p[x]/q[x]); otherwise the residual draw over max(p - q, 0) (argmax of p
// when its mass is 0; the last positive index when no cdf passes the coin).
// out[0] = token, out[1] = accepted.
// In a device-resident round (done != null): the draft token is read from
// x_dev, the emitted token goes to *ctl_out, and a rejection sets
// *ctl_n = row and *done.
__global__ __launch_bounds__(SMP_THREADS) void k_smp_accept(const float *__restrict__ p, const float *__restrict__ q,
                                                            int n, int x_in, const int *__restrict__ x_dev, float u_in,
                                                            int have_u, unsigned long long *__restrict__ rng,
                                                            int *__restrict__ out, int *__restrict__ ctl_out,
                                                            int *__restrict__ ctl_n, int *__restrict__ done, int row) {
    __shared__ SmpLds L;
    if (done && *done) return;
    const int tid = threadIdx.x;
    const int x = x_dev ? *x_dev : x_in;
    auto emit = [&](int tok, int acc) {
        if (out) { out[0] = tok; out[1] = acc; }
        if (ctl_out) *ctl_out = tok;
        if (done && !acc) { *ctl_n = row; *done = 1; }
    };
    if (tid == 0) {
        const float qx = q[x];
        float ratio;
        if (qx <= 0.0f) ratio = 0.0f;
        else { ratio = p[x] / qx; if (ratio > 1.0f) ratio = 1.0f; }
        const float u = have_u ? u_in : d_random_f32(rng);
        L.iv = u < ratio ? 1 : 0;
    }
    __syncthreads();
    if (L.iv) {
        if (tid == 0) emit(x, 1);
        return;
    }
    xprefix(GetResid{p, q, n}, n, XP_TOTAL, 0.0f, L);
    const float total = L.fres;
    if (total <= 0.0f) {
        const int a = blk_argmax(p, n, L);
        if (tid == 0) emit(a, 0);
        return;
    }
    int lp = -1;
#pragma unroll 8
    for (int i = tid; i < n; i += SMP_THREADS) if (p[i] - q[i] > 0.0f) lp = i;
    const int last_pos = (int)blk_max_u32((uint32_t)(lp + 1), L) - 1;
    if (tid == 0) L.fv = d_random_f32(rng) * total;
    __syncthreads();
    xprefix(GetResid{p, q, n}, n, XP_FIRST_GT, L.fv, L);
    if (tid == 0) emit(L.result >= 0 ? L.result : last_pos, 0);
}

// lz_sample_ex with top-p after the candidate sort: r = coin * kept mass,
// the first kept candidate whose cdf passes r (the last kept one when none
// does); no candidate: the argmax.  The coin is drawn before anything else
// reads the generator, as in the reference.
__global__ __launch_bounds__(SMP_THREADS) void k_smp_sample_topp(const float *__restrict__ probs, int n,
                                                                 const uint32_t *__restrict__ skeys,
                                                                 const int *__restrict__ svals,
                                                                 const int *__restrict__ n_cand, float topp,
                                                                 unsigned long long *__restrict__ rng,
                                                                 int *__restrict__ out_tok) {
    __shared__ SmpLds L;
    const int tid = threadIdx.x, nc = *n_cand;
    if (tid == 0) L.fv = d_random_f32(rng);
    __syncthreads();
    const float coin = L.fv;
    if (nc <= 0) {
        const int a = blk_argmax(probs, n, L);
        if (tid == 0) *out_tok = a;
        return;
    }
    xprefix(GetKeys{skeys, nc}, nc, XP_FIRST_GE, topp * 1.0f, L);
    const int last = L.result >= 0 ? L.result : nc - 1;
    const float mass = L.fres;
    __syncthreads();
    xprefix(GetKeys{skeys, last + 1}, last + 1, XP_FIRST_GT, coin * mass, L);
    if (tid == 0) *out_tok = svals[L.result >= 0 ? L.result : last];
}

// Index-order prefix queries on host rows, for the library's check of the
// engine: mode XP_*, c the threshold; out[r] = result index, outv[r] = value.
__global__ __launch_bounds__(SMP_THREADS) void k_smp_xprefix(const float *__restrict__ x, int n, int mode,
                                                             const float *__restrict__ c, int *__restrict__ out,
                                                             float *__restrict__ outv) {
    __shared__ SmpLds L;
    const int r = blockIdx.x;
    xprefix(GetArr{x + (size_t)r * n, n}, n, mode, c ? c[r] : 0.0f, L);
    if (threadIdx.x == 0) { out[r] = L.result; outv[r] = L.fres; }
}

// ------------------------------------------------------ radix sort ---
//
// Stable descending sort of (key, index) pairs, keys below 2^30: three LSD
// passes of 10-bit digits over tiles of RS_TILE elements (one per thread,
// so a tile's elements are in index order across waves and lanes).  A pass
// is (1) k_rs_count: each tile's digit counts -> hist[digit][tile]; (2)
// k_rs_scan: the exclusive prefix of hist in (digit, tile) order, by one
// block; (3) k_rs_scatter: each element to hist[digit][tile] + the count of
// equal digits before it in its tile (lanes of the same digit found with 10
// ballots, then the waves before it).  Digits are taken as 1023 - digit, so
// the order is descending; every pass keeps the order of equal digits, so
// equal keys keep index order.
#define RS_TILE 1024
#define RS_BITS 10
#define RS_DIG (1 << RS_BITS)
#define RS_PASSES 3

__device__ __forceinline__ int rs_digit(uint32_t key, int shift) {
    return (RS_DIG - 1) - (int)((key >> shift) & (RS_DIG - 1));
}

__global__ __launch_bounds__(RS_TILE) void k_rs_count(const uint32_t *__restrict__ keys, int n, int shift,
                                                      int *__restrict__ hist, int ntiles,
                                                      const int *__restrict__ skip) {
    __shared__ int cnt[RS_DIG];
    if (skip && *skip) return;
    const int tid = threadIdx.x, i = blockIdx.x * RS_TILE + tid;
    cnt[tid] = 0;
    __syncthreads();
    if (i < n) atomicAdd(&cnt[rs_digit(keys[i], shift)], 1);
    __syncthreads();
    hist[(size_t)tid * ntiles + blockIdx.x] = cnt[tid];
}

// Exclusive prefix, in place, of the RS_DIG x ntiles counts in (digit,
// tile) order: thread t takes digit t's row of ntiles counts (its loads
// eight 16-byte vectors at a time when ntiles % 4 == 0).
__global__ __launch_bounds__(RS_TILE) void k_rs_scan(int *__restrict__ hist, int ntiles, const int *__restrict__ skip) {
    __shared__ int wsum[RS_TILE / 64];
    if (skip && *skip) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int *row = hist + (size_t)tid * ntiles;
    int sum = 0;
    if ((ntiles & 3) == 0) {
        const int4 *r4 = reinterpret_cast<const int4 *>(row);
        const int n4 = ntiles >> 2;
        for (int i0 = 0; i0 < n4; i0 += 8) {
            int4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = r4[imin(i0 + u, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (i0 + u < n4) sum += v[u].x + v[u].y + v[u].z + v[u].w;
        }
    } else {
        for (int i = 0; i < ntiles; i++) sum += row[i];
    }
    const int incl = (int)wave_scan_u32((uint32_t)sum);
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    if (w == 0) {
        int v = lane < RS_TILE / 64 ? wsum[lane] : 0;
        v = (int)wave_scan_u32((uint32_t)v);
        if (lane < RS_TILE / 64) wsum[lane] = v;
    }
    __syncthreads();
    int run = (w ? wsum[w - 1] : 0) + incl - sum;
    if ((ntiles & 3) == 0) {
        int4 *r4 = reinterpret_cast<int4 *>(row);
        const int n4 = ntiles >> 2;
        for (int i0 = 0; i0 < n4; i0 += 8) {
            int4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = r4[imin(i0 + u, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (i0 + u < n4) {
                    int4 o;
                    o.x = run; run += v[u].x;
                    o.y = run; run += v[u].y;
                    o.z = run; run += v[u].z;
                    o.w = run; run += v[u].w;
                    r4[i0 + u] = o;
                }
            }
        }
    } else {
        for (int i = 0; i < ntiles; i++) {
            const int c = row[i];
            row[i] = run;
            run += c;
        }
    }
}

__global__ __launch_bounds__(RS_TILE) void k_rs_scatter(const uint32_t *__restrict__ keys, const int *__restrict__ vals,
                                                        uint32_t *__restrict__ keys_out, int *__restrict__ vals_out,
                                                        int n, int shift, const int *__restrict__ hist, int ntiles,
                                                        const int *__restrict__ skip) {
    __shared__ unsigned short wcnt[RS_TILE / 64][RS_DIG];   // per wave: elements of each digit
    if (skip && *skip) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, i = blockIdx.x * RS_TILE + tid;
    const bool valid = i < n;
    const uint32_t key = valid ? keys[i] : 0u;
    const int val = valid ? (vals ? vals[i] : i) : 0;
    const int dg = rs_digit(key, shift);
    for (int j = tid; j < (RS_TILE / 64) * RS_DIG; j += RS_TILE) (&wcnt[0][0])[j] = 0;
    // the lanes of this wave holding the same digit
    unsigned long long peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < RS_BITS; b++) {
        const unsigned long long bb = __ballot((dg >> b) & 1);
        peers &= ((dg >> b) & 1) ? bb : ~bb;
    }
    const int rank = __popcll(peers & ((1ull << lane) - 1ull));
    __syncthreads();
    if (valid && rank == 0) wcnt[w][dg] = (unsigned short)__popcll(peers);
    __syncthreads();
    // thread t: digit t's running count over the waves, exclusive
    {
        int run = 0;
#pragma unroll
        for (int ww = 0; ww < RS_TILE / 64; ww++) {
            const int c = wcnt[ww][tid];
            wcnt[ww][tid] = (unsigned short)run;
            run += c;
        }
    }
    __syncthreads();
    if (valid) {
        const int pos = hist[(size_t)dg * ntiles + blockIdx.x] + wcnt[w][dg] + rank;
        keys_out[pos] = key;
        vals_out[pos] = val;
    }
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_smp(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

extern "C" int l98k_smp_softmax(const float *logits, int n, float inv_t, float *probs, float cutoff, uint32_t *keys,
                                int *n_cand, const int *skip, hipStream_t st) {
    if (n < 1) return -1;
    hipLaunchKernelGGL(k_smp_softmax, dim3(1), dim3(SMP_THREADS), 0, st, logits, n, inv_t, probs, cutoff, keys, n_cand,
                       skip);
    return (int)hipGetLastError();
}

extern "C" int l98k_smp_draw(const float *p, int n, unsigned long long *rng, int *out_tok, float *out_p, int *ctl_tok,
                             const int *skip, hipStream_t st) {
    if (n < 1) return -1;
    hipLaunchKernelGGL(k_smp_draw, dim3(1), dim3(SMP_THREADS), 0, st, p, n, rng, out_tok, out_p, ctl_tok, skip);
    return (int)hipGetLastError();
}

extern "C" size_t l98k_smp_sort_tmp_bytes(int n) {
    const size_t ntiles = ((size_t)n + RS_TILE - 1) / RS_TILE;
    return sizeof(int) * RS_DIG * ntiles + 2 * sizeof(int) * (size_t)n;
}

// Stable descending sort of n keys (below 2^30) with their indices 0..n-1:
// keys_out, vals_out.  keys is overwritten (a pass's buffer); tmp holds
// l98k_smp_sort_tmp_bytes(n) bytes.
extern "C" int l98k_smp_sort_desc(uint32_t *keys, uint32_t *keys_out, int *vals_out, int n, void *tmp,
                                  const int *skip, hipStream_t st) {
    if (n < 1 || n > RS_DIG * RS_TILE || !tmp) return -1;
    const int ntiles = (n + RS_TILE - 1) / RS_TILE;
    int *hist = reinterpret_cast<int *>(tmp);
    int *vtmp = hist + (size_t)RS_DIG * ntiles;
    // pass 0: keys -> keys_out (indices implicit) -> vals_out; pass 1:
    // keys_out -> keys, vals_out -> vtmp; pass 2: keys -> keys_out, vtmp ->
    // vals_out
    const uint32_t *kin[RS_PASSES] = {keys, keys_out, keys};
    uint32_t *kout[RS_PASSES] = {keys_out, keys, keys_out};
    const int *vin[RS_PASSES] = {nullptr, vals_out, vtmp};
    int *vout[RS_PASSES] = {vals_out, vtmp, vals_out};
    for (int pass = 0; pass < RS_PASSES; pass++) {
        const int shift = pass * RS_BITS;
        hipLaunchKernelGGL(k_rs_count, dim3(ntiles), dim3(RS_TILE), 0, st, kin[pass], n, shift, hist, ntiles, skip);
        hipLaunchKernelGGL(k_rs_scan, dim3(1), dim3(RS_TILE), 0, st, hist, ntiles, skip);
        hipLaunchKernelGGL(k_rs_scatter, dim3(ntiles), dim3(RS_TILE), 0, st, kin[pass], vin[pass], kout[pass],
                           vout[pass], n, shift, hist, ntiles, skip);
    }
    return (int)hipGetLastError();
}

extern "C" int l98k_smp_topp_dist(const float *probs, int n, const uint32_t *skeys, const int *svals,
                                  const int *n_cand, float topp, float *p_out, const int *skip, hipStream_t st) {
    hipLaunchKernelGGL(k_smp_topp_dist, dim3(1), dim3(SMP_THREADS), 0, st, probs, n, skeys, svals, n_cand, topp,
                       p_out, skip);
    return (int)hipGetLastError();
}

extern "C" int l98k_smp_accept(const float *p, const float *q, int n, int x, const float *u, unsigned long long *rng,
                               int *out, hipStream_t st) {
    if (n < 1 || x < 0 || x >= n) return -1;
    hipLaunchKernelGGL(k_smp_accept, dim3(1), dim3(SMP_THREADS), 0, st, p, q, n, x, nullptr, u ? *u : 0.0f, u ? 1 : 0,
                       rng, out, nullptr, nullptr, nullptr, 0);
    return (int)hipGetLastError();
}

extern "C" int l98k_smp_accept_row(const float *p, const float *q, int n, const int *x_dev, unsigned long long *rng,
                                   int *ctl_out, int *ctl_n, int *done, int row, hipStream_t st) {
    if (n < 1 || !x_dev || !ctl_out || !ctl_n || !done) return -1;
    hipLaunchKernelGGL(k_smp_accept, dim3(1), dim3(SMP_THREADS), 0, st, p, q, n, 0, x_dev, 0.0f, 0, rng, nullptr,
                       ctl_out, ctl_n, done, row);
    return (int)hipGetLastError();
}

extern "C" int l98k_smp_sample_topp(const float *probs, int n, const uint32_t *skeys, const int *svals,
                                    const int *n_cand, float topp, unsigned long long *rng, int *out_tok,
                                    hipStream_t st) {
    hipLaunchKernelGGL(k_smp_sample_topp, dim3(1), dim3(SMP_THREADS), 0, st, probs, n, skeys, svals, n_cand, topp,
                       rng, out_tok);
    return (int)hipGetLastError();
}

extern "C" int l98k_smp_xprefix(const float *x, int rows, int n, int mode, const float *c, int *out, float *outv,
                                hipStream_t st) {
    if (rows < 1 || n < 1 || mode < 0 || mode > 2) return -1;
    hipLaunchKernelGGL(k_smp_xprefix, dim3(rows), dim3(SMP_THREADS), 0, st, x, n, mode, c, out, outv);
    return (int)hipGetLastError();
}

// Device arithmetic shared by the gfx950 kernels of the MTP
// speculative-decoding step.
//
// Every floating-point expression below is evaluated in the reference's
// float-oracle order (reference src/ops_*.c, cited per kernel), and the file
// is compiled with -ffp-contract=off, so results are bit-identical to the
// reference engine, not merely close:
//   * sums the reference accumulates serially stay serial (one lane walks
//     them in index order); integer sums (int8 dot products) and max
//     reductions are order-free and run as wave reductions;
//   * exp / rsqrt / sigmoid / softplus are the reference's own float bodies
//     (magic-number floor, 32-entry 2^(i/32) table, two Newton steps), not
//     the device libm;
//   * int8 rounding is the reference's 1.5*2^23 magic add (round to nearest
//     even).
// Per-round scalars (positions, ring slot, token ids) are read from a device
// control block, so a whole round can be replayed as a HIP graph.
#ifndef L98_DEVMATH_H
#define L98_DEVMATH_H
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "l98_dev.h"
#include "l98_launch.h"

// ---------------------------------------------------------------- math ---

// Each translation unit holds its own copy of the table (static), uploaded
// by its l98k_upload_exp_table_* (all of them run from l98k_upload_exp_table).
static __constant__ float c_exp_tab[32];

// The 2^(i/32) table of d_exp is indexed by a per-lane value, so it is read
// from LDS (one ds_read) rather than constant memory (a vector memory load).
// EXP_TAB_LOAD issues the load of a thread's entry early, with the kernel's
// other loads; EXP_TAB_PUT stores it, and a barrier must follow before the
// first d_exp.
#define EXP_TAB_LOAD(tab)     \
    __shared__ float tab[32]; \
    const float tab##_v = c_exp_tab[threadIdx.x & 31]
#define EXP_TAB_PUT(tab) \
    if (threadIdx.x < 32) tab[threadIdx.x] = tab##_v

__device__ __forceinline__ float f_from_u(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t u_from_f(float f) { return __float_as_uint(f); }

// lz_exp_float_body, src/ops_quant.c:300-349
__device__ __forceinline__ float d_exp(float x, const float *tab) {
    const float C2 = 0.242844437f, C1 = 0.207425515f, C0 = 0.549730133f;
    const float LOG2E32 = 1.44269504f * 32.0f;
    // the body runs for every lane (idx is always in [0, 31]) and the range
    // cases are selected after it: no divergent branch around the table read
    float y32 = x * LOG2E32;
    float m = (y32 - 0.5f) + 12582912.0f;
    int32_t t = (int32_t)(u_from_f(m) & 0x007FFFFFu) - 0x00400000;
    int32_t n = t >> 5;
    int32_t idx = t & 31;
    float r = y32 - (float)t;
    float w = 1.0f + r * 0.03125f;
    float p2n = f_from_u((uint32_t)(n + 127) << 23);
    float c = (C2 * w + C1) * w + C0;
    const float body = p2n * (tab[idx] * c);
    return x > 88.0f ? 3.40282347e+38f : x < -87.3f ? 0.0f : body;
}

// lz_rsqrt_float_body, src/ops_quant.c:126-135
__device__ __forceinline__ float d_rsqrt(float x) {
    float h = 0.5f * x;
    float y = f_from_u(0x5f375a86u - (u_from_f(x) >> 1));
    y = y * (1.5f - h * y * y);
    y = y * (1.5f - h * y * y);
    return y;
}

// lz_sigmoid float branch, src/ops_quant.c:1816-1853
// (x >= 0: 1 / (1 + exp(-x)); else exp(x) / (1 + exp(x)), as one path:
// each lane's exp argument and numerator are those of its branch)
__device__ __forceinline__ float d_sigmoid(float x, const float *tab) {
    const bool nonneg = x >= 0.0f;
    const float z = d_exp(nonneg ? -x : x, tab);
    return (nonneg ? 1.0f : z) / (1.0f + z);
}
__device__ __forceinline__ float d_silu(float x, const float *tab) { return x * d_sigmoid(x, tab); }

// lz_softplus_poly, src/ops_quant.c:1040-1060
__device__ __forceinline__ float d_softplus(float x, const float *tab) {
    const float L[9] = {1.000000000f, -0.499995530f, 0.333203435f, -0.248529464f,
                        0.191451162f, -0.137466222f, 0.079210736f, -0.030110965f,
                        0.005384062f};
    float nx = (x < 0.0f) ? x : -x;
    float u = d_exp(nx, tab);
    float p = L[8];
#pragma unroll
    for (int i = 7; i >= 0; i--) p = p * u + L[i];
    float lp = u * p;
    return x > 16.0f ? x : x > 0.0f ? x + lp : lp;
}

// q8_round (--fastfp off), src/ops_quant.h:145-178
__device__ __forceinline__ int d_q8_round(float v) {
    float t = v + 12582912.0f;
    return (int)(u_from_f(t) & 0x007FFFFFu) - 0x00400000;
}

// q8_group_scale's decisions as selects (straight-line code): amax > 0
// with s = amax * (1/127) >= 1e-30 gives s and inv = 127 / amax; zero, NaN
// and tiny groups give s = 1, inv = 0.  The reference's fallback of
// dividing by s when 127 / amax overflows is unreachable: s >= 1e-30
// means amax > 1.2e-28, so 127 / amax < 1.1e30 is finite.
__device__ __forceinline__ void q8_scale_inv(float amax, float *sg, float *inv) {
    const float INV127 = 1.0f / 127.0f;
    const float sg0 = amax * INV127;
    const float inv0 = 127.0f / amax;
    const bool live = amax > 0.0f && !(sg0 < 1.0e-30f);
    *sg = live ? sg0 : 1.0f;
    *inv = live ? inv0 : 0.0f;
}

// sum of squares / n for power-of-two n is a multiply (src/ops_norm.c:161-170)
__device__ __forceinline__ float d_ss_over_n(float ss, int n) {
    if ((n & (n - 1)) == 0) {
        int e = 31 - __clz(n);
        return ss * f_from_u((uint32_t)(127 - e) << 23);
    }
    return ss / (float)n;
}

// Order-preserving float key (src/sampler.c:121)
__device__ __forceinline__ uint32_t d_fkey(float f) {
    uint32_t u = u_from_f(f);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__device__ __forceinline__ float d_unkey(uint32_t k) {
    return f_from_u((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

__device__ __forceinline__ float wave_max_u(uint32_t v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) {
        uint32_t w = __shfl_xor(v, o, width);
        v = w > v ? w : v;
    }
    return f_from_u(v);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = __shfl_xor(v, o);
        v = w > v ? w : v;
    }
    return v;
}

// Quantize one 32-element group held one element per lane across a
// 32-lane half wave (lane & 31 = element).  Writes q[lane] and, from lane
// 0 of the half, the scale.  src/ops_quant.c:1633-1670, 2152-2286.
__device__ __forceinline__ void d_quant_group32(float x, int8_t *q, float *s) {
    uint32_t a = u_from_f(x) & 0x7FFFFFFFu;
    float amax = wave_max_u(a, 32);
    float sg, inv;
    q8_scale_inv(amax, &sg, &inv);
    int qi = d_q8_round(x * inv);
    qi = qi > 127 ? 127 : qi;
    qi = qi < -127 ? -127 : qi;
    *q = (int8_t)qi;
    if ((threadIdx.x & 31) == 0) *s = sg;
}

// Serial left-to-right float sum of n values in LDS by one lane (v 16-byte
// aligned).  The adds stay in index order.  serial_sum_n unrolls a short
// fixed length; serial_sum walks blocks of 32 values with the next block's
// eight 16-byte reads issued before the current block's adds, so the loop
// body stays small and the LDS latency hides behind the dependent adds.
template <int N>
__device__ __forceinline__ float serial_sum_n(const float *v) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        const float4 q = *reinterpret_cast<const float4 *>(v + i);
        ss += q.x; ss += q.y; ss += q.z; ss += q.w;
    }
    return ss;
}

__device__ __forceinline__ float serial_sum(const float *v, int n) {
    float ss = 0.0f;
    const int nb = n >> 5;
    if (nb > 0) {
        float4 cur[8], nxt[8];
#pragma unroll
        for (int u = 0; u < 8; u++) cur[u] = reinterpret_cast<const float4 *>(v)[u];
#pragma unroll 1
        for (int b = 0; b < nb; b++) {
            const int bn = b + 1 < nb ? b + 1 : b;          // last block re-reads itself
#pragma unroll
            for (int u = 0; u < 8; u++) nxt[u] = reinterpret_cast<const float4 *>(v + 32 * bn)[u];
#pragma unroll
            for (int u = 0; u < 8; u++) { ss += cur[u].x; ss += cur[u].y; ss += cur[u].z; ss += cur[u].w; }
#pragma unroll
            for (int u = 0; u < 8; u++) cur[u] = nxt[u];
        }
    }
    for (int i = nb << 5; i < n; i++) ss += v[i];
    return ss;
}

// -------------------------------------------------------------- helpers ---

__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }

// ------------------------------------------- exact sums, one wave wide ---
//
// wave_sum_nonneg returns, on every lane of a wave, exactly the float that
// the serial loop  s = 0; for i < n: s += v[i]  produces, for non-negative
// v (sums of squares, sums of exponentials), in a fraction of the serial
// loop's 8-cycle-per-add latency.
//
// While the running sum s stays inside one binade [2^E, 2^(E+1)), s is a
// multiple of that binade's ulp u, and s + p rounds to s + RN(p / u) * u:
// the rounding no longer depends on s, except for an exact tie (where the
// parity of s / u decides) and except for the add that leaves the binade.
// So:
//   1. an approximate prefix sum (a wave scan) guesses, per element, the
//      binade of the running sum before and after it;
//   2. every element whose guess changes binade, whose p / u is a tie, or
//      whose p is not small against the binade is "special"; every other
//      element contributes the integer q = RN(p / u) grid steps;
//   3. one walk over the special elements in index order does each of them
//      as a real float add and each run of ordinary elements between two of
//      them as one exact add of (sum of q) * u, after checking that the
//      real running sum is in the guessed binade at the start of the run and
//      does not pass its top at the end (s only grows, so nothing in between
//      can leave it).  A run that fails the check is added serially.
// The guesses only decide how much work is serial; the value is exact for
// any guesses.  Inputs with an infinity or NaN, or more special elements
// than the walk's table holds, take the serial loop.
//
// Element i sits in lane i / C, slot i % C.  rec: LDS table of 128 entries
// for this wave.  v (16-byte aligned) holds the row in the ps_slot layout
// below; C % 4 == 0, n <= 64 * C.
struct __align__(16) PsRec {
    float p;
    uint32_t info;                      // binade guess | (index + 1) << 8
    uint32_t ps;                        // sum of q before the element
    uint32_t pad;
};

__device__ __forceinline__ int f_binade(float x) { return (int)((u_from_f(x) >> 23) & 0xFFu); }
__device__ __forceinline__ float f_rl(float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); }

// Inclusive wave scans: row prefix sums by DPP row_shr, then the row
// carries by row_bcast:15 and row_bcast:31.  The float scan only feeds the
// binade guesses, so its association order is free.
#define L98_DPP_ADD(x, ctrl, rmask) \
    (x) = (x) + __builtin_amdgcn_update_dpp(0, (x), (ctrl), (rmask), 0xF, false)
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
    int x = (int)v;
    L98_DPP_ADD(x, 0x111, 0xF);
    L98_DPP_ADD(x, 0x112, 0xF);
    L98_DPP_ADD(x, 0x114, 0xF);
    L98_DPP_ADD(x, 0x118, 0xF);
    L98_DPP_ADD(x, 0x142, 0xA);
    L98_DPP_ADD(x, 0x143, 0xC);
    return (uint32_t)x;
}
#define L98_DPP_FADD(x, ctrl, rmask) \
    (x) = (x) + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), (ctrl), (rmask), 0xF, false))
__device__ __forceinline__ float wave_scan_f32(float x) {
    L98_DPP_FADD(x, 0x111, 0xF);
    L98_DPP_FADD(x, 0x112, 0xF);
    L98_DPP_FADD(x, 0x114, 0xF);
    L98_DPP_FADD(x, 0x118, 0xF);
    L98_DPP_FADD(x, 0x142, 0xA);
    L98_DPP_FADD(x, 0x143, 0xC);
    return x;
}
// lane l receives lane l-1's value, lane 0 receives 0 (DPP wave_shr:1)
__device__ __forceinline__ float wave_shr1_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x138, 0xF, 0xF, false));
}

// Row layout of wave_sum_nonneg's input: element i at ps_slot<C>(i), i.e.
// lane chunks of C floats, each followed by 4 floats of padding, so that the
// lanes' 16-byte reads of their chunks fall in distinct LDS banks.
template <int C>
__host__ __device__ constexpr int ps_slot(int i) { return (i / C) * (C + 4) + i % C; }
template <int C>
__host__ __device__ constexpr int ps_row_floats() { return 64 * (C + 4); }

// One element of the classification: from the guesses before (E0) and
// after (E1) it, whether it is ordinary (plain) and its grid steps q.
__device__ __forceinline__ uint32_t ps_classify(float p, int E0, int E1, uint32_t *q) {
    const int eb = E0 > 1 ? E0 : 1;
    const float sc = __builtin_amdgcn_ldexpf(p, 150 - eb);
    const uint32_t tiex = u_from_f(__builtin_amdgcn_fractf(sc)) ^ 0x3F000000u;       // 0 iff a tie
    const uint32_t cross = (uint32_t)(E0 ^ E1);
    const uint32_t plain = (tiex < 1u ? tiex : 1u) >> (cross < 1u ? cross : 1u);   // shifts count mod 32
    const uint32_t qq = (uint32_t)__builtin_rintf(sc);
    *q = (qq < 0x1000001u ? qq : 0x1000001u) * plain;
    return plain;
}

template <int C>
__device__ __forceinline__ float wave_sum_nonneg(const float *v, int n, PsRec *rec) {
    static_assert(C % 4 == 0 && C <= 32, "C: multiple of 4, at most 32");
    const int lane = threadIdx.x & 63, i0 = lane * C;
    const float4 *vl = reinterpret_cast<const float4 *>(v + lane * (C + 4));
    // the row holds 64 * (C + 4) floats, so no read is out of range;
    // elements past n read as 0
    float p[C];
#pragma unroll
    for (int g = 0; g < C / 4; g++) {
        const float4 x = vl[g];
        p[4 * g] = i0 + 4 * g < n ? x.x : 0.0f;
        p[4 * g + 1] = i0 + 4 * g + 1 < n ? x.y : 0.0f;
        p[4 * g + 2] = i0 + 4 * g + 2 < n ? x.z : 0.0f;
        p[4 * g + 3] = i0 + 4 * g + 3 < n ? x.w : 0.0f;
    }
    float T = 0.0f;
#pragma unroll
    for (int c = 0; c < C; c++) T += p[c];
    const float incl = wave_scan_f32(T);
    const float off = wave_shr1_f32(incl);
    // Guessed binades before and after each element.  The guess after the
    // lane's last element is `incl` itself, so it equals the next lane's
    // guess before its first element bit for bit.
    int Eb[C + 1];
    {
        float A = off;
        Eb[0] = f_binade(off);
#pragma unroll
        for (int c = 0; c < C; c++) {
            A = (c == C - 1) ? incl : A + p[c];
            Eb[c + 1] = f_binade(A);
        }
    }
    uint32_t plain[C], q[C], cnt = 0, qs = 0;
#pragma unroll
    for (int c = 0; c < C; c++) {
        plain[c] = ps_classify(p[c], Eb[c], Eb[c + 1], &q[c]);
        cnt += 1u - plain[c];
        qs += q[c];
    }
    const uint32_t cincl = wave_scan_u32(cnt);
    const uint32_t qincl = wave_scan_u32(qs);
    // lane sums below 2^26 keep the 32-bit scan from wrapping (64 * 2^26)
    const bool bad = !(T <= 3.0e38f) || f_binade(incl) >= 254 || qs >= 0x4000000u;
    // the number of special elements, counted on the scalar unit from
    // ballots (a readlane feeding a scalar instruction stalls far longer)
    int Kall = 0;
#pragma unroll
    for (int c = 0; c < C; c++) Kall += __popcll(__ballot(plain[c] == 0u));
    const int K = Kall < 62 ? Kall : 62;
    // Each special element's record goes to its rank; ordinary elements
    // write their lane's spare slot 64 + lane (distinct addresses: writes to
    // one address from many lanes would serialize).
    {
        uint32_t r = cincl - cnt + 1, ps = qincl - qs;
#pragma unroll
        for (int c = 0; c < C; c++) {
            PsRec rc;
            rc.p = p[c];
            rc.info = (uint32_t)Eb[c + 1] | ((uint32_t)(i0 + c + 1) << 8);
            rc.ps = ps;
            rc.pad = 0u;
            rec[plain[c] ? 64u + lane : (r < 63u ? r : 63u)] = rc;
            r += 1u - plain[c];
            ps += q[c];
        }
    }
    if (lane == 0) { PsRec e; e.p = 0.0f; e.info = 0u; e.ps = 0u; e.pad = 0u; rec[0] = e; }
    if (lane == 63) { PsRec e; e.p = 0.0f; e.info = (uint32_t)(n + 1) << 8; e.ps = qincl; e.pad = 0u; rec[K + 1] = e; }
    __builtin_amdgcn_s_waitcnt(0xC07F);               // lgkmcnt(0): the table is written
    __builtin_amdgcn_wave_barrier();
    // Lane j: record j and the run after it.  The run may be taken in one
    // add iff lo <= s <= hi for the running sum s after record j: lo is the
    // guessed binade's bottom, hi the largest s with s + Qu at most the
    // binade's top.  Lanes past the last record walk an empty step.
    const PsRec me = rec[imin(lane, K + 1)];
    const PsRec nx = rec[imin(lane + 1, K + 1)];
    const int E = (int)(me.info & 255u), ia = (int)(me.info >> 8), ib = (int)(nx.info >> 8) - 1;
    const int eb = E > 1 ? E : 1;
    const uint32_t Q = nx.ps - me.ps;
    const float top = __builtin_amdgcn_ldexpf(1.0f, eb - 126);
    const float Qu0 = (float)(Q < 16777216u ? Q : 16777216u) * __builtin_amdgcn_ldexpf(1.0f, eb - 150);
    const bool empty = ib <= ia || lane > K;
    const float P = lane > K ? 0.0f : me.p;
    const float lo0 = E ? __builtin_amdgcn_ldexpf(1.0f, E - 127) : 0.0f, hi0 = top - Qu0;
    // an infeasible run (too many steps, or an empty interval) gets lo = hi
    // = -1, which no s >= 0 passes
    const bool feasible = Q <= 16777216u && hi0 >= lo0;
    const float lo = empty ? 0.0f : feasible ? lo0 : -1.0f;
    const float hi = empty ? __builtin_inff() : feasible ? hi0 : -1.0f;
    const float Qu = empty ? 0.0f : Qu0;
    // Fast walk, systolic: each step hands every lane its left neighbour's
    // running sum (DPP wave_shr:1; lane 0 gets 0) and applies the lane's
    // record, so after step j lane j holds its final value.  Then every
    // lane checks its run: med3(s, lo, hi) == s iff lo <= s <= hi.
    float s1 = 0.0f, sout = 0.0f;
    for (int j = 0; j <= K; j++) {
        s1 = wave_shr1_f32(sout) + P;
        sout = s1 + Qu;
    }
    const bool fail = bad || Kall > 62 || __builtin_amdgcn_fmed3f(s1, lo, hi) != s1;
    if (__ballot(fail) == 0) return f_rl(sout, K);
    // Slow path: the serial loop, a lane chunk at a time with the next
    // chunk's reads in flight (elements past n read as 0).
    float s = 0.0f;
    const int nch = (n + C - 1) / C;
    float4 cur[C / 4], nxt[C / 4];
#pragma unroll
    for (int m = 0; m < C / 4; m++) cur[m] = reinterpret_cast<const float4 *>(v)[m];
    for (int l = 0; l < nch; l++) {
        const int ln = l + 1 < nch ? l + 1 : l;
#pragma unroll
        for (int m = 0; m < C / 4; m++) nxt[m] = reinterpret_cast<const float4 *>(v + ln * (C + 4))[m];
#pragma unroll
        for (int m = 0; m < C / 4; m++) {
            const int i = l * C + 4 * m;
            s += i < n ? cur[m].x : 0.0f;
            s += i + 1 < n ? cur[m].y : 0.0f;
            s += i + 2 < n ? cur[m].z : 0.0f;
            s += i + 3 < n ? cur[m].w : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < C / 4; m++) cur[m] = nxt[m];
    }
    return s;
}

// ------------------------------------------------------- rmsnorm (+q8) ---
//
// Row kernels hold a row of n floats in a 64-lane block as float4 f =
// lane + 64*j (PJ per lane), so every 32-element quantization group is an
// aligned lane octet (see quant_octet below).

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Max over the 8 lanes of an aligned lane octet (DPP within a row).
__device__ __forceinline__ uint32_t octet_max(uint32_t m) {
    m = umax(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    m = umax(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    m = umax(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));  // row_half_mirror
    return m;
}

// Per-32 quantization (src/ops_quant.c:1633-1670, 2152-2286) of a group held
// as 4 consecutive elements per lane over an aligned lane octet.  Returns the
// four int8 packed little-endian; *sg receives the group scale.  Every lane
// of the octet must execute it.
__device__ __forceinline__ uint32_t abs_bits4(float4 v) {
    return umax(umax(u_from_f(v.x) & 0x7FFFFFFFu, u_from_f(v.y) & 0x7FFFFFFFu),
                umax(u_from_f(v.z) & 0x7FFFFFFFu, u_from_f(v.w) & 0x7FFFFFFFu));
}

// The element loop of the quantization for a group whose amax is given
// (q8_group_scale's decisions, then the rounding of each element).
__device__ __forceinline__ uint32_t quant4_amax(float4 v, float amax, float *sg_out) {
    float sg, inv;
    q8_scale_inv(amax, &sg, &inv);
    float e[4] = {v.x * inv, v.y * inv, v.z * inv, v.w * inv};
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int qi = d_q8_round(e[i]);
        qi = qi > 127 ? 127 : qi;
        qi = qi < -127 ? -127 : qi;
        packed |= ((uint32_t)qi & 0xFFu) << (8 * i);
    }
    *sg_out = sg;
    return packed;
}

__device__ __forceinline__ uint32_t quant_octet(float4 v, float *sg_out) {
    return quant4_amax(v, f_from_u(octet_max(abs_bits4(v))), sg_out);
}

// epi_q8 of a row with one 32-element group (a per-row weight scale over
// in_dim == 32, so r = gs / 32 == 1: src/ops_epi.c:1012-1021): four
// accumulators, only the first of which takes a term,
//   a0 = 0 + float(acc) * (xs * ws);  o = (a0 + 0) + (0 + 0).
// Rows of more groups take the r > 1 form, 0 + (sum_s float(acc_s) * xs_s)
// * ws.
__device__ __forceinline__ float epi_one_group(int acc, float xs, float ws) {
    float a0 = 0.0f;
    const float a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    a0 += (float)acc * (xs * ws);
    return (a0 + a2) + (a1 + a3);
}

// RMSNorm(1+w) of the block's row v (lz_rmsnorm, src/ops_norm.c:690-747:
// sum of squares in index order, inv = rsqrt(ss/n + eps), o =
// (x*inv)*(1+w)), then the optional store of o and its per-32 quantization.
// The sum is wave_sum_nonneg's (sq: ps_row_floats<4 * PJ>() floats, rec its
// table).  n % 32 == 0.
// NORM == false skips the norm (o = v: the row is only stored and/or
// quantized); TOK selects one scale for the whole row (lz_quantize_q8_tok,
// src/ops_quant.c:2284-2314: the row's amax, the same element loop, the
// scale in every 32-slot) instead of one per 32 elements.
template <int PJ, bool NORM = true, bool TOK = false>
__device__ __forceinline__ void norm_row(const float4 (&v)[PJ], const float4 (&wn)[PJ], int n, float eps,
                                         float *sq, PsRec *rec, float *s_inv, float *__restrict__ out,
                                         int8_t *__restrict__ xq, float *__restrict__ xqs) {
    const int lane = threadIdx.x, nf = n >> 2;
    float inv = 1.0f;
    if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const int f = lane + 64 * j;
            if (f < nf) *reinterpret_cast<float4 *>(sq + ps_slot<4 * PJ>(4 * f)) =
                make_float4(v[j].x * v[j].x, v[j].y * v[j].y, v[j].z * v[j].z, v[j].w * v[j].w);
        }
        __syncthreads();
        const float ss = wave_sum_nonneg<4 * PJ>(sq, n, rec);
        if (lane == 0) *s_inv = d_rsqrt(d_ss_over_n(ss, n) + eps);
        __syncthreads();
        inv = *s_inv;
    }
    if constexpr (!TOK) {
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const int f = lane + 64 * j;
            float4 o = v[j];
            if constexpr (NORM)
                o = make_float4(v[j].x * inv * (1.0f + wn[j].x), v[j].y * inv * (1.0f + wn[j].y),
                                v[j].z * inv * (1.0f + wn[j].z), v[j].w * inv * (1.0f + wn[j].w));
            if (out && f < nf) reinterpret_cast<float4 *>(out)[f] = o;
            if (xq) {
                float sg;
                const uint32_t q = quant_octet(o, &sg);
                if (f < nf) {
                    reinterpret_cast<uint32_t *>(xq)[f] = q;
                    if (!(f & 7)) xqs[f >> 3] = sg;
                }
            }
        }
    } else {
        float4 o[PJ];
        uint32_t am = 0;
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const int f = lane + 64 * j;
            o[j] = v[j];
            if constexpr (NORM)
                o[j] = make_float4(v[j].x * inv * (1.0f + wn[j].x), v[j].y * inv * (1.0f + wn[j].y),
                                   v[j].z * inv * (1.0f + wn[j].z), v[j].w * inv * (1.0f + wn[j].w));
            if (out && f < nf) reinterpret_cast<float4 *>(out)[f] = o[j];
            if (f < nf) am = umax(am, abs_bits4(o[j]));
        }
        if (!xq) return;
        const float row_amax = wave_max_u(am, 64);
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const int f = lane + 64 * j;
            float sg;
            const uint32_t q = quant4_amax(o[j], row_amax, &sg);
            if (f < nf) {
                reinterpret_cast<uint32_t *>(xq)[f] = q;
                if (!(f & 7)) xqs[f >> 3] = sg;
            }
        }
    }
}

// One 64-lane block per row, n <= 256*PJ.  Optionally first folds the
// residual in place: x_row = x_row + (a_row [+ b_row]) (the reference's
// x += xb2 with xb2 = up + shared already summed, src/forward.c:1449-1557,
// src/forward_moe.c:552), then norm_row.  Every load is issued up front.
#endif

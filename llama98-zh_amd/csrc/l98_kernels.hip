// gfx950 kernels of the MTP speculative-decoding step.
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

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "l98_dev.h"
#include "l98_launch.h"

// ---------------------------------------------------------------- math ---

__constant__ float c_exp_tab[32];

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
    if (x > 88.0f) return 3.40282347e+38f;
    if (x < -87.3f) return 0.0f;
    float y32 = x * LOG2E32;
    float m = (y32 - 0.5f) + 12582912.0f;
    int32_t t = (int32_t)(u_from_f(m) & 0x007FFFFFu) - 0x00400000;
    int32_t n = t >> 5;
    int32_t idx = t & 31;
    float r = y32 - (float)t;
    float w = 1.0f + r * 0.03125f;
    float p2n = f_from_u((uint32_t)(n + 127) << 23);
    float c = (C2 * w + C1) * w + C0;
    return p2n * (tab[idx] * c);
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
__device__ __forceinline__ float d_sigmoid(float x, const float *tab) {
    if (x >= 0.0f) {
        float z = d_exp(-x, tab);
        return 1.0f / (1.0f + z);
    }
    float z = d_exp(x, tab);
    return z / (1.0f + z);
}
__device__ __forceinline__ float d_silu(float x, const float *tab) { return x * d_sigmoid(x, tab); }

// lz_softplus_poly, src/ops_quant.c:1040-1060
__device__ __forceinline__ float d_softplus(float x, const float *tab) {
    const float L[9] = {1.000000000f, -0.499995530f, 0.333203435f, -0.248529464f,
                        0.191451162f, -0.137466222f, 0.079210736f, -0.030110965f,
                        0.005384062f};
    if (x > 16.0f) return x;
    float nx = (x < 0.0f) ? x : -x;
    float u = d_exp(nx, tab);
    float p = L[8];
#pragma unroll
    for (int i = 7; i >= 0; i--) p = p * u + L[i];
    float lp = u * p;
    if (x > 0.0f) return x + lp;
    return lp;
}

// q8_round (--fastfp off), src/ops_quant.h:145-178
__device__ __forceinline__ int d_q8_round(float v) {
    float t = v + 12582912.0f;
    return (int)(u_from_f(t) & 0x007FFFFFu) - 0x00400000;
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
    const float INV127 = 1.0f / 127.0f;
    uint32_t a = u_from_f(x) & 0x7FFFFFFFu;
    float amax = wave_max_u(a, 32);
    float sg, inv;
    bool fast;
    if (amax > 0.0f) {
        sg = amax * INV127;
        inv = 127.0f / amax;
        fast = (inv <= 3.40282347e+38f);
        if (sg < 1.0e-30f) { sg = 1.0f; inv = 0.0f; fast = true; }
    } else {
        sg = 1.0f; inv = 0.0f; fast = true;
    }
    int qi = fast ? d_q8_round(x * inv) : d_q8_round(x / sg);
    qi = qi > 127 ? 127 : qi;
    qi = qi < -127 ? -127 : qi;
    *q = (int8_t)qi;
    if ((threadIdx.x & 31) == 0) *s = sg;
}

// Serial left-to-right float sum of n values in LDS by one lane (n % 4 ==
// 0 and v 16-byte aligned).  The adds stay in index order; the loop body
// reads 4 values at a time and is unrolled so the LDS reads run ahead of the
// dependent adds.  The common row width 1024 is a fully unrolled instance.
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
    if (n == 1024) return serial_sum_n<1024>(v);
    float ss = 0.0f;
    int i = 0;
#pragma unroll 8
    for (; i + 4 <= n; i += 4) {
        const float4 q = *reinterpret_cast<const float4 *>(v + i);
        ss += q.x; ss += q.y; ss += q.z; ss += q.w;
    }
    for (; i < n; i++) ss += v[i];
    return ss;
}

// -------------------------------------------------------------- helpers ---

__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }

// -------------------------------------------------------------- embed ---

// lz_t_row_f32 for a Q8_0 per-row table: x = float(q) * scale[row].
__global__ void k_embed(const int8_t *__restrict__ q, const float *__restrict__ s,
                        const int *__restrict__ toks, int d, float *__restrict__ x) {
    int t = blockIdx.y;
    int tok = toks[t];
    const int8_t *row = q + (size_t)tok * d;
    float sc = s[tok];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        x[(size_t)t * d + i] = (float)row[i] * sc;
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
__device__ __forceinline__ uint32_t quant_octet(float4 v, float *sg_out) {
    const float INV127 = 1.0f / 127.0f;
    uint32_t m = umax(umax(u_from_f(v.x) & 0x7FFFFFFFu, u_from_f(v.y) & 0x7FFFFFFFu),
                      umax(u_from_f(v.z) & 0x7FFFFFFFu, u_from_f(v.w) & 0x7FFFFFFFu));
    const float amax = f_from_u(octet_max(m));
    float sg, inv;
    bool fast;
    if (amax > 0.0f) {
        sg = amax * INV127;
        inv = 127.0f / amax;
        fast = (inv <= 3.40282347e+38f);
        if (sg < 1.0e-30f) { sg = 1.0f; inv = 0.0f; fast = true; }
    } else {
        sg = 1.0f; inv = 0.0f; fast = true;
    }
    float e[4] = {v.x, v.y, v.z, v.w};
    if (fast) {
#pragma unroll
        for (int i = 0; i < 4; i++) e[i] = e[i] * inv;
    } else {                             // 127/amax overflowed: divide by the scale instead
#pragma unroll
        for (int i = 0; i < 4; i++) e[i] = e[i] / sg;
    }
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

// RMSNorm(1+w) of the block's row v (lz_rmsnorm, src/ops_norm.c:690-747:
// sum of squares serial in index order by lane 0, inv = rsqrt(ss/n + eps),
// o = (x*inv)*(1+w)), then the optional store of o and its per-32
// quantization.  n % 32 == 0.
template <int PJ>
__device__ __forceinline__ void norm_row(const float4 (&v)[PJ], const float4 (&wn)[PJ], int n, float eps,
                                         float *sq, float *s_inv, float *__restrict__ out,
                                         int8_t *__restrict__ xq, float *__restrict__ xqs) {
    const int lane = threadIdx.x, nf = n >> 2;
#pragma unroll
    for (int j = 0; j < PJ; j++) {
        const int f = lane + 64 * j;
        if (f < nf) reinterpret_cast<float4 *>(sq)[f] =
            make_float4(v[j].x * v[j].x, v[j].y * v[j].y, v[j].z * v[j].z, v[j].w * v[j].w);
    }
    __syncthreads();
    if (lane == 0) *s_inv = d_rsqrt(d_ss_over_n(serial_sum(sq, n), n) + eps);
    __syncthreads();
    const float inv = *s_inv;
#pragma unroll
    for (int j = 0; j < PJ; j++) {
        const int f = lane + 64 * j;
        const float4 o = make_float4(v[j].x * inv * (1.0f + wn[j].x), v[j].y * inv * (1.0f + wn[j].y),
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
}

// One 64-lane block per row, n <= 256*PJ.  Optionally first folds the
// residual in place: x_row = x_row + (a_row [+ b_row]) (the reference's
// x += xb2 with xb2 = up + shared already summed, src/forward.c:1449-1557,
// src/forward_moe.c:552), then norm_row.  Every load is issued up front.
template <int PJ>
__global__ __launch_bounds__(64) void k_rmsnorm(float *__restrict__ x, int x_stride,
                                                const float *__restrict__ a, const float *__restrict__ b,
                                                const float *__restrict__ w, int n, float eps,
                                                float *__restrict__ out, int out_stride,
                                                int8_t *__restrict__ xq, float *__restrict__ xqs) {
    __shared__ __align__(16) float sq[256 * PJ];
    __shared__ float s_inv;
    const int row = blockIdx.x, lane = threadIdx.x, nf = n >> 2;
    float4 *xr = reinterpret_cast<float4 *>(x + (size_t)row * x_stride);
    float4 v[PJ], wn[PJ];
#pragma unroll
    for (int j = 0; j < PJ; j++) {
        const int fc = imin(lane + 64 * j, nf - 1);
        v[j] = xr[fc];
        wn[j] = reinterpret_cast<const float4 *>(w)[fc];
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
    norm_row<PJ>(v, wn, n, eps, sq, &s_inv, out ? out + (size_t)row * out_stride : nullptr,
                 xq ? xq + (size_t)row * n : nullptr, xqs ? xqs + (size_t)row * (n >> 5) : nullptr);
}

// MTP input rows (lz_mtp_draft_step / lz_mtp_prefill, src/forward_mtp.c:
// e = embed(tok); concat = [rmsnorm(e, pre_e) | rmsnorm(h, pre_h)], then the
// per-32 quantization of concat for the fc projection).  blockIdx.y = 0: the
// embedding half, 1: the hidden half.  d % 32 == 0, so the halves quantize
// independently.
template <int PJ>
__global__ __launch_bounds__(64) void k_mtp_pre(const int8_t *__restrict__ emb_q, const float *__restrict__ emb_s,
                                                const int *__restrict__ toks, const float *__restrict__ h,
                                                int d, const float *__restrict__ w_e,
                                                const float *__restrict__ w_h, float eps,
                                                int8_t *__restrict__ xq, float *__restrict__ xqs) {
    __shared__ __align__(16) float sq[256 * PJ];
    __shared__ float s_inv;
    const int r = blockIdx.x, half = blockIdx.y, lane = threadIdx.x, nf = d >> 2;
    const float4 *wn4 = reinterpret_cast<const float4 *>(half == 0 ? w_e : w_h);
    float4 v[PJ], wn[PJ];
    if (half == 0) {
        const int tok = toks[r];
        const uint32_t *er = reinterpret_cast<const uint32_t *>(emb_q + (size_t)tok * d);
        const float sc = emb_s[tok];
#pragma unroll
        for (int j = 0; j < PJ; j++) {
            const uint32_t q = er[imin(lane + 64 * j, nf - 1)];
            v[j] = make_float4((float)(int8_t)(q & 0xFF) * sc, (float)(int8_t)((q >> 8) & 0xFF) * sc,
                               (float)(int8_t)((q >> 16) & 0xFF) * sc, (float)(int8_t)(q >> 24) * sc);
        }
    } else {
#pragma unroll
        for (int j = 0; j < PJ; j++) v[j] = reinterpret_cast<const float4 *>(h + (size_t)r * d)[imin(lane + 64 * j, nf - 1)];
    }
#pragma unroll
    for (int j = 0; j < PJ; j++) wn[j] = wn4[imin(lane + 64 * j, nf - 1)];
    norm_row<PJ>(v, wn, d, eps, sq, &s_inv, nullptr, xq + (size_t)r * 2 * d + (size_t)half * d,
                 xqs + (size_t)r * (2 * d >> 5) + (size_t)half * (d >> 5));
}

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

// LDS bytes of one tile: staged activations, their scales, and the larger of
// the group sums and the RMSNorm squares.
__host__ __device__ inline size_t gemv_lds_bytes(int m, int in_dim, int R, int norm) {
    const size_t part = (size_t)R * m * ((in_dim >> 5) + 1) * 4;
    const size_t sq = norm ? (size_t)m * (in_dim + 4) * 4 : 0;
    return (size_t)m * in_dim + (size_t)m * (in_dim >> 5) * 4 + (part > sq ? part : sq);
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
// of src/forward.c:1449-1557): the squares go to LDS and lane t of wave 0
// walks row t's sum serially, all rows at once; the block with `writer` set
// stores the updated residual and the normed rows.  PRO_SILU:
// lz_ffn_gate_up's silu(g)*u (src/forward_kda.c:1067-1088).  PRO_COMBINE:
// the slot-ordered weighted sum of the experts' outputs
// (src/forward_moe.c:128-200).  Every load is unconditional (rows past nm
// and elements past the row end are clamped to valid addresses and their
// values unused), and each mode is one straight-line block.  Contains block
// barriers: call from every thread.
#define XQ_PER_THREAD 4
template <int M, int PJ, typename IssueW>
__device__ __forceinline__ void build_rows(const Prologue &P, const int8_t *__restrict__ xq,
                                           const float *__restrict__ xqs, int in_dim, const int (&xrow)[M], int nm,
                                           bool writer, int8_t *sx, float *sxs, float *sq, float *s_inv,
                                           float *tab, IssueW issue_w) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nb = in_dim >> 5, nf = in_dim >> 2;
    if (PJ == 0 || P.mode == PRO_XQ) {
        // int4 chunk idx of the tile's rows: token idx / cpr, chunk idx % cpr;
        // the stores are unconditional (clamped: past the end they rewrite
        // the last chunk with its own value).
        const int cpr = in_dim >> 4;
        const int total = M * cpr, stotal = M * nb;
        int4 r[XQ_PER_THREAD];
        float sc[XQ_PER_THREAD];
#pragma unroll
        for (int u = 0; u < XQ_PER_THREAD; u++) {
            const int idx = imin(u * GEMV_THREADS + tid, total - 1);
            const int t = idx / cpr, p = idx - t * cpr;
            r[u] = *reinterpret_cast<const int4 *>(xq + (size_t)xrow[t < nm ? t : 0] * in_dim + p * 16);
            const int si = imin(u * GEMV_THREADS + tid, stotal - 1);
            const int ts = si / nb;
            sc[u] = xqs[(size_t)xrow[ts < nm ? ts : 0] * nb + (si - ts * nb)];
        }
        issue_w();
#pragma unroll
        for (int u = 0; u < XQ_PER_THREAD; u++) {
            reinterpret_cast<int4 *>(sx)[imin(u * GEMV_THREADS + tid, total - 1)] = r[u];
            sxs[imin(u * GEMV_THREADS + tid, stotal - 1)] = sc[u];
        }
        for (int base = XQ_PER_THREAD * GEMV_THREADS; base < total; base += GEMV_THREADS) {
            const int idx = imin(base + tid, total - 1);
            const int t = idx / cpr, p = idx - t * cpr;
            reinterpret_cast<int4 *>(sx)[idx] =
                *reinterpret_cast<const int4 *>(xq + (size_t)xrow[t < nm ? t : 0] * in_dim + p * 16);
        }
        for (int base = XQ_PER_THREAD * GEMV_THREADS; base < stotal; base += GEMV_THREADS) {
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
    switch (P.mode) {
    case PRO_QUANT: {
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++)
                v[r][j] = reinterpret_cast<const float4 *>(P.src + (size_t)xr[r] * P.src_stride)[fc[j]];
        issue_w();
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
        break;
    }
    case PRO_SILU: {
        const float tabv = c_exp_tab[lane & 31];
        float4 q[RW][PJN];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                v[r][j] = reinterpret_cast<const float4 *>(P.src + (size_t)xr[r] * P.src_stride)[fc[j]];
                q[r][j] = reinterpret_cast<const float4 *>(P.src2 + (size_t)xr[r] * P.src_stride)[fc[j]];
            }
        issue_w();
        if (tid < 32) tab[tid] = tabv;
        __syncthreads();
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) v[r][j] = f4_silu_mul(v[r][j], q[r][j], tab);
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
        break;
    }
    case PRO_COMBINE: {
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
        issue_w();
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
        break;
    }
    default: {                           // PRO_NORM
        const bool has_a = P.a != nullptr, has_b = P.b != nullptr;
        const float *pa = has_a ? P.a : P.src;
        const float *pb = has_b ? P.b : pa;
        const int sa = has_a ? in_dim : P.src_stride, sb = has_b ? in_dim : sa;
        float4 wn[PJN], ad[RW][PJN], bd[RW][PJN];
#pragma unroll
        for (int j = 0; j < PJN; j++) wn[j] = reinterpret_cast<const float4 *>(P.w)[fc[j]];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                v[r][j] = reinterpret_cast<const float4 *>(P.src + (size_t)xr[r] * P.src_stride)[fc[j]];
                ad[r][j] = reinterpret_cast<const float4 *>(pa + (size_t)xr[r] * sa)[fc[j]];
                bd[r][j] = reinterpret_cast<const float4 *>(pb + (size_t)xr[r] * sb)[fc[j]];
            }
        issue_w();
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
        // rows padded by 4 floats so the summing lanes read different banks
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int t = wave + 4 * r;
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                const int f = lane + 64 * j;
                if (t < nm && f < nf) {
                    const float4 x = v[r][j];
                    reinterpret_cast<float4 *>(sq + (size_t)t * (in_dim + 4))[f] =
                        make_float4(x.x * x.x, x.y * x.y, x.z * x.z, x.w * x.w);
                }
            }
        }
        __syncthreads();
        if (tid < nm)
            s_inv[tid] = d_rsqrt(d_ss_over_n(serial_sum(sq + (size_t)tid * (in_dim + 4), in_dim), in_dim) + P.eps);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < RW; r++) {
            const int t = wave + 4 * r;
            const float inv = s_inv[t < nm ? t : 0];
#pragma unroll
            for (int j = 0; j < PJN; j++) {
                const int f = lane + 64 * j;
                const float4 x = v[r][j], w = wn[j];
                const float4 o = make_float4(x.x * inv * (1.0f + w.x), x.y * inv * (1.0f + w.y),
                                             x.z * inv * (1.0f + w.z), x.w * inv * (1.0f + w.w));
                if (writer && t < nm && f < nf) {
                    if (P.x_out) reinterpret_cast<float4 *>(P.x_out + (size_t)xr[r] * P.src_stride)[f] = x;
                    if (P.o_out) reinterpret_cast<float4 *>(P.o_out + (size_t)xr[r] * P.o_stride)[f] = o;
                }
                v[r][j] = o;
            }
        }
        quant_rows<RW, PJN>(v, wave, lane, nm, nf, nb, in_dim, sx, sxs);
        break;
    }
    }
}

// One GEMV tile.  xrow[t]: activation row of token slot t (registers);
// s_orow[t]: output row of token slot t (LDS, read after a barrier); nm:
// live token slots.  The caller fills the LDS exp table first.
template <int M, int PJ>
__device__ __forceinline__ void gemv_tile(const int8_t *__restrict__ wt, const float *__restrict__ ws, int rows_here,
                                          int in_dim, const Prologue &P, const int8_t *__restrict__ xq,
                                          const float *__restrict__ xqs, const int (&xrow)[M], const int *s_orow,
                                          int nm, bool writer, float *__restrict__ out, size_t out_stride,
                                          int row0, int32_t *__restrict__ acc_out, int acc_rows, char *smem,
                                          float *s_inv, float *tab) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int cpr = in_dim >> 4, nb = in_dim >> 5;
    const int nchunk = rows_here * cpr;
    int8_t *sx = reinterpret_cast<int8_t *>(smem);                                   // [M][in_dim]
    float *sxs = reinterpret_cast<float *>(smem + (size_t)M * in_dim);                // [M][nb]
    int *part = reinterpret_cast<int *>(sxs + M * nb);                                // [R][M][nb+1]
    // weights: one 8 KiB quarter of the tile per wave, all loads in flight
    int4 wv[GEMV_MAXJ];
    const int er = tid / M, et = tid - er * M;
    float wsv = 0.0f;
    auto issue_w = [&]() {
        const v4i *w4 = reinterpret_cast<const v4i *>(wt);
#pragma unroll
        for (int j = 0; j < GEMV_MAXJ; j++) {
            const int c = imin(wave * (GEMV_WAVE_BYTES / 16) + lane + 64 * j, nchunk - 1);
            const v4i q = __builtin_nontemporal_load(w4 + c);
            wv[j] = make_int4(q.x, q.y, q.z, q.w);
        }
        wsv = ws[row0 + imin(er, rows_here - 1)];     // the epilogue lane's row scale
    };
    build_rows<M, PJ>(P, xq, xqs, in_dim, xrow, nm, writer, sx, sxs, reinterpret_cast<float *>(part), s_inv, tab,
                      issue_w);
    __syncthreads();
    // Partial dot products.  With a power-of-two chunk count per row, lane
    // l's chunks of every row sit at the same in-row offsets (l + 64v) mod
    // cpr for v < cpr/64, so each activation chunk is read from LDS once and
    // reused for all of the lane's weight chunks at that offset.
    const int4 *sx4 = reinterpret_cast<const int4 *>(sx);
    auto dot_store = [&](int j, const int4 (&xv)[M]) {
        const int c = wave * (GEMV_WAVE_BYTES / 16) + lane + 64 * j;
        const int r = c / cpr, p = c - r * cpr;
#pragma unroll
        for (int t = 0; t < M; t++) {
            int a = __builtin_amdgcn_sdot4(wv[j].x, xv[t].x, 0, false);
            a = __builtin_amdgcn_sdot4(wv[j].y, xv[t].y, a, false);
            a = __builtin_amdgcn_sdot4(wv[j].z, xv[t].z, a, false);
            a = __builtin_amdgcn_sdot4(wv[j].w, xv[t].w, a, false);
            a += __builtin_amdgcn_update_dpp(0, a, 0xB1, 0xF, 0xF, false);     // lane ^ 1: chunks 2g, 2g+1
            if (t < nm && c < nchunk && !(lane & 1)) part[(r * M + t) * (nb + 1) + (p >> 1)] = a;
        }
    };
    if ((cpr & (cpr - 1)) == 0 && cpr <= 256) {
        const int nv = cpr > 64 ? cpr >> 6 : 1;
#pragma unroll
        for (int vv = 0; vv < 4; vv++) {
            if (vv < nv) {
                const int p = (lane + 64 * vv) & (cpr - 1);
                int4 xv[M];
#pragma unroll
                for (int t = 0; t < M; t++) xv[t] = sx4[(t < nm ? t : 0) * cpr + p];
#pragma unroll
                for (int j = 0; j < GEMV_MAXJ; j++)
                    if ((j & (nv - 1)) == vv) dot_store(j, xv);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < GEMV_MAXJ; j++) {
            const int c = wave * (GEMV_WAVE_BYTES / 16) + lane + 64 * j;
            const int p = c - (c / cpr) * cpr;
            int4 xv[M];
#pragma unroll
            for (int t = 0; t < M; t++) xv[t] = sx4[(t < nm ? t : 0) * cpr + p];
            dot_store(j, xv);
        }
    }
    __syncthreads();
    if (er < rows_here && et < nm) {
        const int *pp = part + (er * M + et) * (nb + 1);
        const float *xs = sxs + et * nb;
        float dot = 0.0f;
#pragma unroll 8
        for (int g = 0; g < nb; g++) dot += (float)pp[g] * xs[g];
        float sum = 0.0f;
        sum += dot * wsv;
        out[(size_t)s_orow[et] * out_stride + row0 + er] = sum;
        if (acc_out)
            for (int g = 0; g < nb; g++) acc_out[((size_t)et * acc_rows + row0 + er) * nb + g] = pp[g];
    }
}

template <int M, int PJ>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv_q8(GemvBatch batch) {
    extern __shared__ __align__(16) char smem[];
    __shared__ int s_row[M];
    __shared__ float s_inv[M], tab[32];
    int blk = blockIdx.x, j = 0;
    while (j + 1 < batch.n && blk >= batch.job[j + 1].tile0) j++;
    const GemvJob &job = batch.job[j];
    const int row0 = (blk - job.tile0) * job.R;
    const int rows_here = imin(job.R, job.rows - row0);
    if (threadIdx.x < M) s_row[threadIdx.x] = threadIdx.x;
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) xrow[t] = t;
    gemv_tile<M, PJ>(job.w + (size_t)row0 * job.in_dim, job.ws, rows_here, job.in_dim, job.pro, job.xq, job.xqs,
                     xrow, s_row, M, blk == 0, job.out, job.out_stride, row0, job.acc_out, job.rows, smem, s_inv,
                     tab);
}

// Grouped expert GEMV: block -> (projection jb, group gi, tile).  Group gi
// is one distinct expert of the chunk with its member (token, slot) pairs;
// its weight rows stream once for all members.  Output row = pair.
template <int M, int PJ>
__global__ __launch_bounds__(GEMV_THREADS) void k_expert_gemv(ExpertJob j0, ExpertJob j1,
                                                              const MoeGroups *__restrict__ grp,
                                                              int max_groups, int in_dim, int out_rows, int R,
                                                              int tiles) {
    extern __shared__ __align__(16) char smem[];
    __shared__ int s_orow[M];
    __shared__ float s_inv[M], tab[32];
    const int per_job = max_groups * tiles;
    const int jb = blockIdx.x / per_job;
    const int rem = blockIdx.x - jb * per_job;
    const int gi = rem / tiles;
    const int tile = rem - gi * tiles;
    const ExpertJob &J = jb == 0 ? j0 : j1;
    const int ng = grp->n_groups;
    if (gi >= ng) return;
    const int e = grp->expert[gi];
    const int nm = grp->n_members[gi];
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) {
        const int mem = grp->member[gi][t < nm ? t : 0];
        xrow[t] = J.xq_by_pair ? mem : grp->pair_token[mem];
        if (threadIdx.x == t) s_orow[t] = mem;
    }
    const int row0 = tile * R;
    gemv_tile<M, PJ>(J.q + ((size_t)e * out_rows + row0) * in_dim, J.s + (size_t)e * out_rows,
                             imin(R, out_rows - row0), in_dim, J.pro, J.xq, J.xqs, xrow, s_orow, nm, false, J.out,
                             out_rows, row0, nullptr, 0, smem, s_inv, tab);
}

// ------------------------------------------------------------ KDA conv ---

// Depthwise causal conv (K taps) + SiLU over the [q | k | v] channels, one
// thread per channel, token-serial along the state ring
// (lz_causal_conv1d_step, src/ops_conv1d.c:26-87; ring slots
// src/forward_kda.c:680-755).
template <int K>
__global__ __launch_bounds__(256) void k_kda_conv(const float *__restrict__ pq, const float *__restrict__ pk,
                                                  const float *__restrict__ pv, int key, int value,
                                                  const float *__restrict__ wconv,
                                                  float *__restrict__ conv_ring, size_t slot_stride,
                                                  const int *__restrict__ ctl_slot, int depth, int advance,
                                                  int nt, float *__restrict__ qc, float *__restrict__ kc,
                                                  float *__restrict__ vc) {
    EXP_TAB_LOAD(tab);
    constexpr int hist = K - 1;
    const int conv_dim = 2 * key + value;
    const int c = imin(blockIdx.x * blockDim.x + threadIdx.x, conv_dim - 1);   // extra lanes redo the last channel, store nothing
    const bool live = blockIdx.x * blockDim.x + threadIdx.x < conv_dim;
    const float *in;
    float *out;
    int ch, width;
    if (c < key) { in = pq; out = qc; ch = c; width = key; }
    else if (c < 2 * key) { in = pk; out = kc; ch = c - key; width = key; }
    else { in = pv; out = vc; ch = c - 2 * key; width = value; }
    float h[hist > 0 ? hist : 1], wr[K], xs[MAX_CHUNK];
#pragma unroll
    for (int j = 0; j < K; j++) wr[j] = wconv[(size_t)c * K + j];
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) xs[t] = in[(size_t)imin(t, nt - 1) * width + ch];
    const int base = *ctl_slot;
    const float *st0 = conv_ring + (size_t)base * slot_stride + (size_t)c * hist;
#pragma unroll
    for (int j = 0; j < hist; j++) h[j] = st0[j];
    EXP_TAB_PUT(tab);
    __syncthreads();
    if (!live) return;
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        if (t < nt) {
            const float xv = xs[t];
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < hist; j++) sum += wr[j] * h[j];
            sum += wr[hist] * xv;
            out[(size_t)t * width + ch] = d_silu(sum, tab);
#pragma unroll
            for (int j = 0; j + 1 < hist; j++) h[j] = h[j + 1];
            if (hist > 0) h[hist - 1] = xv;
            int so;
            if (advance) { int si = (base + t) % depth; so = si + 1 == depth ? 0 : si + 1; }
            else so = base;
            if (advance || t == nt - 1) {
                float *st = conv_ring + (size_t)so * slot_stride + (size_t)c * hist;
#pragma unroll
                for (int j = 0; j < hist; j++) st[j] = h[j];
            }
        }
    }
}

// ------------------------------------------------------ KDA recurrence ---
//
// One block per value head; lane j owns column j of the fp32 state S[kd][vd]
// (registers).  Per token: l2norm(q)*scale, l2norm(k), beta, the
// per-channel decay gate, u = S^T(g.k), w = S^T(g.q), kq = k.q,
// delta = (v - u)*beta, out = w + delta*kq, S' = g.S + k(x)delta
// (lz_recur_step fp32 arm, src/ops_gdn.c:2516-2560; gate build
// src/forward_kda.c:277-300, 840-850; call site :856-940), every state
// written to its ring slot as the reference does; then the per-head gated
// RMSNorm and the per-32 quantization for o_proj (src/forward_kda.c:
// 1000-1043).  Everything that does not depend on the state (inputs, gates,
// the three serial norms' sums, k.q) is computed for all tokens at once,
// token-parallel; only u, w and the state update run token-serially.
template <int KD, int VD>
__global__ __launch_bounds__(VD) void k_kda_recur(KdaRecurArgs a) {
    static_assert(KD == VD, "one lane per state column and per key channel");
    EXP_TAB_LOAD(tab);
    __shared__ __align__(16) float s_a[MAX_CHUNK][KD];   // q, then q.g*invq*scale (qcw)
    __shared__ __align__(16) float s_b[MAX_CHUNK][KD];   // k, then k*invk (kn)
    __shared__ __align__(16) float s_g[MAX_CHUNK][KD];   // decay gate
    __shared__ __align__(16) float s_c[MAX_CHUNK][KD];   // q^2, then kn*g (kcw), then o^2
    __shared__ __align__(16) float s_d[MAX_CHUNK][KD];   // k^2
    __shared__ float s_invq[MAX_CHUNK], s_invk[MAX_CHUNK], s_beta[MAX_CHUNK], s_kq[MAX_CHUNK],
        s_oinv[MAX_CHUNK];
    const int h = blockIdx.x;
    const int j = threadIdx.x;
    const int nt = a.nt;
    const int kh = (a.nk == a.nv) ? h : (h * a.nk / a.nv);
    const size_t head_off = (size_t)h * KD * VD;
    // token inputs first (independent of the ring slot), then the state
    float vcv[MAX_CHUNK], gzv[MAX_CHUNK], qv[MAX_CHUNK], kv[MAX_CHUNK], pre[MAX_CHUNK];
    const float dtb = a.dt_bias[h * KD + j];
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        const int tc = imin(t, nt - 1);
        qv[t] = a.qc[(size_t)tc * a.key + (size_t)kh * KD + j];
        kv[t] = a.kc[(size_t)tc * a.key + (size_t)kh * KD + j];
        pre[t] = a.gate_pre[(size_t)tc * a.nv * KD + (size_t)h * KD + j];
        vcv[t] = a.vc[(size_t)tc * a.value + (size_t)h * VD + j];
        gzv[t] = a.gz[(size_t)tc * a.value + (size_t)h * VD + j];
    }
    const float bv = a.bvec[(size_t)imin(j, nt - 1) * a.nv + h];
    const float onw = a.o_norm[j];
    const float alog = a.a_log[h];
    const int base = *a.ctl_slot;
    float S[KD];
    {
        const float *src = a.state + (size_t)base * a.slot_stride + head_off;
#pragma unroll
        for (int i = 0; i < KD; i++) S[i] = src[(size_t)i * VD + j];
    }
    EXP_TAB_PUT(tab);
    __syncthreads();
    const float decay = d_exp(alog, tab);
    // rows t >= nt hold the last token's values and are never read
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        s_a[t][j] = qv[t];
        s_b[t][j] = kv[t];
        s_c[t][j] = qv[t] * qv[t];
        s_d[t][j] = kv[t] * kv[t];
        const float p = pre[t] + dtb;
        const float gg = -decay * d_softplus(p, tab);
        s_g[t][j] = d_exp(gg, tab);
    }
    __syncthreads();
    if (j < nt) {                        // lane t: the token's serial norms and k.q
        const int t = j;
        const float invq = d_rsqrt(serial_sum_n<KD>(s_c[t]) + 1e-6f);
        const float invk = d_rsqrt(serial_sum_n<KD>(s_d[t]) + 1e-6f);
        float kq = 0.0f;
        for (int i = 0; i < KD; i++) {
            const float qn = s_a[t][i] * invq * a.scale;
            const float kn = s_b[t][i] * invk;
            kq += kn * qn;
        }
        s_invq[t] = invq;
        s_invk[t] = invk;
        s_kq[t] = kq;
        s_beta[t] = d_sigmoid(bv, tab);
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        if (t < nt) {
            const float g = s_g[t][j];
            const float qn = s_a[t][j] * s_invq[t] * a.scale;
            const float kn = s_b[t][j] * s_invk[t];
            s_a[t][j] = qn * g;
            s_b[t][j] = kn;
            s_c[t][j] = kn * g;
        }
    }
    __syncthreads();
    float ov[MAX_CHUNK];
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        ov[t] = 0.0f;
        if (t < nt) {
            float u = 0.0f, w = 0.0f;
#pragma unroll
            for (int i = 0; i < KD; i++) {
                u += S[i] * s_c[t][i];
                w += S[i] * s_a[t][i];
            }
            u = (vcv[t] - 1.0f * u) * s_beta[t];
            const float o = 1.0f * w + u * s_kq[t];
#pragma unroll
            for (int i = 0; i < KD; i++) S[i] = S[i] * s_g[t][i] + s_b[t][i] * u;
            if (a.advance || t == nt - 1) {
                int so;
                if (a.advance) { int si = (base + t) % a.depth; so = si + 1 == a.depth ? 0 : si + 1; }
                else so = base;
                float *dst = a.state + (size_t)so * a.slot_stride + head_off;
#pragma unroll
                for (int i = 0; i < KD; i++) dst[(size_t)i * VD + j] = S[i];
            }
            if (a.raw_out) a.raw_out[(size_t)t * a.value + (size_t)h * VD + j] = o;
            ov[t] = o;
        }
    }
    __syncthreads();                     // every lane is done reading s_c
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++)
        if (t < nt) s_c[t][j] = ov[t] * ov[t];
    __syncthreads();
    if (j < nt) s_oinv[j] = d_rsqrt(d_ss_over_n(serial_sum_n<VD>(s_c[j]), VD) + a.eps);
    __syncthreads();
    // gated RMSNorm over the head: ((o*inv)*w)*silu(g)  (src/ops_norm.c:749-793)
    const int col = h * VD + j;
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        if (t < nt) {
            const float y = ov[t] * s_oinv[t] * onw * d_silu(gzv[t], tab);
            if (a.normed_out) a.normed_out[(size_t)t * a.value + col] = y;
            d_quant_group32(y, a.xq + (size_t)t * a.value + col, a.xqs + (size_t)t * (a.value >> 5) + (col >> 5));
        }
    }
}

// ------------------------------------------------------------ attention ---

// One 64-lane block per (token, head): RMSNorm(1+w) of a q head (read from
// the interleaved [q | gate] projection) or a k head, NeoX rotary on the
// first rot dims, then q to qh or k quantized per 32 into the KV plane at
// slot pos; the last nkv blocks of a token quantize v heads.
// (attn_impl src/forward_attn.c:878-960; lz_rope src/ops_rope.c:21-67.)
__global__ __launch_bounds__(64) void k_attn_prep(AttnArgs a) {
    __shared__ __align__(16) float sh[256], sq[256];
    __shared__ float s_inv;
    const int nq = a.kv_only ? 0 : a.nh;
    const int per_tok = nq + 2 * a.nkv;
    const int t = blockIdx.x / per_tok;
    const int hh = blockIdx.x - t * per_tok;
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

// Attention of the chunk's tokens against the Q8 KV cache, in two kernels
// (attn_score_loop Q8 branch, src/forward_attn.c:206-660; score_q8_row
// :30-41; lz_softmax src/ops_norm.c:903-990; wsum_q8_row :17-21).
//
// k_attn_scores: one block per (64-position slice, kv head, token).  The
// block prepares what it needs itself: the kv_mul q heads of the token
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

__global__ __launch_bounds__(256) void k_attn_scores(AttnArgs a, float *__restrict__ att, int att_stride) {
    __shared__ __align__(16) float s_x[ATT_MAX_VEC * ATT_MAX_HD];     // vectors being prepared
    __shared__ __align__(16) float s_sq[ATT_MAX_VEC * (ATT_MAX_HD + 4)];
    __shared__ float s_inv[ATT_MAX_VEC];
    __shared__ __align__(16) int8_t s_k[ATT_SLICE * (ATT_MAX_HD + 16)];   // K rows, padded
    __shared__ float s_ks[ATT_SLICE * (ATT_MAX_HD / 32)];
    const int slice = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
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
    for (int base = 0; base < ATT_MAX_VEC * ATT_MAX_HD; base += 256) {
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

// k_attn_av: one block of 8 waves per (q head, token).  Softmax over the
// token's scores (max, exp, serial sum, scale), then the value sum
// out[d] = sum_p a[p] * v[p][d] * vs[p][d/32] walked in position order by
// one lane per d.  The V rows of up to `sc` positions are staged in LDS
// with every load in flight; the products (a*v)*vs of 64 positions at a
// time are formed by the producer waves into a double buffer [d][64] while
// the consumer lanes (hd/64 waves) add the previous 64 in order, so the
// consumer's loop is one LDS read per four adds.  Then the sigmoid output
// gate and the per-32 quantization of the head's output (the o_proj input).
#define AV_CH 64
#define AV_PAD 68                        // floats per d row of the product buffer (bank spread)

// Stages V rows [p0, p0 + n) of kv head kvh (hd int8 + hd/32 scales each)
// into LDS with every load of the block in flight before the first store
// (n * hd / 16 <= AV_THREADS * AV_STAGE_MAX).
#define AV_THREADS 512
#define AV_STAGE_MAX 16
__device__ __forceinline__ void av_stage(const int8_t *__restrict__ vc, const float *__restrict__ vs, int kv_dim,
                                         int kvh, int hd, int p0, int n, int8_t *s_v, float *s_vs) {
    const int tid = threadIdx.x, cpr = hd >> 4, nb = hd >> 5;
    const int total = n * cpr, stotal = n * nb;
    int4 r[AV_STAGE_MAX];
    float q[AV_STAGE_MAX / 2];
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX; u++) {
        const int idx = imin(u * AV_THREADS + tid, total - 1);
        const int row = idx / cpr, c = idx - row * cpr;
        r[u] = *reinterpret_cast<const int4 *>(vc + (size_t)(p0 + row) * kv_dim + kvh * hd + c * 16);
    }
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX / 2; u++) {
        const int sidx = imin(u * AV_THREADS + tid, stotal - 1);
        const int srow = sidx / nb, g = sidx - srow * nb;
        q[u] = vs[(size_t)(p0 + srow) * (kv_dim >> 5) + kvh * nb + g];
    }
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX; u++)
        if (u * AV_THREADS < total) reinterpret_cast<int4 *>(s_v)[imin(u * AV_THREADS + tid, total - 1)] = r[u];
#pragma unroll
    for (int u = 0; u < AV_STAGE_MAX / 2; u++)
        if (u * AV_THREADS < stotal) s_vs[imin(u * AV_THREADS + tid, stotal - 1)] = q[u];
}

__global__ __launch_bounds__(AV_THREADS) void k_attn_av(AttnArgs a, const float *__restrict__ att, int att_stride,
                                                 int sc) {
    EXP_TAB_LOAD(tab);
    extern __shared__ __align__(16) char smem[];
    __shared__ uint32_t s_red[AV_THREADS / 64];
    __shared__ float s_inv;
    const int h = blockIdx.x, t = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int hd = a.hd, nb = hd >> 5, kv_mul = a.nh / a.nkv, kvh = h / kv_mul;
    const int pos_t = *a.ctl_pos + a.pos_off + t, L = pos_t + 1;
    const int Lp = (att_stride + 3) & ~3;
    float *s_a = reinterpret_cast<float *>(smem);                                   // [Lp]
    float *prod = s_a + Lp;                                                          // [2][hd][AV_PAD]
    int8_t *s_v = reinterpret_cast<int8_t *>(prod + 2 * hd * AV_PAD);               // [sc][hd]
    float *s_vs = reinterpret_cast<float *>(s_v + (size_t)sc * hd);                  // [sc][nb]
    const float *arow = att + ((size_t)t * a.nh + h) * att_stride;
    const int cpr = hd >> 4;
    // scores -> LDS, then the V stage (its loads wait behind the score loads)
    for (int p = tid; p < L; p += AV_THREADS) s_a[p] = arow[p];
    av_stage(a.vcache, a.vscale, a.kv_dim, kvh, hd, 0, imin(sc, L), s_v, s_vs);
    EXP_TAB_PUT(tab);
    __syncthreads();
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
    for (int p = tid; p < L; p += AV_THREADS) s_a[p] = d_exp(s_a[p] - mx, tab);
    __syncthreads();
    if (tid == 0) {
        const float sum = serial_sum(s_a, L);
        s_inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
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
            av_stage(a.vcache, a.vscale, a.kv_dim, kvh, hd, sp0, nsc, s_v, s_vs);
            __syncthreads();
        }
        const int nch = (nsc + AV_CH - 1) / AV_CH;
        if (!cons) produce(sp0, sp0, nsc, 0);
        __syncthreads();
        for (int c = 0; c < nch; c++) {
            if (cons) {
                if (d < hd) {
                    const float *pr = prod + (size_t)(c & 1) * hd * AV_PAD + (size_t)d * AV_PAD;
#pragma unroll
                    for (int i = 0; i < AV_CH; i += 4) {
                        const float4 q = *reinterpret_cast<const float4 *>(pr + i);
                        o += q.x; o += q.y; o += q.z; o += q.w;
                    }
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

// ----------------------------------------------------------------- MoE ---

// Routing for every token of the chunk (lz_moe_route, src/ops_moe.c:12-163:
// sigmoid scores, key = score + bias for selection only, repeated
// strict-greater argmax so the lowest index wins ties, weights renormalized
// by their serial sum).  The k-th pick of that loop is the expert whose key
// has rank k in the order (key descending, index ascending), so each
// (token, expert) item counts its rank against the token's keys in LDS.
// Then the chunk's distinct experts (a bit set): group g is the g-th
// selected expert in ascending order, its members the (token, slot) pairs
// that picked it, in pair order (route_group).  Every block of the expert
// launch computes the same tables from the same router logits, so the
// experts' weights need no separate routing launch.  GEMV_THREADS threads;
// nt * E <= 4 * GEMV_THREADS.  Contains block barriers.
struct __align__(16) RouteLds {
    float key[MAX_CHUNK][MAX_EXPERTS];
    float sc[MAX_CHUNK][MAX_EXPERTS];
    __align__(16) int sel[MAX_PAIRS];
    float w[MAX_PAIRS];
    unsigned long long present[2];       // selected experts, one bit each
    int ng;                              // distinct experts
};

__device__ __forceinline__ void route_block(const float *__restrict__ logits, const float *__restrict__ bias, int E,
                                            int topk, int nt, RouteLds &R, float *tab) {
    const int tid = threadIdx.x;
    const float tabv = c_exp_tab[tid & 31];
    float lg[4], bs[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = imin(u * GEMV_THREADS + tid, nt * E - 1);
        const int t = idx / E, i = idx - t * E;
        lg[u] = logits[(size_t)t * E + i];
        bs[u] = bias[i];
    }
    if (tid < MAX_PAIRS) R.sel[tid] = -1;
    if (tid < 32) tab[tid] = tabv;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = u * GEMV_THREADS + tid;
        if (idx < nt * E) {
            const int t = idx / E, i = idx - t * E;
            const float sc = d_sigmoid(lg[u], tab);
            const float kv = sc + bs[u];
            R.sc[t][i] = sc;
            R.key[t][i] = kv == 0.0f ? 0.0f : kv;      // -0 and +0 compare equal in the reference
        }
    }
    __syncthreads();
    // the token's keys are read 16 at a time (all reads in flight) and
    // compared in registers
    for (int idx = tid; idx < nt * E; idx += GEMV_THREADS) {
        const int t = idx / E, i = idx - t * E;
        const float ki = R.key[t][i];
        int rank = 0;
        for (int j0 = 0; j0 < E; j0 += 16) {
            float4 kq[4];
#pragma unroll
            for (int u = 0; u < 4; u++) kq[u] = *reinterpret_cast<const float4 *>(&R.key[t][j0 + 4 * u]);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float kk[4] = {kq[u].x, kq[u].y, kq[u].z, kq[u].w};
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int jj = j0 + 4 * u + v;
                    rank += (jj < E && (kk[v] > ki || (kk[v] == ki && jj < i))) ? 1 : 0;
                }
            }
        }
        if (rank < topk) R.sel[t * topk + rank] = i;
    }
    __syncthreads();
    if (tid < nt) {                      // weights renormalized by their serial sum
        const int t = tid;
        int ek[MAX_TOPK];
        float sk[MAX_TOPK];
#pragma unroll
        for (int k = 0; k < MAX_TOPK; k++) ek[k] = R.sel[t * topk + imin(k, topk - 1)];
#pragma unroll
        for (int k = 0; k < MAX_TOPK; k++) sk[k] = R.sc[t][ek[k] >= 0 ? ek[k] : 0];
        float wsum = 0.0f;
#pragma unroll
        for (int k = 0; k < MAX_TOPK; k++)
            if (k < topk && ek[k] >= 0) wsum += sk[k];
#pragma unroll
        for (int k = 0; k < MAX_TOPK; k++) {
            float w = ek[k] >= 0 ? sk[k] : 0.0f;
            if (ek[k] >= 0 && wsum > 0.0f) w /= wsum;
            if (k < topk) R.w[t * topk + k] = w;
        }
    }
    // distinct experts, ascending: wave 0 holds pair p's expert in lane p
    // (nt * topk <= 64) and ORs the one-hot expert bits across the wave
    if (tid < 64) {
        const int np = nt * topk;
        const int ep = tid < np ? R.sel[tid] : -1;
        unsigned long long lo = (ep >= 0 && ep < 64) ? 1ull << ep : 0ull;
        unsigned long long hi = (ep >= 64) ? 1ull << (ep - 64) : 0ull;
        for (int o = 32; o > 0; o >>= 1) {
            lo |= __shfl_xor(lo, o);
            hi |= __shfl_xor(hi, o);
        }
        if (tid == 0) {
            R.present[0] = lo;
            R.present[1] = hi;
            R.ng = __popcll(lo) + __popcll(hi);
        }
    }
    __syncthreads();
}

// Expert of distinct group gi (the gi-th selected expert in ascending
// order) and its member pairs in pair order (a wave-uniform scan; call from
// whole waves).  Returns the member count; mem[m] for m < count.
__device__ __forceinline__ int route_group(const RouteLds &R, int nt, int topk, int gi, int *e_out,
                                           int (&mem)[MAX_CHUNK]) {
    unsigned long long lo = R.present[0], hi = R.present[1];
    const int nlo = __popcll(lo);
    int e;
    if (gi < nlo) {
        for (int k = 0; k < gi; k++) lo &= lo - 1ull;
        e = __builtin_ctzll(lo);
    } else {
        for (int k = 0; k < gi - nlo; k++) hi &= hi - 1ull;
        e = 64 + __builtin_ctzll(hi);
    }
    const int lane = threadIdx.x & 63, np = nt * topk;
    unsigned long long m = __ballot(lane < np && R.sel[lane < np ? lane : 0] == e);
    int cnt = 0;
#pragma unroll
    for (int k = 0; k < MAX_CHUNK; k++) {
        mem[k] = m ? __builtin_ctzll(m) : (k ? mem[k - 1] : 0);
        if (m) { cnt++; m &= m - 1ull; }
    }
    *e_out = e;
    return cnt;
}

// Routed experts' first projections (w1 and w3 over the latent rows) with
// the routing computed in the block: block -> (projection jb, group gi,
// tile).  Group gi is one distinct expert of the chunk; its weight rows
// stream once for all of its member (token, slot) pairs.  Output row =
// pair.  Block 0 also publishes the routing (sel_idx, sel_w, the group
// table and the distinct-expert tally) for the down projection and the
// combine.
template <int M, int PJ>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_up(ExpertJob j0, ExpertJob j1, const float *__restrict__ logits,
                                                         const float *__restrict__ bias, int E, int topk, int nt,
                                                         int *__restrict__ sel_idx, float *__restrict__ sel_w,
                                                         MoeGroups *__restrict__ grp, int *__restrict__ tally,
                                                         int max_groups, int in_dim, int out_rows, int R, int tiles) {
    extern __shared__ __align__(16) char smem[];
    __shared__ RouteLds rt;
    __shared__ int s_orow[M];
    __shared__ float s_inv[M], tab[32];
    const int per_job = max_groups * tiles;
    const int jb = blockIdx.x / per_job;
    const int rem = blockIdx.x - jb * per_job;
    const int gi = rem / tiles;
    const int tile = rem - gi * tiles;
    route_block(logits, bias, E, topk, nt, rt, tab);
    const int ng = rt.ng;
    if (blockIdx.x == 0) {                 // publish the routing
        const int tid = threadIdx.x;
        if (tid < nt * topk) {
            sel_idx[tid] = rt.sel[tid];
            sel_w[tid] = rt.w[tid];
            grp->pair_token[tid] = tid / topk;
        }
        if (tid < E) {                     // thread e: its group slot and members, in pair order
            const int e = tid;
            const unsigned long long word = rt.present[e >> 6], bit = 1ull << (e & 63);
            if (word & bit) {
                const int g = __popcll(word & (bit - 1ull)) + ((e >> 6) ? __popcll(rt.present[0]) : 0);
                int cnt = 0;
                for (int p = 0; p < nt * topk; p++)
                    if (rt.sel[p] == e && cnt < MAX_CHUNK) grp->member[g][cnt++] = p;
                grp->expert[g] = e;
                grp->n_members[g] = cnt;
            }
        }
        if (tid == 0) {
            grp->n_groups = ng;
            if (tally) *tally += ng;
        }
    }
    if (gi >= ng) return;
    const ExpertJob &J = jb == 0 ? j0 : j1;
    int e, gmem[MAX_CHUNK];
    const int nm = route_group(rt, nt, topk, gi, &e, gmem);
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) {
        const int mem = gmem[t < nm ? t : 0];
        xrow[t] = J.xq_by_pair ? mem : mem / topk;
        if (threadIdx.x == t) s_orow[t] = mem;
    }
    const int row0 = tile * R;
    gemv_tile<M, PJ>(J.q + ((size_t)e * out_rows + row0) * in_dim, J.s + (size_t)e * out_rows,
                             imin(R, out_rows - row0), in_dim, J.pro, J.xq, J.xqs, xrow, s_orow, nm, false, J.out,
                             out_rows, row0, nullptr, 0, smem, s_inv, tab);
}

// -------------------------------------------------------- argmax / ctl ---

#define ARGMAX_BLOCKS 64
#define LZ_ARGMAX_ROWS 8

// Per row argmax, ARGMAX_BLOCKS blocks per row; the last block to finish a
// row reduces the partials and resets the row's counter (so the kernel can
// be replayed from a graph).  mode 0: order-preserving key, first index wins
// (sample_argmax, src/sampler.c:121-137).  mode 1: float '>' compare, first
// index wins (lz_argmax_p1's scan, src/sampler.c:139-155).
__global__ __launch_bounds__(256) void k_argmax(const float *__restrict__ x, int n, int mode,
                                                unsigned long long *__restrict__ partial,
                                                unsigned *__restrict__ counter, int *__restrict__ out) {
    const int row = blockIdx.y, nb = gridDim.x;
    const float *r = x + (size_t)row * n;
    const int seg = (n + nb - 1) / nb;
    const int lo = blockIdx.x * seg, hi = lo + seg < n ? lo + seg : n;
    unsigned long long best = 0;
    for (int i = lo + threadIdx.x; i < hi; i += blockDim.x) {
        float v = r[i];
        uint32_t k;
        if (mode == 0) k = d_fkey(v);
        else k = (v != v) ? 0u : d_fkey(v == 0.0f ? 0.0f : v);
        unsigned long long cand = ((unsigned long long)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
        best = cand > best ? cand : best;
    }
    best = wave_max_u64(best);
    __shared__ unsigned long long sb[4];
    __shared__ bool s_last;
    if ((threadIdx.x & 63) == 0) sb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) b = sb[i] > b ? sb[i] : b;
        partial[(size_t)row * nb + blockIdx.x] = b;
        __threadfence();
        unsigned prev = atomicAdd(&counter[row], 1u);
        s_last = (prev == (unsigned)nb - 1);
    }
    __syncthreads();
    if (s_last) {
        __threadfence();
        unsigned long long b = 0;
        for (int i = threadIdx.x; i < nb; i += blockDim.x) {
            unsigned long long p = __atomic_load_n(&partial[(size_t)row * nb + i], __ATOMIC_RELAXED);
            b = p > b ? p : b;
        }
        b = wave_max_u64(b);
        if ((threadIdx.x & 63) == 0) sb[threadIdx.x >> 6] = b;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long bb = 0;
            for (int i = 0; i < (int)(blockDim.x >> 6); i++) bb = sb[i] > bb ? sb[i] : bb;
            out[row] = (int)(0xFFFFFFFFu - (uint32_t)(bb & 0xFFFFFFFFu));
            counter[row] = 0;
        }
    }
}

// Acceptance of a greedy round (lz_spec_accept, src/generate.c:232-243) and
// the device-side bookkeeping of lz_spec_round (src/generate.c:802-993):
// ring rollback, mtp_chain reseed from the accepted row, catch-up count,
// next anchor and positions.
__global__ void k_accept(DevCtl *ctl, const float *__restrict__ vhidden, int d,
                         float *__restrict__ chain, int depth, int brk) {
    __shared__ int s_n;
    if (threadIdx.x == 0) {
        int k_eff = ctl->k_eff;
        int n = k_eff;
        for (int i = 0; i < k_eff; i++) {
            ctl->out[i] = ctl->targ[i];
            if (ctl->tok[1 + i] != ctl->targ[i]) { n = i; break; }
        }
        if (n == k_eff) ctl->out[k_eff] = ctl->targ[k_eff];
        ctl->n_accept = n;
        int base = ctl->slot_base;
        int slot = (base + k_eff + 1) % depth;           // what the verify left
        if (n < k_eff && !brk) slot = (base + n + 1) % depth;
        ctl->ssm_slot = slot;
        ctl->new_pos = ctl->anchor_pos + 1 + n;
        // catch-up pairs (verify_hidden[j], out[j]) j < n-1 at mtp_pos+1+j
        ctl->catch_n = n > 1 ? n - 1 : 0;
        ctl->catch_pos = ctl->mtp_pos + 1;
        // Catch-up always runs k-1 rows so a round has a fixed shape; rows
        // j >= catch_n land at MTP positions >= the next round's mtp_pos,
        // which that round's draft steps overwrite before any read.
        for (int j = 0; j < 8; j++) ctl->catch_tok[j] = j < ctl->catch_n ? ctl->out[j] : ctl->out[0];
        ctl->mtp_pos_next = ctl->mtp_pos + n;
        s_n = n;
    }
    __syncthreads();
    const int n = s_n;
    for (int i = threadIdx.x; i < d; i += blockDim.x) chain[i] = vhidden[(size_t)n * d + i];
}

// Round bookkeeping on the device.  op 0: draft input 0 = anchor.  op 1:
// record the finished round in hist and advance to the next one as the
// generation driver does with have_seed (src/generate.c:1850-1866,
// 2096-2104): anchor = out[n_accept] at position new_pos, mtp_pos and the
// ring slot carried over.
__global__ void k_set_tokens(DevCtl *ctl, int op, RoundRec *hist, int hist_cap) {
    if (threadIdx.x != 0) return;
    if (op == 0) {
        ctl->tok[0] = ctl->anchor;
    } else if (op == 1) {
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
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

// Rows per GEMV tile: the tile is at most GEMV_TILE_BYTES of weights and
// R*m (row, token) epilogue pairs fit the block.
static int gemv_rows_per_tile(int in_dim, int m) {
    int r = GEMV_TILE_BYTES / in_dim;
    if (r < 1) r = 1;
    if (r > GEMV_THREADS / m) r = GEMV_THREADS / m;
    return r;
}

template <int M, int PJ>
static hipError_t launch_gemv_mp(const GemvBatch &b, size_t lds, int tiles, hipStream_t st) {
    hipLaunchKernelGGL((k_gemv_q8<M, PJ>), dim3(tiles), dim3(GEMV_THREADS), lds, st, b);
    return hipGetLastError();
}

template <int M>
static hipError_t launch_gemv_m(const GemvBatch &b, size_t lds, int tiles, int pj, hipStream_t st) {
    switch (pj) {
    case 0: return launch_gemv_mp<M, 0>(b, lds, tiles, st);
    case 1: return launch_gemv_mp<M, 1>(b, lds, tiles, st);
    case 2: return launch_gemv_mp<M, 2>(b, lds, tiles, st);
    case 4: return launch_gemv_mp<M, 4>(b, lds, tiles, st);
    default: return launch_gemv_mp<M, 8>(b, lds, tiles, st);
    }
}

// Checks one job's prologue against the kernel's limits.
static bool prologue_ok(const Prologue &P, int in_dim, const int8_t *xq, const float *xqs) {
    if (P.mode == PRO_XQ) return xq && xqs;
    if (in_dim > PRO_MAX_IN || !P.src) return false;
    if (P.mode == PRO_QUANT) return P.src_stride >= in_dim && !(P.src_stride & 3);
    if (P.mode == PRO_SILU) return P.src2 && P.src_stride >= in_dim && !(P.src_stride & 3);
    if (P.mode == PRO_NORM) return P.w && P.src_stride >= in_dim && !(P.src_stride & 3) && !(P.o_stride & 3);
    if (P.mode == PRO_COMBINE) return P.sel_idx && P.sel_w && P.topk >= 1 && P.topk <= MAX_TOPK;
    return false;
}

extern "C" int l98k_gemv(GemvBatch *b, int m, hipStream_t st) {
    if (m < 1 || m > MAX_CHUNK || b->n < 1 || b->n > MAX_GEMV_JOBS) return -1;
    int tiles = 0, pj = 0;
    size_t lds = 0;
    for (int j = 0; j < b->n; j++) {
        GemvJob &J = b->job[j];
        if (J.in_dim < 32 || (J.in_dim & 31) || J.in_dim > GEMV_MAX_IN || J.rows < 1 ||
            !prologue_ok(J.pro, J.in_dim, J.xq, J.xqs))
            return -1;
        J.R = gemv_rows_per_tile(J.in_dim, m);
        J.tile0 = tiles;
        tiles += (J.rows + J.R - 1) / J.R;
        size_t l = gemv_lds_bytes(m, J.in_dim, J.R, J.pro.mode == PRO_NORM);
        lds = l > lds ? l : lds;
        if (J.pro.mode != PRO_XQ) pj = pro_pj(J.in_dim) > pj ? pro_pj(J.in_dim) : pj;
    }
    if (lds > 64 * 1024) return -1;
    switch (m) {
    case 1: return (int)launch_gemv_m<1>(*b, lds, tiles, pj, st);
    case 2: return (int)launch_gemv_m<2>(*b, lds, tiles, pj, st);
    case 3: return (int)launch_gemv_m<3>(*b, lds, tiles, pj, st);
    case 4: return (int)launch_gemv_m<4>(*b, lds, tiles, pj, st);
    case 5: return (int)launch_gemv_m<5>(*b, lds, tiles, pj, st);
    case 6: return (int)launch_gemv_m<6>(*b, lds, tiles, pj, st);
    case 7: return (int)launch_gemv_m<7>(*b, lds, tiles, pj, st);
    default: return (int)launch_gemv_m<8>(*b, lds, tiles, pj, st);
    }
}

// Tiles of a GEMV over `rows` rows of in_dim with m token rows.
extern "C" int l98k_gemv_tiles(int rows, int in_dim, int m) {
    const int R = gemv_rows_per_tile(in_dim, m);
    return (rows + R - 1) / R;
}

// Whether a GEMV over m rows of width in_dim with a fused RMSNorm prologue
// fits the kernel's LDS.
extern "C" int l98k_gemv_norm_fits(int in_dim, int m) {
    if (in_dim > PRO_MAX_IN || m < 1 || m > MAX_CHUNK) return 0;
    return gemv_lds_bytes(m, in_dim, gemv_rows_per_tile(in_dim, m), 1) <= 64 * 1024;
}

// Member slots of a grouped expert launch: a power of two >= nt.
static int expert_m(int nt) { return nt <= 1 ? 1 : nt <= 2 ? 2 : nt <= 4 ? 4 : 8; }

#define EXPERT_DISPATCH(KERNEL, M, PJ, ...)                                              \
    do {                                                                                 \
        switch (M * 16 + PJ) {                                                           \
        case 1 * 16 + 1: hipLaunchKernelGGL((KERNEL<1, 1>), __VA_ARGS__); break;         \
        case 1 * 16 + 2: hipLaunchKernelGGL((KERNEL<1, 2>), __VA_ARGS__); break;         \
        case 1 * 16 + 4: hipLaunchKernelGGL((KERNEL<1, 4>), __VA_ARGS__); break;         \
        case 2 * 16 + 1: hipLaunchKernelGGL((KERNEL<2, 1>), __VA_ARGS__); break;         \
        case 2 * 16 + 2: hipLaunchKernelGGL((KERNEL<2, 2>), __VA_ARGS__); break;         \
        case 2 * 16 + 4: hipLaunchKernelGGL((KERNEL<2, 4>), __VA_ARGS__); break;         \
        case 4 * 16 + 1: hipLaunchKernelGGL((KERNEL<4, 1>), __VA_ARGS__); break;         \
        case 4 * 16 + 2: hipLaunchKernelGGL((KERNEL<4, 2>), __VA_ARGS__); break;         \
        case 4 * 16 + 4: hipLaunchKernelGGL((KERNEL<4, 4>), __VA_ARGS__); break;         \
        case 8 * 16 + 1: hipLaunchKernelGGL((KERNEL<8, 1>), __VA_ARGS__); break;         \
        case 8 * 16 + 2: hipLaunchKernelGGL((KERNEL<8, 2>), __VA_ARGS__); break;         \
        case 8 * 16 + 4: hipLaunchKernelGGL((KERNEL<8, 4>), __VA_ARGS__); break;         \
        default: return -1;                                                              \
        }                                                                                \
    } while (0)

// Both expert launches build their activation rows with a float prologue
// (quantize, or SiLU-mul then quantize) of width <= 1024.
static bool expert_jobs_ok(const ExpertJob *jobs, int n_jobs, int in_dim) {
    if (n_jobs < 1 || n_jobs > 2 || in_dim < 32 || (in_dim & 31) || in_dim > 1024) return false;
    for (int j = 0; j < n_jobs; j++)
        if ((jobs[j].pro.mode != PRO_QUANT && jobs[j].pro.mode != PRO_SILU) ||
            !prologue_ok(jobs[j].pro, in_dim, jobs[j].xq, jobs[j].xqs))
            return false;
    return true;
}

extern "C" int l98k_expert_gemv(const ExpertJob *jobs, int n_jobs, const MoeGroups *grp, int max_groups,
                                int in_dim, int out_rows, int nt, hipStream_t st) {
    if (!expert_jobs_ok(jobs, n_jobs, in_dim) || max_groups < 1 || max_groups > MAX_PAIRS || nt < 1 ||
        nt > MAX_CHUNK)
        return -1;
    const int M = expert_m(nt);
    const int R = gemv_rows_per_tile(in_dim, M);
    const int tiles = (out_rows + R - 1) / R;
    const size_t lds = gemv_lds_bytes(M, in_dim, R, 0);
    if (lds > 64 * 1024) return -1;
    const int pj = pro_pj(in_dim);
    const dim3 grid(n_jobs * max_groups * tiles), blk(GEMV_THREADS);
    const ExpertJob &a = jobs[0], &b2 = n_jobs > 1 ? jobs[1] : jobs[0];
    EXPERT_DISPATCH(k_expert_gemv, M, pj, grid, blk, lds, st, a, b2, grp, max_groups, in_dim, out_rows, R, tiles);
    return (int)hipGetLastError();
}

extern "C" int l98k_moe_up(const ExpertJob *jobs, int n_jobs, const float *logits, const float *bias, int E,
                           int topk, int nt, int *sel_idx, float *sel_w, MoeGroups *grp, int *tally, int in_dim,
                           int out_rows, hipStream_t st) {
    if (E > MAX_EXPERTS || E < topk || topk < 1 || topk > MAX_TOPK || nt < 1 || nt > MAX_CHUNK ||
        nt * topk > MAX_PAIRS || nt * E > 4 * GEMV_THREADS || !expert_jobs_ok(jobs, n_jobs, in_dim))
        return -1;
    const int max_groups = nt * topk < E ? nt * topk : E;
    const int M = expert_m(nt);
    const int R = gemv_rows_per_tile(in_dim, M);
    const int tiles = (out_rows + R - 1) / R;
    const size_t lds = gemv_lds_bytes(M, in_dim, R, 0);
    if (lds > 64 * 1024) return -1;
    const int pj = pro_pj(in_dim);
    const dim3 grid(n_jobs * max_groups * tiles), blk(GEMV_THREADS);
    const ExpertJob &a = jobs[0], &b2 = n_jobs > 1 ? jobs[1] : jobs[0];
    EXPERT_DISPATCH(k_moe_up, M, pj, grid, blk, lds, st, a, b2, logits, bias, E, topk, nt, sel_idx, sel_w, grp, tally,
                    max_groups, in_dim, out_rows, R, tiles);
    return (int)hipGetLastError();
}

extern "C" int l98k_embed(const int8_t *q, const float *s, const int *toks, int d, int nt,
                          float *x, hipStream_t st) {
    hipLaunchKernelGGL(k_embed, dim3((d + 255) / 256, nt), dim3(256), 0, st, q, s, toks, d, x);
    return (int)hipGetLastError();
}

#define NORM_CASES(X) X(1) X(2) X(4) X(8)

extern "C" int l98k_rmsnorm(float *x, int x_stride, const float *a, const float *b, const float *w,
                            int n, float eps, int rows, float *out, int out_stride, int8_t *xq,
                            float *xqs, hipStream_t st) {
    if (n < 32 || n > 256 * 8 || (n & 31) || (x_stride & 3) || (out && (out_stride & 3)) || rows < 1) return -1;
#define NORM_LAUNCH(PJ)                                                                          \
    if (n <= 256 * PJ) {                                                                         \
        hipLaunchKernelGGL(k_rmsnorm<PJ>, dim3(rows), dim3(64), 0, st, x, x_stride, a, b, w, n, \
                           eps, out, out_stride, xq, xqs);                                       \
        return (int)hipGetLastError();                                                           \
    }
    NORM_CASES(NORM_LAUNCH)
#undef NORM_LAUNCH
    return -1;
}

extern "C" int l98k_mtp_pre(const int8_t *emb_q, const float *emb_s, const int *toks, const float *h, int d,
                            const float *w_e, const float *w_h, float eps, int rows, int8_t *xq, float *xqs,
                            hipStream_t st) {
    if (d < 32 || d > 256 * 8 || (d & 31) || rows < 1) return -1;
#define PRE_LAUNCH(PJ)                                                                                  \
    if (d <= 256 * PJ) {                                                                                \
        hipLaunchKernelGGL(k_mtp_pre<PJ>, dim3(rows, 2), dim3(64), 0, st, emb_q, emb_s, toks, h, d, w_e, \
                           w_h, eps, xq, xqs);                                                          \
        return (int)hipGetLastError();                                                                  \
    }
    NORM_CASES(PRE_LAUNCH)
#undef PRE_LAUNCH
    return -1;
}

extern "C" int l98k_kda_conv(const float *pq, const float *pk, const float *pv, int key, int value,
                             const float *wconv, float *ring, size_t slot_stride, int K,
                             const int *ctl_slot, int depth, int advance, int nt, float *qc,
                             float *kc, float *vc, hipStream_t st) {
    if (nt < 1 || nt > MAX_CHUNK) return -1;
    const int n = 2 * key + value;
    const dim3 grid((n + 255) / 256);
    if (K == 4)
        hipLaunchKernelGGL(k_kda_conv<4>, grid, dim3(256), 0, st, pq, pk, pv, key, value, wconv, ring,
                           slot_stride, ctl_slot, depth, advance, nt, qc, kc, vc);
    else if (K == 3)
        hipLaunchKernelGGL(k_kda_conv<3>, grid, dim3(256), 0, st, pq, pk, pv, key, value, wconv, ring,
                           slot_stride, ctl_slot, depth, advance, nt, qc, kc, vc);
    else if (K == 2)
        hipLaunchKernelGGL(k_kda_conv<2>, grid, dim3(256), 0, st, pq, pk, pv, key, value, wconv, ring,
                           slot_stride, ctl_slot, depth, advance, nt, qc, kc, vc);
    else
        return -1;
    return (int)hipGetLastError();
}

extern "C" int l98k_kda_recur(const KdaRecurArgs *a, int kd, int vd, hipStream_t st) {
    if (a->nt < 1 || a->nt > MAX_CHUNK) return -1;
    if (kd == 64 && vd == 64)
        hipLaunchKernelGGL((k_kda_recur<64, 64>), dim3(a->nv), dim3(64), 0, st, *a);
    else if (kd == 128 && vd == 128)
        hipLaunchKernelGGL((k_kda_recur<128, 128>), dim3(a->nv), dim3(128), 0, st, *a);
    else if (kd == 32 && vd == 32)
        hipLaunchKernelGGL((k_kda_recur<32, 32>), dim3(a->nv), dim3(32), 0, st, *a);
    else
        return -1;
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

extern "C" int l98k_attn(const AttnArgs *a, int nt, int max_len, float *att, hipStream_t st) {
    if (a->nkv < 1 || a->nh % a->nkv || (a->hd & 31) || a->hd > ATT_MAX_HD || a->rot > a->hd || (a->rot & 1) ||
        nt < 1 || nt > MAX_CHUNK || max_len < 1 || !a->oq || !a->oqs || !att)
        return -1;
    const int kv_mul = a->nh / a->nkv;
    if (kv_mul + MAX_CHUNK > ATT_MAX_VEC) return -1;
    const int att_stride = (max_len + 3) & ~3;
    const int slices = (max_len + ATT_SLICE - 1) / ATT_SLICE;
    hipLaunchKernelGGL(k_attn_scores, dim3(slices, a->nkv, nt), dim3(256), 0, st, *a, att, att_stride);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    // value-sum kernel: scores, the product double buffer, then as many
    // staged V positions (multiple of 64) as the LDS limit leaves
    const int hd = a->hd;
    const size_t fixed = ((size_t)att_stride + 2 * (size_t)hd * AV_PAD) * sizeof(float);
    const size_t per_pos = (size_t)hd + (size_t)(hd >> 5) * sizeof(float);
    const int lim = lds_limit() - 1024;          // the kernel's static LDS (exp table, reductions) fits in the rest
    if (fixed + AV_CH * per_pos > (size_t)lim) return -1;
    int sc = (int)(((size_t)lim - fixed) / per_pos) & ~(AV_CH - 1);
    const int need = (max_len + AV_CH - 1) & ~(AV_CH - 1);
    if (sc > need) sc = need;
    const int sc_regs = (AV_THREADS * AV_STAGE_MAX / (hd >> 4)) & ~(AV_CH - 1);   // one register-staged pass
    if (sc > sc_regs) sc = sc_regs;
    const size_t lds = fixed + (size_t)sc * per_pos;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_av),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lim);
        attr_set = true;
    }
    hipLaunchKernelGGL(k_attn_av, dim3(a->nh, nt), dim3(AV_THREADS), lds, st, *a, att, att_stride, sc);
    return (int)hipGetLastError();
}

extern "C" int l98k_argmax(const float *x, int n, int rows, int mode, int *out,
                           unsigned long long *partial, unsigned *counter, hipStream_t st) {
    if (rows < 1 || rows > LZ_ARGMAX_ROWS || n < 1) return -1;
    hipLaunchKernelGGL(k_argmax, dim3(ARGMAX_BLOCKS, rows), dim3(256), 0, st, x, n, mode, partial,
                       counter, out);
    return (int)hipGetLastError();
}

extern "C" int l98k_accept(DevCtl *ctl, const float *vhidden, int d, float *chain, int depth,
                           int brk, hipStream_t st) {
    hipLaunchKernelGGL(k_accept, dim3(1), dim3(256), 0, st, ctl, vhidden, d, chain, depth, brk);
    return (int)hipGetLastError();
}

extern "C" int l98k_set_tokens(DevCtl *ctl, int op, RoundRec *hist, int hist_cap, hipStream_t st) {
    hipLaunchKernelGGL(k_set_tokens, dim3(1), dim3(64), 0, st, ctl, op, hist, hist_cap);
    return (int)hipGetLastError();
}

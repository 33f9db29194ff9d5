// Block-diagonal Walsh-Hadamard transforms of rows (the SubLN variant's
// o_proj / down_proj input path), one 256-thread block per row with the row
// staged in LDS:
//   k_fwht_i32   lz_fwht_i32 on each block of a row       src/fwht.c:65-196
//   k_fwht_f32   lz_fwht on each block, optionally times rsqrt(blk)
//                (subn_rot_f32)                          src/fwht.c:198-320,
//                                                        src/forward_kda.c:130-135
//   k_subn_quant subn_fwht_quant: power-of-two fixed point, integer
//                transform, per-group int8 codes        src/forward_kda.c:43-92
// Every stage is the Sylvester butterfly (u + v, u - v) at stride len for
// len = 1, 2, ... blk / 2; blk is a power of two, so applying the stages to
// the whole row is the block-diagonal transform.  The integer transform
// wraps in uint32, as int32 two's complement does.  The float transform
// rounds each add and subtract once, as the serial loop does, and the order
// of butterflies within a stage does not change any value.
#include "l98_dev.h"
#include "l98_devmath.h"

#define FWHT_THREADS 256
#define FWHT_MAX_N 8192

// pow2f, src/ops_quant.c:77-83
__device__ __forceinline__ float d_pow2f(int e) {
    if (e < -126) return 0.0f;
    if (e > 127) e = 127;
    return f_from_u((uint32_t)(e + 127) << 23);
}

template <typename T>
__device__ __forceinline__ void fwht_stages(T *v, int n, int blk) {
    for (int len = 1; len < blk; len <<= 1) {
        for (int p = threadIdx.x; p < (n >> 1); p += FWHT_THREADS) {
            const int i = ((p & ~(len - 1)) << 1) | (p & (len - 1));
            const T a = v[i], b = v[i + len];
            v[i] = a + b;
            v[i + len] = a - b;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(FWHT_THREADS) void k_fwht_i32(const int32_t *__restrict__ x, int32_t *__restrict__ y,
                                                           int n, int blk) {
    __shared__ uint32_t t[FWHT_MAX_N];
    const size_t off = (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) t[i] = (uint32_t)x[off + i];
    __syncthreads();
    fwht_stages(t, n, blk);
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) y[off + i] = (int32_t)t[i];
}

__global__ __launch_bounds__(FWHT_THREADS) void k_fwht_f32(float *__restrict__ v, int n, int blk, int rot) {
    __shared__ float t[FWHT_MAX_N];
    const size_t off = (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) t[i] = v[off + i];
    __syncthreads();
    fwht_stages(t, n, blk);
    const float inv = d_rsqrt((float)blk);
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) v[off + i] = rot ? t[i] * inv : t[i];
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t m, uint32_t *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = umax(m, (uint32_t)__shfl_xor((int)m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = umax(umax(red[0], red[1]), umax(red[2], red[3]));
    return m;
}

// One row of n floats -> n int8 codes and n / 32 scales (each group's scale
// in each of its 32-element slots).  gw: elements per stored scale (n
// unless a multiple of 32 dividing n).
__global__ __launch_bounds__(FWHT_THREADS) void k_subn_quant(const float *__restrict__ x, int n, int blk, int gw,
                                                             int8_t *__restrict__ q, float *__restrict__ s) {
    static const float INV127 = 1.0f / 127.0f;
    __shared__ uint32_t t[FWHT_MAX_N];
    __shared__ int32_t cmax[FWHT_MAX_N / 32];
    __shared__ float gsc[FWHT_MAX_N / 32], ginv[FWHT_MAX_N / 32];
    __shared__ uint32_t red[FWHT_THREADS / 64];
    const size_t off = (size_t)blockIdx.x * n;
    const float *xr = x + off;
    int8_t *qr = q + off;
    float *sr = s + (size_t)blockIdx.x * (n >> 5);

    uint32_t am = 0;
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) am = umax(am, u_from_f(xr[i]) & 0x7FFFFFFFu);
    am = block_max_u32(am, red);
    if (f_from_u(am) <= 0.0f) {                    // an all-zero row: q = 0, s = 1
        for (int i = threadIdx.x; i < n; i += FWHT_THREADS) qr[i] = 0;
        for (int i = threadIdx.x; i < (n >> 5); i += FWHT_THREADS) sr[i] = 1.0f;
        return;
    }
    // S puts the row max in [2^14, 2^15): the transform's outputs stay
    // below blk * 2^15
    const int e = (int)((am >> 23) & 0xFFu) - 127;
    const float S = d_pow2f(14 - e);
    const float inv_S = 1.0f / S;
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) t[i] = (uint32_t)d_q8_round(xr[i] * S);
    __syncthreads();
    fwht_stages(t, n, blk);
    if (gw <= 0 || (gw & 31) != 0 || n % gw != 0) gw = n;
    // |t| maxima of the 32-element chunks, then of the groups
    for (int c = threadIdx.x; c < (n >> 5); c += FWHT_THREADS) {
        int32_t m = 0;
        for (int k = 0; k < 32; k++) {
            const int32_t v = (int32_t)t[32 * c + k];
            const int32_t a = v < 0 ? (int32_t)(0u - (uint32_t)v) : v;
            m = a > m ? a : m;
        }
        cmax[c] = m;
    }
    __syncthreads();
    const float rs = d_rsqrt((float)blk);
    const int cpg = gw >> 5;
    for (int g = threadIdx.x; g < n / gw; g += FWHT_THREADS) {
        int32_t tam = 0;
        for (int c = g * cpg; c < (g + 1) * cpg; c++) tam = cmax[c] > tam ? cmax[c] : tam;
        float scale = (float)tam * inv_S * rs * INV127;
        float inv_q;
        if (tam == 0 || scale < 1.0e-30f) {
            scale = 1.0f;
            inv_q = 0.0f;
        } else {
            inv_q = 127.0f / (float)tam;
        }
        gsc[g] = scale;
        ginv[g] = inv_q;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += FWHT_THREADS) {
        int qv = d_q8_round((float)(int32_t)t[i] * ginv[i / gw]);
        qv = qv > 127 ? 127 : qv;
        qr[i] = (int8_t)(qv < -127 ? -127 : qv);
    }
    for (int c = threadIdx.x; c < (n >> 5); c += FWHT_THREADS) sr[c] = gsc[(c << 5) / gw];
}

static bool fwht_shape_ok(int rows, int n, int blk) {
    return rows >= 1 && n >= 1 && n <= FWHT_MAX_N && blk >= 1 && blk <= n && (blk & (blk - 1)) == 0 &&
           n % blk == 0;
}

extern "C" int l98k_fwht_i32(const int32_t *x, int32_t *y, int rows, int n, int blk, hipStream_t st) {
    if (!x || !y || !fwht_shape_ok(rows, n, blk)) return -1;
    hipLaunchKernelGGL(k_fwht_i32, dim3(rows), dim3(FWHT_THREADS), 0, st, x, y, n, blk);
    return (int)hipGetLastError();
}

extern "C" int l98k_fwht_f32(float *v, int rows, int n, int blk, int rot, hipStream_t st) {
    if (!v || !fwht_shape_ok(rows, n, blk)) return -1;
    hipLaunchKernelGGL(k_fwht_f32, dim3(rows), dim3(FWHT_THREADS), 0, st, v, n, blk, rot ? 1 : 0);
    return (int)hipGetLastError();
}

extern "C" int l98k_subn_quant(const float *x, int rows, int n, int blk, int gw, int8_t *q, float *s,
                               hipStream_t st) {
    if (!x || !q || !s || !fwht_shape_ok(rows, n, blk) || n % 32 != 0) return -1;
    hipLaunchKernelGGL(k_subn_quant, dim3(rows), dim3(FWHT_THREADS), 0, st, x, n, blk, gw, q, s);
    return (int)hipGetLastError();
}

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

// ---------------------------------------------------------------- math ---

__constant__ float c_exp_tab[32];

__device__ __forceinline__ float f_from_u(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t u_from_f(float f) { return __float_as_uint(f); }

// lz_exp_float_body, src/ops_quant.c:300-349
__device__ __forceinline__ float d_exp(float x) {
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
    return p2n * (c_exp_tab[idx] * c);
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
__device__ __forceinline__ float d_sigmoid(float x) {
    if (x >= 0.0f) {
        float z = d_exp(-x);
        return 1.0f / (1.0f + z);
    }
    float z = d_exp(x);
    return z / (1.0f + z);
}
__device__ __forceinline__ float d_silu(float x) { return x * d_sigmoid(x); }

// lz_softplus_poly, src/ops_quant.c:1040-1060
__device__ __forceinline__ float d_softplus(float x) {
    const float L[9] = {1.000000000f, -0.499995530f, 0.333203435f, -0.248529464f,
                        0.191451162f, -0.137466222f, 0.079210736f, -0.030110965f,
                        0.005384062f};
    if (x > 16.0f) return x;
    float nx = (x < 0.0f) ? x : -x;
    float u = d_exp(nx);
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

__device__ __forceinline__ float wave_max_u(uint32_t v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) {
        uint32_t w = __shfl_xor(v, o, width);
        v = w > v ? w : v;
    }
    return f_from_u(v);
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

// Serial left-to-right float sum of n values in LDS (one lane).
__device__ __forceinline__ float serial_sum(const float *v, int n) {
    float ss = 0.0f;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        float4 q = *reinterpret_cast<const float4 *>(v + i);
        ss += q.x; ss += q.y; ss += q.z; ss += q.w;
    }
    for (; i < n; i++) ss += v[i];
    return ss;
}

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

// One 64-lane block per row.  Optionally first folds the residual:
//   x_row = x_row + (a_row [+ b_row])      (the reference's x += xb2 with
//   xb2 = up + shared already summed, src/forward.c:1449-1557,
//   src/forward_moe.c:552)
// then o = (x*inv)*(1+w) (lz_rmsnorm, src/ops_norm.c:690-747) and, when xq
// is given, the per-32 int8 quantization of o.
// LDS: n floats of squares.
__global__ void k_rmsnorm(float *__restrict__ x, int x_stride, const float *__restrict__ a,
                          const float *__restrict__ b, const float *__restrict__ w, int n,
                          float eps, float *__restrict__ out, int out_stride,
                          int8_t *__restrict__ xq, float *__restrict__ xqs) {
    extern __shared__ float sh[];
    int row = blockIdx.x;
    float *xr = x + (size_t)row * x_stride;
    const int lane = threadIdx.x;
    for (int i = lane; i < n; i += 64) {
        float v = xr[i];
        if (a) {
            float add = a[(size_t)row * n + i];
            if (b) add = add + b[(size_t)row * n + i];
            v = v + add;
            xr[i] = v;
        }
        sh[i] = v * v;
    }
    __syncthreads();
    __shared__ float s_inv;
    if (lane == 0) s_inv = d_rsqrt(d_ss_over_n(serial_sum(sh, n), n) + eps);
    __syncthreads();
    float inv = s_inv;
    for (int base = 0; base < n; base += 64) {
        int i = base + lane;
        float o = 0.0f;
        if (i < n) {
            o = xr[i] * inv * (1.0f + w[i]);
            if (out) out[(size_t)row * out_stride + i] = o;
        }
        if (xq && base + (lane & ~31) < n)
            d_quant_group32(o, xq + (size_t)row * n + i, xqs + (size_t)row * (n >> 5) + (i >> 5));
    }
}

// Per-32 quantization of rows (lz_quantize_q8).  block = 64 lanes, one row.
__global__ void k_quant_rows(const float *__restrict__ x, int n, int x_stride,
                             int8_t *__restrict__ xq, float *__restrict__ xqs) {
    int row = blockIdx.x;
    for (int base = 0; base < n; base += 64) {
        int i = base + threadIdx.x;
        if (base + (int)(threadIdx.x & ~31) >= n) break;
        float v = x[(size_t)row * x_stride + i];
        d_quant_group32(v, xq + (size_t)row * n + i, xqs + (size_t)row * (n >> 5) + (i >> 5));
    }
}

// g = silu(h1)*h3 then per-32 quantization (lz_ffn_gate_up default branch,
// src/forward_kda.c:1067-1088, followed by lz_quantize_q8).  Row r reads
// h1/h3 at r*stride; count may come from device memory (rows beyond it
// exit).
__global__ void k_act_quant(const float *__restrict__ h1, const float *__restrict__ h3,
                            int n, const int *__restrict__ count,
                            int8_t *__restrict__ xq, float *__restrict__ xqs,
                            float *__restrict__ g_out) {
    int row = blockIdx.x;
    if (count && row >= *count) return;
    for (int base = 0; base < n; base += 64) {
        int i = base + threadIdx.x;
        if (base + (int)(threadIdx.x & ~31) >= n) break;
        float g = d_silu(h1[(size_t)row * n + i]) * h3[(size_t)row * n + i];
        if (g_out) g_out[(size_t)row * n + i] = g;
        d_quant_group32(g, xq + (size_t)row * n + i, xqs + (size_t)row * (n >> 5) + (i >> 5));
    }
}

// ------------------------------------------------------------- GEMV/q8 ---
//
// o[t][row] = 0.0f + (sum_s float(acc[t,row,s]) * xqs[t][s]) * ws[row]
// with acc the exact int32 sum over each 32-element group
// (lz_matmul_xq_nt -> matmul_q8_impl + epi_q8, src/ops_matmul.c:336-466,
// src/ops_epi.c:983-1017).
//
// One 64-lane block streams a tile of R consecutive rows (R*in <= 8 KiB):
// lane l reads 16-byte chunks l, l+64, ... of the tile, so every 1 KiB of a
// row is one coalesced wave load.  Each chunk's 16-element partial dot
// products for all M tokens go to LDS; then R*M lanes each run one
// (row, token) epilogue, serially over the groups, in the reference order.
// Weights stream from HBM once per launch regardless of M (M <= 8).

template <int M>
__global__ __launch_bounds__(64) void k_gemv_q8(GemvBatch batch, const int8_t *__restrict__ xq_base,
                                                 const float *__restrict__ xqs_base, int in_dim,
                                                 int R) {
    extern __shared__ int part[];               // [R][M][cpr]
    int blk = blockIdx.x, j = 0;
    while (j + 1 < batch.n && blk >= batch.job[j + 1].tile0) j++;
    const GemvJob &job = batch.job[j];
    if (job.count && *job.count <= 0) return;
    const int tile = blk - job.tile0;
    const int row0 = tile * R;
    const int rows = job.rows;
    const int cpr = in_dim >> 4;                // 16-byte chunks per row
    const int nb = in_dim >> 5;
    const int8_t *xq = job.xq ? job.xq : xq_base;
    const float *xqs = job.xqs ? job.xqs : xqs_base;
    const int8_t *w = job.w + (size_t)row0 * in_dim;
    const int nchunk = R * cpr;
    const int lane = threadIdx.x;
    for (int c = lane; c < nchunk; c += 64) {
        int r = c / cpr;
        int p = c - r * cpr;
        int acc[M];
        if (row0 + r < rows) {
            int4 wv = *reinterpret_cast<const int4 *>(w + (size_t)c * 16);
#pragma unroll
            for (int t = 0; t < M; t++) {
                int4 xv = *reinterpret_cast<const int4 *>(xq + (size_t)t * in_dim + p * 16);
                int s0 = __builtin_amdgcn_sdot4(wv.x, xv.x, 0, false);
                s0 = __builtin_amdgcn_sdot4(wv.y, xv.y, s0, false);
                s0 = __builtin_amdgcn_sdot4(wv.z, xv.z, s0, false);
                s0 = __builtin_amdgcn_sdot4(wv.w, xv.w, s0, false);
                acc[t] = s0;
            }
        } else {
#pragma unroll
            for (int t = 0; t < M; t++) acc[t] = 0;
        }
#pragma unroll
        for (int t = 0; t < M; t++) part[(r * M + t) * cpr + p] = acc[t];
    }
    __syncthreads();
    if (lane < R * M) {
        int r = lane / M, t = lane - r * M;
        int row = row0 + r;
        if (row < rows) {
            const int *pp = part + (r * M + t) * cpr;
            const float *xs = xqs + (size_t)t * nb;
            float dot = 0.0f;
            for (int g = 0; g < nb; g++) {
                int a = pp[2 * g] + pp[2 * g + 1];
                dot += (float)a * xs[g];
            }
            float sum = 0.0f;
            sum += dot * job.ws[row];
            job.out[(size_t)t * job.out_stride + row] = sum;
            if (job.acc_out) {
                for (int g = 0; g < nb; g++)
                    job.acc_out[((size_t)t * rows + row) * nb + g] = pp[2 * g] + pp[2 * g + 1];
            }
        }
    }
}

// Grouped expert GEMV: job e = one distinct expert of the chunk with its
// member (token, slot) pairs; activations are the members' own quantized
// rows.  Weight rows stream once per distinct expert.
//   xq rows:   xq_base + member_row * in_dim  (member_row from the group table)
//   output:    out + member_pair * out_rows + row
template <int M>
__global__ __launch_bounds__(64) void k_expert_gemv(const ExpertBank bank, const MoeGroups *__restrict__ grp,
                                                    const int8_t *__restrict__ xq_base,
                                                    const float *__restrict__ xqs_base,
                                                    int xq_by_pair, float *__restrict__ out,
                                                    int in_dim, int out_rows, int R, int tiles) {
    extern __shared__ int part[];
    const int gi = blockIdx.x / tiles;
    const int tile = blockIdx.x - gi * tiles;
    if (gi >= grp->n_groups) return;
    const int e = grp->expert[gi];
    const int nm = grp->n_members[gi];
    const int row0 = tile * R;
    const int cpr = in_dim >> 4;
    const int nb = in_dim >> 5;
    const int8_t *w = bank.q + ((size_t)e * out_rows + row0) * in_dim;
    const float *ws = bank.s + (size_t)e * out_rows;
    const int lane = threadIdx.x;
    const int nchunk = R * cpr;
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) {
        int mem = t < nm ? grp->member[gi][t] : grp->member[gi][0];
        xrow[t] = xq_by_pair ? mem : grp->pair_token[mem];
    }
    for (int c = lane; c < nchunk; c += 64) {
        int r = c / cpr;
        int p = c - r * cpr;
        int acc[M];
        if (row0 + r < out_rows) {
            int4 wv = *reinterpret_cast<const int4 *>(w + (size_t)c * 16);
#pragma unroll
            for (int t = 0; t < M; t++) {
                acc[t] = 0;
                if (t < nm) {
                    int4 xv = *reinterpret_cast<const int4 *>(xq_base + (size_t)xrow[t] * in_dim + p * 16);
                    int s0 = __builtin_amdgcn_sdot4(wv.x, xv.x, 0, false);
                    s0 = __builtin_amdgcn_sdot4(wv.y, xv.y, s0, false);
                    s0 = __builtin_amdgcn_sdot4(wv.z, xv.z, s0, false);
                    s0 = __builtin_amdgcn_sdot4(wv.w, xv.w, s0, false);
                    acc[t] = s0;
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < M; t++) acc[t] = 0;
        }
#pragma unroll
        for (int t = 0; t < M; t++) part[(r * M + t) * cpr + p] = acc[t];
    }
    __syncthreads();
    if (lane < R * M) {
        int r = lane / M, t = lane - r * M;
        int row = row0 + r;
        if (row < out_rows && t < nm) {
            const int *pp = part + (r * M + t) * cpr;
            const float *xs = xqs_base + (size_t)xrow[t] * nb;
            float dot = 0.0f;
            for (int g = 0; g < nb; g++) {
                int a = pp[2 * g] + pp[2 * g + 1];
                dot += (float)a * xs[g];
            }
            float sum = 0.0f;
            sum += dot * ws[row];
            int pair = grp->member[gi][t];
            out[(size_t)pair * out_rows + row] = sum;
        }
    }
}

// ------------------------------------------------------------ KDA conv ---

// Depthwise causal conv (k taps) + SiLU over the [q | k | v] channels, one
// thread per channel, token-serial along the state ring
// (lz_causal_conv1d_step, src/ops_conv1d.c:26-87; ring slots
// src/forward_kda.c:680-755).  proj rows: q at qkv[t], k, v at separate
// strides.
__global__ void k_kda_conv(const float *__restrict__ pq, const float *__restrict__ pk,
                           const float *__restrict__ pv, int key, int value,
                           const float *__restrict__ wconv,      // [conv_dim][K]
                           float *__restrict__ conv_ring, size_t slot_stride, int K,
                           const int *__restrict__ ctl_slot, int depth, int advance, int nt,
                           float *__restrict__ qc, float *__restrict__ kc, float *__restrict__ vc) {
    int c = blockIdx.x * blockDim.x + threadIdx.x;
    int conv_dim = 2 * key + value;
    if (c >= conv_dim) return;
    const int hist = K - 1;
    const float *in;
    float *out;
    int ch, width;
    if (c < key) { in = pq; out = qc; ch = c; width = key; }
    else if (c < 2 * key) { in = pk; out = kc; ch = c - key; width = key; }
    else { in = pv; out = vc; ch = c - 2 * key; width = value; }
    const int base = *ctl_slot;
    float h[8];
    const float *st0 = conv_ring + (size_t)base * slot_stride + (size_t)c * hist;
    for (int j = 0; j < hist; j++) h[j] = st0[j];
    const float *wr = wconv + (size_t)c * K;
    for (int t = 0; t < nt; t++) {
        float xv = in[(size_t)t * width + ch];
        float sum = 0.0f;
        for (int j = 0; j < hist; j++) sum += wr[j] * h[j];
        sum += wr[hist] * xv;
        out[(size_t)t * width + ch] = d_silu(sum);
        for (int j = 0; j + 1 < hist; j++) h[j] = h[j + 1];
        if (hist > 0) h[hist - 1] = xv;
        int so;
        if (advance) { int si = (base + t) % depth; so = si + 1 == depth ? 0 : si + 1; }
        else so = base;
        float *st = conv_ring + (size_t)so * slot_stride + (size_t)c * hist;
        for (int j = 0; j < hist; j++) st[j] = h[j];
    }
}

// ------------------------------------------------------ KDA recurrence ---
//
// One block per value head; lane j owns column j of the fp32 state S[kd][vd]
// (registers).  Per token, serially: l2norm(q)*scale, l2norm(k), beta,
// the per-channel decay gate, u = S^T(g.k), w = S^T(g.q), kq = k.q,
// delta = (v - u)*beta, out = w + delta*kq, S' = g.S + k(x)delta
// (lz_recur_step fp32 arm, src/ops_gdn.c:2516-2560; gate build
// src/forward_kda.c:277-300, 840-850; call site :856-940), with every
// state written to its ring slot as the reference does.  Then the per-head
// gated RMSNorm and the per-32 quantization for o_proj
// (src/forward_kda.c:1000-1043).
template <int KD, int VD>
__global__ __launch_bounds__(VD) void k_kda_recur(KdaRecurArgs a) {
    __shared__ float s_q[KD], s_k[KD], s_g[KD], s_o[VD];
    const int h = blockIdx.x;
    const int j = threadIdx.x;
    const int kh = (a.nk == a.nv) ? h : (h * a.nk / a.nv);
    const int base = *a.ctl_slot;
    const size_t head_off = (size_t)h * KD * VD;
    float S[KD];
    {
        const float *src = a.state + (size_t)base * a.slot_stride + head_off;
#pragma unroll
        for (int i = 0; i < KD; i++) S[i] = src[(size_t)i * VD + j];
    }
    const float decay = d_exp(a.a_log[h]);
    for (int t = 0; t < a.nt; t++) {
        // stage q, k, gate for this head/token
        for (int i = j; i < KD; i += VD) {
            s_q[i] = a.qc[(size_t)t * a.key + (size_t)kh * KD + i];
            s_k[i] = a.kc[(size_t)t * a.key + (size_t)kh * KD + i];
            float pre = a.gate_pre[(size_t)t * a.nv * KD + (size_t)h * KD + i] + a.dt_bias[h * KD + i];
            float gg = -decay * d_softplus(pre);
            s_g[i] = d_exp(gg);
        }
        __syncthreads();
        // l2 norms (every lane walks the same serial sums)
        float ssq = 0.0f, ssk = 0.0f;
        for (int i = 0; i < KD; i++) ssq += s_q[i] * s_q[i];
        for (int i = 0; i < KD; i++) ssk += s_k[i] * s_k[i];
        const float invq = d_rsqrt(ssq + 1e-6f), invk = d_rsqrt(ssk + 1e-6f);
        const float beta = d_sigmoid(a.bvec[(size_t)t * a.nv + h]);
        float u = 0.0f, w = 0.0f, kq = 0.0f;
#pragma unroll 8
        for (int i = 0; i < KD; i++) {
            float qn = s_q[i] * invq * a.scale;
            float kn = s_k[i] * invk;
            float kcw = kn * s_g[i], qcw = qn * s_g[i];
            kq += kn * qn;
            u += S[i] * kcw;
            w += S[i] * qcw;
        }
        const float vcv = a.vc[(size_t)t * a.value + (size_t)h * VD + j];
        u = (vcv - 1.0f * u) * beta;
        float o = 1.0f * w + u * kq;
#pragma unroll 8
        for (int i = 0; i < KD; i++) {
            float kn = s_k[i] * invk;
            S[i] = S[i] * s_g[i] + kn * u;
        }
        // write this token's state to its ring slot
        int so;
        if (a.advance) { int si = (base + t) % a.depth; so = si + 1 == a.depth ? 0 : si + 1; }
        else so = base;
        {
            float *dst = a.state + (size_t)so * a.slot_stride + head_off;
#pragma unroll
            for (int i = 0; i < KD; i++) dst[(size_t)i * VD + j] = S[i];
        }
        if (a.raw_out) a.raw_out[(size_t)t * a.value + (size_t)h * VD + j] = o;
        // gated RMSNorm over the head: ((o*inv)*w)*silu(g)  (src/ops_norm.c:749-793)
        s_o[j] = o * o;
        __syncthreads();
        float ss = 0.0f;
        for (int i = 0; i < VD; i++) ss += s_o[i];
        float inv = d_rsqrt(d_ss_over_n(ss, VD) + a.eps);
        float gz = a.gz[(size_t)t * a.value + (size_t)h * VD + j];
        float y = o * inv * a.o_norm[j] * d_silu(gz);
        if (a.normed_out) a.normed_out[(size_t)t * a.value + (size_t)h * VD + j] = y;
        const int col = h * VD + j;
        d_quant_group32(y, a.xq + (size_t)t * a.value + col,
                        a.xqs + (size_t)t * (a.value >> 5) + (col >> 5));
        __syncthreads();
    }
}

// ------------------------------------------------------------ attention ---

// Per token: RMSNorm(1+w) of every q head (read from the interleaved
// [q | gate] projection) and k head, NeoX rotary on the first rot dims, then
// per-32 int8 quantization of k and v into the KV plane at slot pos
// (attn_impl, src/forward_attn.c:878-960; lz_rope, src/ops_rope.c:21-67).
// One block of 64 lanes per token; heads walked in turn.
__global__ void k_attn_prep(AttnArgs a) {
    extern __shared__ float sh[];               // hd floats
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    const int hd = a.hd, half = a.rot >> 1;
    const int pos = *a.ctl_pos + a.pos_off + t;
    const float *cs = a.rope_cs + (size_t)pos * half * 2;
    const int n_heads_total = (a.kv_only ? 0 : a.nh) + a.nkv;
    for (int hh = 0; hh < n_heads_total; hh++) {
        const bool isq = hh < (a.kv_only ? 0 : a.nh);
        const int h = isq ? hh : hh - (a.kv_only ? 0 : a.nh);
        const float *src = isq ? a.qg + (size_t)t * a.qg_dim + (size_t)h * 2 * hd
                               : a.kp + (size_t)t * a.kv_dim + (size_t)h * hd;
        const float *nw = isq ? a.q_norm : a.k_norm;
        float v0 = 0.0f;
        for (int i = lane; i < hd; i += 64) { v0 = src[i]; sh[i] = v0 * v0; }
        __syncthreads();
        float ss = 0.0f;
        for (int i = 0; i < hd; i++) ss += sh[i];
        float inv = d_rsqrt(d_ss_over_n(ss, hd) + a.eps);
        __syncthreads();
        for (int i = lane; i < hd; i += 64) sh[i] = src[i] * inv * (1.0f + nw[i]);
        __syncthreads();
        // rotary (in LDS), each lane one pair
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
                if (base + (lane & ~31) >= hd) break;
                int col = h * hd + i;
                d_quant_group32(sh[i], a.kcache + (size_t)pos * a.kv_dim + col,
                                a.kscale + (size_t)pos * (a.kv_dim >> 5) + (col >> 5));
            }
        }
        __syncthreads();
    }
    // v: quantize the raw projection
    for (int base = 0; base < a.kv_dim; base += 64) {
        int i = base + lane;
        if (base + (lane & ~31) >= a.kv_dim) break;
        float v = a.vp[(size_t)t * a.kv_dim + i];
        d_quant_group32(v, a.vcache + (size_t)pos * a.kv_dim + i,
                        a.vscale + (size_t)pos * (a.kv_dim >> 5) + (i >> 5));
    }
}

// Scores, softmax and weighted sum for one (token, head) per block
// (attn_score_loop Q8 branch, src/forward_attn.c:206-660: score_q8_row
// :30-41, lz_softmax src/ops_norm.c:903-990, wsum_q8_row :17-21), then the
// sigmoid output gate.  Position-parallel scores; the softmax sum and the
// weighted sums over positions are serial, as in the reference.
__global__ __launch_bounds__(256) void k_attn_decode(AttnArgs a) {
    extern __shared__ float att[];              // pos+1 floats (+ q head)
    const int t = blockIdx.x / a.nh;
    const int h = blockIdx.x - t * a.nh;
    const int hd = a.hd;
    const int kvh = h / (a.nh / a.nkv);
    const int pos = *a.ctl_pos + a.pos_off + t;
    const int L = pos + 1;
    float *qsh = att + ((L + 3) & ~3);
    const int tid = threadIdx.x;
    for (int i = tid; i < hd; i += blockDim.x) qsh[i] = a.qh[(size_t)t * a.q_dim + (size_t)h * hd + i];
    __syncthreads();
    const float scale = a.attn_scale;
    for (int tt = tid; tt < L; tt += blockDim.x) {
        const int8_t *kr = a.kcache + (size_t)tt * a.kv_dim + (size_t)kvh * hd;
        const float *ks = a.kscale + (size_t)tt * (a.kv_dim >> 5) + (size_t)kvh * (hd >> 5);
        float sum = 0.0f;
        for (int dd = 0; dd < hd; dd += 32) {
            float acc = 0.0f;
            for (int e = 0; e < 32; e++) acc += qsh[dd + e] * (float)kr[dd + e];
            sum += acc * ks[dd >> 5];
        }
        att[tt] = sum * scale;
    }
    __syncthreads();
    // softmax: exact max (any order), exp, serial sum, scale
    __shared__ uint32_t s_best;
    __shared__ float s_inv;
    if (tid == 0) s_best = 0;
    __syncthreads();
    {
        uint32_t best = 0;
        for (int tt = tid; tt < L; tt += blockDim.x) {
            uint32_t k = d_fkey(att[tt]);
            best = k > best ? k : best;
        }
        atomicMax(&s_best, best);
    }
    __syncthreads();
    {
        uint32_t kb = s_best;
        uint32_t u = (kb & 0x80000000u) ? (kb ^ 0x80000000u) : ~kb;
        float mx = f_from_u(u);
        for (int tt = tid; tt < L; tt += blockDim.x) att[tt] = d_exp(att[tt] - mx);
    }
    __syncthreads();
    if (tid == 0) {
        float sum = serial_sum(att, L);
        s_inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    {
        float inv = s_inv;
        for (int tt = tid; tt < L; tt += blockDim.x) att[tt] *= inv;
    }
    __syncthreads();
    for (int dd = tid; dd < hd; dd += blockDim.x) {
        float o = 0.0f;
        const int8_t *vr = a.vcache + (size_t)kvh * hd + dd;
        const float *vs = a.vscale + (size_t)(kvh * hd + dd) / 32;
        const size_t vstride = a.kv_dim, sstride = a.kv_dim >> 5;
        for (int tt = 0; tt < L; tt++)
            o += att[tt] * (float)vr[(size_t)tt * vstride] * vs[(size_t)tt * sstride];
        const float gate = a.qg[(size_t)t * a.qg_dim + (size_t)h * 2 * hd + hd + dd];
        o *= d_sigmoid(gate);
        a.out[(size_t)t * a.q_dim + (size_t)h * hd + dd] = o;
    }
}

// ----------------------------------------------------------------- MoE ---

// Routing for every token of the chunk (lz_moe_route, src/ops_moe.c:12-163:
// sigmoid scores, key = score + bias for selection only, repeated
// strict-greater argmax so the lowest index wins ties, weights renormalized
// by their serial sum), then the chunk's distinct-expert table with each
// expert's member (token, slot) pairs, in first-appearance order.
// One block of 64 lanes; lanes parallel over experts.
__global__ void k_moe_route(const float *__restrict__ logits, const float *__restrict__ bias,
                            int E, int topk, int nt, int *__restrict__ sel_idx,
                            float *__restrict__ sel_w, MoeGroups *__restrict__ grp,
                            int *__restrict__ tally) {
    __shared__ float key[MAX_EXPERTS], score[MAX_EXPERTS];
    __shared__ int s_idx[MAX_TOPK];
    const int lane = threadIdx.x;
    for (int t = 0; t < nt; t++) {
        for (int i = lane; i < E; i += 64) {
            float sc = d_sigmoid(logits[(size_t)t * E + i]);
            float kv = sc + bias[i];
            score[i] = sc;
            key[i] = kv == 0.0f ? 0.0f : kv;      // -0 and +0 compare equal in the reference
        }
        __syncthreads();
        for (int k = 0; k < topk; k++) {
            // argmax with lowest index on ties: reduce (fkey, -index)
            uint64_t best = 0;
            for (int i = lane; i < E; i += 64) {
                if (key[i] <= -1e30f) continue;
                uint64_t cand = ((uint64_t)d_fkey(key[i]) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
                best = cand > best ? cand : best;
            }
            for (int o = 32; o > 0; o >>= 1) {
                uint64_t w = __shfl_xor(best, o);
                best = w > best ? w : best;
            }
            if (lane == 0) {
                int bi = best ? (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu)) : -1;
                s_idx[k] = bi;
                if (bi >= 0) key[bi] = -1e30f;
            }
            __syncthreads();
        }
        if (lane == 0) {
            float wsum = 0.0f, w[MAX_TOPK];
            for (int k = 0; k < topk; k++) {
                int bi = s_idx[k];
                w[k] = bi >= 0 ? score[bi] : 0.0f;
                if (bi >= 0) wsum += w[k];
            }
            for (int k = 0; k < topk; k++) {
                if (s_idx[k] >= 0 && wsum > 0.0f) w[k] /= wsum;
                sel_idx[t * topk + k] = s_idx[k];
                sel_w[t * topk + k] = w[k];
            }
        }
        __syncthreads();
    }
    if (lane == 0) {
        int ng = 0;
        for (int t = 0; t < nt; t++)
            for (int k = 0; k < topk; k++) {
                int e = sel_idx[t * topk + k];
                int pair = t * topk + k;
                grp->pair_token[pair] = t;
                if (e < 0) continue;
                int g = 0;
                while (g < ng && grp->expert[g] != e) g++;
                if (g == ng) { grp->expert[ng] = e; grp->n_members[ng] = 0; ng++; }
                grp->member[g][grp->n_members[g]++] = pair;
            }
        grp->n_groups = ng;
        if (tally) *tally += ng;
    }
}

// lat_y[t] = sum over slots in order of w * h2 (src/forward_moe.c:128-200),
// then its per-32 quantization for the up projection.  One 64-lane block per
// token.
__global__ void k_moe_combine(const float *__restrict__ h2, const int *__restrict__ sel_idx,
                              const float *__restrict__ sel_w, int topk, int lat,
                              float *__restrict__ lat_y, int8_t *__restrict__ xq,
                              float *__restrict__ xqs) {
    const int t = blockIdx.x;
    for (int base = 0; base < lat; base += 64) {
        int v = base + threadIdx.x;
        if (base + (int)(threadIdx.x & ~31) >= lat) break;
        float y = 0.0f;
        for (int k = 0; k < topk; k++) {
            if (sel_idx[t * topk + k] < 0) continue;
            y += sel_w[t * topk + k] * h2[((size_t)t * topk + k) * lat + v];
        }
        if (lat_y) lat_y[(size_t)t * lat + v] = y;
        d_quant_group32(y, xq + (size_t)t * lat + v, xqs + (size_t)t * (lat >> 5) + (v >> 5));
    }
}

// -------------------------------------------------------- argmax / ctl ---

// Per row argmax.  mode 0: order-preserving key, first index wins
// (sample_argmax, src/sampler.c:121-137).  mode 1: float '>' compare, first
// index wins (lz_argmax_p1's scan, src/sampler.c:139-155).
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ x, int n, int mode,
                                                 int *__restrict__ out) {
    const int row = blockIdx.x;
    const float *r = x + (size_t)row * n;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = r[i];
        uint32_t k;
        if (mode == 0) k = d_fkey(v);
        else k = (v != v) ? 0u : d_fkey(v == 0.0f ? 0.0f : v);
        uint64_t cand = ((uint64_t)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
        best = cand > best ? cand : best;
    }
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = __shfl_xor(best, o);
        best = w > best ? w : best;
    }
    __shared__ uint64_t sb[16];
    if ((threadIdx.x & 63) == 0) sb[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = 0;
        for (int i = 0; i < (int)(blockDim.x >> 6); i++) b = sb[i] > b ? sb[i] : b;
        out[row] = (int)(0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFu));
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

template <int M>
static hipError_t launch_gemv_m(const GemvBatch &b, const int8_t *xq, const float *xqs, int in_dim,
                                int R, int tiles, hipStream_t st) {
    size_t lds = (size_t)R * M * (in_dim >> 4) * sizeof(int);
    hipLaunchKernelGGL(k_gemv_q8<M>, dim3(tiles), dim3(64), lds, st, b, xq, xqs, in_dim, R);
    return hipGetLastError();
}

extern "C" int l98k_gemv_rows_per_tile(int in_dim, int m) {
    int r = 8192 / in_dim;
    if (r < 1) r = 1;
    if (r > 64 / m) r = 64 / m;
    return r;
}

extern "C" int l98k_gemv(GemvBatch *b, const int8_t *xq, const float *xqs, int in_dim, int m,
                         hipStream_t st) {
    if (m < 1 || m > 8 || (in_dim & 31) || b->n < 1 || b->n > MAX_GEMV_JOBS) return -1;
    int R = l98k_gemv_rows_per_tile(in_dim, m);
    int tiles = 0;
    for (int j = 0; j < b->n; j++) {
        b->job[j].tile0 = tiles;
        tiles += (b->job[j].rows + R - 1) / R;
    }
    switch (m) {
    case 1: return (int)launch_gemv_m<1>(*b, xq, xqs, in_dim, R, tiles, st);
    case 2: return (int)launch_gemv_m<2>(*b, xq, xqs, in_dim, R, tiles, st);
    case 3: return (int)launch_gemv_m<3>(*b, xq, xqs, in_dim, R, tiles, st);
    case 4: return (int)launch_gemv_m<4>(*b, xq, xqs, in_dim, R, tiles, st);
    case 5: return (int)launch_gemv_m<5>(*b, xq, xqs, in_dim, R, tiles, st);
    case 6: return (int)launch_gemv_m<6>(*b, xq, xqs, in_dim, R, tiles, st);
    case 7: return (int)launch_gemv_m<7>(*b, xq, xqs, in_dim, R, tiles, st);
    default: return (int)launch_gemv_m<8>(*b, xq, xqs, in_dim, R, tiles, st);
    }
}

extern "C" int l98k_expert_gemv(const ExpertBank *bank, const MoeGroups *grp, int max_groups,
                                const int8_t *xq, const float *xqs, int xq_by_pair, float *out,
                                int in_dim, int out_rows, int m, hipStream_t st) {
    int R = l98k_gemv_rows_per_tile(in_dim, 8);
    int tiles = (out_rows + R - 1) / R;
    size_t lds = (size_t)R * 8 * (in_dim >> 4) * sizeof(int);
    (void)m;
    hipLaunchKernelGGL(k_expert_gemv<8>, dim3(max_groups * tiles), dim3(64), lds, st, *bank, grp, xq,
                       xqs, xq_by_pair, out, in_dim, out_rows, R, tiles);
    return (int)hipGetLastError();
}

extern "C" int l98k_embed(const int8_t *q, const float *s, const int *toks, int d, int nt,
                          float *x, hipStream_t st) {
    hipLaunchKernelGGL(k_embed, dim3((d + 255) / 256, nt), dim3(256), 0, st, q, s, toks, d, x);
    return (int)hipGetLastError();
}

extern "C" int l98k_rmsnorm(float *x, int x_stride, const float *a, const float *b, const float *w,
                            int n, float eps, int rows, float *out, int out_stride, int8_t *xq,
                            float *xqs, hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(64), (size_t)n * sizeof(float), st, x, x_stride,
                       a, b, w, n, eps, out, out_stride, xq, xqs);
    return (int)hipGetLastError();
}

extern "C" int l98k_quant_rows(const float *x, int n, int x_stride, int rows, int8_t *xq, float *xqs,
                               hipStream_t st) {
    hipLaunchKernelGGL(k_quant_rows, dim3(rows), dim3(64), 0, st, x, n, x_stride, xq, xqs);
    return (int)hipGetLastError();
}

extern "C" int l98k_act_quant(const float *h1, const float *h3, int n, int rows, const int *count,
                              int8_t *xq, float *xqs, float *g_out, hipStream_t st) {
    hipLaunchKernelGGL(k_act_quant, dim3(rows), dim3(64), 0, st, h1, h3, n, count, xq, xqs, g_out);
    return (int)hipGetLastError();
}

extern "C" int l98k_kda_conv(const float *pq, const float *pk, const float *pv, int key, int value,
                             const float *wconv, float *ring, size_t slot_stride, int K,
                             const int *ctl_slot, int depth, int advance, int nt, float *qc,
                             float *kc, float *vc, hipStream_t st) {
    int n = 2 * key + value;
    hipLaunchKernelGGL(k_kda_conv, dim3((n + 255) / 256), dim3(256), 0, st, pq, pk, pv, key, value,
                       wconv, ring, slot_stride, K, ctl_slot, depth, advance, nt, qc, kc, vc);
    return (int)hipGetLastError();
}

extern "C" int l98k_kda_recur(const KdaRecurArgs *a, int kd, int vd, hipStream_t st) {
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
    hipLaunchKernelGGL(k_attn_prep, dim3(nt), dim3(64), (size_t)a->hd * sizeof(float), st, *a);
    return (int)hipGetLastError();
}

extern "C" int l98k_attn_decode(const AttnArgs *a, int nt, int max_len, hipStream_t st) {
    size_t lds = ((size_t)((max_len + 3) & ~3) + a->hd) * sizeof(float);
    hipLaunchKernelGGL(k_attn_decode, dim3(nt * a->nh), dim3(256), lds, st, *a);
    return (int)hipGetLastError();
}

extern "C" int l98k_moe_route(const float *logits, const float *bias, int E, int topk, int nt,
                              int *sel_idx, float *sel_w, MoeGroups *grp, int *tally, hipStream_t st) {
    if (E > MAX_EXPERTS || topk > MAX_TOPK) return -1;
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(64), 0, st, logits, bias, E, topk, nt, sel_idx,
                       sel_w, grp, tally);
    return (int)hipGetLastError();
}

extern "C" int l98k_moe_combine(const float *h2, const int *sel_idx, const float *sel_w, int topk,
                                int lat, int nt, float *lat_y, int8_t *xq, float *xqs,
                                hipStream_t st) {
    hipLaunchKernelGGL(k_moe_combine, dim3(nt), dim3(64), 0, st, h2, sel_idx, sel_w, topk, lat,
                       lat_y, xq, xqs);
    return (int)hipGetLastError();
}

extern "C" int l98k_argmax(const float *x, int n, int rows, int mode, int *out, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(1024), 0, st, x, n, mode, out);
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

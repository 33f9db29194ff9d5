// Wide int8 GEMM on the gfx950 matrix cores, for forwards of many token
// rows at once (prefill chunks, batched verify across sessions), and the
// elementwise producers of its quantized inputs.
//
// o[t][n] = 0.0f + (sum_s float(acc[t,n,s]) * xs[t][s]) * ws[n]
// with acc the exact int32 sum over the 32-element group s
// (lz_matmul_xq_nt -> matmul_q8_impl + epi_q8, src/ops_matmul.c:336-466,
// src/ops_epi.c:983-1017).  v_mfma_i32_16x16x32_i8 contracts exactly one
// 32-element group: started from a zero accumulator it returns the exact
// group sums of a 16 x 16 (row, token) tile, which the lanes then fold into
// fp32 in group order, one multiply and one add per group and output, as
// the reference's epilogue does (a one-group row, K == 32, takes the
// reference's r == 1 association instead: epi_one_group).  The result is bit-identical to the GEMV
// path for every token, whatever the number of tokens.
//
// Operand layout of the 16x16x32 int8 MFMA (64 lanes): lane l supplies
// A[l % 16][8 (l / 16) .. +8) and B[8 (l / 16) .. +8)[l % 16] as eight
// bytes each, and receives D[4 (l / 16) + v][l % 16] in result register v.
// A is the weight tile (rows), B the activation tile (tokens).
#include "l98_devmath.h"

typedef int v4i_t __attribute__((ext_vector_type(4)));

#define MF_THREADS 256
#define MF_ROWS 64        // weight rows per block (four 16-row MFMA tiles per wave)
#define MF_COLS 64        // token columns per block (16 per wave)
#define MF_GU 4           // groups whose operands are loaded ahead of their MFMAs

// Columns of a launch: dense (column t is activation row t and output row
// t, t < M) or grouped (block z is group g: expert gexp[g], columns
// list[goff[g] .. goff[g] + gcnt[g]), activation row xmap[col] or col,
// output row col).
struct MfCols {
    const int *gexp, *goff, *gcnt, *list, *xmap;
    const int *ng;           // groups actually present (device)
};

__device__ __forceinline__ long ld8(const int8_t *p) { return *reinterpret_cast<const long *>(p); }

__global__ __launch_bounds__(MF_THREADS) void k_mfma_q8(const int8_t *__restrict__ W, const float *__restrict__ ws,
                                                         int N, int K, size_t w_group_stride,
                                                         const int8_t *__restrict__ X, const float *__restrict__ Xs,
                                                         int M, MfCols cols, float *__restrict__ out,
                                                         int out_stride) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * MF_ROWS, c0 = blockIdx.y * MF_COLS;
    const int nb = K >> 5;
    int ncols = M, cbase = 0;
    const int8_t *Wg = W;
    const float *wsg = ws;
    if (cols.list) {
        const int g = blockIdx.z;
        if (g >= *cols.ng) return;
        ncols = cols.gcnt[g];
        cbase = cols.goff[g];
        const int e = cols.gexp[g];
        Wg = W + (size_t)e * w_group_stride;
        wsg = ws + (size_t)e * N;
    }
    if (c0 >= ncols) return;
    // this lane's B column and its activation / output rows
    const int cl = c0 + 16 * wave + (lane & 15);
    const int cc = cl < ncols ? cl : ncols - 1;
    int orow = cc, xrow = cc;
    if (cols.list) {
        orow = cols.list[cbase + cc];
        xrow = cols.xmap ? cols.xmap[orow] : orow;
    }
    const int kq = 8 * (lane >> 4);
    const int8_t *xp = X + (size_t)xrow * K + kq;
    const float *xsp = Xs + (size_t)xrow * nb;
    const int8_t *wp[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = n0 + 16 * i + (lane & 15);
        wp[i] = Wg + (size_t)(r < N ? r : N - 1) * K + kq;
    }
    float f[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int v = 0; v < 4; v++) f[i][v] = 0.0f;
    const v4i_t zero = {0, 0, 0, 0};
    int g = 0;
    for (; g + MF_GU <= nb; g += MF_GU) {
        long a[MF_GU][4], b[MF_GU];
        float s[MF_GU];
#pragma unroll
        for (int u = 0; u < MF_GU; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) a[u][i] = ld8(wp[i] + 32 * (g + u));
            b[u] = ld8(xp + 32 * (g + u));
            s[u] = xsp[g + u];
        }
#pragma unroll
        for (int u = 0; u < MF_GU; u++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[u][i], b[u], zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) f[i][v] += (float)d[v] * s[u];
            }
        }
    }
    // one group (K == 32): f holds the exact group sum (|acc| < 2^24) for
    // epi_one_group's association
    const bool one = nb == 1;
    float s0 = 0.0f;
    for (; g < nb; g++) {
        long a[4];
#pragma unroll
        for (int i = 0; i < 4; i++) a[i] = ld8(wp[i] + 32 * g);
        const long b = ld8(xp + 32 * g);
        const float s = xsp[g];
        s0 = s;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b, zero, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++) f[i][v] += one ? (float)d[v] : (float)d[v] * s;
        }
    }
    if (cl >= ncols) return;
    float *op = out + (size_t)orow * out_stride;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int n = n0 + 16 * i + 4 * (lane >> 4) + v;
            if (n < N) {
                float sum = 0.0f;
                if (one) sum = epi_one_group((int)f[i][v], s0, wsg[n]);
                else sum += f[i][v] * wsg[n];
                op[n] = sum;
            }
        }
    }
}

// ------------------------------------------------------ wide producers ---
//
// The quantized GEMM inputs of many rows, one 64-lane block per row, with
// the arithmetic of the GEMV prologues (l98_gemv.h) element for element:
//   mode 0: quantize src rows                       (PRO_QUANT)
//   mode 1: silu(src) * src2, then quantize          (PRO_SILU,
//           lz_ffn_gate_up, src/forward_kda.c:1067-1088)
//   mode 2: sum over the row's slots k < topk with sel_idx >= 0 of
//           sel_w * src[pair], in slot order from 0, then quantize
//           (PRO_COMBINE, src/forward_moe.c:128-200)
// Lane l holds float4 f = l + 64 j of the row, so a quantization group is
// an aligned lane octet.  n % 32 == 0, n <= 4096.
#define WP_MAXJ 16
__global__ __launch_bounds__(64) void k_wide_pro(int mode, const float *__restrict__ src,
                                                 const float *__restrict__ src2, int src_stride,
                                                 const int *__restrict__ sel_idx, const float *__restrict__ sel_w,
                                                 int topk, int n, int8_t *__restrict__ xq, float *__restrict__ xqs,
                                                 float *__restrict__ fout) {
    EXP_TAB_LOAD(tab);
    EXP_TAB_PUT(tab);
    __syncthreads();
    const int row = blockIdx.x, lane = threadIdx.x;
    const int nf = n >> 2, nb = n >> 5;
    for (int j = 0; j < WP_MAXJ; j++) {
        if (64 * j >= nf) break;                   // wave-uniform
        const int f = lane + 64 * j;
        const int fc = f < nf ? f : nf - 1;
        float4 v;
        if (mode == 0) {
            v = reinterpret_cast<const float4 *>(src + (size_t)row * src_stride)[fc];
        } else if (mode == 1) {
            const float4 p = reinterpret_cast<const float4 *>(src + (size_t)row * src_stride)[fc];
            const float4 q = reinterpret_cast<const float4 *>(src2 + (size_t)row * src_stride)[fc];
            v = make_float4(d_silu(p.x, tab) * q.x, d_silu(p.y, tab) * q.y, d_silu(p.z, tab) * q.z,
                            d_silu(p.w, tab) * q.w);
        } else {
            float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            for (int k = 0; k < topk; k++) {
                const int pair = row * topk + k;
                if (sel_idx[pair] < 0) continue;
                const float wk = sel_w[pair];
                const float4 hk = reinterpret_cast<const float4 *>(src + (size_t)pair * n)[fc];
                y = make_float4(y.x + wk * hk.x, y.y + wk * hk.y, y.z + wk * hk.z, y.w + wk * hk.w);
            }
            v = y;
        }
        if (fout && f < nf) reinterpret_cast<float4 *>(fout + (size_t)row * n)[f] = v;
        if (xq) {
            float sg;
            const uint32_t q = quant_octet(v, &sg);
            if (f < nf) {
                reinterpret_cast<uint32_t *>(xq + (size_t)row * n)[f] = q;
                if (!(f & 7)) xqs[(size_t)row * nb + (f >> 3)] = sg;
            }
        }
    }
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_mfma(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

// Dense: out[t][n] (row stride out_stride) for t < M over activation rows
// t.  Returns 0, a HIP error, or -1 for shapes outside the kernel.
extern "C" int l98k_mfma_gemm(const int8_t *W, const float *ws, int N, int K, const int8_t *X, const float *Xs, int M,
                              float *out, int out_stride, hipStream_t st) {
    if (N < 1 || M < 1 || K < 32 || (K & 31) || out_stride < N) return -1;
    MfCols c{};
    hipLaunchKernelGGL(k_mfma_q8, dim3((N + MF_ROWS - 1) / MF_ROWS, (M + MF_COLS - 1) / MF_COLS, 1),
                       dim3(MF_THREADS), 0, st, W, ws, N, K, (size_t)0, X, Xs, M, c, out, out_stride);
    return (int)hipGetLastError();
}

// Grouped (experts): group g (< *ng <= max_groups) multiplies bank rows of
// expert gexp[g] with its columns list[goff[g] ..], at most max_cols each.
extern "C" int l98k_mfma_gemm_grouped(const int8_t *bank, const float *bank_s, int N, int K, const int8_t *X,
                                      const float *Xs, const int *ng, int max_groups, const int *gexp,
                                      const int *goff, const int *gcnt, const int *list, const int *xmap,
                                      int max_cols, float *out, int out_stride, hipStream_t st) {
    if (N < 1 || K < 32 || (K & 31) || max_groups < 1 || max_cols < 1 || out_stride < N) return -1;
    MfCols c{gexp, goff, gcnt, list, xmap, ng};
    hipLaunchKernelGGL(k_mfma_q8,
                       dim3((N + MF_ROWS - 1) / MF_ROWS, (max_cols + MF_COLS - 1) / MF_COLS, max_groups),
                       dim3(MF_THREADS), 0, st, bank, bank_s, N, K, (size_t)N * K, X, Xs, 0, c, out, out_stride);
    return (int)hipGetLastError();
}

extern "C" int l98k_wide_pro(int mode, const float *src, const float *src2, int src_stride, const int *sel_idx,
                             const float *sel_w, int topk, int n, int rows, int8_t *xq, float *xqs, hipStream_t st) {
    if (rows < 1 || n < 32 || (n & 31) || n > 4 * 64 * WP_MAXJ || mode < 0 || mode > 2) return -1;
    if (mode < 2 && (src_stride < n || (src_stride & 3))) return -1;
    if (mode == 2 && (topk < 1 || topk > MAX_TOPK || !sel_idx || !sel_w)) return -1;
    if (!xq || !xqs) return -1;
    hipLaunchKernelGGL(k_wide_pro, dim3(rows), dim3(64), 0, st, mode, src, src2, src_stride, sel_idx, sel_w, topk, n,
                       xq, xqs, (float *)nullptr);
    return (int)hipGetLastError();
}

// The same rows in float, unquantized (row stride n): the input of a norm
// that comes before the quantization.
extern "C" int l98k_wide_pro_f(int mode, const float *src, const float *src2, int src_stride, const int *sel_idx,
                               const float *sel_w, int topk, int n, int rows, float *fout, hipStream_t st) {
    if (rows < 1 || n < 32 || (n & 31) || n > 4 * 64 * WP_MAXJ || mode < 0 || mode > 2 || !fout) return -1;
    if (mode < 2 && (src_stride < n || (src_stride & 3))) return -1;
    if (mode == 2 && (topk < 1 || topk > MAX_TOPK || !sel_idx || !sel_w)) return -1;
    hipLaunchKernelGGL(k_wide_pro, dim3(rows), dim3(64), 0, st, mode, src, src2, src_stride, sel_idx, sel_w, topk, n,
                       (int8_t *)nullptr, (float *)nullptr, fout);
    return (int)hipGetLastError();
}

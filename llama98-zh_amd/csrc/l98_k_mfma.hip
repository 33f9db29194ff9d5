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
//
// A block computes 64 weight rows x 64 token columns (a wave per 16
// columns).  K goes through LDS in stages of MF_KC bytes (eight groups),
// double-buffered: each thread loads its 16-byte pieces of the next stage
// (coalesced: 16 threads per 256-byte row) while the block's MFMAs run on
// the current one, so a stage costs one memory round trip overlapped with
// compute instead of one per group batch.
#include "l98_devmath.h"

typedef int v4i_t __attribute__((ext_vector_type(4)));

#define MF_THREADS 256
#define MF_ROWS 64        // weight rows per block (four 16-row MFMA tiles per wave)
#define MF_COLS 64        // token columns per block (16 per wave)
#define MF_KC 256         // K bytes (eight groups) per LDS stage
#define MF_LDS_ROW (MF_KC + 16)   // padded stage row: the lanes' 8-byte operand reads spread over the banks

// Columns of a launch: dense (column t is activation row t and output row
// t, t < M) or grouped (block z is group g: expert gexp[g], columns
// list[goff[g] .. goff[g] + gcnt[g]), activation row xmap[col] or col,
// output row col).
struct MfCols {
    const int *gexp, *goff, *gcnt, *list, *xmap;
    const int *ng;           // groups actually present (device)
};

__device__ __forceinline__ long ld8(const int8_t *p) { return *reinterpret_cast<const long *>(p); }

// One LDS stage of k_mfma_q8 in a thread's registers: its four 16-byte
// pieces of weight rows and of activation columns, and its B column's eight
// group scales (named members, so they stay in registers across the stage
// loop).
static_assert(MF_KC == 256, "MfStage holds eight group scales");
struct MfStage {
    int4 w0, w1, w2, w3, x0, x1, x2, x3;
    float s0, s1, s2, s3, s4, s5, s6, s7;
    __device__ __forceinline__ void load(const int8_t *const (&wl)[4], const int8_t *const (&xl)[4],
                                         const float *xsp, int st, int pc, int K, int nb) {
        const int off = imin(st * MF_KC + 16 * pc, K - 16);
        w0 = *reinterpret_cast<const int4 *>(wl[0] + off);
        w1 = *reinterpret_cast<const int4 *>(wl[1] + off);
        w2 = *reinterpret_cast<const int4 *>(wl[2] + off);
        w3 = *reinterpret_cast<const int4 *>(wl[3] + off);
        x0 = *reinterpret_cast<const int4 *>(xl[0] + off);
        x1 = *reinterpret_cast<const int4 *>(xl[1] + off);
        x2 = *reinterpret_cast<const int4 *>(xl[2] + off);
        x3 = *reinterpret_cast<const int4 *>(xl[3] + off);
        const int g0 = st * (MF_KC / 32), gl = nb - 1;
        s0 = xsp[imin(g0, gl)]; s1 = xsp[imin(g0 + 1, gl)]; s2 = xsp[imin(g0 + 2, gl)]; s3 = xsp[imin(g0 + 3, gl)];
        s4 = xsp[imin(g0 + 4, gl)]; s5 = xsp[imin(g0 + 5, gl)]; s6 = xsp[imin(g0 + 6, gl)]; s7 = xsp[imin(g0 + 7, gl)];
    }
    __device__ __forceinline__ void put(int8_t (*sw)[MF_LDS_ROW], int8_t (*sx)[MF_LDS_ROW], int rr, int pc) const {
        *reinterpret_cast<int4 *>(&sw[rr][16 * pc]) = w0;
        *reinterpret_cast<int4 *>(&sw[rr + 16][16 * pc]) = w1;
        *reinterpret_cast<int4 *>(&sw[rr + 32][16 * pc]) = w2;
        *reinterpret_cast<int4 *>(&sw[rr + 48][16 * pc]) = w3;
        *reinterpret_cast<int4 *>(&sx[rr][16 * pc]) = x0;
        *reinterpret_cast<int4 *>(&sx[rr + 16][16 * pc]) = x1;
        *reinterpret_cast<int4 *>(&sx[rr + 32][16 * pc]) = x2;
        *reinterpret_cast<int4 *>(&sx[rr + 48][16 * pc]) = x3;
    }
};

__global__ __launch_bounds__(MF_THREADS) void k_mfma_q8(const int8_t *__restrict__ W, const float *__restrict__ ws,
                                                         int N, int K, size_t w_group_stride,
                                                         const int8_t *__restrict__ X, const float *__restrict__ Xs,
                                                         int M, MfCols cols, float *__restrict__ out,
                                                         int out_stride) {
    __shared__ __align__(16) int8_t s_w[2][MF_ROWS][MF_LDS_ROW];
    __shared__ __align__(16) int8_t s_x[2][MF_COLS][MF_LDS_ROW];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n0 = blockIdx.x * MF_ROWS;
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
    // column tiles blockIdx.y, + gridDim.y, ... (a grouped launch has one
    // block row per group, which walks the group's tiles)
#pragma unroll 1
    for (int c0 = blockIdx.y * MF_COLS; c0 < ncols; c0 += gridDim.y * MF_COLS) {
        // this lane's B column and its activation / output rows
        const int cl = c0 + 16 * wave + (lane & 15);
        const int cc = cl < ncols ? cl : ncols - 1;
        int orow = cc, xrow = cc;
        if (cols.list) {
            orow = cols.list[cbase + cc];
            xrow = cols.xmap ? cols.xmap[orow] : orow;
        }
        const int kq = 8 * (lane >> 4);
        const float *xsp = Xs + (size_t)xrow * nb;
        // Stage loads: thread t takes the 16-byte piece pc of weight rows and
        // activation columns rr + 16 j of the block (j < 4): every row's
        // MF_KC-byte stage is read by 16 consecutive threads.  Rows past N and
        // columns past ncols repeat the last; pieces past K repeat the row's
        // last piece (their groups are not used).
        const int pc = tid & 15, rr = tid >> 4;
        const int8_t *wl[4], *xl[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = n0 + rr + 16 * j;
            wl[j] = Wg + (size_t)(r < N ? r : N - 1) * K;
            const int c = imin(c0 + rr + 16 * j, ncols - 1);
            int xr = c;
            if (cols.list) {
                const int o = cols.list[cbase + c];
                xr = cols.xmap ? cols.xmap[o] : o;
            }
            xl[j] = X + (size_t)xr * K;
        }
        const int nst = (K + MF_KC - 1) / MF_KC;
        MfStage nx;
        float f[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) f[i][v] = 0.0f;
        const v4i_t zero = {0, 0, 0, 0};
        // one group (K == 32): f holds the exact group sum (|acc| < 2^24) for
        // epi_one_group's association
        const bool one = nb == 1;
        float s0 = 0.0f;
        nx.load(wl, xl, xsp, 0, pc, K, nb);
        nx.put(s_w[0], s_x[0], rr, pc);
        __syncthreads();
#pragma unroll 1
        for (int st = 0; st < nst; st++) {
            const int buf = st & 1;
            const float sc[MF_KC / 32] = {nx.s0, nx.s1, nx.s2, nx.s3, nx.s4, nx.s5, nx.s6, nx.s7};
            // the next stage's loads are in flight during this stage's MFMAs (the
            // last stage reloads itself into the idle buffer)
            nx.load(wl, xl, xsp, st + 1 < nst ? st + 1 : st, pc, K, nb);
#pragma unroll
            for (int gl = 0; gl < MF_KC / 32; gl++) {
                if (st * (MF_KC / 32) + gl >= nb) break;          // uniform
                long a[4];
#pragma unroll
                for (int i = 0; i < 4; i++) a[i] = *reinterpret_cast<const long *>(&s_w[buf][16 * i + (lane & 15)][32 * gl + kq]);
                const long b = *reinterpret_cast<const long *>(&s_x[buf][16 * wave + (lane & 15)][32 * gl + kq]);
                const float s = sc[gl];
                s0 = s;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b, zero, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++) f[i][v] += one ? (float)d[v] : (float)d[v] * s;
                }
            }
            nx.put(s_w[buf ^ 1], s_x[buf ^ 1], rr, pc);
            __syncthreads();
        }
        // (after the last stage's barrier no wave reads this tile's LDS, so the
        // next tile may refill it)
        if (cl < ncols) {
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
    hipLaunchKernelGGL(k_mfma_q8, dim3((N + MF_ROWS - 1) / MF_ROWS, 1, max_groups),
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

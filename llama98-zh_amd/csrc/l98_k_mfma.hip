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
// A block computes MF_ROWS = 16 MF_RT weight rows x 64 token columns (a
// wave per 16 columns, MF_RT 16-row MFMA tiles each; two tiles keep a
// wave's per-group fp32 fold short and give a 1024-row GEMM a block per CU).  K goes through LDS in stages of MF_KC bytes (eight groups),
// double-buffered: each thread loads its 16-byte pieces of the next stage
// (coalesced: 16 threads per 256-byte row) while the block's MFMAs run on
// the current one, so a stage costs one memory round trip overlapped with
// compute instead of one per group batch.
#include "l98_devmath.h"

typedef int v4i_t __attribute__((ext_vector_type(4)));

#define MF_THREADS 256
#define MF_RT 1           // 16-row MFMA tiles per wave
#define MF_ROWS (16 * MF_RT)  // weight rows per block
#define MF_COLS 64        // token columns per block (16 per wave)
#define MF_KC 256         // K bytes (eight groups) per LDS stage
#define MF_LDS_ROW (MF_KC + 16)   // padded stage row: the lanes' 8-byte operand reads spread over the banks

// Columns of a launch: dense (column t is activation row t and output row
// t, t < M) or grouped (block z is group g: expert gexp[g], columns
// list[goff[g] .. goff[g] + gcnt[g]), activation row xmap[col] or col,
// output row col).
// Dense GEMMs over the same rows sharing a launch: job j covers block rows
// [blk0, next job's blk0) of the grid's x, with its own weights, input (X,
// Xs, K) and output; n == 0: the launch's own arguments.
#define MF_MAX_JOBS 6
struct MfJob {
    const int8_t *W;
    const float *ws;
    float *out;
    const int8_t *X;
    const float *Xs;
    int N, out_stride, blk0, K;
};
struct MfJobs {
    MfJob j[MF_MAX_JOBS];
    int n, pad[3];
};

struct MfCols {
    const int *gexp, *goff, *gcnt, *list, *xmap;
    const int *ng;           // groups actually present (device)
};

__device__ __forceinline__ long ld8(const int8_t *p) { return *reinterpret_cast<const long *>(p); }

// One LDS stage of k_mfma_q8 in a thread's registers (set R: Aw0 .. At1):
// its four 16-byte pieces of weight rows and of activation
// columns, and two of the block's 64 x 8 activation group scales (column
// tid / 4, groups 2 (tid % 4) and the next).  Plain locals (a struct would
// be kept in scratch memory across the scheduling barriers that hold the
// loads' issue in place).
static_assert(MF_KC == 256 && MF_THREADS == 256, "a stage: eight group scales per column, two per thread");
#define MF_STAGE_LOAD(R, st_)                                                                  \
    do {                                                                                       \
        const int off_ = imin((st_) * MF_KC + 16 * pc, K - 16);                                \
        R##w0 = *reinterpret_cast<const int4 *>(wl0 + off_);                                   \
        if constexpr (MF_RT >= 2) R##w1 = *reinterpret_cast<const int4 *>(wl1 + off_);         \
        if constexpr (MF_RT == 4) {                                                            \
            R##w2 = *reinterpret_cast<const int4 *>(wl2 + off_);                               \
            R##w3 = *reinterpret_cast<const int4 *>(wl3 + off_);                               \
        }                                                                                      \
        R##x0 = *reinterpret_cast<const int4 *>(xl0 + off_);                                   \
        R##x1 = *reinterpret_cast<const int4 *>(xl1 + off_);                                   \
        R##x2 = *reinterpret_cast<const int4 *>(xl2 + off_);                                   \
        R##x3 = *reinterpret_cast<const int4 *>(xl3 + off_);                                   \
        const int g_ = (st_) * (MF_KC / 32) + 2 * (tid & 3);                                   \
        R##t0 = xsl[imin(g_, nb - 1)];                                                         \
        R##t1 = xsl[imin(g_ + 1, nb - 1)];                                                     \
    } while (0)
#define MF_STAGE_PUT(R, b_)                                                                    \
    do {                                                                                       \
        *reinterpret_cast<int4 *>(&s_w[b_][rr][16 * pc]) = R##w0;                              \
        if constexpr (MF_RT >= 2) *reinterpret_cast<int4 *>(&s_w[b_][rr + 16][16 * pc]) = R##w1; \
        if constexpr (MF_RT == 4) {                                                            \
            *reinterpret_cast<int4 *>(&s_w[b_][rr + 32][16 * pc]) = R##w2;                     \
            *reinterpret_cast<int4 *>(&s_w[b_][rr + 48][16 * pc]) = R##w3;                     \
        }                                                                                      \
        *reinterpret_cast<int4 *>(&s_x[b_][rr][16 * pc]) = R##x0;                              \
        *reinterpret_cast<int4 *>(&s_x[b_][rr + 16][16 * pc]) = R##x1;                         \
        *reinterpret_cast<int4 *>(&s_x[b_][rr + 32][16 * pc]) = R##x2;                         \
        *reinterpret_cast<int4 *>(&s_x[b_][rr + 48][16 * pc]) = R##x3;                         \
        *reinterpret_cast<float2 *>(&s_xs[b_][tid >> 2][2 * (tid & 3)]) = make_float2(R##t0, R##t1); \
    } while (0)

__device__ __forceinline__ void mf_fold(float (&f)[4], v4i_t d, float s, bool one) {
    f[0] += one ? (float)d[0] : (float)d[0] * s;
    f[1] += one ? (float)d[1] : (float)d[1] * s;
    f[2] += one ? (float)d[2] : (float)d[2] * s;
    f[3] += one ? (float)d[3] : (float)d[3] * s;
}
template <bool FULL>
__device__ __forceinline__ void mf_stage(float (&f)[MF_RT][4], const int8_t (*sw)[MF_LDS_ROW],
                                         const int8_t (*sx)[MF_LDS_ROW], const float *sc, int ng, bool one,
                                         int wave, int lane, int kq) {
    const v4i_t zero = {0, 0, 0, 0};
#pragma unroll
    for (int gl = 0; gl < MF_KC / 32; gl++) {
        if (!FULL && gl >= ng) break;                  // uniform
        const long b = *reinterpret_cast<const long *>(&sx[16 * wave + (lane & 15)][32 * gl + kq]);
        const long a0 = *reinterpret_cast<const long *>(&sw[(lane & 15)][32 * gl + kq]);
        const v4i_t d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b, zero, 0, 0, 0);
        const float s = sc[gl];
        if constexpr (MF_RT == 1) {
            mf_fold(f[0], d0, s, one);
            continue;
        }
        const long a1 = *reinterpret_cast<const long *>(&sw[16 + (lane & 15)][32 * gl + kq]);
        const v4i_t d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b, zero, 0, 0, 0);
        if constexpr (MF_RT == 4) {
            const long a2 = *reinterpret_cast<const long *>(&sw[32 + (lane & 15)][32 * gl + kq]);
            const long a3 = *reinterpret_cast<const long *>(&sw[48 + (lane & 15)][32 * gl + kq]);
            const v4i_t d2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a2, b, zero, 0, 0, 0);
            const v4i_t d3 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a3, b, zero, 0, 0, 0);
            mf_fold(f[0], d0, s, one);
            mf_fold(f[1], d1, s, one);
            mf_fold(f[MF_RT - 2], d2, s, one);
            mf_fold(f[MF_RT - 1], d3, s, one);
        } else {
            mf_fold(f[0], d0, s, one);
            mf_fold(f[MF_RT - 1], d1, s, one);
        }
    }
}

template <bool FULLK>
__global__ __launch_bounds__(MF_THREADS) void k_mfma_q8(const int8_t *__restrict__ W0, const float *__restrict__ ws0,
                                                         int N0, int K0, size_t w_group_stride,
                                                         const int8_t *__restrict__ X0, const float *__restrict__ Xs0,
                                                         int M, MfCols cols, float *__restrict__ out0,
                                                         int out_stride0, MfJobs jobs) {
    __shared__ __align__(16) int8_t s_w[2][MF_ROWS][MF_LDS_ROW];
    __shared__ __align__(16) int8_t s_x[2][MF_COLS][MF_LDS_ROW];
    __shared__ __align__(16) float s_xs[2][MF_COLS][MF_KC / 32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int8_t *W = W0;
    const float *ws = ws0;
    float *out = out0;
    const int8_t *X = X0;
    const float *Xs = Xs0;
    int N = N0, K = K0, out_stride = out_stride0, bx = blockIdx.x;
    if (jobs.n) {
        // the job whose block rows hold this block (the index is uniform)
        int ji = 0;
#pragma unroll
        for (int k = 1; k < MF_MAX_JOBS; k++)
            if (k < jobs.n && bx >= jobs.j[k].blk0) ji = k;
        const MfJob jb = jobs.j[ji];
        W = jb.W;
        ws = jb.ws;
        out = jb.out;
        X = jb.X;
        Xs = jb.Xs;
        K = jb.K;
        N = jb.N;
        out_stride = jb.out_stride;
        bx -= jb.blk0;
    }
    const int n0 = bx * MF_ROWS;
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
        // this lane's B column and its output row
        const int cl = c0 + 16 * wave + (lane & 15);
        const int cc = cl < ncols ? cl : ncols - 1;
        const int orow = cols.list ? cols.list[cbase + cc] : cc;
        const int kq = 8 * (lane >> 4);
        // Stage loads: thread t takes the 16-byte piece pc of weight rows
        // rr + 16 j (j < MF_RT) and activation columns rr + 16 j (j < 4) of
        // the block: every row's
        // MF_KC-byte stage is read by 16 consecutive threads.  Rows past N and
        // columns past ncols repeat the last; pieces past K repeat the row's
        // last piece (their groups are not used).
        const int pc = tid & 15, rr = tid >> 4;
        auto wrow = [&](int j) { const int r = n0 + rr + 16 * j; return Wg + (size_t)(r < N ? r : N - 1) * K; };
        auto xcol = [&](int j) {
            const int c = imin(c0 + rr + 16 * j, ncols - 1);
            int xr = c;
            if (cols.list) {
                const int o = cols.list[cbase + c];
                xr = cols.xmap ? cols.xmap[o] : o;
            }
            return X + (size_t)xr * K;
        };
        const int8_t *wl0 = wrow(0), *wl1 = wrow(imin(1, MF_RT - 1)), *wl2 = wrow(imax(0, MF_RT - 2)),
                     *wl3 = wrow(MF_RT - 1);
        const int8_t *xl0 = xcol(0), *xl1 = xcol(1), *xl2 = xcol(2), *xl3 = xcol(3);
        // the activation scales this thread stages: column tid / 4
        const float *xsl;
        {
            const int c = imin(c0 + (tid >> 2), ncols - 1);
            int xr = c;
            if (cols.list) {
                const int o = cols.list[cbase + c];
                xr = cols.xmap ? cols.xmap[o] : o;
            }
            xsl = Xs + (size_t)xr * nb;
        }
        const int nst = (K + MF_KC - 1) / MF_KC;
        int4 Aw0, Aw1 = {}, Aw2 = {}, Aw3 = {}, Ax0, Ax1, Ax2, Ax3;
        float At0, At1;
        float f[MF_RT][4];
#pragma unroll
        for (int i = 0; i < MF_RT; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) f[i][v] = 0.0f;
        // one group (K == 32): f holds the exact group sum (|acc| < 2^24) for
        // epi_one_group's association
        const bool one = nb == 1;
        float s0 = 0.0f;
        MF_STAGE_LOAD(A, 0);
        MF_STAGE_PUT(A, 0);
        __syncthreads();
#pragma unroll 1
        for (int st = 0; st < nst; st++) {
            const int buf = st & 1;
            const float *sc = s_xs[buf][16 * wave + (lane & 15)];
            // the next stage's loads are in flight during this stage's MFMAs (the
            // last stage reloads itself into the idle buffer); the scheduling
            // barrier keeps their issue ahead of the MFMAs.  FULLK: every stage
            // holds eight groups and the stage is one basic block (with a
            // branch between them the compiler sinks the loads to their LDS
            // stores).
            MF_STAGE_LOAD(A, st + 1 < nst ? st + 1 : st);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (FULLK) {
                mf_stage<true>(f, s_w[buf], s_x[buf], sc, MF_KC / 32, false, wave, lane, kq);
            } else {
                mf_stage<false>(f, s_w[buf], s_x[buf], sc, nb - st * (MF_KC / 32), one, wave, lane, kq);
                if (one) s0 = sc[0];
            }
            MF_STAGE_PUT(A, buf ^ 1);
            __syncthreads();
        }
        // (after the last stage's barrier no wave reads this tile's LDS, so the
        // next tile may refill it)
        if (cl < ncols) {
            float *op = out + (size_t)orow * out_stride;
#pragma unroll
            for (int i = 0; i < MF_RT; i++) {
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

#undef MF_STAGE_LOAD
#undef MF_STAGE_PUT

// The narrow form: a block computes 64 weight rows x 16 token columns
// (wave w: rows 16 w .. 16 w + 15 of the same 16 columns), so each block
// streams four times the weights of k_mfma_q8's 16-row tile and stages
// only the 16 columns it uses, and the loads run two stages ahead (register
// sets A and B alternate) - for few columns per weight tile (the experts of
// a batched verify, whose groups average a few pairs; dense GEMMs over the
// batch's rows), where a stage's round trip, not the arithmetic, bounds the
// block.  Dense (cols.list null: column t is activation and output row t,
// t < M; jobs as in k_mfma_q8; a 1-D grid mapped onto the XCDs so that the
// column tiles of a weight tile share an L2) or grouped (block z is group g; a group's
// column tiles spread over the grid's y, whose extra blocks exit at once).
// Same stages, MFMAs and fold per (row, column) as k_mfma_q8, so the same
// bits.
#define MFN_ROWS 64
#define MFN_COLS 16
#define MFN_DENSE_MAX 128      // dense GEMMs of at most this many rows take the narrow tiles
#define MFN_STAGE_LOAD(R, st_)                                                                 \
    do {                                                                                       \
        const int off_ = imin((st_) * MF_KC + 16 * pc, K - 16);                                \
        R##w0 = *reinterpret_cast<const int4 *>(wl0 + off_);                                   \
        R##w1 = *reinterpret_cast<const int4 *>(wl1 + off_);                                   \
        R##w2 = *reinterpret_cast<const int4 *>(wl2 + off_);                                   \
        R##w3 = *reinterpret_cast<const int4 *>(wl3 + off_);                                   \
        R##x0 = *reinterpret_cast<const int4 *>(xl0 + off_);                                   \
        if (tid < 64) {                                                                        \
            const int g_ = (st_) * (MF_KC / 32) + 2 * (tid & 3);                               \
            R##t0 = xsl[imin(g_, nb - 1)];                                                     \
            R##t1 = xsl[imin(g_ + 1, nb - 1)];                                                 \
        }                                                                                      \
    } while (0)
#define MFN_STAGE_PUT(R, b_)                                                                   \
    do {                                                                                       \
        *reinterpret_cast<int4 *>(&s_w[b_][rr][16 * pc]) = R##w0;                              \
        *reinterpret_cast<int4 *>(&s_w[b_][rr + 16][16 * pc]) = R##w1;                         \
        *reinterpret_cast<int4 *>(&s_w[b_][rr + 32][16 * pc]) = R##w2;                         \
        *reinterpret_cast<int4 *>(&s_w[b_][rr + 48][16 * pc]) = R##w3;                         \
        *reinterpret_cast<int4 *>(&s_x[b_][rr][16 * pc]) = R##x0;                              \
        if (tid < 64) *reinterpret_cast<float2 *>(&s_xs[b_][tid >> 2][2 * (tid & 3)]) = make_float2(R##t0, R##t1); \
    } while (0)
template <bool FULLK>
__global__ __launch_bounds__(MF_THREADS) void k_mfma_q8n(const int8_t *__restrict__ W0, const float *__restrict__ ws0,
                                                          int N0, int K0, size_t w_group_stride,
                                                          const int8_t *__restrict__ X0, const float *__restrict__ Xs0,
                                                          int M, MfCols cols, float *__restrict__ out0,
                                                          int out_stride0, MfJobs jobs) {
    __shared__ __align__(16) int8_t s_w[2][MFN_ROWS][MF_LDS_ROW];
    __shared__ __align__(16) int8_t s_x[2][MFN_COLS][MF_LDS_ROW];
    __shared__ __align__(16) float s_xs[2][MFN_COLS][MF_KC / 32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int8_t *W = W0;
    const float *ws = ws0;
    float *out = out0;
    const int8_t *X = X0;
    const float *Xs = Xs0;
    int N = N0, K = K0, out_stride = out_stride0, bx = blockIdx.x;
    int cy = blockIdx.y, cys = gridDim.y;
    if (!cols.list) {
        // Dense: a 1-D grid of (row tiles rounded up to 8) x column tiles.
        // Blocks go to the 8 XCDs in turn by linear index, so block L runs on
        // XCD L % 8; give XCD x the row tiles x, x + 8, ... with all their
        // column tiles one after another, so the column tiles that share a
        // weight tile share that XCD's L2 (weights read from HBM once).
        const int ny = (M + MFN_COLS - 1) / MFN_COLS, xcd = bx & 7, sl = bx >> 3, q = sl / ny;
        bx = q * 8 + xcd;
        cy = sl - q * ny;
        cys = ny;
        const int nrt = jobs.n ? jobs.j[jobs.n - 1].blk0 + (jobs.j[jobs.n - 1].N + MFN_ROWS - 1) / MFN_ROWS
                               : (N0 + MFN_ROWS - 1) / MFN_ROWS;
        if (bx >= nrt) return;
    }
    if (jobs.n) {
        int ji = 0;
#pragma unroll
        for (int k = 1; k < MF_MAX_JOBS; k++)
            if (k < jobs.n && bx >= jobs.j[k].blk0) ji = k;
        const MfJob jb = jobs.j[ji];
        W = jb.W;
        ws = jb.ws;
        out = jb.out;
        X = jb.X;
        Xs = jb.Xs;
        K = jb.K;
        N = jb.N;
        out_stride = jb.out_stride;
        bx -= jb.blk0;
    }
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
    const int n0 = bx * MFN_ROWS, nb = K >> 5;
    const int pc = tid & 15, rr = tid >> 4;
    auto wrow = [&](int j) { const int r = n0 + rr + 16 * j; return Wg + (size_t)(r < N ? r : N - 1) * K; };
    const int8_t *wl0 = wrow(0), *wl1 = wrow(1), *wl2 = wrow(2), *wl3 = wrow(3);
    const int kq = 8 * (lane >> 4);
    const int nst = (K + MF_KC - 1) / MF_KC;
#pragma unroll 1
    for (int c0 = cy * MFN_COLS; c0 < ncols; c0 += cys * MFN_COLS) {
        auto xrow = [&](int c) {
            const int cc = imin(c0 + c, ncols - 1);
            if (!cols.list) return cc;
            const int o = cols.list[cbase + cc];
            return cols.xmap ? cols.xmap[o] : o;
        };
        const int8_t *xl0 = X + (size_t)xrow(rr) * K;                  // column rr's piece pc
        const float *xsl = Xs + (size_t)xrow(tid >> 2) * nb;            // threads < 64: column tid / 4
        const int cl = c0 + (lane & 15);
        int4 Aw0, Aw1, Aw2, Aw3, Ax0, Bw0, Bw1, Bw2, Bw3, Bx0;
        float At0 = 0.0f, At1 = 0.0f, Bt0 = 0.0f, Bt1 = 0.0f;
        float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const bool one = nb == 1;
        float s0 = 0.0f;
        auto compute = [&](int buf, int st) {
            const float *sc = s_xs[buf][lane & 15];
            const v4i_t zero = {0, 0, 0, 0};
            const int ng = FULLK ? MF_KC / 32 : nb - st * (MF_KC / 32);
#pragma unroll
            for (int gl = 0; gl < MF_KC / 32; gl++) {
                if (!FULLK && gl >= ng) break;                     // uniform
                const long b = *reinterpret_cast<const long *>(&s_x[buf][lane & 15][32 * gl + kq]);
                const long a = *reinterpret_cast<const long *>(&s_w[buf][16 * wave + (lane & 15)][32 * gl + kq]);
                const v4i_t dd = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
                mf_fold(f, dd, sc[gl], one);
            }
            if (!FULLK && one) s0 = sc[0];
        };
        // stage st in buffer st % 2; the loads of stages st + 1 and st + 2
        // in flight while it runs (stages past the last reload the last)
        MFN_STAGE_LOAD(A, 0);
        MFN_STAGE_PUT(A, 0);
        __syncthreads();
        MFN_STAGE_LOAD(A, imin(1, nst - 1));
#pragma unroll 1
        for (int st = 0; st < nst; st += 2) {
            MFN_STAGE_LOAD(B, imin(st + 2, nst - 1));
            __builtin_amdgcn_sched_barrier(0);
            compute(0, st);
            MFN_STAGE_PUT(A, 1);
            __syncthreads();
            if (st + 1 >= nst) break;                          // uniform
            MFN_STAGE_LOAD(A, imin(st + 3, nst - 1));
            __builtin_amdgcn_sched_barrier(0);
            compute(1, st + 1);
            MFN_STAGE_PUT(B, 0);
            __syncthreads();
        }
        if (cl < ncols) {
            float *op = out + (size_t)(cols.list ? cols.list[cbase + cl] : cl) * out_stride;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int n = n0 + 16 * wave + 4 * (lane >> 4) + v;
                if (n < N) {
                    float sum = 0.0f;
                    if (one) sum = epi_one_group((int)f[v], s0, wsg[n]);
                    else sum += f[v] * wsg[n];
                    op[n] = sum;
                }
            }
        }
    }
}
#undef MFN_STAGE_LOAD
#undef MFN_STAGE_PUT


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
struct WideProArgs {
    const float *src, *src2;
    const int *sel_idx;
    const float *sel_w;
    int8_t *xq;
    float *xqs, *fout;
    int mode, src_stride, topk, n;
};
__device__ __forceinline__ void wide_pro_body(int mode, const float *__restrict__ src, const float *__restrict__ src2,
                                              int src_stride, const int *__restrict__ sel_idx,
                                              const float *__restrict__ sel_w, int topk, int n,
                                              int8_t *__restrict__ xq, float *__restrict__ xqs,
                                              float *__restrict__ fout, int row, const float *tab) {
    const int lane = threadIdx.x;
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
__global__ __launch_bounds__(64) void k_wide_pro(int mode, const float *__restrict__ src,
                                                 const float *__restrict__ src2, int src_stride,
                                                 const int *__restrict__ sel_idx, const float *__restrict__ sel_w,
                                                 int topk, int n, int8_t *__restrict__ xq, float *__restrict__ xqs,
                                                 float *__restrict__ fout) {
    EXP_TAB_LOAD(tab);
    EXP_TAB_PUT(tab);
    __syncthreads();
    wide_pro_body(mode, src, src2, src_stride, sel_idx, sel_w, topk, n, xq, xqs, fout, blockIdx.x, tab);
}
// Two independent producers in one launch: blocks [0, rows_a) run a's rows,
// the rest b's.
__global__ __launch_bounds__(64) void k_wide_pro2(WideProArgs a, int rows_a, WideProArgs b) {
    EXP_TAB_LOAD(tab);
    EXP_TAB_PUT(tab);
    __syncthreads();
    const bool first = (int)blockIdx.x < rows_a;
    const WideProArgs &p = first ? a : b;
    wide_pro_body(p.mode, p.src, p.src2, p.src_stride, p.sel_idx, p.sel_w, p.topk, p.n, p.xq, p.xqs, p.fout,
                  first ? blockIdx.x : blockIdx.x - rows_a, tab);
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
    if (M <= MFN_DENSE_MAX) {
        const int nrt8 = ((N + MFN_ROWS - 1) / MFN_ROWS + 7) & ~7;
        const dim3 gridn(nrt8 * ((M + MFN_COLS - 1) / MFN_COLS), 1, 1);
        if (K % MF_KC == 0)
            hipLaunchKernelGGL(k_mfma_q8n<true>, gridn, dim3(MF_THREADS), 0, st, W, ws, N, K, (size_t)0, X, Xs, M, c,
                               out, out_stride, MfJobs{});
        else
            hipLaunchKernelGGL(k_mfma_q8n<false>, gridn, dim3(MF_THREADS), 0, st, W, ws, N, K, (size_t)0, X, Xs, M, c,
                               out, out_stride, MfJobs{});
        return (int)hipGetLastError();
    }
    const dim3 grid((N + MF_ROWS - 1) / MF_ROWS, (M + MF_COLS - 1) / MF_COLS, 1);
    if (K % MF_KC == 0)
        hipLaunchKernelGGL(k_mfma_q8<true>, grid, dim3(MF_THREADS), 0, st, W, ws, N, K, (size_t)0, X, Xs, M, c, out,
                           out_stride, MfJobs{});
    else
        hipLaunchKernelGGL(k_mfma_q8<false>, grid, dim3(MF_THREADS), 0, st, W, ws, N, K, (size_t)0, X, Xs, M, c, out,
                           out_stride, MfJobs{});
    return (int)hipGetLastError();
}

// Several dense GEMMs over the same M rows in one launch: job j multiplies
// W[j] (N[j] x K[j], scales ws[j]) over the rows of X[j] / Xs[j] into out[j]
// (row stride out_stride[j]).  The blocks of job j follow those of job
// j - 1.  The full-stage instance needs every K a multiple of 256.
extern "C" int l98k_mfma_gemm_multi(int n_jobs, const int8_t *const *W, const float *const *ws, const int *N,
                                    float *const *out, const int *out_stride, const int *K,
                                    const int8_t *const *X, const float *const *Xs, int M, hipStream_t st) {
    if (n_jobs < 1 || n_jobs > MF_MAX_JOBS || M < 1) return -1;
    const bool narrow = M <= MFN_DENSE_MAX;
    const int tile = narrow ? MFN_ROWS : MF_ROWS;
    MfJobs jobs{};
    int blocks = 0;
    bool full = true;
    for (int j = 0; j < n_jobs; j++) {
        if (N[j] < 1 || out_stride[j] < N[j] || K[j] < 32 || (K[j] & 31)) return -1;
        full = full && K[j] % MF_KC == 0;
        jobs.j[j] = MfJob{W[j], ws[j], out[j], X[j], Xs[j], N[j], out_stride[j], blocks, K[j]};
        blocks += (N[j] + tile - 1) / tile;
    }
    jobs.n = n_jobs;
    MfCols c{};
    if (narrow) {
        const dim3 gridn(((blocks + 7) & ~7) * ((M + MFN_COLS - 1) / MFN_COLS), 1, 1);
        if (full)
            hipLaunchKernelGGL(k_mfma_q8n<true>, gridn, dim3(MF_THREADS), 0, st, W[0], ws[0], N[0], K[0], (size_t)0,
                               X[0], Xs[0], M, c, out[0], out_stride[0], jobs);
        else
            hipLaunchKernelGGL(k_mfma_q8n<false>, gridn, dim3(MF_THREADS), 0, st, W[0], ws[0], N[0], K[0], (size_t)0,
                               X[0], Xs[0], M, c, out[0], out_stride[0], jobs);
        return (int)hipGetLastError();
    }
    const dim3 grid(blocks, (M + MF_COLS - 1) / MF_COLS, 1);
    if (full)
        hipLaunchKernelGGL(k_mfma_q8<true>, grid, dim3(MF_THREADS), 0, st, W[0], ws[0], N[0], K[0], (size_t)0, X[0],
                           Xs[0], M, c, out[0], out_stride[0], jobs);
    else
        hipLaunchKernelGGL(k_mfma_q8<false>, grid, dim3(MF_THREADS), 0, st, W[0], ws[0], N[0], K[0], (size_t)0, X[0],
                           Xs[0], M, c, out[0], out_stride[0], jobs);
    return (int)hipGetLastError();
}

// Grouped (experts): group g (< *ng <= max_groups) multiplies bank rows of
// expert gexp[g] with its columns list[goff[g] ..], at most max_cols each.
// Groups of about 16 columns or fewer (mean_cols, the caller's estimate)
// take the 64-row x 16-column tiles, larger ones the 16 x 64 tiles.
extern "C" int l98k_mfma_gemm_grouped(const int8_t *bank, const float *bank_s, int N, int K, const int8_t *X,
                                      const float *Xs, const int *ng, int max_groups, const int *gexp,
                                      const int *goff, const int *gcnt, const int *list, const int *xmap,
                                      int max_cols, int mean_cols, float *out, int out_stride, hipStream_t st) {
    if (N < 1 || K < 32 || (K & 31) || max_groups < 1 || max_cols < 1 || out_stride < N) return -1;
    MfCols c{gexp, goff, gcnt, list, xmap, ng};
    if (mean_cols <= MFN_COLS) {
        const int ys = max_cols > 3 * MFN_COLS ? 4 : (max_cols + MFN_COLS - 1) / MFN_COLS;
        const dim3 gridn((N + MFN_ROWS - 1) / MFN_ROWS, ys, max_groups);
        if (K % MF_KC == 0)
            hipLaunchKernelGGL(k_mfma_q8n<true>, gridn, dim3(MF_THREADS), 0, st, bank, bank_s, N, K, (size_t)N * K, X,
                               Xs, 0, c, out, out_stride, MfJobs{});
        else
            hipLaunchKernelGGL(k_mfma_q8n<false>, gridn, dim3(MF_THREADS), 0, st, bank, bank_s, N, K, (size_t)N * K,
                               X, Xs, 0, c, out, out_stride, MfJobs{});
        return (int)hipGetLastError();
    }
    const dim3 grid((N + MF_ROWS - 1) / MF_ROWS, 1, max_groups);
    if (K % MF_KC == 0)
        hipLaunchKernelGGL(k_mfma_q8<true>, grid, dim3(MF_THREADS), 0, st, bank, bank_s, N, K, (size_t)N * K, X, Xs, 0,
                           c, out, out_stride, MfJobs{});
    else
        hipLaunchKernelGGL(k_mfma_q8<false>, grid, dim3(MF_THREADS), 0, st, bank, bank_s, N, K, (size_t)N * K, X, Xs,
                           0, c, out, out_stride, MfJobs{});
    return (int)hipGetLastError();
}

// Two grouped GEMMs over the same columns and groups (an expert's w1 and w3
// banks, both N x K): on the narrow tiles one launch whose first half of
// block columns runs bank 1 and the second half bank 3 (jobs); otherwise
// two launches.
extern "C" int l98k_mfma_gemm_grouped2(const int8_t *bank1, const float *bank1_s, float *out1, const int8_t *bank3,
                                       const float *bank3_s, float *out3, int N, int K, const int8_t *X,
                                       const float *Xs, const int *ng, int max_groups, const int *gexp,
                                       const int *goff, const int *gcnt, const int *list, const int *xmap,
                                       int max_cols, int mean_cols, int out_stride, hipStream_t st) {
    if (N < 1 || K < 32 || (K & 31) || max_groups < 1 || max_cols < 1 || out_stride < N) return -1;
    if (mean_cols > MFN_COLS) {
        const int rc = l98k_mfma_gemm_grouped(bank1, bank1_s, N, K, X, Xs, ng, max_groups, gexp, goff, gcnt, list, xmap,
                                              max_cols, mean_cols, out1, out_stride, st);
        if (rc) return rc;
        return l98k_mfma_gemm_grouped(bank3, bank3_s, N, K, X, Xs, ng, max_groups, gexp, goff, gcnt, list, xmap,
                                      max_cols, mean_cols, out3, out_stride, st);
    }
    MfCols c{gexp, goff, gcnt, list, xmap, ng};
    const int nrt = (N + MFN_ROWS - 1) / MFN_ROWS;
    MfJobs jobs{};
    jobs.j[0] = MfJob{bank1, bank1_s, out1, X, Xs, N, out_stride, 0, K};
    jobs.j[1] = MfJob{bank3, bank3_s, out3, X, Xs, N, out_stride, nrt, K};
    jobs.n = 2;
    const int ys = max_cols > 3 * MFN_COLS ? 4 : (max_cols + MFN_COLS - 1) / MFN_COLS;
    const dim3 gridn(2 * nrt, ys, max_groups);
    if (K % MF_KC == 0)
        hipLaunchKernelGGL(k_mfma_q8n<true>, gridn, dim3(MF_THREADS), 0, st, bank1, bank1_s, N, K, (size_t)N * K, X, Xs,
                           0, c, out1, out_stride, jobs);
    else
        hipLaunchKernelGGL(k_mfma_q8n<false>, gridn, dim3(MF_THREADS), 0, st, bank1, bank1_s, N, K, (size_t)N * K, X, Xs,
                           0, c, out1, out_stride, jobs);
    return (int)hipGetLastError();
}

static bool wide_pro_ok(int mode, int src_stride, const int *sel_idx, const float *sel_w, int topk, int n, int rows) {
    if (rows < 1 || n < 32 || (n & 31) || n > 4 * 64 * WP_MAXJ || mode < 0 || mode > 2) return false;
    if (mode < 2 && (src_stride < n || (src_stride & 3))) return false;
    if (mode == 2 && (topk < 1 || topk > MAX_TOPK || !sel_idx || !sel_w)) return false;
    return true;
}

// Two quantizing producers (modes as l98k_wide_pro) in one launch.
extern "C" int l98k_wide_pro2(int mode_a, const float *src_a, const float *src2_a, int stride_a, int n_a, int rows_a,
                              int8_t *xq_a, float *xqs_a, int mode_b, const float *src_b, const float *src2_b,
                              int stride_b, const int *sel_idx_b, const float *sel_w_b, int topk_b, int n_b,
                              int rows_b, int8_t *xq_b, float *xqs_b, hipStream_t st) {
    if (mode_a == 2 || !wide_pro_ok(mode_a, stride_a, nullptr, nullptr, 0, n_a, rows_a) ||
        !wide_pro_ok(mode_b, stride_b, sel_idx_b, sel_w_b, topk_b, n_b, rows_b) || !xq_a || !xqs_a || !xq_b || !xqs_b)
        return -1;
    const WideProArgs a{src_a, src2_a, nullptr, nullptr, xq_a, xqs_a, nullptr, mode_a, stride_a, 0, n_a};
    const WideProArgs b{src_b, src2_b, sel_idx_b, sel_w_b, xq_b, xqs_b, nullptr, mode_b, stride_b, topk_b, n_b};
    hipLaunchKernelGGL(k_wide_pro2, dim3(rows_a + rows_b), dim3(64), 0, st, a, rows_a, b);
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

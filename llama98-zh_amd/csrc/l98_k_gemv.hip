// Dense fused int8 GEMV kernels of the MTP speculative-decoding step
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_gemv.h"
#include <climits>

// The argmax epilogue (instances with MA; one job): each block stores its
// tile's per-row maxima (exact 64-bit candidates) for l98k_argmax_part.
template <int M>
__device__ __forceinline__ void amax_store(const GemvBatch &b, const GemvJob &job, int m,
                                           const unsigned long long *s_am) {
    __syncthreads();
    if ((int)threadIdx.x < m) b.amax_part[(size_t)threadIdx.x * job.tiles + blockIdx.x] = s_am[threadIdx.x];
}

// One launch over b.n jobs; m <= M live token rows.
// Block (x, y) is tile x of job y: the job index is the workgroup id, so
// the job's fields are read with the kernel's first batch of scalar loads
// (no dependent lookup); tiles past a job's last exit at once.
template <int M, int PJ, int MODES>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv_q8(GemvBatch batch, int m) {
    extern __shared__ __align__(16) char smem[];
    __shared__ int s_row[M];
    __shared__ float s_inv[M], tab[32];
    __shared__ unsigned long long s_am[(MODES & MA) ? M : 1];
    const GemvJob job = batch.job[blockIdx.y];
    if ((int)blockIdx.x >= job.tiles) return;
    if ((MODES & MA) && threadIdx.x < M) s_am[threadIdx.x] = 0;
    const int row0 = blockIdx.x * job.R;
    const int rows_here = imin(job.R, job.rows - row0);
    if (threadIdx.x < M) s_row[threadIdx.x] = threadIdx.x < m ? threadIdx.x : 0;
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) xrow[t] = t < m ? t : 0;
    gemv_tile<M, PJ, MODES>(job.w + (size_t)row0 * job.in_dim, job.ws, rows_here, job.R, job.in_dim, job.pro, job.xq,
                            job.xqs, xrow, s_row, m, blockIdx.x == 0 && blockIdx.y == 0, job.out, job.out_stride,
                            row0, job.acc_out, job.rows,
                            smem, s_inv, tab, job.gs, s_am, batch.amax_mode);
    if (MODES & MA) amax_store<M>(batch, job, m, s_am);
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_gemv(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

// Instances: token slots M in {1, 2, 4, 5, 6, 8}; prologue sets: pre-quantized
// (PJ 0), RMSNorm (PJ 1..8), RMSNorm with fold-only jobs (PJ 1..8),
// SiLU-mul (PJ 1..4), combine + SiLU-mul (PJ 1..4); each with one scale per
// weight row or with grouped scales (MG); pre-quantized with the argmax
// epilogue (MA).
#define GEMV_CASE(M_, PJ_, MODES_)                                                                         \
    case (M_) * 100000 + (PJ_) * 1000 + (MODES_):                                                            \
        ALLOW_BIG_LDS((k_gemv_q8<M_, PJ_, MODES_>));                                                      \
        hipLaunchKernelGGL((k_gemv_q8<M_, PJ_, MODES_>), dim3(tiles, b->n), dim3(GEMV_THREADS), lds, st, *b, m); \
        break;
#define GEMV_CASES_MG(M_, G_)                                                                          \
    GEMV_CASE(M_, 0, MODES_X | G_)                                                                     \
    GEMV_CASE(M_, 1, MODES_N | G_) GEMV_CASE(M_, 2, MODES_N | G_) GEMV_CASE(M_, 4, MODES_N | G_)       \
    GEMV_CASE(M_, 8, MODES_N | G_)                                                                     \
    GEMV_CASE(M_, 1, MODES_NF | G_) GEMV_CASE(M_, 2, MODES_NF | G_) GEMV_CASE(M_, 4, MODES_NF | G_)    \
    GEMV_CASE(M_, 8, MODES_NF | G_)                                                                    \
    GEMV_CASE(M_, 1, MODES_S | G_) GEMV_CASE(M_, 2, MODES_S | G_) GEMV_CASE(M_, 4, MODES_S | G_)       \
    GEMV_CASE(M_, 1, MODES_CS | G_) GEMV_CASE(M_, 2, MODES_CS | G_) GEMV_CASE(M_, 4, MODES_CS | G_)
#define GEMV_CASES_M(M_)                                                                              \
    GEMV_CASES_MG(M_, 0) GEMV_CASES_MG(M_, MG) GEMV_CASE(M_, 0, MODES_X | MA) GEMV_CASE(M_, 0, MODES_X | MG | MA)

// Checks every job's prologue against the kernel's limits, lays the jobs'
// tiles out in one grid and launches the instance for the jobs' prologue
// set (pre-quantized, RMSNorm, SiLU-mul, or combine + SiLU-mul).
extern "C" int l98k_gemv(GemvBatch *b, int m, hipStream_t st) {
    if (m < 1 || m > MAX_CHUNK || b->n < 1 || b->n > MAX_GEMV_JOBS) return -1;
    const int M = gemv_slots(m);
    int tiles = 0, pj = 0, modes = 0, grouped = 0;       // tiles: the largest job's
    size_t lds = 0;
    for (int j = 0; j < b->n; j++) {
        GemvJob &J = b->job[j];
        if (J.in_dim < 32 || (J.in_dim & 31) || J.in_dim > GEMV_MAX_IN || J.rows < 1 ||
            !prologue_ok(J.pro, J.in_dim, J.xq, J.xqs) || (J.gs && ((J.gs & 31) || J.in_dim % J.gs)))
            return -1;
        J.R = gemv_rows_per_tile(J.in_dim, M);
        J.tiles = (J.rows + J.R - 1) / J.R;
        tiles = J.tiles > tiles ? J.tiles : tiles;
        modes |= MB(J.pro.mode);
        if (J.gs && J.gs < J.in_dim) grouped = MG;
        if (J.pro.mode != PRO_XQ) pj = pro_pj(J.in_dim) > pj ? pro_pj(J.in_dim) : pj;
    }
    for (int j = 0; j < b->n; j++) {
        const GemvJob &J = b->job[j];
        const size_t l = gemv_lds_bytes(M, J.in_dim, J.R, J.pro.mode == PRO_NORM, pj);
        lds = l > lds ? l : lds;
    }
    if (lds > gemv_lds_limit()) return -1;
    if (modes == MODES_X) pj = 0;
    else if (modes == MB(PRO_COMBINE)) modes = MODES_CS;
    else if (modes == MB(PRO_FOLD)) modes = MODES_NF;
    else if (modes != MODES_N && modes != MODES_NF && modes != MODES_S && modes != MODES_CS) return -1;
    if (b->amax_part) {
        // the argmax epilogue: one pre-quantized job, partials for every tile
        if (b->n != 1 || modes != MODES_X || (b->amax_mode != 0 && b->amax_mode != 1) ||
            (size_t)tiles * (size_t)m > (size_t)b->amax_cap)
            return -1;
        modes |= MA;
    }
    modes |= grouped;
    switch (M * 100000 + pj * 1000 + modes) {
        GEMV_CASES_M(1)
        GEMV_CASES_M(2)
        GEMV_CASES_M(4)
        GEMV_CASES_M(5)
        GEMV_CASES_M(6)
        GEMV_CASES_M(8)
    default:
        return -1;
    }
    return (int)hipGetLastError();
}

// Tiles of a GEMV over `rows` rows of in_dim with m token rows.
extern "C" int l98k_gemv_tiles(int rows, int in_dim, int m) {
    const int R = gemv_rows_per_tile(in_dim, gemv_slots(m));
    return (rows + R - 1) / R;
}

// Whether a GEMV over m rows of width in_dim with a fused RMSNorm prologue
// fits the kernel's LDS.
extern "C" int l98k_gemv_norm_fits(int in_dim, int m) {
    if (in_dim > PRO_MAX_IN || m < 1 || m > MAX_CHUNK) return 0;
    const int M = gemv_slots(m);
    return gemv_lds_bytes(M, in_dim, gemv_rows_per_tile(in_dim, M), 1, pro_pj(in_dim)) <= gemv_lds_limit();
}


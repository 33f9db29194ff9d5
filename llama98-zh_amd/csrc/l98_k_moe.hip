// Routed-expert kernels: in-block routing and grouped expert GEMVs
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_gemv.h"

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
    gemv_tile<M, PJ, MODES_S>(J.q + ((size_t)e * out_rows + row0) * in_dim, J.s + (size_t)e * out_rows,
                             imin(R, out_rows - row0), R, in_dim, J.pro, J.xq, J.xqs, xrow, s_orow, nm, false, J.out,
                             out_rows, row0, nullptr, 0, smem, s_inv, tab);
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
    gemv_tile<M, PJ, MODES_Q>(J.q + ((size_t)e * out_rows + row0) * in_dim, J.s + (size_t)e * out_rows,
                             imin(R, out_rows - row0), R, in_dim, J.pro, J.xq, J.xqs, xrow, s_orow, nm, false, J.out,
                             out_rows, row0, nullptr, 0, smem, s_inv, tab);
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_moe(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

// Member slots of a grouped expert launch: a power of two >= nt.
static int expert_m(int nt) { return nt <= 1 ? 1 : nt <= 2 ? 2 : nt <= 4 ? 4 : 8; }

#define EXPERT_CASE(KERNEL, M_, PJ_, ...)                                                \
    case M_ * 16 + PJ_:                                                                  \
        ALLOW_BIG_LDS((KERNEL<M_, PJ_>));                                                \
        hipLaunchKernelGGL((KERNEL<M_, PJ_>), __VA_ARGS__);                              \
        break;
#define EXPERT_DISPATCH(KERNEL, M, PJ, ...)                                              \
    do {                                                                                 \
        switch (M * 16 + PJ) {                                                           \
            EXPERT_CASE(KERNEL, 1, 1, __VA_ARGS__) EXPERT_CASE(KERNEL, 1, 2, __VA_ARGS__)  \
            EXPERT_CASE(KERNEL, 1, 4, __VA_ARGS__) EXPERT_CASE(KERNEL, 2, 1, __VA_ARGS__)  \
            EXPERT_CASE(KERNEL, 2, 2, __VA_ARGS__) EXPERT_CASE(KERNEL, 2, 4, __VA_ARGS__)  \
            EXPERT_CASE(KERNEL, 4, 1, __VA_ARGS__) EXPERT_CASE(KERNEL, 4, 2, __VA_ARGS__)  \
            EXPERT_CASE(KERNEL, 4, 4, __VA_ARGS__) EXPERT_CASE(KERNEL, 8, 1, __VA_ARGS__)  \
            EXPERT_CASE(KERNEL, 8, 2, __VA_ARGS__) EXPERT_CASE(KERNEL, 8, 4, __VA_ARGS__)  \
        default: return -1;                                                              \
        }                                                                                \
    } while (0)

// The expert launches build their activation rows with one float prologue
// of width <= 1024: quantize (the up projections, k_moe_up) or SiLU-mul then
// quantize (the down projection, k_expert_gemv).
static bool expert_jobs_ok(const ExpertJob *jobs, int n_jobs, int in_dim, int mode) {
    if (n_jobs < 1 || n_jobs > 2 || in_dim < 32 || (in_dim & 31) || in_dim > 1024) return false;
    for (int j = 0; j < n_jobs; j++)
        if (jobs[j].pro.mode != mode || !prologue_ok(jobs[j].pro, in_dim, jobs[j].xq, jobs[j].xqs)) return false;
    return true;
}

extern "C" int l98k_expert_gemv(const ExpertJob *jobs, int n_jobs, const MoeGroups *grp, int max_groups,
                                int in_dim, int out_rows, int nt, hipStream_t st) {
    if (!expert_jobs_ok(jobs, n_jobs, in_dim, PRO_SILU) || max_groups < 1 || max_groups > MAX_PAIRS || nt < 1 ||
        nt > MAX_CHUNK)
        return -1;
    const int M = expert_m(nt);
    const int R = gemv_rows_per_tile(in_dim, M);
    const int tiles = (out_rows + R - 1) / R;
    const size_t lds = gemv_lds_bytes(M, in_dim, R, 0, 0);
    if (lds > gemv_lds_limit()) return -1;
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
        nt * topk > MAX_PAIRS || nt * E > 4 * GEMV_THREADS || !expert_jobs_ok(jobs, n_jobs, in_dim, PRO_QUANT))
        return -1;
    const int max_groups = nt * topk < E ? nt * topk : E;
    const int M = expert_m(nt);
    const int R = gemv_rows_per_tile(in_dim, M);
    const int tiles = (out_rows + R - 1) / R;
    const size_t lds = gemv_lds_bytes(M, in_dim, R, 0, 0);
    if (lds > gemv_lds_limit()) return -1;
    const int pj = pro_pj(in_dim);
    const dim3 grid(n_jobs * max_groups * tiles), blk(GEMV_THREADS);
    const ExpertJob &a = jobs[0], &b2 = n_jobs > 1 ? jobs[1] : jobs[0];
    EXPERT_DISPATCH(k_moe_up, M, pj, grid, blk, lds, st, a, b2, logits, bias, E, topk, nt, sel_idx, sel_w, grp, tally,
                    max_groups, in_dim, out_rows, R, tiles);
    return (int)hipGetLastError();
}


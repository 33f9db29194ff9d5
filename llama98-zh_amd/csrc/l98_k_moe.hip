// Routed-expert kernels: in-block routing and grouped expert GEMVs
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_gemv.h"

// Grouped expert GEMV: block -> (projection jb, group gi, tile).  Group gi
// is one distinct expert of the chunk with its member (token, slot) pairs;
// its weight rows stream once for all members.  Output row = pair.
template <int M, int PJ, int G>
__global__ __launch_bounds__(GEMV_THREADS) void k_expert_gemv(ExpertJob j0, ExpertJob j1,
                                                              const MoeGroups *__restrict__ grp,
                                                              int max_groups, int in_dim, int out_rows, int R,
                                                              int tiles) {
    extern __shared__ __align__(16) char smem[];
    __shared__ int s_orow[M];
    __shared__ float s_inv[M], tab[32];
    const int tile = blockIdx.x, gi = blockIdx.y, jb = blockIdx.z;   // grid (tiles, max_groups, jobs)
    (void)max_groups;
    const ExpertJob J = jb == 0 ? j0 : j1;
    // the group's table entries in one batch, before the group count is
    // known (gi < max_groups <= MAX_PAIRS keeps every read inside the table;
    // a block past the count returns before it uses them), so the weights
    // and activations wait on one round trip instead of three
    const int ng = grp->n_groups, e = grp->expert[gi], nm = grp->n_members[gi];
    int memv[M];
#pragma unroll
    for (int t = 0; t < M; t++) memv[t] = grp->member[gi][t];
    if (gi >= ng) return;
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) {
        int mem = memv[0];
#pragma unroll
        for (int u = 1; u < M; u++)
            if (u == t && t < nm) mem = memv[u];
        xrow[t] = J.xq_by_pair ? mem : grp->pair_token[mem];
        if (threadIdx.x == t) s_orow[t] = mem;
    }
    const int row0 = tile * R;
    const int nws = (G && J.gs > 0 && J.gs < in_dim) ? in_dim / J.gs : 1;
    gemv_tile<M, PJ, MODES_S | G>(J.q + ((size_t)e * out_rows + row0) * in_dim, J.s + (size_t)e * out_rows * nws,
                             imin(R, out_rows - row0), R, in_dim, J.pro, J.xq, J.xqs, xrow, s_orow, nm, false, J.out,
                             out_rows, row0, nullptr, 0, smem, s_inv, tab, J.gs);
}

// ----------------------------------------------------------------- MoE ---

// Routing for every token of the chunk (lz_moe_route, src/ops_moe.c:12-163:
// sigmoid scores, key = score + bias for selection only, top_k rounds of a
// strict-greater argmax over the keys not yet taken, weights renormalized
// by their serial sum).  Wave w routes tokens w and w + 4, lane l holds
// experts l and l + 64.  One round is the reference's scan restated for a
// wave (src/ops_moe.c:130-142): the candidates are the keys not <= the
// sentinel -1e30 (taken ones leave the set); when the first candidate's key
// is NaN nothing beats it and it wins, otherwise the winner is the lowest
// index whose key equals the largest non-NaN candidate key (ties and
// -0 == +0 go to the earlier index).  Without NaN keys a round is one
// integer max over order-preserving images of the keys.  Then the chunk's distinct experts (a
// bit set): group g is the g-th selected expert in ascending order, its
// members the (token, slot) pairs that picked it, in pair order
// (route_group).  Every block of the expert launch computes the same tables
// from the same router logits, so the experts' weights need no separate
// routing launch.  GEMV_THREADS threads; E <= 128, nt <= 8.  Contains
// block barriers.
struct __align__(16) RouteLds {
    __align__(16) int sel[MAX_PAIRS];
    float w[MAX_PAIRS];
    int tok[MAX_PAIRS];                       // token of pair p (p / topk)
    unsigned long long tmask[MAX_CHUNK][2];   // token t's selected experts
};
struct RouteSet {
    unsigned long long lo, hi;           // selected experts of the chunk, one bit each
    int ng;                              // distinct experts
};

// Inclusive DPP max scan step (lanes outside the source row read -inf);
// after the six row_shr / row_bcast steps lane 63 holds the wave's largest
// value
#define L98_DPP_FMAX(x, ctrl, rmask) \
    (x) = fmaxf((x), __int_as_float(__builtin_amdgcn_update_dpp((int)0xFF800000u, __float_as_int(x), (ctrl), (rmask), 0xF, false)))

// Order-preserving unsigned image of a non-NaN float (-0 taken as +0, as
// the selection loop's comparisons see it); every image is >= 1.
__device__ __forceinline__ uint32_t route_ord(float x) {
    const uint32_t b = u_from_f(x == 0.0f ? 0.0f : x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
#define L98_DPP_UMAX(x, ctrl, rmask)                                                              \
    do {                                                                                          \
        const uint32_t o_ = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(x), (ctrl), (rmask), 0xF, true); \
        (x) = o_ > (x) ? o_ : (x);                                                                \
    } while (0)

// One token's top_k rounds in one wave: S key slots per lane (experts lane
// and lane + 64).  Lanes k < topk write the token's pair k.
template <int S>
__device__ __forceinline__ void route_token(const float (&lg)[2], const float (&bs)[2], int E, int topk, int t,
                                            RouteLds &R, const float *tab) {
    const float SENT = -1e30f;
    const int lane = threadIdx.x & 63;
    float sc[S], key[S];
    bool live[S];
    unsigned long long nanm = 0ull;
#pragma unroll
    for (int s = 0; s < S; s++) {
        sc[s] = d_sigmoid(lg[s], tab);
        key[s] = sc[s] + bs[s];
        live[s] = lane + 64 * s < E;
        nanm |= __ballot(live[s] && key[s] != key[s]);
    }
    int ek[MAX_TOPK];
    float wk[MAX_TOPK];
    float wsum = 0.0f;
    unsigned long long mlo = 0ull, mhi = 0ull;
    const int rounds = imin(topk, E);
    if (nanm == 0ull) {
        // no NaN key: the winner is the lowest index holding the largest
        // candidate key, found as the largest order image (0 = none left)
        uint32_t u[S];
#pragma unroll
        for (int s = 0; s < S; s++) u[s] = (live[s] && !(key[s] <= SENT)) ? route_ord(key[s]) : 0u;
#pragma unroll
        for (int k = 0; k < MAX_TOPK; k++) {
            ek[k] = -1;
            wk[k] = 0.0f;
            if (k >= rounds) continue;
            uint32_t v = u[0];
            if (S == 2) v = u[S - 1] > v ? u[S - 1] : v;
            L98_DPP_UMAX(v, 0x111, 0xF);
            L98_DPP_UMAX(v, 0x112, 0xF);
            L98_DPP_UMAX(v, 0x114, 0xF);
            L98_DPP_UMAX(v, 0x118, 0xF);
            L98_DPP_UMAX(v, 0x142, 0xA);
            L98_DPP_UMAX(v, 0x143, 0xC);
            const uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
            if (m == 0u) continue;
            const unsigned long long b0 = __ballot(u[0] == m);
            int best;
            if (S == 1 || b0) {
                best = __builtin_ctzll(b0);
                mlo |= 1ull << best;
                if (lane == best) u[0] = 0u;
            } else {
                best = 64 + __builtin_ctzll(__ballot(u[S - 1] == m));
                mhi |= 1ull << (best - 64);
                if (lane == best - 64) u[S - 1] = 0u;
            }
            ek[k] = best;
            wk[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best < 64 ? sc[0] : sc[S - 1]), best & 63));
            wsum += wk[k];
        }
    } else {
        // a NaN key: the loop's own order (the first remaining candidate
        // wins when its key is NaN; NaN never beats a number)
#pragma unroll
        for (int k = 0; k < MAX_TOPK; k++) {
            ek[k] = -1;
            wk[k] = 0.0f;
            if (k >= rounds) continue;
            bool c[S];
            unsigned long long b[2] = {0ull, 0ull};
#pragma unroll
            for (int s = 0; s < S; s++) {
                c[s] = live[s] && !(key[s] <= SENT);
                b[s] = __ballot(c[s]);
            }
            if ((b[0] | b[1]) == 0ull) continue;
            const int f = b[0] ? __builtin_ctzll(b[0]) : 64 + __builtin_ctzll(b[1]);
            const float kf =
                __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f < 64 ? key[0] : key[S - 1]), f & 63));
            int best = f;
            if (kf == kf) {
                float mx = -INFINITY;
#pragma unroll
                for (int s = 0; s < S; s++)
                    if (c[s] && key[s] == key[s]) mx = fmaxf(mx, key[s]);
                L98_DPP_FMAX(mx, 0x111, 0xF);
                L98_DPP_FMAX(mx, 0x112, 0xF);
                L98_DPP_FMAX(mx, 0x114, 0xF);
                L98_DPP_FMAX(mx, 0x118, 0xF);
                L98_DPP_FMAX(mx, 0x142, 0xA);
                L98_DPP_FMAX(mx, 0x143, 0xC);
                mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 63));
                const unsigned long long e0 = __ballot(c[0] && key[0] == mx);
                best = (S == 1 || e0) ? __builtin_ctzll(e0) : 64 + __builtin_ctzll(__ballot(c[S - 1] && key[S - 1] == mx));
            }
            ek[k] = best;
            wk[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best < 64 ? sc[0] : sc[S - 1]), best & 63));
            wsum += wk[k];
            if (best < 64) {
                mlo |= 1ull << best;
                if (lane == best) key[0] = SENT;
            } else {
                mhi |= 1ull << (best - 64);
                if (lane == best - 64) key[S - 1] = SENT;
            }
        }
    }
    int my_e = -1;
    float my_w = 0.0f;
#pragma unroll
    for (int k = 0; k < MAX_TOPK; k++)
        if (lane == k) { my_e = ek[k]; my_w = wk[k]; }
    if (my_e >= 0 && wsum > 0.0f) my_w /= wsum;
    if (lane < topk) {
        R.sel[t * topk + lane] = my_e;
        R.w[t * topk + lane] = my_w;
        R.tok[t * topk + lane] = t;
    }
    if (lane == 0) {
        R.tmask[t][0] = mlo;
        R.tmask[t][1] = mhi;
    }
}

__device__ __forceinline__ RouteSet route_block(const float *__restrict__ logits, const float *__restrict__ bias,
                                                int E, int topk, int nt, RouteLds &R, float *tab) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float tabv = c_exp_tab[tid & 31];
    float lg[2][2], bs[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int e = imin(lane + 64 * s, E - 1);
        bs[s] = bias[e];
#pragma unroll
        for (int h = 0; h < 2; h++) lg[h][s] = logits[(size_t)imin(wave + 4 * h, nt - 1) * E + e];
    }
    if (tid < 32) tab[tid] = tabv;
    __syncthreads();
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int t = wave + 4 * h;
        if (t >= nt) break;                  // wave-uniform
        if (E <= 64)
            route_token<1>(lg[h], bs, E, topk, t, R, tab);
        else
            route_token<2>(lg[h], bs, E, topk, t, R, tab);
    }
    __syncthreads();
    RouteSet rs{0ull, 0ull, 0};
    for (int t = 0; t < nt; t++) {
        rs.lo |= R.tmask[t][0];
        rs.hi |= R.tmask[t][1];
    }
    rs.ng = __popcll(rs.lo) + __popcll(rs.hi);
    return rs;
}

// Expert of distinct group gi (the gi-th selected expert in ascending
// order) and its member pairs in pair order (a wave-uniform scan; call from
// whole waves).  Returns the member count; mem[m] for m < count.
__device__ __forceinline__ int route_group(const RouteLds &R, const RouteSet &rs, int nt, int topk, int gi,
                                           int *e_out, int (&mem)[MAX_CHUNK]) {
    unsigned long long lo = rs.lo, hi = rs.hi;
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
template <int M, int PJ, int G>
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_up(ExpertJob j0, ExpertJob j1, const float *__restrict__ logits,
                                                         const float *__restrict__ bias, int E, int topk, int nt,
                                                         int *__restrict__ sel_idx, float *__restrict__ sel_w,
                                                         MoeGroups *__restrict__ grp, int *__restrict__ tally,
                                                         int max_groups, int in_dim, int out_rows, int R, int tiles) {
    extern __shared__ __align__(16) char smem[];
    __shared__ RouteLds rt;
    __shared__ int s_orow[M];
    __shared__ float s_inv[M], tab[32];
    const int tile = blockIdx.x, gi = blockIdx.y, jb = blockIdx.z;   // grid (tiles, max_groups, jobs)
    (void)max_groups;
    // the projection's arguments read now, so their loads overlap the routing
    const ExpertJob J = jb == 0 ? j0 : j1;
    const RouteSet rs = route_block(logits, bias, E, topk, nt, rt, tab);
    const int ng = rs.ng;
    if ((blockIdx.x | blockIdx.y | blockIdx.z) == 0) {   // publish the routing
        const int tid = threadIdx.x;
        if (tid < nt * topk) {
            sel_idx[tid] = rt.sel[tid];
            sel_w[tid] = rt.w[tid];
            grp->pair_token[tid] = tid / topk;
        }
        if (tid < E) {                     // thread e: its group slot and members, in pair order
            const int e = tid;
            const unsigned long long word = (e >> 6) ? rs.hi : rs.lo, bit = 1ull << (e & 63);
            if (word & bit) {
                const int g = __popcll(word & (bit - 1ull)) + ((e >> 6) ? __popcll(rs.lo) : 0);
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
    int e, gmem[MAX_CHUNK];
    const int nm = route_group(rt, rs, nt, topk, gi, &e, gmem);
    int xrow[M];
#pragma unroll
    for (int t = 0; t < M; t++) {
        const int mem = gmem[t < nm ? t : 0];
        xrow[t] = J.xq_by_pair ? mem : rt.tok[mem];
        if (threadIdx.x == t) s_orow[t] = mem;
    }
    const int row0 = tile * R;
    const int nws = (G && J.gs > 0 && J.gs < in_dim) ? in_dim / J.gs : 1;
    gemv_tile<M, PJ, MODES_Q | G>(J.q + ((size_t)e * out_rows + row0) * in_dim, J.s + (size_t)e * out_rows * nws,
                             imin(R, out_rows - row0), R, in_dim, J.pro, J.xq, J.xqs, xrow, s_orow, nm, false, J.out,
                             out_rows, row0, nullptr, 0, smem, s_inv, tab, J.gs);
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_moe(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

// Member slots of a grouped expert launch (>= nt): the GEMV's token slots.
static int expert_m(int nt) { return gemv_slots(nt); }

// Instances: member slots M, prologue width PJ, and G = MG for weights with
// grouped scales (0: one scale per row).
#define EXPERT_CASE(KERNEL, M_, PJ_, G_, ...)                                            \
    case ((G_) != 0 ? 256 : 0) + M_ * 16 + PJ_:                                                 \
        ALLOW_BIG_LDS((KERNEL<M_, PJ_, G_>));                                            \
        hipLaunchKernelGGL((KERNEL<M_, PJ_, G_>), __VA_ARGS__);                          \
        break;
#define EXPERT_CASES_G(KERNEL, G_, ...)                                                  \
    EXPERT_CASE(KERNEL, 1, 1, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 1, 2, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 1, 4, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 2, 1, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 2, 2, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 2, 4, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 4, 1, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 4, 2, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 4, 4, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 5, 1, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 5, 2, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 5, 4, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 6, 1, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 6, 2, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 6, 4, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 8, 1, G_, __VA_ARGS__)  \
    EXPERT_CASE(KERNEL, 8, 2, G_, __VA_ARGS__) EXPERT_CASE(KERNEL, 8, 4, G_, __VA_ARGS__)
#define EXPERT_DISPATCH(KERNEL, M, PJ, GROUPED, ...)                                     \
    do {                                                                                 \
        switch ((GROUPED ? 256 : 0) + M * 16 + PJ) {                                     \
            EXPERT_CASES_G(KERNEL, 0, __VA_ARGS__)                                       \
            EXPERT_CASES_G(KERNEL, MG, __VA_ARGS__)                                      \
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
    const dim3 grid(tiles, max_groups, n_jobs), blk(GEMV_THREADS);
    const ExpertJob &a = jobs[0], &b2 = n_jobs > 1 ? jobs[1] : jobs[0];
    const bool grouped = (a.gs && a.gs < in_dim) || (b2.gs && b2.gs < in_dim);
    EXPERT_DISPATCH(k_expert_gemv, M, pj, grouped, grid, blk, lds, st, a, b2, grp, max_groups, in_dim, out_rows, R,
                    tiles);
    return (int)hipGetLastError();
}

extern "C" int l98k_moe_up(const ExpertJob *jobs, int n_jobs, const float *logits, const float *bias, int E,
                           int topk, int nt, int *sel_idx, float *sel_w, MoeGroups *grp, int *tally, int in_dim,
                           int out_rows, hipStream_t st) {
    if (E > MAX_EXPERTS || E < topk || topk < 1 || topk > MAX_TOPK || nt < 1 || nt > MAX_CHUNK ||
        nt * topk > MAX_PAIRS || !expert_jobs_ok(jobs, n_jobs, in_dim, PRO_QUANT))
        return -1;
    const int max_groups = nt * topk < E ? nt * topk : E;
    const int M = expert_m(nt);
    const int R = gemv_rows_per_tile(in_dim, M);
    const int tiles = (out_rows + R - 1) / R;
    const size_t lds = gemv_lds_bytes(M, in_dim, R, 0, 0);
    if (lds > gemv_lds_limit()) return -1;
    const int pj = pro_pj(in_dim);
    const dim3 grid(tiles, max_groups, n_jobs), blk(GEMV_THREADS);
    const ExpertJob &a = jobs[0], &b2 = n_jobs > 1 ? jobs[1] : jobs[0];
    const bool grouped = (a.gs && a.gs < in_dim) || (b2.gs && b2.gs < in_dim);
    EXPERT_DISPATCH(k_moe_up, M, pj, grouped, grid, blk, lds, st, a, b2, logits, bias, E, topk, nt, sel_idx, sel_w, grp,
                    tally, max_groups, in_dim, out_rows, R, tiles);
    return (int)hipGetLastError();
}

// The routing of k_moe_up alone (one block): sel_idx / sel_w as k_moe_up
// publishes them, nt * topk pairs in (token, slot) order.
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_route(const float *__restrict__ logits,
                                                            const float *__restrict__ bias, int E, int topk, int nt,
                                                            int *__restrict__ sel_idx, float *__restrict__ sel_w) {
    __shared__ RouteLds rt;
    __shared__ float tab[32];
    (void)route_block(logits, bias, E, topk, nt, rt, tab);
    const int tid = threadIdx.x;
    if (tid < nt * topk) {
        sel_idx[tid] = rt.sel[tid];
        sel_w[tid] = rt.w[tid];
    }
}

extern "C" int l98k_moe_route(const float *logits, const float *bias, int E, int topk, int nt, int *sel_idx,
                              float *sel_w, hipStream_t st) {
    if (E < 1 || E > MAX_EXPERTS || topk < 1 || topk > MAX_TOPK || nt < 1 || nt > MAX_CHUNK || nt * topk > MAX_PAIRS)
        return -1;
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(GEMV_THREADS), 0, st, logits, bias, E, topk, nt, sel_idx, sel_w);
    return (int)hipGetLastError();
}


// ------------------------------------------------------ wide routing ---
// Routing of many token rows: block g routes rows [8 g, 8 g + 8) with the
// in-block router above (lz_moe_route per token, src/ops_moe.c:12-163), so
// every row's selection and weights are those of the chunked path.  With
// lx, the same rows of the latent lx[row][lat] (lat % 32 == 0, <= 4096)
// are quantized per 32 into lq / lqs by the block's waves, a row per wave
// at a time, lane l taking float4 l + 64 j: the wide producers' quantize
// mode (quant_octet), so the expert GEMMs' input takes no launch of its own.
__global__ __launch_bounds__(GEMV_THREADS) void k_moe_route_wide(const float *__restrict__ logits,
                                                                 const float *__restrict__ bias, int E, int topk,
                                                                 int rows, int *__restrict__ sel_idx,
                                                                 float *__restrict__ sel_w,
                                                                 const float *__restrict__ lx, int lat,
                                                                 int8_t *__restrict__ lq, float *__restrict__ lqs) {
    __shared__ RouteLds rt;
    __shared__ float tab[32];
    const int r0 = blockIdx.x * MAX_CHUNK;
    const int nt = imin(MAX_CHUNK, rows - r0);
    (void)route_block(logits + (size_t)r0 * E, bias, E, topk, nt, rt, tab);
    const int tid = threadIdx.x;
    if (tid < nt * topk) {
        sel_idx[(size_t)r0 * topk + tid] = rt.sel[tid];
        sel_w[(size_t)r0 * topk + tid] = rt.w[tid];
    }
    if (lx) {
        const int lane = tid & 63, nf = lat >> 2, nb = lat >> 5;
        for (int r = tid >> 6; r < nt; r += GEMV_THREADS / 64) {
            const size_t row = (size_t)(r0 + r);
            for (int j = 0; 64 * j < nf; j++) {           // wave-uniform
                const int f = lane + 64 * j, fc = f < nf ? f : nf - 1;
                const float4 v = reinterpret_cast<const float4 *>(lx + row * lat)[fc];
                float sg;
                const uint32_t q = quant_octet(v, &sg);
                if (f < nf) {
                    reinterpret_cast<uint32_t *>(lq + row * lat)[f] = q;
                    if (!(f & 7)) lqs[row * nb + (f >> 3)] = sg;
                }
            }
        }
    }
}

// The rows' (token, slot) pairs grouped by expert, for the grouped GEMMs:
// group g < *ng is expert gexp[g] (ascending) with gcnt[g] pairs at
// list[goff[g] ..]; pair_token[p] = p / topk.  Pairs without an expert
// (sel_idx < 0) join no group.  One block; the order of a group's pairs is
// free (every pair's output is computed on its own).
__global__ __launch_bounds__(1024) void k_moe_group(const int *__restrict__ sel_idx, int npairs, int topk, int E,
                                                    int *__restrict__ ng, int *__restrict__ gexp,
                                                    int *__restrict__ goff, int *__restrict__ gcnt,
                                                    int *__restrict__ list, int *__restrict__ pair_token) {
    __shared__ int cnt[MAX_EXPERTS], off[MAX_EXPERTS], cur[MAX_EXPERTS];
    const int tid = threadIdx.x;
    if (tid < MAX_EXPERTS) { cnt[tid] = 0; cur[tid] = 0; }
    __syncthreads();
    for (int p = tid; p < npairs; p += blockDim.x) {
        pair_token[p] = p / topk;
        const int e = sel_idx[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // offsets (exclusive prefix of the counts in expert order) and group
    // slots (rank of each present expert) on one wave: lane l takes experts
    // l and l + 64
    static_assert(MAX_EXPERTS <= 128, "two experts per lane");
    if (tid < 64) {
        const int c0 = tid < E ? cnt[tid] : 0, c1 = tid + 64 < E ? cnt[tid + 64] : 0;
        const uint32_t i0 = wave_scan_u32((uint32_t)c0), i1 = wave_scan_u32((uint32_t)c1);
        const int tot0 = __builtin_amdgcn_readlane((int)i0, 63);
        const int o0 = (int)i0 - c0, o1 = tot0 + (int)i1 - c1;
        const unsigned long long b0 = __ballot(c0 > 0), b1 = __ballot(c1 > 0);
        const unsigned long long below = (1ull << tid) - 1ull;
        const int n0 = __popcll(b0);
        const int g0 = __popcll(b0 & below), g1 = n0 + __popcll(b1 & below);
        off[tid] = o0;
        off[tid + 64] = o1;
        if (c0) { gexp[g0] = tid; goff[g0] = o0; gcnt[g0] = c0; }
        if (c1) { gexp[g1] = tid + 64; goff[g1] = o1; gcnt[g1] = c1; }
        if (tid == 0) *ng = n0 + __popcll(b1);
    }
    __syncthreads();
    for (int p = tid; p < npairs; p += blockDim.x) {
        const int e = sel_idx[p];
        if (e >= 0 && e < E) list[off[e] + atomicAdd(&cur[e], 1)] = p;
    }
}

extern "C" int l98k_moe_route_wide(const float *logits, const float *bias, int E, int topk, int rows, int *sel_idx,
                                   float *sel_w, const float *lx, int lat, int8_t *lq, float *lqs, hipStream_t st) {
    if (E < 1 || E > MAX_EXPERTS || topk < 1 || topk > MAX_TOPK || rows < 1) return -1;
    if (lx && (!lq || !lqs || lat < 32 || (lat & 31) || lat > 4096)) return -1;
    hipLaunchKernelGGL(k_moe_route_wide, dim3((rows + MAX_CHUNK - 1) / MAX_CHUNK), dim3(GEMV_THREADS), 0, st, logits,
                       bias, E, topk, rows, sel_idx, sel_w, lx, lat, lq, lqs);
    return (int)hipGetLastError();
}

extern "C" int l98k_moe_group(const int *sel_idx, int npairs, int topk, int E, int *ng, int *gexp, int *goff,
                              int *gcnt, int *list, int *pair_token, hipStream_t st) {
    if (npairs < 1 || E < 1 || E > MAX_EXPERTS || topk < 1) return -1;
    hipLaunchKernelGGL(k_moe_group, dim3(1), dim3(1024), 0, st, sel_idx, npairs, topk, E, ng, gexp, goff, gcnt, list,
                       pair_token);
    return (int)hipGetLastError();
}

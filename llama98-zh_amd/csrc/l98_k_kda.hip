// KDA gated-delta kernels: causal conv and the fp32-state recurrence
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_devmath.h"

typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------- KDA layer ---
//
// One block of 4*kd threads per head (nk == nv).  The conv phase gives
// thread group g = tid / kd row type g (q, k, v, output gate input) of
// channel tid % kd for every token, the gate rows go to the groups token by
// token, and the later channel phases use the first group; the recurrence
// uses a lane quad per state column: thread 4c + r holds rows
// [r*kd/4, (r+1)*kd/4) of column c of the fp32 state S[kd][vd].  The ring
// slot stores a head's state in that thread order: float4 i of thread t
// (rows r*kd/4 + 4i .. + 3 of column c) at float4 index i * 4kd + t of the
// head, so each load or store instruction of the block moves 4kd
// consecutive float4s (the recurrence kernels are the state's only
// readers and writers).
// For the chunk's tokens, in one launch:
//   * the depthwise causal conv + SiLU of the q, k and v channels along the
//     ring (lz_causal_conv1d_step, src/ops_conv1d.c:26-87: taps summed in
//     order, then the current input; ring slots src/forward_kda.c:680-755);
//   * the gate up-projection row h*kd + j of f_b over the per-32 quantized
//     low-rank input (lz_matmul_xq_nt + epi_q8, src/ops_matmul.c:468-660,
//     src/ops_epi.c:983-1017: exact int32 group sums, groups summed in
//     order, times the row scale);
//   * the gate (src/forward_kda.c:277-300, 840-850), l2norm(q)*scale,
//     l2norm(k), beta, kq = k.q, then per token u = S^T(g.k), w = S^T(g.q),
//     delta = (v - u)*beta, out = w + delta*kq, S' = g.S + k(x)delta
//     (lz_recur_step fp32 arm, src/ops_gdn.c:2516-2560; call site
//     src/forward_kda.c:856-940), every state written to its ring slot.
//     u and w keep the reference's row order: the quad's first lane sums
//     its rows from 0, passes the partial to the next lane (DPP), which
//     continues with its rows, and so on; the row products and the state
//     update are spread over the quad;
//   * the per-head gated RMSNorm and the per-32 quantization for o_proj
//     (src/forward_kda.c:1000-1043).
// Work that does not depend on the state is done for all NT token slots at
// once (NT in {1, 2, 4, 5, 6, 8}, >= nt; slots past nt repeat the last token and
// store nothing), as straight-line code with independent work per token.
__device__ __forceinline__ float dpp_quad_shr1(float v) {        // lane r <- lane r-1 (lane 0 keeps its own)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x90, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad_bcast3(float v) {      // every lane <- lane 3 of its quad
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xFF, 0xF, 0xF, false));
}

// One token of the recurrence on the lane quads: c = kn.g, q = qn.g*scale,
// g and b = kn are LDS rows of the token (the lane reads its rows row0 ..
// row0 + kd/4), vt its v for the lane's column.  Every LDS read is issued at
// the top (one wait, not one per use).  Returns o on every lane of the quad
// and leaves S' in S.
template <int KD>
__device__ __forceinline__ float kda_token(float (&S)[KD / 4], const float *sc, const float *sa, const float *sg,
                                           const float *sb, const float *pv, const float *pbeta,
                                           const float *pkq, int row0) {
    constexpr int RPL = KD / 4;
    float4 c4[RPL / 4], a4[RPL / 4], g4[RPL / 4], b4[RPL / 4];
#pragma unroll
    for (int i = 0; i < RPL / 4; i++) {
        c4[i] = *reinterpret_cast<const float4 *>(&sc[row0 + 4 * i]);
        a4[i] = *reinterpret_cast<const float4 *>(&sa[row0 + 4 * i]);
        g4[i] = *reinterpret_cast<const float4 *>(&sg[row0 + 4 * i]);
        b4[i] = *reinterpret_cast<const float4 *>(&sb[row0 + 4 * i]);
    }
    const float vt = *pv, bt = *pbeta, kqt = *pkq;
    __builtin_amdgcn_sched_barrier(0);
    float pu[RPL], pw[RPL];
#pragma unroll
    for (int i = 0; i < RPL / 4; i++) {
        pu[4 * i] = S[4 * i] * c4[i].x; pu[4 * i + 1] = S[4 * i + 1] * c4[i].y;
        pu[4 * i + 2] = S[4 * i + 2] * c4[i].z; pu[4 * i + 3] = S[4 * i + 3] * c4[i].w;
        pw[4 * i] = S[4 * i] * a4[i].x; pw[4 * i + 1] = S[4 * i + 1] * a4[i].y;
        pw[4 * i + 2] = S[4 * i + 2] * a4[i].z; pw[4 * i + 3] = S[4 * i + 3] * a4[i].w;
    }
    float u = 0.0f, w = 0.0f;
#pragma unroll
    for (int ph = 0; ph < 4; ph++) {
        if (ph) { u = dpp_quad_shr1(u); w = dpp_quad_shr1(w); }
#pragma unroll
        for (int i = 0; i < RPL; i++) { u += pu[i]; w += pw[i]; }
    }
    u = dpp_quad_bcast3(u);
    w = dpp_quad_bcast3(w);
    const float ut = (vt - 1.0f * u) * bt;
    const float o = 1.0f * w + ut * kqt;
#pragma unroll
    for (int i = 0; i < RPL / 4; i++) {
        S[4 * i] = S[4 * i] * g4[i].x + b4[i].x * ut;
        S[4 * i + 1] = S[4 * i + 1] * g4[i].y + b4[i].y * ut;
        S[4 * i + 2] = S[4 * i + 2] * g4[i].z + b4[i].z * ut;
        S[4 * i + 3] = S[4 * i + 3] * g4[i].w + b4[i].w * ut;
    }
    return o;
}

// The per-head gated RMSNorm of the recurrence outputs s_o[t][0..vd) with
// the silu'd output gate s_z (src/ops_norm.c:749-793: the sum of o^2 in
// index order, inv = rsqrt(ss/vd + eps), ((o*inv)*w)*z), then the per-32
// quantization of the rows for o_proj (src/forward_kda.c:1000-1043).  s_sq,
// s_y: LDS rows the tail may overwrite.  All 4*kd threads of the block.
template <int KD, int NT>
__device__ __forceinline__ void kda_gated_tail(const KdaStepArgs &a, int h, int nt, int j, float onw,
                                               float (*s_o)[KD], const float (*s_z)[KD], float (*s_sq)[KD],
                                               float (*s_y)[KD], float *s_oinv) {
    constexpr int VD = KD, NTHR = 4 * KD;
    constexpr int NO4 = (NT * VD / 4 + NTHR - 1) / NTHR;                // float4 of the output per thread
    const int tid = threadIdx.x, value = a.value;
    const bool chan = tid < KD;
    if (chan) {
#pragma unroll
        for (int t = 0; t < NT; t++)
            if (t < nt) s_sq[t][j] = s_o[t][j] * s_o[t][j];
    }
    __syncthreads();
    if (tid < nt) s_oinv[tid] = d_rsqrt(d_ss_over_n(serial_sum_n<VD>(s_sq[tid]), VD) + a.eps);
    __syncthreads();
    float yv[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tc = imin(t, nt - 1);
        yv[t] = s_o[tc][j] * s_oinv[tc] * onw * s_z[t][j];
    }
    if (chan) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < nt) {
                if (a.normed_out) a.normed_out[(size_t)t * value + h * VD + j] = yv[t];
                s_y[t][j] = yv[t];
            }
        }
    }
    __syncthreads();
    const int no4 = nt * VD / 4;
#pragma unroll
    for (int u = 0; u < NO4; u++) {
        const int f = u * NTHR + tid;
        const int fc = imin(f, no4 - 1);
        const int t = (4 * fc) / VD, c = 4 * fc - t * VD;
        float sg;
        const uint32_t q = quant_octet(*reinterpret_cast<const float4 *>(&s_y[t][c]), &sg);
        if (f < no4) {
            reinterpret_cast<uint32_t *>(a.xq + (size_t)t * value + h * VD)[c >> 2] = q;
            if (!(c & 31)) a.xqs[(size_t)t * (value >> 5) + ((h * VD + c) >> 5)] = sg;
        }
    }
}

template <int KD, int K, int NT, bool PRE = false>
__device__ __forceinline__ void kda_step_body(const KdaStepArgs &a, int h) {
    constexpr int VD = KD, HIST = K - 1, NTHR = 4 * KD, RPL = KD / 4;
    constexpr int NF4 = (NT * KDA_MAX_RANK / 4 + NTHR - 1) / NTHR;      // float4 of the gate input per thread
    EXP_TAB_LOAD(tab);
    __shared__ __align__(16) float s_a[MAX_CHUNK][KD];   // q, then q.g*invq*scale (qcw), then y
    __shared__ __align__(16) float s_b[MAX_CHUNK][KD];   // k, then k*invk (kn)
    __shared__ __align__(16) float s_g[MAX_CHUNK][KD];   // decay gate
    __shared__ __align__(16) float s_c[MAX_CHUNK][KD];   // q^2, then kn*g (kcw), then o^2
    __shared__ __align__(16) float s_d[MAX_CHUNK][KD];   // k^2, then o
    __shared__ __align__(16) float s_v[MAX_CHUNK][KD];   // conv v
    __shared__ __align__(16) int8_t s_fq[MAX_CHUNK * KDA_MAX_RANK];
    __shared__ float s_fs[MAX_CHUNK * KDA_MAX_RANK / 32];
    __shared__ float s_invq[MAX_CHUNK], s_invk[MAX_CHUNK], s_beta[MAX_CHUNK], s_kq[MAX_CHUNK],
        s_oinv[MAX_CHUNK];
    __shared__ __align__(16) float s_z[MAX_CHUNK][KD];   // silu of the output gate input
    const int tid = threadIdx.x;
    // Channel phases: thread group grp = tid / kd takes row type grp (0: q,
    // 1: k, 2: v, 3: the output gate input) of channel j for every token, and
    // the gate rows of tokens grp, grp + 4, ...; the later phases use the
    // first group (tid < kd, j = tid).
    const int grp = tid / KD, j = tid - grp * KD;
    const int col = tid >> 2, quarter = tid & 3, row0 = quarter * RPL;
    const int nt = a.nt, key = a.key, value = a.value, rank = a.rank;
    const size_t head_off = (size_t)h * KD * VD;
    const int base = *a.ctl_slot;
    // ring slot written after token 0: (base % depth) + 1, wrapping, when
    // advancing (token t: t slots further, wrapping), else base
    int so0 = base;
    if (a.advance) {
        const int si0 = base % a.depth;
        so0 = si0 + 1 == a.depth ? 0 : si0 + 1;
    }
    // ---- loads: the thread's row of every token, conv taps and history,
    // gate input, f_b row, state
    const int cch = grp == 0 ? h * KD + j : grp == 1 ? key + h * KD + j : 2 * key + h * VD + imin(j, VD - 1);
    const float *xsrc = grp == 0 ? a.pq : grp == 1 ? a.pk : grp == 2 ? a.pv : a.gz;
    const int xstride = grp < 2 ? key : value;
    float xin[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) xin[t] = xsrc[(size_t)imin(t, nt - 1) * xstride + h * KD + j];
    const int nfa4 = nt * rank / 4;
    float4 fa4[NF4];
#pragma unroll
    for (int u = 0; u < NF4; u++) fa4[u] = reinterpret_cast<const float4 *>(a.pfa)[imin(u * NTHR + tid, nfa4 - 1)];
    float wc[K], hc[HIST > 0 ? HIST : 1];
#pragma unroll
    for (int i = 0; i < K; i++) wc[i] = a.conv_w[(size_t)cch * K + i];
    if (PRE && a.hist_rows) {
        // the inputs of the HIST rows before row 0 (earlier rows of the same prefill)
#pragma unroll
        for (int i = 0; i < HIST; i++) hc[i] = xsrc[(ptrdiff_t)(i - HIST) * xstride + h * KD + j];
    } else {
        const float *r0 = a.conv_ring + (size_t)base * a.conv_slot_stride;
#pragma unroll
        for (int i = 0; i < HIST; i++) hc[i] = r0[(size_t)cch * HIST + i];
    }
    const int4 *fbrow = reinterpret_cast<const int4 *>(a.fb_q + (size_t)(h * KD + j) * rank);
    int4 fbw[KDA_MAX_RANK / 16];
#pragma unroll
    for (int u = 0; u < KDA_MAX_RANK / 16; u++) fbw[u] = fbrow[imin(u, (rank >> 4) - 1)];
    // f_b's scales: one per row, or rank/fb_gs per row (groups of fb_gs)
    const int fb_nws = (a.fb_gs > 0 && a.fb_gs < rank) ? rank / a.fb_gs : 1;
    float fbsv[KDA_MAX_RANK / 32];
#pragma unroll
    for (int u = 0; u < KDA_MAX_RANK / 32; u++) fbsv[u] = a.fb_s[(size_t)(h * KD + j) * fb_nws + imin(u, fb_nws - 1)];
    const float fbs = fbsv[0];
    const float bv = a.bvec[(size_t)imin(j, nt - 1) * a.nv + h];
    const float dtb = a.dt_bias[h * KD + j];
    const float onw = a.o_norm[j];
    const float alog = a.a_log[h];
    float S[RPL];
    if constexpr (!PRE) {
        const float4 *src = reinterpret_cast<const float4 *>(a.state + (size_t)base * a.slot_stride + head_off) + tid;
#pragma unroll
        for (int i = 0; i < RPL / 4; i++) {
            const float4 q = src[i * NTHR];
            S[4 * i] = q.x; S[4 * i + 1] = q.y; S[4 * i + 2] = q.z; S[4 * i + 3] = q.w;
        }
    }
    EXP_TAB_PUT(tab);
    // ---- per-32 quantization of the gate input: four values per thread, a
    // group per aligned lane octet (rank % 32 == 0)
#pragma unroll
    for (int u = 0; u < NF4; u++) {
        float sg;
        const uint32_t q = quant_octet(fa4[u], &sg);
        const int f = u * NTHR + tid;
        if (f < nfa4) {
            reinterpret_cast<uint32_t *>(s_fq)[f] = q;
            if (!(f & 7)) s_fs[f >> 3] = sg;
        }
    }
    __syncthreads();                     // gate input quantized, exp table in place
    // ---- conv + silu of the thread's row, all token slots: token t reads
    // history seq[t .. t+HIST-1] and input seq[t+HIST], seq = [ring history |
    // the chunk's inputs]; the output gate input only takes the silu
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float sc = 0.0f;
#pragma unroll
        for (int i = 0; i < HIST; i++) {
            const int si = t + i;                          // position in seq
            sc += wc[i] * (si < HIST ? hc[si < HIST ? si : 0] : xin[si >= HIST ? si - HIST : 0]);
        }
        sc += wc[HIST] * xin[t];
        const float y = d_silu(grp == 3 ? xin[t] : sc, tab);
        if (grp == 0) { s_a[t][j] = y; s_c[t][j] = y * y; }
        else if (grp == 1) { s_b[t][j] = y; s_d[t][j] = y * y; }
        else if (grp == 2) { s_v[t][j] = y; }
        else s_z[t][j] = y;
    }
    // ring: the history after token t is seq[t+1 .. t+HIST] (the split
    // prefill writes it after its last row instead)
    if (!PRE && grp < 3) {
        int so_t = so0;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            if (t < nt && (a.advance || t == nt - 1)) {
                const int so = a.advance ? so_t : base;
                float *r1 = a.conv_ring + (size_t)so * a.conv_slot_stride;
#pragma unroll
                for (int i = 0; i < HIST; i++) {
                    const int si = t + 1 + i;
                    r1[(size_t)cch * HIST + i] = si < HIST ? hc[si < HIST ? si : 0] : xin[si >= HIST ? si - HIST : 0];
                }
            }
            so_t = so_t + 1 == a.depth ? 0 : so_t + 1;
        }
    }
    // ---- gate rows of tokens grp, grp + 4, ..., then the decay gate
    const float decay = d_exp(alog, tab);
#pragma unroll
    for (int t0 = 0; t0 < NT; t0 += 4) {
        const int t = t0 + grp;
        if (t < NT) {
            const int tc = imin(t, nt - 1);
            float dot = 0.0f;
            int acc0 = 0;
            int accg[KDA_MAX_RANK / 32];
#pragma unroll
            for (int g = 0; g < KDA_MAX_RANK / 32; g++) {
                accg[g] = 0;
                if (g * 32 < rank) {
                    const int4 *xr = reinterpret_cast<const int4 *>(s_fq + tc * rank + g * 32);
                    const int4 x0 = xr[0], x1 = xr[1];
                    const int4 w0 = fbw[2 * g], w1 = fbw[2 * g + 1];
                    int acc = __builtin_amdgcn_sdot4(w0.x, x0.x, 0, false);
                    acc = __builtin_amdgcn_sdot4(w0.y, x0.y, acc, false);
                    acc = __builtin_amdgcn_sdot4(w0.z, x0.z, acc, false);
                    acc = __builtin_amdgcn_sdot4(w0.w, x0.w, acc, false);
                    acc = __builtin_amdgcn_sdot4(w1.x, x1.x, acc, false);
                    acc = __builtin_amdgcn_sdot4(w1.y, x1.y, acc, false);
                    acc = __builtin_amdgcn_sdot4(w1.z, x1.z, acc, false);
                    acc = __builtin_amdgcn_sdot4(w1.w, x1.w, acc, false);
                    dot += (float)acc * s_fs[(tc * rank >> 5) + g];
                    if (g == 0) acc0 = acc;
                    accg[g] = acc;
                }
            }
            float pre = 0.0f;
            if (fb_nws > 1) {
                // grouped scales (epi_q8 with r = fb_gs/32 < rank/32)
                const int nb = rank >> 5, r = a.fb_gs >> 5;
                const float *xs = s_fs + (tc * rank >> 5);
                if (r > 1) {
                    // runs of r groups (static register indices)
                    int run = 0;
                    float d2 = 0.0f;
#pragma unroll
                    for (int g = 0; g < KDA_MAX_RANK / 32; g++) {
                        if (g < nb) {
                            d2 += (float)accg[g] * xs[g];
                            if ((g + 1) % r == 0) {
                                const float wr = run == 0 ? fbsv[0] : run == 1 ? fbsv[1] : run == 2 ? fbsv[2] : fbsv[3];
                                pre += d2 * wr;
                                d2 = 0.0f;
                                run++;
                            }
                        }
                    }
                } else {
                    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
                    if (nb == 4) {
                        a0 += (float)accg[0] * (xs[0] * fbsv[0]);
                        a1 += (float)accg[1] * (xs[1] * fbsv[1]);
                        a2 += (float)accg[2] * (xs[2] * fbsv[2]);
                        a3 += (float)accg[3] * (xs[3] * fbsv[3]);
                    } else {
#pragma unroll
                        for (int g = 0; g < KDA_MAX_RANK / 32; g++)
                            if (g < nb) a0 += (float)accg[g] * (xs[g] * fbsv[g]);
                    }
                    pre = (a0 + a2) + (a1 + a3);
                }
            } else if (rank == 32) {
                pre = epi_one_group(acc0, s_fs[tc * rank >> 5], fbs);
            } else {
                pre += dot * fbs;
            }
            // kda_gate_build_float, src/forward_kda.c:285-293
            const float p = pre + dtb;
            const float gg = a.has_lb ? a.gate_lb * d_sigmoid(decay * p, tab) : -decay * d_softplus(p, tab);
            s_g[t][j] = d_exp(gg, tab);
        }
    }
    __syncthreads();
    // Token norms (lz_l2norm at src/forward_kda.c:889-901, src/ops_norm.c:795;
    // k.q in lz_recur_step, src/ops_gdn.c:2516-2560): lane t of the first wave sums
    // q_t^2 and lane t of the second wave k_t^2, each in index order from a
    // row read whole into registers; then every thread forms its elements'
    // normalized q and k (qn = q*invq*scale, kn = k*invk) and the stored
    // products qn*g, kn*g, kn*qn; then lane t sums kn*qn in index order.
    if ((tid < nt) || (tid >= 64 && tid < 64 + nt)) {
        const int t = tid & 63;
        const float *row = tid < 64 ? s_c[t] : s_d[t];
        float4 r4[KD / 4];
#pragma unroll
        for (int i = 0; i < KD / 4; i++) r4[i] = reinterpret_cast<const float4 *>(row)[i];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < KD / 4; i++) { ss += r4[i].x; ss += r4[i].y; ss += r4[i].z; ss += r4[i].w; }
        const float inv = d_rsqrt(ss + 1e-6f);
        if (tid < 64) s_invq[t] = inv;
        else s_invk[t] = inv;
    }
    if (tid < nt) s_beta[tid] = d_sigmoid(bv, tab);
    __syncthreads();
#pragma unroll
    for (int t0 = 0; t0 < NT; t0 += 4) {
        const int t = t0 + grp;
        if (t < NT) {
            const int tc = imin(t, nt - 1);
            const float g = s_g[t][j];
            const float qn = s_a[t][j] * s_invq[tc] * a.scale;
            const float kn = s_b[t][j] * s_invk[tc];
            s_a[t][j] = qn * g;
            s_b[t][j] = kn;
            s_c[t][j] = kn * g;
            s_d[t][j] = kn * qn;
        }
    }
    __syncthreads();
    if (tid < nt) {
        float4 r4[KD / 4];
#pragma unroll
        for (int i = 0; i < KD / 4; i++) r4[i] = reinterpret_cast<const float4 *>(s_d[tid])[i];
        float kq = 0.0f;
#pragma unroll
        for (int i = 0; i < KD / 4; i++) { kq += r4[i].x; kq += r4[i].y; kq += r4[i].z; kq += r4[i].w; }
        s_kq[tid] = kq;
    }
    __syncthreads();
    if constexpr (PRE) {
        // the rows' token records for the split prefill's recurrence launch:
        // [kn.g | qn.g | g | kn | v] of the head, then beta, k.q, 0, 0
        constexpr int Q4 = KD / 4, RS4 = 5 * Q4 + 1;
        for (int f = tid; f < nt * RS4; f += NTHR) {
            const int t = f / RS4, e = f - t * RS4, seg = e / Q4, k4 = e - seg * Q4;
            const float(*arr)[KD] = seg == 0 ? s_c : seg == 1 ? s_a : seg == 2 ? s_g : seg == 3 ? s_b : s_v;
            const float4 val = seg < 5 ? reinterpret_cast<const float4 *>(arr[t])[k4]
                                       : make_float4(s_beta[t], s_kq[t], 0.0f, 0.0f);
            reinterpret_cast<float4 *>(a.rec + (size_t)t * a.nv * (4 * RS4) + (size_t)h * (4 * RS4))[e] = val;
        }
        return;
    }
    // ---- the token-serial recurrence on the lane quads; the state slot
    // advances without a division
    int so_t = so0;
#pragma unroll 1
    for (int t = 0; t < nt; t++) {
        const float o = kda_token<KD>(S, s_c[t], s_a[t], s_g[t], s_b[t], &s_v[t][col], &s_beta[t], &s_kq[t], row0);
        if (a.advance || t == nt - 1) {
            // slot (base + t) % depth + 1 (wrapping) when advancing, else base
            const int so = a.advance ? so_t : base;
            float4 *dst = reinterpret_cast<float4 *>(a.state + (size_t)so * a.slot_stride + head_off) + tid;
#pragma unroll
            for (int i = 0; i < RPL / 4; i++)
                __builtin_nontemporal_store(v4f{S[4 * i], S[4 * i + 1], S[4 * i + 2], S[4 * i + 3]},
                                            reinterpret_cast<v4f *>(dst + i * NTHR));
        }
        so_t = so_t + 1 == a.depth ? 0 : so_t + 1;
        if (quarter == 0) {
            if (a.raw_out) a.raw_out[(size_t)t * value + (size_t)h * VD + col] = o;
            s_d[t][col] = o;
        }
    }
    __syncthreads();
    kda_gated_tail<KD, NT>(a, h, nt, j, onw, s_d, s_z, s_c, s_a, s_oinv);
}

template <int KD, int K, int NT>
__global__ __launch_bounds__(4 * KD) void k_kda_step(KdaStepArgs a) {
    kda_step_body<KD, K, NT>(a, blockIdx.x);
}

// Several sessions' rows in one launch: block (head, item); item i is a
// session's rows [row0, row0 + n) against its own state and conv rings
// (layer offsets added here), in NT-row sub-chunks in order (a sub-chunk
// reads back the state and conv history the previous one wrote, from the
// same threads).  The launch's args carry the layer's weights and the row
// buffers at row 0.  Rows advance the ring only for n <= NT.  NT = 4 when
// every item has at most 4 rows (a session batch's verify at k <= 3), so
// that the token-slot work is not done for slots no item has.
template <int KD, int K, int NT>
__global__ __launch_bounds__(4 * KD) void k_kda_items(KdaStepArgs b, const KdaItem *__restrict__ items,
                                                      size_t state_off, size_t conv_off) {
    const KdaItem it = items[blockIdx.y];
    KdaStepArgs a = b;
    a.state = it.state + state_off;
    a.conv_ring = it.conv_ring + conv_off;
    a.ctl_slot = it.ctl_slot;
    a.slot_stride = it.slot_stride;
    a.conv_slot_stride = it.conv_slot_stride;
    a.depth = it.depth;
    for (int c0 = 0; c0 < it.n; c0 += NT) {
        const int r = it.row0 + c0;
        a.nt = imin(NT, it.n - c0);
        a.pq = b.pq + (size_t)r * b.key;
        a.pk = b.pk + (size_t)r * b.key;
        a.pv = b.pv + (size_t)r * b.value;
        a.pfa = b.pfa + (size_t)r * b.rank;
        a.bvec = b.bvec + (size_t)r * b.nv;
        a.gz = b.gz + (size_t)r * b.value;
        a.xq = b.xq + (size_t)r * b.value;
        a.xqs = b.xqs + (size_t)r * (b.value >> 5);
        a.raw_out = b.raw_out ? b.raw_out + (size_t)r * b.value : nullptr;
        a.normed_out = b.normed_out ? b.normed_out + (size_t)r * b.value : nullptr;
        if (c0) __syncthreads();
        kda_step_body<KD, K, NT>(a, blockIdx.x);
    }
}

// One session's prefill rows (n > MAX_CHUNK, no ring advance) in three
// launches, the same arithmetic as k_kda_items' sub-chunks:
//   k_kda_pre  - every (MAX_CHUNK-row block, head) at once: the conv (history
//                from the ring for the first rows, else from the rows before),
//                the gate rows, the l2 norms, beta and k.q, i.e. everything
//                that does not read the state, stored as one record per
//                (row, head): [kn.g | qn.g*scale... | g | kn | v | beta, k.q];
//   k_kda_rec  - one block per head: the token-serial recurrence over all n
//                rows from the records, staged through LDS one block of rows
//                ahead (the next block's records are in flight while the
//                current block's tokens run); o to orow, the final state to
//                the base slot;
//   k_kda_post - every (row block, head) at once: the gated norm and the
//                quantization for o_proj, and the conv history after the last
//                row into the base slot (after every read of it).
template <int KD, int K>
__global__ __launch_bounds__(4 * KD) void k_kda_pre(KdaStepArgs b, int n) {
    const int r = blockIdx.x * MAX_CHUNK;
    KdaStepArgs a = b;
    a.nt = imin(MAX_CHUNK, n - r);
    a.hist_rows = r > 0;
    a.pq = b.pq + (size_t)r * b.key;
    a.pk = b.pk + (size_t)r * b.key;
    a.pv = b.pv + (size_t)r * b.value;
    a.pfa = b.pfa + (size_t)r * b.rank;
    a.bvec = b.bvec + (size_t)r * b.nv;
    a.gz = b.gz + (size_t)r * b.value;
    a.rec = b.rec + (size_t)r * b.nv * (5 * KD + 4);
    kda_step_body<KD, K, MAX_CHUNK, true>(a, blockIdx.y);
}

// A stage of k_kda_rec: the records of rows s0 .. s0 + MAX_CHUNK - 1 (those
// below n) of one head, RS4 float4 each, spread over the block's threads
// (three float4 per thread for every kd here; indices past the stage clamp
// to its last float4); fetched into registers, later stored to the stage's
// LDS buffer.
template <int KD>
struct RecStage {
    static constexpr int RS4 = (5 * KD + 4) / 4, NTHR = 4 * KD;
    static_assert(MAX_CHUNK * RS4 <= 3 * NTHR && MAX_CHUNK * RS4 > 2 * NTHR, "three float4 per thread");
    float4 v0, v1, v2;
    __device__ __forceinline__ int idx(int u, int m) const { return imin(u * NTHR + (int)threadIdx.x, m - 1); }
    __device__ __forceinline__ float4 ld(const float *src, size_t rstride, int s0, int f) const {
        const int t = f / RS4;
        return reinterpret_cast<const float4 *>(src + (size_t)(s0 + t) * rstride)[f - t * RS4];
    }
    __device__ __forceinline__ void fetch(const float *src, size_t rstride, int s0, int n) {
        const int m = imin(MAX_CHUNK, n - s0) * RS4;
        v0 = ld(src, rstride, s0, idx(0, m));
        v1 = ld(src, rstride, s0, idx(1, m));
        v2 = ld(src, rstride, s0, idx(2, m));
    }
    __device__ __forceinline__ void put(float (*buf)[5 * KD + 4], int s0, int n) const {
        const int m = imin(MAX_CHUNK, n - s0) * RS4;
        const int f0 = idx(0, m), f1 = idx(1, m), f2 = idx(2, m);      // clamped lanes rewrite the last value
        reinterpret_cast<float4 *>(buf[f0 / RS4])[f0 % RS4] = v0;
        reinterpret_cast<float4 *>(buf[f1 / RS4])[f1 % RS4] = v1;
        reinterpret_cast<float4 *>(buf[f2 / RS4])[f2 % RS4] = v2;
    }
};

template <int KD>
__global__ __launch_bounds__(4 * KD) void k_kda_rec(KdaStepArgs a, int n) {
    constexpr int RPL = KD / 4, RS = 5 * KD + 4, T = MAX_CHUNK;
    __shared__ __align__(16) float s_rec[2][T][RS];
    const int h = blockIdx.x, tid = threadIdx.x, col = tid >> 2, row0 = (tid & 3) * RPL;
    float4 *sp = reinterpret_cast<float4 *>(a.state + (size_t)(*a.ctl_slot) * a.slot_stride + (size_t)h * KD * KD) + tid;
    float S[RPL];
#pragma unroll
    for (int i = 0; i < RPL / 4; i++) {
        const float4 q = sp[i * 4 * KD];
        S[4 * i] = q.x; S[4 * i + 1] = q.y; S[4 * i + 2] = q.z; S[4 * i + 3] = q.w;
    }
    const size_t rstride = (size_t)a.nv * RS;
    const float *src = a.rec + (size_t)h * RS;
    RecStage<KD> nb;
    nb.fetch(src, rstride, 0, n);
    nb.put(s_rec[0], 0, n);
    __syncthreads();
    const int nst = (n + T - 1) / T;
#pragma unroll 1
    for (int sk = 0; sk < nst; sk++) {
        // the next stage's records are in flight while this stage runs (the
        // last stage refetches itself into the idle buffer)
        const int sb = sk & 1, s0 = sk * T, nt = imin(T, n - s0), sn = sk + 1 < nst ? s0 + T : s0;
        nb.fetch(src, rstride, sn, n);
#pragma unroll 1
        for (int t = 0; t < nt; t++) {
            const float *rc = s_rec[sb][t];
            const float o = kda_token<KD>(S, rc, rc + KD, rc + 2 * KD, rc + 3 * KD, rc + 4 * KD + col, rc + 5 * KD,
                                          rc + 5 * KD + 1, row0);
            if ((tid & 3) == 0) {
                const size_t oi = (size_t)(s0 + t) * a.value + (size_t)h * KD + col;
                a.orow[oi] = o;
                if (a.raw_out) a.raw_out[oi] = o;
            }
        }
        nb.put(s_rec[sb ^ 1], sn, n);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < RPL / 4; i++) sp[i * 4 * KD] = make_float4(S[4 * i], S[4 * i + 1], S[4 * i + 2], S[4 * i + 3]);
}

template <int KD, int K>
__global__ __launch_bounds__(4 * KD) void k_kda_post(KdaStepArgs b, int n) {
    constexpr int VD = KD, HIST = K - 1, NT = MAX_CHUNK;
    EXP_TAB_LOAD(tab);
    __shared__ __align__(16) float s_o[NT][KD];
    __shared__ __align__(16) float s_z[NT][KD];
    __shared__ __align__(16) float s_sq[NT][KD];
    __shared__ __align__(16) float s_y[NT][KD];
    __shared__ float s_oinv[NT];
    const int h = blockIdx.y, r = blockIdx.x * NT, nt = imin(NT, n - r), tid = threadIdx.x;
    const int grp = tid / KD, j = tid - grp * KD;
    float ov[NT / 4], zv[NT / 4];
#pragma unroll
    for (int i = 0; i < NT / 4; i++) {
        const size_t ri = (size_t)(r + imin(4 * i + grp, nt - 1)) * b.value + (size_t)h * VD + j;
        ov[i] = b.orow[ri];
        zv[i] = b.gz[ri];
    }
    const float onw = b.o_norm[j];
    EXP_TAB_PUT(tab);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NT / 4; i++) {
        s_o[4 * i + grp][j] = ov[i];
        s_z[4 * i + grp][j] = d_silu(zv[i], tab);
    }
    __syncthreads();
    KdaStepArgs a = b;
    a.xq = b.xq + (size_t)r * b.value;
    a.xqs = b.xqs + (size_t)r * (b.value >> 5);
    a.normed_out = b.normed_out ? b.normed_out + (size_t)r * b.value : nullptr;
    kda_gated_tail<KD, NT>(a, h, nt, j, onw, s_o, s_z, s_sq, s_y, s_oinv);
    if (r + nt == n && grp < 3) {
        const int cch = grp == 0 ? h * KD + j : grp == 1 ? b.key + h * KD + j : 2 * b.key + h * VD + j;
        const float *xsrc = grp == 0 ? b.pq : grp == 1 ? b.pk : b.pv;
        const int xstride = grp < 2 ? b.key : b.value;
        float *r1 = b.conv_ring + (size_t)(*b.ctl_slot) * b.conv_slot_stride;
#pragma unroll
        for (int i = 0; i < HIST; i++) r1[(size_t)cch * HIST + i] = xsrc[(size_t)(n - HIST + i) * xstride + h * KD + j];
    }
}

// ---------------------------------------------------------- host glue ---

extern "C" int l98k_upload_exp_table_kda(const float *tab) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(c_exp_tab), tab, 32 * sizeof(float));
}

extern "C" int l98k_kda_step(const KdaStepArgs *a, int kd, int K, hipStream_t st) {
    if (a->nt < 1 || a->nt > MAX_CHUNK || a->rank < 32 || (a->rank & 31) || a->rank > KDA_MAX_RANK ||
        a->key != a->nv * kd || a->value != a->nv * kd || K < 2 || K > 4)
        return -1;
    const int nt = a->nt, NT = nt <= 1 ? 1 : nt <= 2 ? 2 : nt <= 4 ? 4 : nt <= 6 ? nt : 8;
    // conv width 4 (every synthetic config) has an instance per token bound;
    // other widths run the 8-slot instance
#define KDA_STEP(KD_, K_, NT_) hipLaunchKernelGGL((k_kda_step<KD_, K_, NT_>), dim3(a->nv), dim3(4 * (KD_)), 0, st, *a)
#define KDA_K4(KD_)                                 \
    switch (NT) {                                   \
    case 1: KDA_STEP(KD_, 4, 1); break;             \
    case 2: KDA_STEP(KD_, 4, 2); break;             \
    case 4: KDA_STEP(KD_, 4, 4); break;             \
    case 5: KDA_STEP(KD_, 4, 5); break;             \
    case 6: KDA_STEP(KD_, 4, 6); break;             \
    default: KDA_STEP(KD_, 4, 8); break;            \
    }
    switch (kd * 8 + K) {
    case 64 * 8 + 4: KDA_K4(64); break;
    case 64 * 8 + 3: KDA_STEP(64, 3, 8); break;
    case 64 * 8 + 2: KDA_STEP(64, 2, 8); break;
    case 128 * 8 + 4: KDA_K4(128); break;
    case 128 * 8 + 3: KDA_STEP(128, 3, 8); break;
    case 128 * 8 + 2: KDA_STEP(128, 2, 8); break;
    case 32 * 8 + 4: KDA_K4(32); break;
    case 32 * 8 + 3: KDA_STEP(32, 3, 8); break;
    case 32 * 8 + 2: KDA_STEP(32, 2, 8); break;
    default: return -1;
    }
#undef KDA_K4
#undef KDA_STEP
    return (int)hipGetLastError();
}

extern "C" int l98k_kda_items(const KdaStepArgs *a, const KdaItem *items, int n_items, int max_n, size_t state_off,
                              size_t conv_off, int kd, int K, hipStream_t st) {
    if (n_items < 1 || a->rank < 32 || (a->rank & 31) || a->rank > KDA_MAX_RANK || a->key != a->nv * kd ||
        a->value != a->nv * kd || K < 2 || K > 4)
        return -1;
#define KDA_ITEMS(KD_, K_)                                                                                     \
    if (max_n <= 4)                                                                                            \
        hipLaunchKernelGGL((k_kda_items<KD_, K_, 4>), dim3(a->nv, n_items), dim3(4 * (KD_)), 0, st, *a, items, \
                           state_off, conv_off);                                                               \
    else                                                                                                       \
        hipLaunchKernelGGL((k_kda_items<KD_, K_, MAX_CHUNK>), dim3(a->nv, n_items), dim3(4 * (KD_)), 0, st, *a, \
                           items, state_off, conv_off)
    switch (kd * 8 + K) {
    case 64 * 8 + 4: KDA_ITEMS(64, 4); break;
    case 64 * 8 + 3: KDA_ITEMS(64, 3); break;
    case 64 * 8 + 2: KDA_ITEMS(64, 2); break;
    case 128 * 8 + 4: KDA_ITEMS(128, 4); break;
    case 128 * 8 + 3: KDA_ITEMS(128, 3); break;
    case 128 * 8 + 2: KDA_ITEMS(128, 2); break;
    case 32 * 8 + 4: KDA_ITEMS(32, 4); break;
    case 32 * 8 + 3: KDA_ITEMS(32, 3); break;
    case 32 * 8 + 2: KDA_ITEMS(32, 2); break;
    default: return -1;
    }
#undef KDA_ITEMS
    return (int)hipGetLastError();
}

extern "C" int l98k_kda_split(const KdaStepArgs *a, int n, int kd, int K, hipStream_t st) {
    if (n <= MAX_CHUNK || a->advance || !a->rec || !a->orow || a->rank < 32 || (a->rank & 31) ||
        a->rank > KDA_MAX_RANK || a->key != a->nv * kd || a->value != a->nv * kd || K < 2 || K > 4)
        return -1;
    const dim3 rows((n + MAX_CHUNK - 1) / MAX_CHUNK, a->nv);
#define KDA_SPLIT(KD_, K_)                                                                            \
    do {                                                                                              \
        hipLaunchKernelGGL((k_kda_pre<KD_, K_>), rows, dim3(4 * (KD_)), 0, st, *a, n);               \
        hipLaunchKernelGGL((k_kda_rec<KD_>), dim3(a->nv), dim3(4 * (KD_)), 0, st, *a, n);            \
        hipLaunchKernelGGL((k_kda_post<KD_, K_>), rows, dim3(4 * (KD_)), 0, st, *a, n);              \
    } while (0)
    switch (kd * 8 + K) {
    case 64 * 8 + 4: KDA_SPLIT(64, 4); break;
    case 64 * 8 + 3: KDA_SPLIT(64, 3); break;
    case 64 * 8 + 2: KDA_SPLIT(64, 2); break;
    case 128 * 8 + 4: KDA_SPLIT(128, 4); break;
    case 128 * 8 + 3: KDA_SPLIT(128, 3); break;
    case 128 * 8 + 2: KDA_SPLIT(128, 2); break;
    case 32 * 8 + 4: KDA_SPLIT(32, 4); break;
    case 32 * 8 + 3: KDA_SPLIT(32, 3); break;
    case 32 * 8 + 2: KDA_SPLIT(32, 2); break;
    default: return -1;
    }
#undef KDA_SPLIT
    return (int)hipGetLastError();
}

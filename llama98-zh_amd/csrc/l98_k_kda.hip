// KDA gated-delta kernels: causal conv and the fp32-state recurrence
// (bit-exact restatement of the reference float-oracle path; see
// l98_devmath.h for the numeric contract).
#include "l98_devmath.h"

// ---------------------------------------------------------- KDA layer ---
//
// One block per head (nk == nv); lane j owns q/k channel j of the head, v
// channel j, and column j of the fp32 state S[kd][vd] (registers).  For the
// chunk's tokens, in one launch:
//   * the depthwise causal conv + SiLU of the lane's q, k and v channels
//     along the ring (lz_causal_conv1d_step, src/ops_conv1d.c:26-87: taps
//     summed in order, then the current input; ring slots
//     src/forward_kda.c:680-755);
//   * the gate up-projection row h*kd + j of f_b over the per-32 quantized
//     low-rank input (lz_matmul_xq_nt + epi_q8, src/ops_matmul.c:468-660,
//     src/ops_epi.c:983-1017: exact int32 group sums, groups summed in
//     order, times the row scale);
//   * the gate (src/forward_kda.c:277-300, 840-850), l2norm(q)*scale,
//     l2norm(k), beta, kq = k.q, then per token u = S^T(g.k), w = S^T(g.q),
//     delta = (v - u)*beta, out = w + delta*kq, S' = g.S + k(x)delta
//     (lz_recur_step fp32 arm, src/ops_gdn.c:2516-2560; call site
//     src/forward_kda.c:856-940), every state written to its ring slot;
//   * the per-head gated RMSNorm and the per-32 quantization for o_proj
//     (src/forward_kda.c:1000-1043).
// Everything that does not depend on the state is computed for all tokens
// at once; only u, w and the state update run token-serially.
template <int KD, int K>
__global__ __launch_bounds__(KD) void k_kda_step(KdaStepArgs a) {
    constexpr int VD = KD, HIST = K - 1;
    EXP_TAB_LOAD(tab);
    __shared__ __align__(16) float s_a[MAX_CHUNK][KD];   // q, then q.g*invq*scale (qcw)
    __shared__ __align__(16) float s_b[MAX_CHUNK][KD];   // k, then k*invk (kn)
    __shared__ __align__(16) float s_g[MAX_CHUNK][KD];   // decay gate
    __shared__ __align__(16) float s_c[MAX_CHUNK][KD];   // q^2, then kn*g (kcw), then o^2
    __shared__ __align__(16) float s_d[MAX_CHUNK][KD];   // k^2
    __shared__ __align__(16) int8_t s_fq[MAX_CHUNK][KDA_MAX_RANK];
    __shared__ float s_fs[MAX_CHUNK][KDA_MAX_RANK / 32];
    __shared__ float s_invq[MAX_CHUNK], s_invk[MAX_CHUNK], s_beta[MAX_CHUNK], s_kq[MAX_CHUNK],
        s_oinv[MAX_CHUNK];
    const int h = blockIdx.x;
    const int j = threadIdx.x;
    const int nt = a.nt, key = a.key, value = a.value, rank = a.rank;
    const size_t head_off = (size_t)h * KD * VD;
    const int base = *a.ctl_slot;
    // ---- loads: token inputs, conv taps and history, f_b row, state
    const int cq = h * KD + j, ck = key + h * KD + j, cv = 2 * key + h * VD + j;   // conv channels
    float xq[MAX_CHUNK], xk[MAX_CHUNK], xv[MAX_CHUNK], gzv[MAX_CHUNK], fa[MAX_CHUNK][KDA_MAX_RANK / KD + 1];
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        const int tc = imin(t, nt - 1);
        xq[t] = a.pq[(size_t)tc * key + h * KD + j];
        xk[t] = a.pk[(size_t)tc * key + h * KD + j];
        xv[t] = a.pv[(size_t)tc * value + h * VD + j];
        gzv[t] = a.gz[(size_t)tc * value + h * VD + j];
#pragma unroll
        for (int r = 0; r < KDA_MAX_RANK / KD + 1; r++)
            fa[t][r] = a.pfa[(size_t)tc * rank + imin(r * KD + j, rank - 1)];
    }
    float wq[K], wk[K], wv[K], hq[HIST > 0 ? HIST : 1], hk[HIST > 0 ? HIST : 1], hv[HIST > 0 ? HIST : 1];
#pragma unroll
    for (int i = 0; i < K; i++) {
        wq[i] = a.conv_w[(size_t)cq * K + i];
        wk[i] = a.conv_w[(size_t)ck * K + i];
        wv[i] = a.conv_w[(size_t)cv * K + i];
    }
    {
        const float *r0 = a.conv_ring + (size_t)base * a.conv_slot_stride;
#pragma unroll
        for (int i = 0; i < HIST; i++) {
            hq[i] = r0[(size_t)cq * HIST + i];
            hk[i] = r0[(size_t)ck * HIST + i];
            hv[i] = r0[(size_t)cv * HIST + i];
        }
    }
    const int4 *fbrow = reinterpret_cast<const int4 *>(a.fb_q + (size_t)(h * KD + j) * rank);
    int4 fbw[KDA_MAX_RANK / 16];
#pragma unroll
    for (int u = 0; u < KDA_MAX_RANK / 16; u++) fbw[u] = fbrow[imin(u, (rank >> 4) - 1)];
    const float fbs = a.fb_s[h * KD + j];
    const float bv = a.bvec[(size_t)imin(j, nt - 1) * a.nv + h];
    const float dtb = a.dt_bias[h * KD + j];
    const float onw = a.o_norm[j];
    const float alog = a.a_log[h];
    float S[KD];
    {
        const float *src = a.state + (size_t)base * a.slot_stride + head_off;
#pragma unroll
        for (int i = 0; i < KD; i++) S[i] = src[(size_t)i * VD + j];
    }
    EXP_TAB_PUT(tab);
    // ---- per-32 quantization of the low-rank gate input (groups are lane
    // halves: rank % 32 == 0, chunks of KD elements)
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        if (t < nt) {
#pragma unroll
            for (int r = 0; r < KDA_MAX_RANK / KD + 1; r++) {
                if (r * KD < rank) {
                    const int ri = r * KD + j;
                    int8_t q;
                    float sg;
                    d_quant_group32(fa[t][r], &q, &sg);
                    if (ri < rank) {
                        s_fq[t][ri] = q;
                        if ((ri & 31) == 0) s_fs[t][ri >> 5] = sg;
                    }
                }
            }
        }
    }
    __syncthreads();
    const float decay = d_exp(alog, tab);
    // ---- conv (token-serial along the history) and the gate row
    float qv[MAX_CHUNK], kv[MAX_CHUNK], vcv[MAX_CHUNK];
    const int ring_owner = 1;              // nk == nv: every head owns its channels
    (void)ring_owner;
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        qv[t] = kv[t] = vcv[t] = 0.0f;
        if (t < nt) {
            float sq = 0.0f, sk = 0.0f, sv = 0.0f;
#pragma unroll
            for (int i = 0; i < HIST; i++) {
                sq += wq[i] * hq[i];
                sk += wk[i] * hk[i];
                sv += wv[i] * hv[i];
            }
            sq += wq[HIST] * xq[t];
            sk += wk[HIST] * xk[t];
            sv += wv[HIST] * xv[t];
            qv[t] = d_silu(sq, tab);
            kv[t] = d_silu(sk, tab);
            vcv[t] = d_silu(sv, tab);
#pragma unroll
            for (int i = 0; i + 1 < HIST; i++) { hq[i] = hq[i + 1]; hk[i] = hk[i + 1]; hv[i] = hv[i + 1]; }
            if (HIST > 0) { hq[HIST - 1] = xq[t]; hk[HIST - 1] = xk[t]; hv[HIST - 1] = xv[t]; }
            if (a.advance || t == nt - 1) {
                int so;
                if (a.advance) { const int si = (base + t) % a.depth; so = si + 1 == a.depth ? 0 : si + 1; }
                else so = base;
                float *r1 = a.conv_ring + (size_t)so * a.conv_slot_stride;
#pragma unroll
                for (int i = 0; i < HIST; i++) {
                    r1[(size_t)cq * HIST + i] = hq[i];
                    r1[(size_t)ck * HIST + i] = hk[i];
                    r1[(size_t)cv * HIST + i] = hv[i];
                }
            }
        }
    }
    // gate pre-activation of row h*kd + j for each token, then the decay gate
#pragma unroll
    for (int t = 0; t < MAX_CHUNK; t++) {
        if (t < nt) {
            float dot = 0.0f;
#pragma unroll
            for (int g = 0; g < KDA_MAX_RANK / 32; g++) {
                if (g * 32 < rank) {
                    const int4 *xr = reinterpret_cast<const int4 *>(&s_fq[t][g * 32]);
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
                    dot += (float)acc * s_fs[t][g];
                }
            }
            float pre = 0.0f;
            pre += dot * fbs;
            const float p = pre + dtb;
            const float gg = -decay * d_softplus(p, tab);
            s_g[t][j] = d_exp(gg, tab);
            s_a[t][j] = qv[t];
            s_b[t][j] = kv[t];
            s_c[t][j] = qv[t] * qv[t];
            s_d[t][j] = kv[t] * kv[t];
        }
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
                if (a.advance) { const int si = (base + t) % a.depth; so = si + 1 == a.depth ? 0 : si + 1; }
                else so = base;
                float *dst = a.state + (size_t)so * a.slot_stride + head_off;
#pragma unroll
                for (int i = 0; i < KD; i++) dst[(size_t)i * VD + j] = S[i];
            }
            if (a.raw_out) a.raw_out[(size_t)t * value + (size_t)h * VD + j] = o;
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
            if (a.normed_out) a.normed_out[(size_t)t * value + col] = y;
            d_quant_group32(y, a.xq + (size_t)t * value + col, a.xqs + (size_t)t * (value >> 5) + (col >> 5));
        }
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
#define KDA_STEP(KD_, K_) hipLaunchKernelGGL((k_kda_step<KD_, K_>), dim3(a->nv), dim3(KD_), 0, st, *a)
    switch (kd * 8 + K) {
    case 64 * 8 + 4: KDA_STEP(64, 4); break;
    case 64 * 8 + 3: KDA_STEP(64, 3); break;
    case 64 * 8 + 2: KDA_STEP(64, 2); break;
    case 128 * 8 + 4: KDA_STEP(128, 4); break;
    case 128 * 8 + 3: KDA_STEP(128, 3); break;
    case 128 * 8 + 2: KDA_STEP(128, 2); break;
    case 32 * 8 + 4: KDA_STEP(32, 4); break;
    case 32 * 8 + 3: KDA_STEP(32, 3); break;
    case 32 * 8 + 2: KDA_STEP(32, 2); break;
    default: return -1;
    }
#undef KDA_STEP
    return (int)hipGetLastError();
}

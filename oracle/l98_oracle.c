/* l98_oracle.c -- CPU restatement of the reference's MTP speculative-decoding
 * path, in its float-oracle mode (--fixed off --fastfp off, fp32 KDA state,
 * Q8 KV cache, no attention window).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the
 * checker.  The product (llama98-zh_amd/) never links or calls it.
 *
 * Every function states the reference file:line it follows (paths relative
 * to the reference tree).  Arithmetic is written in the reference's exact
 * evaluation order; compile with -O2 -ffp-contract=off and no fast-math so
 * the rounding sequence is the reference's.
 *
 * Pinning (what checks each function beyond this restatement; see
 * tests/test_oracle_*.py):
 *   - the composed engine (capture, verify, draft, prefill, catch-up, the
 *     greedy and temperature rounds) is compared bit for bit against the
 *     reference engine built from its own sources (oracle/_ref), on seeded
 *     random-init models, and against the committed golden fixtures;
 *   - o_exp / o_rsqrt / o_sigmoid / o_softplus are swept against the
 *     reference's exported lz_exp / lz_rsqrt / lz_sigmoid / lz_softplus and
 *     against libm within their documented error;
 *   - quantize / matmul / argmax / route / accept are checked against closed
 *     forms and brute force (integer sums, first-index tie breaks, injected
 *     u boundaries);
 *   - o_fwht_i32 / o_fwht_f32 are compared with the reference's exported
 *     lz_fwht_i32 / lz_fwht and with a dense Sylvester matrix product;
 *     o_subn_fwht_quant / o_subn_rot_f32 restate static functions of
 *     src/forward_kda.c: they are checked bit for bit against those very
 *     functions, exported by a test-only translation unit that compiles
 *     the reference's forward_kda.c in place (oracle/ref_subn.c), which
 *     pins the scale's multiply order (tam * inv_S) * rsqrt(blk) / 127; and
 *     by closed forms (a zero row, each group's largest code being 127, the
 *     dequantized row against H.x / sqrt(blk), the float rotation against
 *     the dense product).
 */
#define _POSIX_C_SOURCE 200809L
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ORA_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------------- */
/* Scalar transcendentals of the float tier.                               */
/* ---------------------------------------------------------------------- */

/* 2^(i/32), i = 0..31, as float (reference src/ops_quant.c:244-253 holds the
 * same 32 values as decimal literals). */
static float g_exp_tab[32];
static int g_exp_tab_ready;
static void exp_tab_init(void) {
    for (int i = 0; i < 32; i++) g_exp_tab[i] = (float)exp2((double)i / 32.0);
    g_exp_tab_ready = 1;
}

/* Fitted constants of the reference's float exp (src/ops_quant.c:300-349)
 * and softplus log1p polynomial (src/ops_quant.c:986-990); the values must
 * be identical for bitwise agreement. */
static const float EXP_C2 = 0.242844437f;
static const float EXP_C1 = 0.207425515f;
static const float EXP_C0 = 0.549730133f;
static const float EXP_LOG2E32 = 1.44269504f * 32.0f;
static const float EXP_LO = -87.3f;
static const float SP_LOG1P[9] = {
    1.000000000f, -0.499995530f, 0.333203435f, -0.248529464f, 0.191451162f,
    -0.137466222f, 0.079210736f, -0.030110965f, 0.005384062f,
};

/* lz_exp_float_body, src/ops_quant.c:300-349: floor(x log2e 32) by a float
 * magic add, 2^(n) by exponent bits, 2^(idx/32) from the table and a
 * quadratic in w = 1 + r/32. */
ORA_API float o_exp(float x) {
    union { float f; int32_t i; } u, p2n;
    float y32, r, w, c;
    int32_t t, n, idx;
    if (!g_exp_tab_ready) exp_tab_init();
    if (x > 88.0f) return FLT_MAX;
    if (x < EXP_LO) return 0.0f;
    y32 = x * EXP_LOG2E32;
    u.f = y32 - 0.5f + 12582912.0f;
    t = (u.i & 0x007FFFFF) - 0x00400000;
    n = t >> 5;
    idx = t & 31;
    r = y32 - (float)t;
    w = 1.0f + r * 0.03125f;
    p2n.i = (n + 127) << 23;
    c = (EXP_C2 * w + EXP_C1) * w + EXP_C0;
    return p2n.f * (g_exp_tab[idx] * c);
}

/* lz_rsqrt_float_body, src/ops_quant.c:126-135: magic seed + two Newtons. */
ORA_API float o_rsqrt(float x) {
    union { float f; uint32_t u; } t;
    float h = 0.5f * x, y;
    t.f = x;
    t.u = 0x5f375a86u - (t.u >> 1);
    y = t.f;
    y = y * (1.5f - h * y * y);
    y = y * (1.5f - h * y * y);
    return y;
}

/* lz_sigmoid float branch, src/ops_quant.c:1816-1853. */
ORA_API float o_sigmoid(float x) {
    if (x >= 0.0f) {
        float z = o_exp(-x);
        return 1.0f / (1.0f + z);
    } else {
        float z = o_exp(x);
        return z / (1.0f + z);
    }
}

/* lz_silu, src/ops_quant.c:1862-1865. */
ORA_API float o_silu(float x) { return x * o_sigmoid(x); }

/* lz_softplus -> lz_softplus_poly, src/ops_quant.c:1040-1060, 2068-2070. */
ORA_API float o_softplus(float x) {
    float nx, u, p, lp;
    int i;
    if (x > 16.0f) return x;
    nx = (x < 0.0f) ? x : -x;
    u = o_exp(nx);
    p = SP_LOG1P[8];
    for (i = 7; i >= 0; i--) p = p * u + SP_LOG1P[i];
    lp = u * p;
    if (x > 0.0f) return x + lp;
    return lp;
}

/* ---------------------------------------------------------------------- */
/* Vector primitives.                                                      */
/* ---------------------------------------------------------------------- */

static float ss_over_n(float ss, int n) {      /* src/ops_norm.c:161-170 */
    if (n > 0 && (n & (n - 1)) == 0) {
        int e = 0;
        while ((1 << e) < n) e++;
        return ss * ldexpf(1.0f, -e);
    }
    return ss / (float)n;
}

/* lz_rmsnorm, src/ops_norm.c:690-747: serial sum of squares, (x*inv)*(1+w). */
ORA_API void o_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f, inv;
    int i;
    for (i = 0; i < n; i++) ss += x[i] * x[i];
    inv = o_rsqrt(ss_over_n(ss, n) + eps);
    for (i = 0; i < n; i++) o[i] = x[i] * inv * (1.0f + w[i]);
}

/* lz_rmsnorm_gated float branch, src/ops_norm.c:749-793: ((x*inv)*w)*silu(g). */
ORA_API void o_rmsnorm_gated(float *o, const float *x, const float *g, const float *w,
                             int n, float eps) {
    float ss = 0.0f, inv;
    int i;
    for (i = 0; i < n; i++) ss += x[i] * x[i];
    inv = o_rsqrt(ss_over_n(ss, n) + eps);
    for (i = 0; i < n; i++) o[i] = x[i] * inv * w[i] * o_silu(g[i]);
}

/* lz_l2norm float branch, src/ops_norm.c:795-868. */
ORA_API void o_l2norm(float *o, const float *x, int n, float eps) {
    float ss = 0.0f, inv;
    int i;
    for (i = 0; i < n; i++) ss += x[i] * x[i];
    inv = o_rsqrt(ss + eps);
    for (i = 0; i < n; i++) o[i] = x[i] * inv;
}

static uint32_t fkey_bits(uint32_t u) {        /* src/sampler.c:121 LZ_FKEY */
    return u ^ (((uint32_t)((int32_t)u >> 31)) | 0x80000000u);
}
static uint32_t fkey(float f) {
    union { float f; uint32_t u; } b;
    b.f = f;
    return fkey_bits(b.u);
}

/* lz_softmax, src/ops_norm.c:903-990 (float tier): exact max, serial sum. */
ORA_API void o_softmax(float *x, int n) {
    float mx = x[0], sum = 0.0f, inv;
    uint32_t best = fkey(mx);
    int i;
    for (i = 1; i < n; i++) {
        uint32_t k = fkey(x[i]);
        if (k > best) { best = k; mx = x[i]; }
    }
    for (i = 0; i < n; i++) {
        x[i] = o_exp(x[i] - mx);
        sum += x[i];
    }
    inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
    for (i = 0; i < n; i++) x[i] *= inv;
}

/* q8_round with --fastfp off: the 1.5*2^23 magic add is round-to-nearest-
 * even for |v| < 2^22 (src/ops_quant.h:145-178). */
static int q8_round(float v) {
    union { float f; uint32_t u; } t;
    t.f = v + 12582912.0f;
    return (int)(t.u & 0x007FFFFFu) - 0x00400000;
}

/* q8_group_scale + the element loop of lz_quantize_q8 over one group of n
 * elements (src/ops_quant.c:1444-1475, 1633-1670, 2152-2286): amax by |bits|,
 * s = amax/127 (as amax*(1/127f)), inv = 127/amax, q = clamp(rne(x*inv),
 * +-127); a zero or tiny group gets s = 1, q = 0; a group whose 127/amax
 * overflows divides by s instead.  Returns the group's scale. */
static float quant_group(const float *grp, int n, int8_t *q) {
    static const float INV127 = 1.0f / 127.0f;
    union { float f; uint32_t u; } b;
    uint32_t am = 0;
    float amax, sg, inv;
    int fast, k;
    for (k = 0; k < n; k++) {
        uint32_t a;
        b.f = grp[k];
        a = b.u & 0x7FFFFFFFu;
        if (a > am) am = a;
    }
    b.u = am;
    amax = b.f;
    if (amax > 0.0f) {
        sg = amax * INV127;
        inv = 127.0f / amax;
        fast = (inv <= FLT_MAX);
        if (sg < 1.0e-30f) { sg = 1.0f; inv = 0.0f; fast = 1; }
    } else {
        sg = 1.0f; inv = 0.0f; fast = 1;
    }
    for (k = 0; k < n; k++) {
        int qi = fast ? q8_round(grp[k] * inv) : q8_round(grp[k] / sg);
        qi = (qi > 127) ? 127 : qi;
        q[k] = (int8_t)((qi < -127) ? -127 : qi);
    }
    return sg;
}

/* lz_quantize_q8 for gs = 32: one quant_group per 32 elements. */
ORA_API void o_quantize_q8(const float *x, int n, int8_t *q, float *s) {
    for (int g = 0; g < n / 32; g++) s[g] = quant_group(x + g * 32, 32, q + g * 32);
}

/* lz_quantize_q8_tok (src/ops_quant.c:2284-2314): q8_group_scale over the
 * whole row, the same element loop, and the one scale replicated into all
 * n/32 slots. */
ORA_API void o_quantize_q8_tok(const float *x, int n, int8_t *q, float *s) {
    if (n < 32) return;
    const float sg = quant_group(x, n, q);
    for (int g = 0; g < n / 32; g++) s[g] = sg;
}

/* lz_fwht_i32's scalar body (src/fwht.c:65-196; the loop at :186-195): the
 * Sylvester butterflies u+v, u-v at strides 1, 2, 4, ... n/2 over a copy of
 * x, in wrapping int32 (computed in uint32 so the wrap is defined). */
ORA_API void o_fwht_i32(int32_t *y, const int32_t *x, int n) {
    int len, i, j;
    for (i = 0; i < n; i++) y[i] = x[i];
    for (len = 1; len < n; len <<= 1)
        for (i = 0; i < n; i += len << 1)
            for (j = 0; j < len; j++) {
                uint32_t u = (uint32_t)y[i + j], v = (uint32_t)y[i + j + len];
                y[i + j] = (int32_t)(u + v);
                y[i + j + len] = (int32_t)(u - v);
            }
}

/* lz_fwht (src/fwht.c:198-320; the loop at :310-319): the same butterflies
 * in float, in place. */
ORA_API void o_fwht_f32(float *v, int n) {
    int len, i, j;
    for (len = 1; len < n; len <<= 1)
        for (i = 0; i < n; i += len << 1)
            for (j = 0; j < len; j++) {
                float a = v[i + j], b = v[i + j + len];
                v[i + j] = a + b;
                v[i + j + len] = a - b;
            }
}

/* pow2f (src/ops_quant.c:77-83): 2^e from the exponent field; 0 below
 * 2^-126, 2^127 above. */
static float o_pow2f(int e) {
    union { float f; uint32_t u; } b;
    if (e < -126) return 0.0f;
    if (e > 127) e = 127;
    b.u = (uint32_t)(e + 127) << 23;
    return b.f;
}

/* subn_fwht_quant (src/forward_kda.c:43-92), the SubLN o_proj / down_proj
 * input quantization of one row of n floats:
 *   amax by |bits|; a zero row gives q = 0, s = 1;
 *   S = pow2f(14 - e(amax)), so the row max lands in [2^14, 2^15);
 *   t = block-diagonal FWHT (block blk) of q8_round(x * S), exact int32;
 *   per group of gw elements (gw = n unless gw is a multiple of 32 dividing
 *   n): tam = max |t|, scale = (float)tam * (1/S) * rsqrt(blk) * (1/127)
 *   left to right; tam == 0 or scale < 1e-30 gives scale 1 and q = 0;
 *   else q = clamp(q8_round(t * (127/tam)), +-127);
 *   s holds the group's scale in each of its n/32 slots. */
ORA_API void o_subn_fwht_quant(const float *x, int n, int blk, int gw, int8_t *q, float *s) {
    static const float INV127 = 1.0f / 127.0f;
    union { float f; uint32_t u; } b;
    uint32_t am = 0;
    float S, inv_S, rs;
    int i, e, base;
    int32_t *f = (int32_t *)malloc(sizeof(int32_t) * 2 * (size_t)n);
    for (i = 0; i < n; i++) {
        b.f = x[i];
        if ((b.u & 0x7FFFFFFFu) > am) am = b.u & 0x7FFFFFFFu;
    }
    b.u = am;
    if (b.f <= 0.0f) {
        for (i = 0; i < n; i++) q[i] = 0;
        for (i = 0; i < n / 32; i++) s[i] = 1.0f;
        free(f);
        return;
    }
    e = (int)((am >> 23) & 0xFFu) - 127;
    S = o_pow2f(14 - e);
    inv_S = 1.0f / S;
    for (i = 0; i < n; i++) f[i] = q8_round(x[i] * S);
    for (base = 0; base < n; base += blk) o_fwht_i32(f + n + base, f + base, blk);
    if (gw <= 0 || (gw & 31) != 0 || (n % gw) != 0) gw = n;
    rs = o_rsqrt((float)blk);
    for (base = 0; base < n; base += gw) {
        int32_t tam = 0;
        float scale, inv_q;
        for (i = base; i < base + gw; i++) {
            int32_t a = f[n + i] < 0 ? (int32_t)(0u - (uint32_t)f[n + i]) : f[n + i];
            if (a > tam) tam = a;
        }
        scale = (float)tam * inv_S * rs * INV127;
        if (tam == 0 || scale < 1.0e-30f) {
            scale = 1.0f;
            inv_q = 0.0f;
        } else {
            inv_q = 127.0f / (float)tam;
        }
        for (i = base; i < base + gw; i++) {
            int qv = q8_round((float)f[n + i] * inv_q);
            qv = qv > 127 ? 127 : qv;
            q[i] = (int8_t)(qv < -127 ? -127 : qv);
        }
        for (i = base / 32; i < (base + gw) / 32; i++) s[i] = scale;
    }
    free(f);
}

/* subn_rot_f32 (src/forward_kda.c:130-135): the same block-diagonal
 * Hadamard on the float row, then each element times rsqrt(blk). */
ORA_API void o_subn_rot_f32(float *x, int n, int blk) {
    float inv = o_rsqrt((float)blk);
    int i;
    for (i = 0; i < n; i += blk) o_fwht_f32(x + i, blk);
    for (i = 0; i < n; i++) x[i] *= inv;
}

/* lz_matmul_xq_nt for a Q8_0 weight with groups of gs (a multiple of 32
 * dividing in), the SIMD row kernel + epi_q8 (src/ops_matmul.c:336-466;
 * src/ops_epi.c:983-1022), r = gs/32, wsr the row's in/gs scales:
 *   acc[t,i,s] = sum_{e<32} w[i,32s+e] xq[t,32s+e]       (exact int32)
 *   r > 1: per run of r groups from 0.0f, dot = sum float(acc)*xqs (in s
 *          order); sum (from 0.0f) += dot*wsr[run], runs in order; o = sum
 *   r == 1: four accumulators a[j] (from 0.0f), group s adds
 *          float(acc)*(xqs[s]*wsr[s]) to a[s % 4] for the groups of whole
 *          fours and to a[0] for the rest; o = (a0 + a2) + (a1 + a3)
 * The SIMD kernel's x256 accumulator and 2^-8 post-scale are exact powers of
 * two and cancel.  acc_out (optional) receives acc[t][i][s]. */
ORA_API void o_matmul_q8g(float *o, const int8_t *xq, const float *xqs,
                          const int8_t *w, const float *ws, int in, int out, int nt, int gs,
                          int32_t *acc_out) {
    const int nb = in / 32, r = gs / 32, nws = in / gs;
    int32_t acc[512];
    for (int i = 0; i < out; i++) {
        const int8_t *wr = w + (size_t)i * in;
        const float *wsr = ws + (size_t)i * nws;
        for (int t = 0; t < nt; t++) {
            const int8_t *xr = xq + (size_t)t * in;
            const float *xs = xqs + (size_t)t * nb;
            for (int g = 0; g < nb; g++) {
                int32_t a = 0;
                for (int e = 0; e < 32; e++) a += (int32_t)wr[g * 32 + e] * (int32_t)xr[g * 32 + e];
                acc[g] = a;
                if (acc_out) acc_out[((size_t)t * out + i) * nb + g] = a;
            }
            float sum = 0.0f;
            if (r > 1) {
                for (int run = 0; run < nb / r; run++) {
                    float dot = 0.0f;
                    for (int g = 0; g < r; g++) dot += (float)acc[run * r + g] * xs[run * r + g];
                    sum += dot * wsr[run];
                }
            } else {
                float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
                int g = 0;
                for (; g + 3 < nb; g += 4) {
                    a0 += (float)acc[g] * (xs[g] * wsr[g]);
                    a1 += (float)acc[g + 1] * (xs[g + 1] * wsr[g + 1]);
                    a2 += (float)acc[g + 2] * (xs[g + 2] * wsr[g + 2]);
                    a3 += (float)acc[g + 3] * (xs[g + 3] * wsr[g + 3]);
                }
                for (; g < nb; g++) a0 += (float)acc[g] * (xs[g] * wsr[g]);
                sum = (a0 + a2) + (a1 + a3);
            }
            o[(size_t)t * out + i] = sum;
        }
    }
}

/* The per-row weight (gs = in). */
ORA_API void o_matmul_q8(float *o, const int8_t *xq, const float *xqs,
                         const int8_t *w, const float *ws, int in, int out, int nt,
                         int32_t *acc_out) {
    o_matmul_q8g(o, xq, xqs, w, ws, in, out, nt, in, acc_out);
}

/* lz_rope non-SIMD body, src/ops_rope.c:21-67 (NeoX half split). */
static void rope(float *v, int n_heads, int hd, int rot, int pos, const float *cs) {
    int half = rot / 2;
    const float *row = cs + (size_t)pos * half * 2;
    for (int i = 0; i < half; i++) {
        float c = row[i * 2], sn = row[i * 2 + 1];
        for (int h = 0; h < n_heads; h++) {
            float *b = v + (size_t)h * hd;
            float x0 = b[i], x1 = b[i + half];
            b[i] = x0 * c - x1 * sn;
            b[i + half] = x1 * c + x0 * sn;
        }
    }
}

/* Intermediate recorder mirroring the reference's LZ_TAP sites
 * (src/forward.h:27-36): (tag[8], layer, n, n floats) records. */
static FILE *g_tap;
ORA_API void ora_set_tap(const char *path) {
    if (g_tap) fclose(g_tap);
    g_tap = path ? fopen(path, "wb") : NULL;
}
static void tap(const char *tag, int layer, const float *p, int n) {
    char t[8];
    if (!g_tap) return;
    memset(t, 0, sizeof t);
    strncpy(t, tag, sizeof t);
    fwrite(t, 1, 8, g_tap);
    fwrite(&layer, 4, 1, g_tap);
    fwrite(&n, 4, 1, g_tap);
    fwrite(p, 4, (size_t)n, g_tap);
    fflush(g_tap);
}

/* ---------------------------------------------------------------------- */
/* Model.                                                                  */
/* ---------------------------------------------------------------------- */

typedef struct { int rows, cols, gs; int8_t *q; float *s; } QMat;   /* s: rows*cols/gs */

typedef struct {
    int type;                                    /* 1 full, 2 KDA */
    float *in_norm, *post_norm;
    /* attention */
    QMat q, k, v, o;
    float *q_norm, *k_norm;
    /* KDA */
    QMat kq, kk, kv, fa, fb, kb, kg, ko;
    float *conv_q, *conv_k, *conv_v;             /* [ch][K] */
    float *a_log, *dt_bias, *o_norm;
    /* MoE */
    QMat router, down, up, sg, su, sd;
    float *bias;
    QMat *w1, *w2, *w3;
    /* SubLN per-projection input norms (use_subn only; src/model.c:1511-1665):
     * attention q/k/v/o, KDA q/k/v/g/o, MoE router / routed down / routed up
     * / shared gate / up / down, dense FFN gate / up / down (the MTP head's) */
    float *sn_q, *sn_k, *sn_v, *sn_o;
    float *kn_q, *kn_k, *kn_v, *kn_g, *kn_o;
    float *mn_gate, *mn_down, *mn_up, *mn_sg, *mn_su, *mn_sd;
    float *fn_gate, *fn_up, *fn_down;
} OLayer;

typedef struct {
    int vocab, d, n_layers, seq_len, nh, nkv, hd, inter;
    int nk, nv, kd, vd, K, n_lin, n_full;
    float eps, theta;
    int q_dim, qg_dim, kv_dim, key, value, conv_dim, rot;
    int types[128];
    int gate_rank, n_experts, topk, moe_inter, latent, shared_w;
    int has_lb;                                  /* kda_has_gate_lower_bound */
    float gate_lb;                               /* kda_gate_lower_bound */
    int mtp_inter;
    int use_subn, hadamard_o, hadamard_down;
    int version, scale_layout, has_mtp;
    int n_draft;                                 /* mtp_n_draft: > 1 is a DSpark head */
    QMat embed;
    float *final_norm;
    OLayer *L;
    OLayer mtp;                                  /* attention block + dense FFN */
    QMat mtp_gate, mtp_up, mtp_down, mtp_fc;
    float *mtp_norm, *mtp_pre_h, *mtp_pre_e;
    QMat mtp_main;                               /* DSpark main_proj [d][3d] */
    float *mtp_depth, *mtp_mask;                 /* depth_embed rows [n_draft][d], mask_embed [d] */
    float *rope_cs;                              /* [seq_len][rot/2][2] */
} OModel;

#define SPEC_K_MAX_REF 6                         /* LZ_SPEC_K_MAX, src/ops.h:2098 */

typedef struct { FILE *f; int bad; int layout; } Rd;
static void rd(Rd *r, void *p, size_t n) {
    if (!r->bad && fread(p, 1, n, r->f) != n) r->bad = 1;
}
static int32_t rd_i32(Rd *r) { int32_t v = 0; rd(r, &v, 4); return v; }
static float rd_f32(Rd *r) { float v = 0; rd(r, &v, 4); return v; }

/* lz_f16_to_f32 (src/compat.c:283-312): binary16 widened exactly. */
static float f16_to_f32(unsigned h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    union { uint32_t u; float f; } b;
    if (e == 0) {
        if (m == 0) u = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            u = sign | ((uint32_t)(127 - 14 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 0x1Fu) {
        u = sign | 0x7F800000u | (m << 13);
    } else {
        u = sign | ((e + 127u - 15u) << 23) | (m << 13);
    }
    b.u = u;
    return b.f;
}

/* An F32 tensor of n elements, stored as f32 or as BF16 (dtype 6: the high
 * half of each f32, widened by <<16 as lz_t_f32 does, src/ops_epi.c:1210). */
static float *rd_f32_body(Rd *r, int n, uint8_t dt, uint32_t cnt) {
    float *p;
    if ((dt != 0 && dt != 6) || (int)cnt != n) { r->bad = 1; return NULL; }
    p = (float *)malloc(sizeof(float) * (size_t)n);
    if (!p) { r->bad = 1; return NULL; }
    if (dt == 0) {
        rd(r, p, sizeof(float) * (size_t)n);
    } else {
        uint16_t *h = (uint16_t *)malloc(2 * (size_t)n);
        if (!h) { r->bad = 1; free(p); return NULL; }
        rd(r, h, 2 * (size_t)n);
        for (int i = 0; i < n; i++) {
            union { uint32_t u; float f; } b;
            b.u = (uint32_t)h[i] << 16;
            p[i] = b.f;
        }
        free(h);
    }
    return p;
}
static float *rd_f32v(Rd *r, int n) {
    uint8_t dt = 0xFF;
    uint32_t cnt = 0;
    rd(r, &dt, 1); rd(r, &cnt, 4);
    return rd_f32_body(r, n, dt, cnt);
}

/* layout-2 decode (src/compat.c:340-345): base * (u / 255), each step
 * rounded to float. */
static float u8_decode(float base, float u) {
    volatile float levels = 255.0f;
    volatile float q = u / levels;
    volatile float p = base * q;
    return p;
}

static void free_q(QMat *m) { free(m->q); free(m->s); }

/* A Q8_0 tensor: u32 gs (a multiple of 32 dividing the row), the codes,
 * then the scale plane in the file's layout (read_scale_plane,
 * src/model.c:3510-3554): 0 f32 per group; 1 binary16 per group; 2 a
 * binary16 base per row, then a u8 per group decoded as base * (u / 255). */
static void rd_q8_body(Rd *r, QMat *m, int rows, int cols, uint8_t dt, uint32_t cnt) {
    uint32_t gs = 0;
    size_t ng;
    rd(r, &gs, 4);
    m->rows = rows; m->cols = cols; m->gs = (int)gs; m->q = NULL; m->s = NULL;
    if (dt != 1 || cnt != (uint32_t)rows * (uint32_t)cols || gs == 0 || gs % 32 || (uint32_t)cols % gs) {
        r->bad = 1; return;
    }
    ng = (size_t)rows * (cols / gs);
    m->q = (int8_t *)malloc((size_t)rows * cols);
    m->s = (float *)malloc(sizeof(float) * ng);
    if (!m->q || !m->s) { r->bad = 1; return; }
    rd(r, m->q, (size_t)rows * cols);
    if (r->layout == 0) {
        rd(r, m->s, sizeof(float) * ng);
    } else if (r->layout == 1) {
        uint16_t *h = (uint16_t *)malloc(2 * ng);
        if (!h) { r->bad = 1; return; }
        rd(r, h, 2 * ng);
        for (size_t i = 0; i < ng; i++) m->s[i] = f16_to_f32(h[i]);
        free(h);
    } else {
        uint16_t *h = (uint16_t *)malloc(2 * (size_t)rows);
        uint8_t *u = (uint8_t *)malloc(ng);
        const size_t gpr = ng / (size_t)rows;
        if (!h || !u) { r->bad = 1; free(h); free(u); return; }
        rd(r, h, 2 * (size_t)rows);
        rd(r, u, ng);
        for (size_t i = 0; i < ng; i++) m->s[i] = u8_decode(f16_to_f32(h[i / gpr]), (float)u[i]);
        free(h); free(u);
    }
}
static void rd_q8(Rd *r, QMat *m, int rows, int cols) {
    uint8_t dt = 0xFF;
    uint32_t cnt = 0;
    rd(r, &dt, 1); rd(r, &cnt, 4);
    rd_q8_body(r, m, rows, cols, dt, cnt);
}
/* A table of rows read as lz_t_row_f32 reads it (src/ops_epi.c:1260-1290):
 * a Q8_0 row is its codes times their group's scale, an F32 / BF16 row its
 * values.  Returns rows * cols floats. */
static float *rd_rows_f32(Rd *r, int rows, int cols) {
    uint8_t dt = 0xFF;
    uint32_t cnt = 0;
    float *p;
    QMat q;
    rd(r, &dt, 1); rd(r, &cnt, 4);
    if (dt != 1) return rd_f32_body(r, rows * cols, dt, cnt);
    rd_q8_body(r, &q, rows, cols, dt, cnt);
    p = (float *)malloc(sizeof(float) * (size_t)rows * cols);
    if (r->bad || !p) { r->bad = 1; free_q(&q); free(p); return NULL; }
    for (size_t i = 0; i < (size_t)rows * cols; i++) p[i] = (float)q.q[i] * q.s[i / (size_t)q.gs];
    free_q(&q);
    return p;
}

/* Cos/sin table of lz_rope_build_table, rope scaling type 0
 * (src/forward_rope.c:75-210).  The float powf/sinf/cosf restatement is the
 * product's host-side one (a model constant, not on the GPU path); its output
 * is pinned entry by entry against the table the reference engine builds. */
#include "../llama98-zh_amd/csrc/mathf.c"
static void rope_table(OModel *m) {
    m->rope_cs = (float *)malloc(sizeof(float) * (size_t)m->seq_len * m->rot);
    l98_rope_table(m->rope_cs, m->seq_len, m->rot, m->theta);
}

ORA_API void ora_close(void *h) {
    OModel *m = (OModel *)h;
    if (!m) return;
    free_q(&m->embed);
    free(m->final_norm);
    for (int l = 0; m->L && l < m->n_layers; l++) {
        OLayer *L = &m->L[l];
        free(L->in_norm); free(L->post_norm);
        free_q(&L->q); free_q(&L->k); free_q(&L->v); free_q(&L->o);
        free(L->q_norm); free(L->k_norm);
        free_q(&L->kq); free_q(&L->kk); free_q(&L->kv); free_q(&L->fa); free_q(&L->fb);
        free_q(&L->kb); free_q(&L->kg); free_q(&L->ko);
        free(L->conv_q); free(L->conv_k); free(L->conv_v);
        free(L->a_log); free(L->dt_bias); free(L->o_norm);
        free_q(&L->router); free_q(&L->down); free_q(&L->up);
        free_q(&L->sg); free_q(&L->su); free_q(&L->sd);
        free(L->bias);
        for (int e = 0; L->w1 && e < m->n_experts; e++) {
            free_q(&L->w1[e]); free_q(&L->w2[e]); free_q(&L->w3[e]);
        }
        free(L->w1); free(L->w2); free(L->w3);
        free(L->sn_q); free(L->sn_k); free(L->sn_v); free(L->sn_o);
        free(L->kn_q); free(L->kn_k); free(L->kn_v); free(L->kn_g); free(L->kn_o);
        free(L->mn_gate); free(L->mn_down); free(L->mn_up);
        free(L->mn_sg); free(L->mn_su); free(L->mn_sd);
    }
    free(m->L);
    free(m->mtp.in_norm); free(m->mtp.post_norm);
    free_q(&m->mtp.q); free_q(&m->mtp.k); free_q(&m->mtp.v); free_q(&m->mtp.o);
    free(m->mtp.q_norm); free(m->mtp.k_norm);
    free(m->mtp.sn_q); free(m->mtp.sn_k); free(m->mtp.sn_v); free(m->mtp.sn_o);
    free(m->mtp.fn_gate); free(m->mtp.fn_up); free(m->mtp.fn_down);
    free_q(&m->mtp_gate); free_q(&m->mtp_up); free_q(&m->mtp_down); free_q(&m->mtp_fc);
    free(m->mtp_norm); free(m->mtp_pre_h); free(m->mtp_pre_e);
    free_q(&m->mtp_main); free(m->mtp_depth); free(m->mtp_mask);
    free(m->rope_cs);
    free(m);
}

/* Reads the version-5 model.bin layout (reference src/model.c:3993-4200,
 * tensors in model_walk order src/model.c:2240-2625). */
ORA_API void *ora_open(const char *dir, char *err, int errlen) {
    char path[1024];
    Rd r;
    char magic[4];
    OModel *m = (OModel *)calloc(1, sizeof(OModel));
    if (!m) return NULL;
    snprintf(path, sizeof path, "%s/model.bin", dir);
    r.f = fopen(path, "rb");
    r.bad = 0;
    r.layout = 0;
    if (!r.f) { snprintf(err, (size_t)errlen, "open %s", path); free(m); return NULL; }
    rd(&r, magic, 4);
    m->version = rd_i32(&r);
    if (memcmp(magic, "L98Z", 4) != 0 || m->version < 4 || m->version > 9) {
        snprintf(err, (size_t)errlen, "bad magic/version");
        fclose(r.f); free(m); return NULL;
    }
    m->vocab = rd_i32(&r); m->d = rd_i32(&r); m->n_layers = rd_i32(&r);
    m->seq_len = rd_i32(&r); m->nh = rd_i32(&r); m->nkv = rd_i32(&r); m->hd = rd_i32(&r);
    m->inter = rd_i32(&r); m->nk = rd_i32(&r); m->nv = rd_i32(&r);
    m->kd = rd_i32(&r); m->vd = rd_i32(&r); m->K = rd_i32(&r);
    m->n_lin = rd_i32(&r); m->n_full = rd_i32(&r); (void)rd_i32(&r);
    (void)rd_i32(&r); (void)rd_i32(&r);
    m->eps = rd_f32(&r); m->theta = rd_f32(&r); (void)rd_f32(&r);
    m->q_dim = rd_i32(&r); m->qg_dim = rd_i32(&r); m->kv_dim = rd_i32(&r);
    m->key = rd_i32(&r); m->value = rd_i32(&r); m->conv_dim = rd_i32(&r);
    m->rot = rd_i32(&r);
    for (int i = 0; i < 128; i++) m->types[i] = rd_i32(&r);
    m->gate_rank = rd_i32(&r); m->has_lb = rd_i32(&r); m->gate_lb = rd_f32(&r);
    m->n_experts = rd_i32(&r); m->topk = rd_i32(&r); (void)rd_i32(&r);
    m->moe_inter = rd_i32(&r); m->latent = rd_i32(&r);
    (void)rd_i32(&r); (void)rd_i32(&r); (void)rd_i32(&r); (void)rd_i32(&r);
    m->shared_w = rd_i32(&r);
    /* lz_open_bin's version ladder (src/model.c:3925-3989, 4105-4460): v4
     * stops after the 13-word tail (no MTP head, hadamard blocks derived);
     * v5 carries the rest of the tail and the 522 appended words; v6 the
     * application table, mtp_n_draft, the rotated-vocabulary words and
     * the scale layout; v7 / v8 / v9 one word each.  The path restated
     * here has the identity schedule, no rotated vocabulary and none of the
     * v7-v9 mechanisms; mtp_n_draft > 1 (at most LZ_SPEC_K_MAX, alloc_mtp
     * src/model.c:2905-2909) is a DSpark head. */
    m->has_mtp = 0;
    m->n_draft = 1;
    m->hadamard_o = m->hadamard_down = -1;
    if (m->version >= 5) {
        m->has_mtp = rd_i32(&r); m->mtp_inter = rd_i32(&r);
        for (int i = 0; i < 5; i++) (void)rd_i32(&r);             /* rope scaling */
        m->use_subn = rd_i32(&r);
        m->hadamard_o = rd_i32(&r);
        m->hadamard_down = rd_i32(&r);
        for (int i = 0; i < 7 + 3 * 128 + 6 + 128; i++) (void)rd_i32(&r);   /* mla .. csa2 */
    }
    if (m->version >= 6) {
        int exec_len = rd_i32(&r), bad = exec_len != m->n_layers;
        for (int i = 0; i < 128; i++) bad |= rd_i32(&r) != (i < m->n_layers ? i : 0);   /* app_layer */
        for (int i = 0; i < 128; i++) bad |= rd_i32(&r) != 0;                          /* app_loop */
        m->n_draft = rd_i32(&r);                                                        /* mtp_n_draft */
        bad |= m->n_draft > SPEC_K_MAX_REF;
        bad |= rd_i32(&r) != 0;                                                         /* embed_hadamard */
        (void)rd_i32(&r);                                                               /* embed_signs_seed */
        r.layout = rd_i32(&r);
        bad |= r.layout < 0 || r.layout > 2;
        if (m->version >= 7) bad |= rd_i32(&r) != 0;                                    /* loop_input_mix */
        if (m->version >= 8) bad |= rd_i32(&r) != 0;                                    /* ced_local */
        if (m->version >= 9) (void)rd_i32(&r);                                          /* loop_input_mix_from */
        if (bad) r.bad = 1;
    }
    m->scale_layout = r.layout;
    if (m->has_mtp != 0 && m->has_mtp != 1) r.bad = 1;
    if (m->n_draft < 1) m->n_draft = 1;
    if (m->n_draft > 1 && !m->has_mtp) r.bad = 1;
    /* resolve_hadamard (src/model.c:139-182): -1 derives (hadamard_o: the
     * whole lin_value_dim on a dense model when it is a power of two, else
     * 0; hadamard_down: the largest power of two <= 512 dividing
     * intermediate_size); an explicit block must be 0 or a power of two
     * dividing its width, and hadamard_down must divide the MTP width. */
    if (m->hadamard_o == -1) {
        int oblk = m->n_experts == 0 ? m->value : 0;
        if (oblk < 2 || (oblk & (oblk - 1))) oblk = 0;
        m->hadamard_o = oblk;
    } else if (m->hadamard_o < 0 || (m->hadamard_o & (m->hadamard_o - 1)) ||
               (m->hadamard_o && m->value % m->hadamard_o)) {
        r.bad = 1;
    }
    if (m->hadamard_down == -1) {
        int dblk = 512;
        while (dblk > 1 && m->inter % dblk) dblk >>= 1;
        m->hadamard_down = dblk == 1 ? 0 : dblk;
    } else if (m->hadamard_down < 0 || (m->hadamard_down & (m->hadamard_down - 1)) ||
               (m->hadamard_down && m->inter % m->hadamard_down)) {
        r.bad = 1;
    }
    if (m->use_subn && m->hadamard_down > 1 && m->mtp_inter % m->hadamard_down) r.bad = 1;
    const int d = m->d;
    rd_q8(&r, &m->embed, m->vocab, d);
    m->final_norm = rd_f32v(&r, d);
    m->L = (OLayer *)calloc((size_t)m->n_layers, sizeof(OLayer));
    for (int l = 0; l < m->n_layers && !r.bad; l++) {
        OLayer *L = &m->L[l];
        L->type = m->types[l];
        L->in_norm = rd_f32v(&r, d);
        L->post_norm = rd_f32v(&r, d);
        if (L->type == 1) {
            rd_q8(&r, &L->q, m->qg_dim, d);
            rd_q8(&r, &L->k, m->kv_dim, d);
            rd_q8(&r, &L->v, m->kv_dim, d);
            rd_q8(&r, &L->o, d, m->q_dim);
            L->q_norm = rd_f32v(&r, m->hd);
            L->k_norm = rd_f32v(&r, m->hd);
            if (m->use_subn) {
                L->sn_q = rd_f32v(&r, d);
                L->sn_k = rd_f32v(&r, d);
                L->sn_v = rd_f32v(&r, d);
                L->sn_o = rd_f32v(&r, m->q_dim);
            }
        } else {
            rd_q8(&r, &L->kq, m->key, d);
            rd_q8(&r, &L->kk, m->key, d);
            rd_q8(&r, &L->kv, m->value, d);
            L->conv_q = rd_f32v(&r, m->key * m->K);
            L->conv_k = rd_f32v(&r, m->key * m->K);
            L->conv_v = rd_f32v(&r, m->value * m->K);
            L->a_log = rd_f32v(&r, m->nv);
            rd_q8(&r, &L->fa, m->gate_rank, d);
            rd_q8(&r, &L->fb, m->nv * m->kd, m->gate_rank);
            L->dt_bias = rd_f32v(&r, m->nv * m->kd);
            rd_q8(&r, &L->kb, m->nv, d);
            rd_q8(&r, &L->kg, m->value, d);
            L->o_norm = rd_f32v(&r, m->vd);
            rd_q8(&r, &L->ko, d, m->value);
            if (m->use_subn) {
                L->kn_q = rd_f32v(&r, d);
                L->kn_k = rd_f32v(&r, d);
                L->kn_v = rd_f32v(&r, d);
                L->kn_g = rd_f32v(&r, d);
                L->kn_o = rd_f32v(&r, m->value);
            }
        }
        rd_q8(&r, &L->router, m->n_experts, d);
        L->bias = rd_f32v(&r, m->n_experts);
        rd_q8(&r, &L->down, m->latent, d);
        rd_q8(&r, &L->up, d, m->latent);
        rd_q8(&r, &L->sg, m->shared_w, d);
        rd_q8(&r, &L->su, m->shared_w, d);
        rd_q8(&r, &L->sd, d, m->shared_w);
        if (m->use_subn) {
            L->mn_gate = rd_f32v(&r, d);
            L->mn_down = rd_f32v(&r, d);
            L->mn_up = rd_f32v(&r, m->latent);
            L->mn_sg = rd_f32v(&r, d);
            L->mn_su = rd_f32v(&r, d);
            L->mn_sd = rd_f32v(&r, m->shared_w);
        }
        L->w1 = (QMat *)calloc((size_t)m->n_experts, sizeof(QMat));
        L->w2 = (QMat *)calloc((size_t)m->n_experts, sizeof(QMat));
        L->w3 = (QMat *)calloc((size_t)m->n_experts, sizeof(QMat));
        for (int e = 0; e < m->n_experts; e++) {
            rd_q8(&r, &L->w1[e], m->moe_inter, m->latent);
            rd_q8(&r, &L->w2[e], m->latent, m->moe_inter);
            rd_q8(&r, &L->w3[e], m->moe_inter, m->latent);
        }
    }
    m->mtp.type = 1;
    if (m->has_mtp) {
    m->mtp.in_norm = rd_f32v(&r, d);
    m->mtp.post_norm = rd_f32v(&r, d);
    if (m->use_subn) {
        m->mtp.fn_gate = rd_f32v(&r, d);
        m->mtp.fn_up = rd_f32v(&r, d);
    }
    rd_q8(&r, &m->mtp.q, m->qg_dim, d);
    rd_q8(&r, &m->mtp.k, m->kv_dim, d);
    rd_q8(&r, &m->mtp.v, m->kv_dim, d);
    rd_q8(&r, &m->mtp.o, d, m->q_dim);
    m->mtp.q_norm = rd_f32v(&r, m->hd);
    m->mtp.k_norm = rd_f32v(&r, m->hd);
    if (m->use_subn) {
        m->mtp.sn_q = rd_f32v(&r, d);
        m->mtp.sn_k = rd_f32v(&r, d);
        m->mtp.sn_v = rd_f32v(&r, d);
        m->mtp.sn_o = rd_f32v(&r, m->q_dim);
    }
    rd_q8(&r, &m->mtp_gate, m->mtp_inter, d);
    rd_q8(&r, &m->mtp_up, m->mtp_inter, d);
    rd_q8(&r, &m->mtp_down, d, m->mtp_inter);
    if (m->use_subn) m->mtp.fn_down = rd_f32v(&r, m->mtp_inter);
    /* MTP_SPECS (src/model.c:2529-2552): fc for one draft slot, or the
     * DSpark main_proj / depth_embed / mask_embed / markov_embed /
     * markov_proj after the three norms.  A model.bin holds no Markov rank
     * (only config.json names it, src/model.c:539), so the two Markov
     * tensors are [vocab][0]: empty, and the correction adds zero. */
    if (m->n_draft <= 1) rd_q8(&r, &m->mtp_fc, d, 2 * d);
    m->mtp_norm = rd_f32v(&r, d);
    m->mtp_pre_h = rd_f32v(&r, d);
    m->mtp_pre_e = rd_f32v(&r, d);
    if (m->n_draft > 1) {
        rd_q8(&r, &m->mtp_main, d, 3 * d);
        m->mtp_depth = rd_rows_f32(&r, m->n_draft, d);
        m->mtp_mask = rd_f32v(&r, d);
        free(rd_f32v(&r, 0));                   /* markov_embed */
        free(rd_f32v(&r, 0));                   /* markov_proj */
    }
    }
    {
        char extra;
        if (!r.bad && fread(&extra, 1, 1, r.f) == 1) r.bad = 1;   /* trailing bytes */
    }
    fclose(r.f);
    if (r.bad) {
        snprintf(err, (size_t)errlen, "model.bin layout mismatch");
        ora_close(m);
        return NULL;
    }
    rope_table(m);
    return m;
}

ORA_API int ora_config(void *h, int *out, int n) {
    OModel *m = (OModel *)h;
    int v[30] = {m->vocab, m->d, m->n_layers, m->seq_len, m->nh, m->nkv, m->hd,
                 m->nk, m->nv, m->kd, m->vd, m->K, m->n_lin, m->n_full,
                 m->gate_rank, m->n_experts, m->topk, m->latent, m->moe_inter,
                 m->shared_w, m->mtp_inter, m->q_dim, m->kv_dim, m->conv_dim,
                 m->version, m->scale_layout, m->has_mtp, m->embed.gs, m->use_subn, m->n_draft};
    for (int i = 0; i < n && i < 30; i++) out[i] = v[i];
    return 30;
}

ORA_API const float *ora_rope_table(void *h) { return ((OModel *)h)->rope_cs; }

/* ---------------------------------------------------------------------- */
/* Run state.                                                              */
/* ---------------------------------------------------------------------- */

#define MAXB 8                                   /* LZ_BATCH_MAX, src/ops.h:1457 */
#define SPEC_K_MAX 6                             /* src/ops.h:2098 */
/* The GPU library's own loops also run k = 7 (a verify of 8 rows), which the
 * reference's cap refuses; the rounds below take k up to SPEC_K_EXT with the
 * same algorithm and an 8-slot ring, so that width has a CPU checker too. */
#define SPEC_K_EXT 7

typedef struct {
    OModel *m;
    int seq_len, depth, nt_cap;
    int ssm_slot, mtp_pos;
    float *kda_state;                            /* [depth][n_lin][nv][kd][vd] */
    float *conv_state;                           /* [depth][n_lin][conv_dim][K-1] */
    int8_t *kq, *vq;                             /* [planes][seq][kv_dim] */
    float *ks, *vs;                              /* [planes][seq][kv_dim/32] */
    int planes;                                  /* n_full + 1 (MTP plane last) */
    float *x, *xb, *xb2;                         /* [MAXB][d] */
    int8_t *xq; float *xqs;
    float *logits, *mtp_logits, *mtp_hidden, *mtp_chain, *mtp_draft, *mtp_draft_q;
    float *mtp_kdraft;                           /* DSpark slot logits [SPEC_K_EXT][V] */
    float *target_p;
    int lin_index[128], full_index[128];
    /* scratch */
    float *t0, *t1, *t2, *t3, *t4, *t5, *att;
} OState;

ORA_API void ora_state_free(void *h) {
    OState *s = (OState *)h;
    if (!s) return;
    free(s->kda_state); free(s->conv_state);
    free(s->kq); free(s->vq); free(s->ks); free(s->vs);
    free(s->x); free(s->xb); free(s->xb2); free(s->xq); free(s->xqs);
    free(s->logits); free(s->mtp_logits); free(s->mtp_hidden); free(s->mtp_chain);
    free(s->mtp_draft); free(s->mtp_draft_q); free(s->target_p); free(s->mtp_kdraft);
    free(s->t0); free(s->t1); free(s->t2); free(s->t3); free(s->t4); free(s->t5);
    free(s->att);
    free(s);
}

static size_t kda_slot_floats(const OModel *m) {
    return (size_t)m->n_lin * m->nv * m->kd * m->vd;
}
static size_t conv_slot_floats(const OModel *m) {
    return (size_t)m->n_lin * m->conv_dim * (m->K - 1);
}

ORA_API void ora_state_reset(void *h) {
    OState *s = (OState *)h;
    const OModel *m = s->m;
    memset(s->kda_state, 0, sizeof(float) * kda_slot_floats(m) * s->depth);
    memset(s->conv_state, 0, sizeof(float) * conv_slot_floats(m) * s->depth);
    memset(s->kq, 0, (size_t)s->planes * s->seq_len * m->kv_dim);
    memset(s->vq, 0, (size_t)s->planes * s->seq_len * m->kv_dim);
    memset(s->ks, 0, sizeof(float) * (size_t)s->planes * s->seq_len * m->kv_dim / 32);
    memset(s->vs, 0, sizeof(float) * (size_t)s->planes * s->seq_len * m->kv_dim / 32);
    memset(s->mtp_chain, 0, sizeof(float) * (size_t)m->d);
    s->ssm_slot = 0;
    s->mtp_pos = 0;
}

/* lz_state_alloc, src/forward_state.c:1245: ring depth = spec_k_max + 1,
 * nt_cap = LZ_BATCH_DEFAULT = 4 (src/ops.h:1462). */
ORA_API void *ora_state_new(void *hm, int seq_len, int spec_k_max) {
    OModel *m = (OModel *)hm;
    OState *s = (OState *)calloc(1, sizeof(OState));
    int wide;
    if (!s) return NULL;
    s->m = m;
    s->seq_len = seq_len > 0 ? seq_len : m->seq_len;
    s->depth = spec_k_max > 0 ? (spec_k_max > SPEC_K_EXT ? SPEC_K_EXT : spec_k_max) + 1 : 1;
    s->nt_cap = 4;
    s->planes = m->n_full + 1;
    {
        int li = 0, fi = 0;
        for (int l = 0; l < m->n_layers; l++) {
            if (m->types[l] == 1) { s->full_index[l] = fi++; s->lin_index[l] = -1; }
            else { s->lin_index[l] = li++; s->full_index[l] = -1; }
        }
    }
    s->kda_state = (float *)calloc(kda_slot_floats(m) * s->depth, sizeof(float));
    s->conv_state = (float *)calloc(conv_slot_floats(m) * s->depth, sizeof(float));
    s->kq = (int8_t *)calloc((size_t)s->planes * s->seq_len * m->kv_dim, 1);
    s->vq = (int8_t *)calloc((size_t)s->planes * s->seq_len * m->kv_dim, 1);
    s->ks = (float *)calloc((size_t)s->planes * s->seq_len * m->kv_dim / 32, sizeof(float));
    s->vs = (float *)calloc((size_t)s->planes * s->seq_len * m->kv_dim / 32, sizeof(float));
    wide = m->d;
    if (3 * m->d > wide) wide = 3 * m->d;
    if (m->qg_dim > wide) wide = m->qg_dim;
    if (m->conv_dim > wide) wide = m->conv_dim;
    if (m->shared_w > wide) wide = m->shared_w;
    if (m->mtp_inter > wide) wide = m->mtp_inter;
    if (m->nv * m->kd > wide) wide = m->nv * m->kd;
    s->x = (float *)calloc((size_t)MAXB * wide, sizeof(float));
    s->xb = (float *)calloc((size_t)MAXB * wide, sizeof(float));
    s->xb2 = (float *)calloc((size_t)MAXB * wide, sizeof(float));
    s->xq = (int8_t *)calloc((size_t)MAXB * wide, 1);
    s->xqs = (float *)calloc((size_t)MAXB * wide / 32 + 8, sizeof(float));
    s->logits = (float *)calloc((size_t)m->vocab, sizeof(float));
    s->mtp_logits = (float *)calloc((size_t)(SPEC_K_EXT + 1) * m->vocab, sizeof(float));
    s->mtp_hidden = (float *)calloc((size_t)(SPEC_K_EXT + 1) * m->d, sizeof(float));
    s->mtp_chain = (float *)calloc((size_t)m->d, sizeof(float));
    s->mtp_draft = (float *)calloc((size_t)m->vocab, sizeof(float));
    s->mtp_draft_q = (float *)calloc((size_t)SPEC_K_EXT * m->vocab, sizeof(float));
    s->mtp_kdraft = (float *)calloc((size_t)SPEC_K_EXT * m->vocab, sizeof(float));
    s->target_p = (float *)calloc((size_t)m->vocab, sizeof(float));
    s->t0 = (float *)calloc((size_t)MAXB * wide * 4, sizeof(float));
    s->t1 = (float *)calloc((size_t)MAXB * wide * 4, sizeof(float));
    s->t2 = (float *)calloc((size_t)MAXB * wide * 4, sizeof(float));
    s->t3 = (float *)calloc((size_t)MAXB * wide * 4, sizeof(float));
    s->t4 = (float *)calloc((size_t)MAXB * wide * 4, sizeof(float));
    s->t5 = (float *)calloc((size_t)MAXB * wide * 4, sizeof(float));
    s->att = (float *)calloc((size_t)s->seq_len + 8, sizeof(float));
    return s;
}

static float *kda_slot(OState *s, int slot, int li, int h) {
    const OModel *m = s->m;
    return s->kda_state + (size_t)slot * kda_slot_floats(m) +
           ((size_t)li * m->nv + h) * m->kd * m->vd;
}
static float *conv_slot(OState *s, int slot, int li) {
    const OModel *m = s->m;
    return s->conv_state + (size_t)slot * conv_slot_floats(m) +
           (size_t)li * m->conv_dim * (m->K - 1);
}

/* ---------------------------------------------------------------------- */
/* Layers.                                                                 */
/* ---------------------------------------------------------------------- */

static void quant_rows(OState *s, const float *x, int n, int nt) {
    for (int t = 0; t < nt; t++)
        o_quantize_q8(x + (size_t)t * n, n, s->xq + (size_t)t * n, s->xqs + (size_t)t * (n / 32));
}
static void mm(OState *s, float *o, const QMat *w, int nt) {
    o_matmul_q8g(o, s->xq, s->xqs, w->q, w->s, w->cols, w->rows, nt, w->gs, NULL);
}

/* One SubLN projection (subn_norm_q8, src/forward_kda.c:203-236, and its
 * twins in forward_attn / forward_moe / dense_ffn_step): RMSNorm(1+w) of
 * each input row with the projection's own weight into tmp, its int8
 * quantization (per 32 elements, or one scale per row when tok), then the
 * matmul. */
static void subn_proj(OState *s, const float *x, const float *wn, const QMat *W, float *out, int nt, int tok,
                      float *tmp) {
    const int n = W->cols;
    for (int t = 0; t < nt; t++) o_rmsnorm(tmp + (size_t)t * n, x + (size_t)t * n, wn, n, s->m->eps);
    for (int t = 0; t < nt; t++) {
        if (tok) o_quantize_q8_tok(tmp + (size_t)t * n, n, s->xq + (size_t)t * n, s->xqs + (size_t)t * (n / 32));
        else o_quantize_q8(tmp + (size_t)t * n, n, s->xq + (size_t)t * n, s->xqs + (size_t)t * (n / 32));
    }
    mm(s, out, W, nt);
}

/* subn_scale_gs + lz_subn_scale_group with the default scale choice
 * (src/forward_kda.c:106-110, src/ops_sched.c:517-520): per-32 scales on a
 * MoE model, one scale per row on a dense (BitLinear) one. */
static int subn_tok(const OModel *m) { return m->n_experts == 0; }

/* lz_causal_conv1d_step, src/ops_conv1d.c:26-87. */
static void conv_step(float *o, const float *x, const float *st_in, float *st_out,
                      const float *w, int n_ch, int k) {
    int hist = k - 1;
    for (int c = 0; c < n_ch; c++) {
        const float *si = st_in + (size_t)c * hist;
        float *so = st_out + (size_t)c * hist;
        const float *wr = w + (size_t)c * k;
        float sum = 0.0f, xc = x[c];
        float keep[16];
        for (int j = 0; j < hist; j++) { sum += wr[j] * si[j]; keep[j] = si[j]; }
        sum += wr[hist] * xc;
        o[c] = o_silu(sum);
        for (int j = 0; j + 1 < hist; j++) so[j] = keep[j + 1];
        if (hist > 0) so[hist - 1] = xc;
    }
}

/* lz_recur_step fp32-state arm, src/ops_gdn.c:2516-2560 (gt = 1). */
ORA_API void o_recur_step(float *out, const float *sf_in, float *sf_out,
                          const float *q, const float *k, const float *v,
                          const float *gvec, float beta, int kd, int vd) {
    float u[512], w[512], kq = 0.0f;
    for (int j = 0; j < vd; j++) { u[j] = 0.0f; w[j] = 0.0f; }
    for (int i = 0; i < kd; i++) {
        const float *row = sf_in + (size_t)i * vd;
        float kc = k[i], qc = q[i];
        float kcw = kc * gvec[i], qcw = qc * gvec[i];
        kq += kc * qc;
        for (int j = 0; j < vd; j++) {
            u[j] += row[j] * kcw;
            w[j] += row[j] * qcw;
        }
    }
    for (int j = 0; j < vd; j++) {
        float vc = v[j];
        u[j] = (vc - 1.0f * u[j]) * beta;
        out[j] = 1.0f * w[j] + u[j] * kq;
    }
    for (int i = 0; i < kd; i++) {
        const float *ri = sf_in + (size_t)i * vd;
        float *ro = sf_out + (size_t)i * vd;
        float kc = k[i], dec = gvec[i];
        for (int j = 0; j < vd; j++) ro[j] = ri[j] * dec + kc * u[j];
    }
}

/* forward_kda float/oracle tier with use_subn = 0, src/forward_kda.c:410-1065.
 * in: s->xb [nt][d]; out: s->xb2 [nt][d]. */
static void forward_kda(OState *s, const OLayer *L, int li, int nt, int advance, int base, int layer) {
    const OModel *m = s->m;
    const int d = m->d, key = m->key, value = m->value, nv = m->nv, kd = m->kd, vd = m->vd;
    const int nvk = nv * kd, D = s->depth, hist = m->K - 1;
    float *q = s->t0, *k = s->t1, *v = s->t2, *g = s->t3, *fa = s->t4, *bvec = s->t5;
    float qc[MAXB * 1024], kc[MAXB * 1024], vc[MAXB * 1024];
    float gate[MAXB * 1024], ssm_out[MAXB * 1024], decay[64];
    float qn[512], kn[512];
    (void)d;
    if (m->use_subn) {
        /* SubLN (:559-612): q/k/v/g each normalize the raw residual with
         * their own weight; f_a and b share one quantization of the raw row */
        const int tok = subn_tok(m);
        subn_proj(s, s->xb, L->kn_q, &L->kq, q, nt, tok, s->xb2);
        subn_proj(s, s->xb, L->kn_k, &L->kk, k, nt, tok, s->xb2);
        subn_proj(s, s->xb, L->kn_v, &L->kv, v, nt, tok, s->xb2);
        subn_proj(s, s->xb, L->kn_g, &L->kg, g, nt, tok, s->xb2);
        for (int t = 0; t < nt; t++) {
            if (tok) o_quantize_q8_tok(s->xb + (size_t)t * d, d, s->xq + (size_t)t * d, s->xqs + (size_t)t * (d / 32));
            else o_quantize_q8(s->xb + (size_t)t * d, d, s->xq + (size_t)t * d, s->xqs + (size_t)t * (d / 32));
        }
        mm(s, fa, &L->fa, nt);
        mm(s, bvec, &L->kb, nt);
    } else {
        /* one quantization of xb shared by q/k/v/f_a/b/g (:615-633) */
        quant_rows(s, s->xb, m->d, nt);
        mm(s, q, &L->kq, nt);
        mm(s, k, &L->kk, nt);
        mm(s, v, &L->kv, nt);
        mm(s, fa, &L->fa, nt);
        mm(s, bvec, &L->kb, nt);
        mm(s, g, &L->kg, nt);
    }
    tap("kq", layer, q, key); tap("kk", layer, k, key); tap("kv", layer, v, value);
    tap("kfa", layer, fa, m->gate_rank); tap("kb", layer, bvec, nv); tap("kg", layer, g, value);
    /* causal conv + SiLU, token-serial over the ring (:680-755) */
    for (int t = 0; t < nt; t++) {
        int si = advance ? (base + t) % D : base;
        int so = advance ? (si + 1 == D ? 0 : si + 1) : base;
        float *bi = conv_slot(s, si, li), *bo = conv_slot(s, so, li);
        conv_step(qc + (size_t)t * key, q + (size_t)t * key, bi, bo, L->conv_q, key, m->K);
        conv_step(kc + (size_t)t * key, k + (size_t)t * key, bi + (size_t)key * hist,
                  bo + (size_t)key * hist, L->conv_k, key, m->K);
        conv_step(vc + (size_t)t * value, v + (size_t)t * value, bi + (size_t)2 * key * hist,
                  bo + (size_t)2 * key * hist, L->conv_v, value, m->K);
    }
    tap("kqc", layer, qc, key); tap("kkc", layer, kc, key); tap("kvc", layer, vc, value);
    /* f_b per token on its own quantization of the f_a row (:760-815) */
    for (int t = 0; t < nt; t++) {
        o_quantize_q8(fa + (size_t)t * m->gate_rank, m->gate_rank, s->xq, s->xqs);
        o_matmul_q8g(gate + (size_t)t * nvk, s->xq, s->xqs, L->fb.q, L->fb.s,
                     m->gate_rank, nvk, 1, L->fb.gs, NULL);
    }
    /* decay gate (kda_gate_build_float, src/forward_kda.c:277-300, :840-850):
     * with a lower bound lb the gate is lb * sigmoid(exp(A_log) * pre),
     * without one -exp(A_log) * softplus(pre) */
    for (int h = 0; h < nv; h++) decay[h] = o_exp(L->a_log[h]);
    for (int t = 0; t < nt; t++)
        for (int h = 0; h < nv; h++)
            for (int i = 0; i < kd; i++) {
                int idx = h * kd + i;
                float pre = gate[(size_t)t * nvk + idx] + L->dt_bias[idx];
                float gg = m->has_lb ? m->gate_lb * o_sigmoid(decay[h] * pre) : -decay[h] * o_softplus(pre);
                gate[(size_t)t * nvk + idx] = o_exp(gg);
            }
    tap("kgate", layer, gate, nvk);
    /* recurrence, head-major then token (:856-940) */
    {
        float scale = o_rsqrt((float)kd);          /* ssm_scale, src/forward_state.c:1409 */
        for (int h = 0; h < nv; h++) {
            int kh = (m->nk == nv) ? h : (h * m->nk / nv);
            for (int t = 0; t < nt; t++) {
                int si = advance ? (base + t) % D : base;
                int so = advance ? (si + 1 == D ? 0 : si + 1) : base;
                const float *qp = qc + (size_t)t * key + (size_t)kh * kd;
                const float *kp = kc + (size_t)t * key + (size_t)kh * kd;
                const float *vp = vc + (size_t)t * value + (size_t)h * vd;
                float beta;
                o_l2norm(qn, qp, kd, 1e-6f);
                o_l2norm(kn, kp, kd, 1e-6f);
                for (int i = 0; i < kd; i++) qn[i] *= scale;
                beta = o_sigmoid(bvec[(size_t)t * nv + h]);
                o_recur_step(ssm_out + (size_t)t * value + (size_t)h * vd,
                             kda_slot(s, si, li, h), kda_slot(s, so, li, h),
                             qn, kn, vp, gate + (size_t)t * nvk + (size_t)h * kd,
                             beta, kd, vd);
            }
        }
    }
    tap("kraw", layer, ssm_out, value);
    /* gated RMSNorm per head, quantize, o_proj (:1000-1043) */
    for (int t = 0; t < nt; t++)
        for (int h = 0; h < nv; h++)
            o_rmsnorm_gated(ssm_out + (size_t)t * value + (size_t)h * vd,
                            ssm_out + (size_t)t * value + (size_t)h * vd,
                            g + (size_t)t * value + (size_t)h * vd, L->o_norm, vd, m->eps);
    if (m->use_subn) {
        /* o_proj's own RMSNorm over the whole value row, then the block
         * Hadamard quantization, or the plain one when hadamard_o <= 1
         * (:954-996) */
        const int tok = subn_tok(m), gw = tok ? 0 : 32;
        for (int t = 0; t < nt; t++) {
            float *row = ssm_out + (size_t)t * value;
            o_rmsnorm(row, row, L->kn_o, value, m->eps);
            if (m->hadamard_o > 1)
                o_subn_fwht_quant(row, value, m->hadamard_o, gw, s->xq + (size_t)t * value,
                                  s->xqs + (size_t)t * (value / 32));
            else if (tok)
                o_quantize_q8_tok(row, value, s->xq + (size_t)t * value, s->xqs + (size_t)t * (value / 32));
            else
                o_quantize_q8(row, value, s->xq + (size_t)t * value, s->xqs + (size_t)t * (value / 32));
        }
        tap("sgdn", layer, ssm_out, value);
    } else {
        tap("sgdn", layer, ssm_out, value);
        quant_rows(s, ssm_out, value, nt);
    }
    mm(s, s->xb2, &L->ko, nt);
}

/* attn_impl + attn_score_loop with a Q8 KV cache and no window
 * (src/forward_attn.c:17-57, 206-660, 663-1073).  plane = KV plane index. */
static void forward_attn(OState *s, const OLayer *L, int plane, int pos0, int nt, int kv_only, int layer) {
    const OModel *m = s->m;
    const int d = m->d, hd = m->hd, nh = m->nh, nkv = m->nkv, kvd = m->kv_dim;
    const int qd = m->q_dim, qgd = m->qg_dim, kv_mul = nh / nkv;
    float *qg = s->t0, *kt = s->t1, *vt = s->t2, *qh = s->t3, *ao = s->t4;
    int8_t *kcache = s->kq + (size_t)plane * s->seq_len * kvd;
    int8_t *vcache = s->vq + (size_t)plane * s->seq_len * kvd;
    float *kscale = s->ks + (size_t)plane * s->seq_len * kvd / 32;
    float *vscale = s->vs + (size_t)plane * s->seq_len * kvd / 32;
    float scale = o_rsqrt((float)hd);              /* attn_scale, src/forward_state.c:1408 */
    if (m->use_subn) {
        /* SubLN (:787-822): q/k/v each normalize the raw residual with their
         * own weight, per-32 quantization */
        if (!kv_only) subn_proj(s, s->xb, L->sn_q, &L->q, qg, nt, 0, s->xb2);
        subn_proj(s, s->xb, L->sn_k, &L->k, kt, nt, 0, s->xb2);
        subn_proj(s, s->xb, L->sn_v, &L->v, vt, nt, 0, s->xb2);
    } else {
        quant_rows(s, s->xb, d, nt);
        mm(s, kt, &L->k, nt);
        mm(s, vt, &L->v, nt);
        if (!kv_only) mm(s, qg, &L->q, nt);
    }
    for (int t = 0; t < nt; t++) {
        int pos = pos0 + t;
        float *qgt = qg + (size_t)t * qgd, *qht = qh + (size_t)t * qd;
        float *ktt = kt + (size_t)t * kvd, *vtt = vt + (size_t)t * kvd;
        if (!kv_only)
            for (int h = 0; h < nh; h++)
                o_rmsnorm(qht + (size_t)h * hd, qgt + (size_t)h * 2 * hd, L->q_norm, hd, m->eps);
        for (int h = 0; h < nkv; h++)
            o_rmsnorm(ktt + (size_t)h * hd, ktt + (size_t)h * hd, L->k_norm, hd, m->eps);
        if (!kv_only) rope(qht, nh, hd, m->rot, pos, m->rope_cs);
        rope(ktt, nkv, hd, m->rot, pos, m->rope_cs);
        o_quantize_q8(ktt, kvd, kcache + (size_t)pos * kvd, kscale + (size_t)pos * kvd / 32);
        o_quantize_q8(vtt, kvd, vcache + (size_t)pos * kvd, vscale + (size_t)pos * kvd / 32);
    }
    if (kv_only) return;
    tap("aq", layer, qh, qd); tap("ak", layer, kt, kvd);
    for (int t = 0; t < nt; t++) {
        int pos = pos0 + t;
        const float *qht = qh + (size_t)t * qd, *qgt = qg + (size_t)t * qgd;
        float *aot = ao + (size_t)t * qd;
        for (int h = 0; h < nh; h++) {
            int kvh = h / kv_mul;
            const float *qhh = qht + (size_t)h * hd;
            float *out = aot + (size_t)h * hd;
            for (int tt = 0; tt <= pos; tt++) {           /* score_q8_row :30-41 */
                const int8_t *kr = kcache + (size_t)tt * kvd + (size_t)kvh * hd;
                const float *ksr = kscale + (size_t)tt * kvd / 32 + (size_t)kvh * hd / 32;
                float sum = 0.0f;
                for (int dd = 0; dd < hd; dd += 32) {
                    float acc = 0.0f;
                    for (int e = 0; e < 32; e++) acc += qhh[dd + e] * (float)kr[dd + e];
                    sum += acc * ksr[dd >> 5];
                }
                s->att[tt] = sum * scale;
            }
            o_softmax(s->att, pos + 1);
            for (int dd = 0; dd < hd; dd++) out[dd] = 0.0f;
            for (int tt = 0; tt <= pos; tt++) {           /* wsum_q8_row :17-21 */
                const int8_t *vr = vcache + (size_t)tt * kvd + (size_t)kvh * hd;
                const float *vsr = vscale + (size_t)tt * kvd / 32 + (size_t)kvh * hd / 32;
                float a = s->att[tt];
                for (int dd = 0; dd < hd; dd++) out[dd] += a * (float)vr[dd] * vsr[dd >> 5];
            }
        }
        for (int h = 0; h < nh; h++) {                    /* output gate :636-643 */
            const float *gate = qgt + (size_t)h * 2 * hd + hd;
            float *out = aot + (size_t)h * hd;
            for (int dd = 0; dd < hd; dd++) out[dd] *= o_sigmoid(gate[dd]);
        }
    }
    tap("ax", layer, ao, qd);
    if (m->use_subn)                                      /* o_proj's own norm (:1015-1024) */
        for (int t = 0; t < nt; t++) o_rmsnorm(ao + (size_t)t * qd, ao + (size_t)t * qd, L->sn_o, qd, m->eps);
    quant_rows(s, ao, qd, nt);
    mm(s, s->xb2, &L->o, nt);
}

/* lz_moe_route with sigmoid scores, bias for selection only, repeated
 * strict-greater argmax, renormalized by the serial sum (src/ops_moe.c:12-163). */
ORA_API void o_moe_route(const float *logits, const float *bias, int E, int topk,
                         int *idx, float *w) {
    float score[256], key[256], wsum = 0.0f;
    for (int t = 0; t < topk; t++) { idx[t] = -1; w[t] = 0.0f; }
    for (int i = 0; i < E; i++) score[i] = o_sigmoid(logits[i]);
    for (int i = 0; i < E; i++) key[i] = score[i] + (bias ? bias[i] : 0.0f);
    for (int t = 0; t < topk && t < E; t++) {
        int best = -1;
        float bk = 0.0f;
        for (int i = 0; i < E; i++) {
            if (key[i] <= -1e30f) continue;
            if (best < 0 || key[i] > bk) { best = i; bk = key[i]; }
        }
        if (best < 0) break;
        idx[t] = best;
        w[t] = score[best];
        wsum += w[t];
        key[best] = -1e30f;
    }
    if (wsum > 0.0f)
        for (int t = 0; t < topk; t++)
            if (idx[t] >= 0) w[t] /= wsum;
}

/* forward_moe + moe_expert_loop, use_subn = 0, latent norm off
 * (src/forward_moe.c:55-212, 220-553).  in: s->xb; out: s->xb2. */
static void forward_moe(OState *s, const OLayer *L, int nt, int layer) {
    const OModel *m = s->m;
    const int d = m->d, E = m->n_experts, lat = m->latent, inter = m->moe_inter;
    const int sw = m->shared_w;
    float *rl = s->t0, *latx = s->t1, *laty = s->t2, *h1 = s->t3, *h3 = s->t4, *h2 = s->t5;
    int8_t lq[2048]; float lqs[64];
    int8_t hq[4096]; float hqs[128];
    float *nx = (float *)malloc(sizeof(float) * (size_t)nt * d);
    if (m->use_subn) {
        /* SubLN (:349-389): the router and the latent down-projection each
         * normalize the raw residual with their own weight */
        subn_proj(s, s->xb, L->mn_gate, &L->router, rl, nt, 0, nx);
        subn_proj(s, s->xb, L->mn_down, &L->down, latx, nt, 0, nx);
    } else {
        quant_rows(s, s->xb, d, nt);                      /* shared by router, down, shared expert */
        mm(s, rl, &L->router, nt);
        mm(s, latx, &L->down, nt);
    }
    tap("mrt", layer, rl, E); tap("mlat", layer, latx, lat);
    for (int t = 0; t < nt; t++) {
        int idx[16]; float w[16];
        float *ly = laty + (size_t)t * lat;
        o_moe_route(rl + (size_t)t * E, L->bias, E, m->topk, idx, w);
        for (int v = 0; v < lat; v++) ly[v] = 0.0f;
        o_quantize_q8(latx + (size_t)t * lat, lat, lq, lqs);   /* reused across experts */
        for (int kk = 0; kk < m->topk; kk++) {
            int e = idx[kk];
            if (e < 0) continue;
            o_matmul_q8g(h1, lq, lqs, L->w1[e].q, L->w1[e].s, lat, inter, 1, L->w1[e].gs, NULL);
            o_matmul_q8g(h3, lq, lqs, L->w3[e].q, L->w3[e].s, lat, inter, 1, L->w3[e].gs, NULL);
            for (int i = 0; i < inter; i++) h1[i] = o_silu(h1[i]) * h3[i];
            o_quantize_q8(h1, inter, hq, hqs);
            o_matmul_q8g(h2, hq, hqs, L->w2[e].q, L->w2[e].s, inter, lat, 1, L->w2[e].gs, NULL);
            for (int v = 0; v < lat; v++) ly[v] += w[kk] * h2[v];
        }
    }
    {
        float *sgo = (float *)malloc(sizeof(float) * (size_t)nt * sw);
        float *suo = (float *)malloc(sizeof(float) * (size_t)nt * sw);
        float *sdo = (float *)malloc(sizeof(float) * (size_t)nt * d);
        tap("mrou", layer, laty, lat);
        if (m->use_subn) {
            /* shared gate / up with their own norms (:455-480); the routed
             * output's own norm before up_proj (:418-430) */
            subn_proj(s, s->xb, L->mn_sg, &L->sg, sgo, nt, 0, nx);
            subn_proj(s, s->xb, L->mn_su, &L->su, suo, nt, 0, nx);
            for (int t = 0; t < nt; t++)
                o_rmsnorm(laty + (size_t)t * lat, laty + (size_t)t * lat, L->mn_up, lat, m->eps);
        } else {
            /* shared expert gate/up read the router's quantization of xb */
            mm(s, sgo, &L->sg, nt);
            mm(s, suo, &L->su, nt);
        }
        quant_rows(s, laty, lat, nt);
        mm(s, s->xb2, &L->up, nt);
        for (int i = 0; i < nt * sw; i++) sgo[i] = o_silu(sgo[i]) * suo[i];
        if (m->use_subn)                                  /* shared down's own norm (:515-525) */
            for (int t = 0; t < nt; t++)
                o_rmsnorm(sgo + (size_t)t * sw, sgo + (size_t)t * sw, L->mn_sd, sw, m->eps);
        quant_rows(s, sgo, sw, nt);
        mm(s, sdo, &L->sd, nt);
        for (int i = 0; i < nt * d; i++) s->xb2[i] += sdo[i];
        free(sgo); free(suo); free(sdo);
    }
    free(nx);
}

/* dense_ffn_step (src/forward_kda.c:1089-1250).  SubLN: gate and up each
 * normalize the raw input with their own weight and quantize it with one
 * scale per row (the float arm's lz_quantize_q8_tok, :1102-1160); the
 * SwiGLU output gets down's own norm, then the block Hadamard quantization
 * (hadamard_down > 1), else the plain one (:1195-1240). */
static void dense_ffn(OState *s, const OLayer *F, const QMat *gp, const QMat *up, const QMat *dp, int nt) {
    const OModel *m = s->m;
    int inter = gp->rows;
    float *hb = s->t0, *hb2 = s->t1;
    if (m->use_subn) {
        subn_proj(s, s->xb, F->fn_gate, gp, hb, nt, 1, s->xb2);
        subn_proj(s, s->xb, F->fn_up, up, hb2, nt, 1, s->xb2);
    } else {
        quant_rows(s, s->xb, m->d, nt);
        mm(s, hb, gp, nt);
        mm(s, hb2, up, nt);
    }
    for (int i = 0; i < nt * inter; i++) hb[i] = o_silu(hb[i]) * hb2[i];
    if (m->use_subn) {
        const int tok = subn_tok(m), gw = tok ? 0 : 32;
        for (int t = 0; t < nt; t++) {
            float *row = hb2 + (size_t)t * inter;
            o_rmsnorm(row, hb + (size_t)t * inter, F->fn_down, inter, m->eps);
            if (m->hadamard_down > 1)
                o_subn_fwht_quant(row, inter, m->hadamard_down, gw, s->xq + (size_t)t * inter,
                                  s->xqs + (size_t)t * (inter / 32));
            else if (tok)
                o_quantize_q8_tok(row, inter, s->xq + (size_t)t * inter, s->xqs + (size_t)t * (inter / 32));
            else
                o_quantize_q8(row, inter, s->xq + (size_t)t * inter, s->xqs + (size_t)t * (inter / 32));
        }
    } else {
        quant_rows(s, hb, inter, nt);
    }
    mm(s, s->xb2, dp, nt);
}

/* lz_t_row_f32 of a Q8_0 row (src/ops_epi.c:1276-1280): q * its group's scale. */
static void embed_row(const OModel *m, int tok, float *out) {
    const int8_t *q = m->embed.q + (size_t)tok * m->d;
    const float *sc = m->embed.s + (size_t)tok * (m->d / m->embed.gs);
    for (int i = 0; i < m->d; i++) out[i] = (float)q[i] * sc[i / m->embed.gs];
}

/* forward_chunk, src/forward.c:1210-1617, for one chunk of nt <= 8 tokens.
 * capture: rows of the final-normed hidden; all_logits: logits of every row
 * into logits_out and advance the ring; otherwise skip_logits or last row
 * logits into s->logits. */
static int forward_chunk(OState *s, const int *tokens, int nt, int pos0, float *capture,
                         int all_logits, float *logits_out, int skip_logits) {
    OModel *m = s->m;
    const int d = m->d;
    int base = s->ssm_slot;
    for (int t = 0; t < nt; t++) {
        if (tokens[t] < 0 || tokens[t] >= m->vocab) return 1;
        if (pos0 + t < 0 || pos0 + t >= s->seq_len) return 1;
    }
    for (int t = 0; t < nt; t++) embed_row(m, tokens[t], s->x + (size_t)t * d);
    tap("emb", -1, s->x, d);
    for (int l = 0; l < m->n_layers; l++) {
        const OLayer *L = &m->L[l];
        if (m->use_subn)                                 /* SubLN: no pre-layer norm (:1426-1449) */
            memcpy(s->xb, s->x, sizeof(float) * (size_t)nt * d);
        else
            for (int t = 0; t < nt; t++)
                o_rmsnorm(s->xb + (size_t)t * d, s->x + (size_t)t * d, L->in_norm, d, m->eps);
        tap("an", l, s->xb, d);
        if (L->type == 1) forward_attn(s, L, s->full_index[l], pos0, nt, 0, l);
        else forward_kda(s, L, s->lin_index[l], nt, all_logits, base, l);
        tap("blk", l, s->xb2, d);
        for (int i = 0; i < nt * d; i++) s->x[i] += s->xb2[i];
        tap("res", l, s->x, d);
        if (m->use_subn)                                 /* (:1535-1542) */
            memcpy(s->xb, s->x, sizeof(float) * (size_t)nt * d);
        else
            for (int t = 0; t < nt; t++)
                o_rmsnorm(s->xb + (size_t)t * d, s->x + (size_t)t * d, L->post_norm, d, m->eps);
        tap("pn", l, s->xb, d);
        forward_moe(s, L, nt, l);
        tap("ffn", l, s->xb2, d);
        for (int i = 0; i < nt * d; i++) s->x[i] += s->xb2[i];
        tap("out", l, s->x, d);
    }
    if (all_logits) s->ssm_slot = (base + nt) % s->depth;
    if (capture)
        for (int t = 0; t < nt; t++)
            o_rmsnorm(capture + (size_t)t * d, s->x + (size_t)t * d, m->final_norm, d, m->eps);
    if (all_logits) {                                    /* chunk_logits_all :931-982 */
        for (int t = 0; t < nt; t++) {
            float *xt = s->x + (size_t)t * d;
            o_rmsnorm(xt, xt, m->final_norm, d, m->eps);
        }
        quant_rows(s, s->x, d, nt);
        mm(s, logits_out, &m->embed, nt);
        return 0;
    }
    if (skip_logits) return 0;
    {                                                    /* chunk_logits_last */
        float *xl = s->x + (size_t)(nt - 1) * d;
        o_rmsnorm(xl, xl, m->final_norm, d, m->eps);
        o_quantize_q8(xl, d, s->xq, s->xqs);
        mm(s, s->logits, &m->embed, 1);
    }
    return 0;
}

/* lz_forward_batch_capture, src/forward.c:1810-1843. */
ORA_API int ora_forward_batch_capture(void *hs, const int *tokens, int n, int pos0, float *h_out) {
    OState *s = (OState *)hs;
    int done = 0;
    if (n < 1 || !h_out) return 1;
    while (done < n) {
        int k = n - done;
        if (k > s->nt_cap) k = s->nt_cap;
        if (forward_chunk(s, tokens + done, k, pos0 + done, h_out + (size_t)done * s->m->d,
                          0, NULL, done + k < n))
            return 1;
        done += k;
    }
    return 0;
}

/* lz_forward_capture, src/forward.c:1623-1632: logits of one token, the
 * final-normed hidden into mtp_chain. */
ORA_API float *ora_forward_capture(void *hs, int token, int pos) {
    OState *s = (OState *)hs;
    if (forward_chunk(s, &token, 1, pos, s->mtp_chain, 0, NULL, 0)) return NULL;
    return s->logits;
}

/* lz_forward_verify, src/forward.c:1774-1808. */
ORA_API int ora_forward_verify(void *hs, const int *tokens, int n, int pos0) {
    OState *s = (OState *)hs;
    int done = 0;
    const OModel *m = s->m;
    if (n < 1 || !m->has_mtp) return 1;                 /* the verify needs the MTP head (:1780) */
    while (done < n) {
        int k = n - done;
        if (k > s->nt_cap) k = s->nt_cap;
        if (forward_chunk(s, tokens + done, k, pos0 + done, s->mtp_hidden + (size_t)done * m->d,
                          1, s->mtp_logits + (size_t)done * m->vocab, 0))
            return 1;
        done += k;
    }
    return 0;
}

/* lz_mtp_draft_step, src/forward_mtp.c:32-144. */
ORA_API float *ora_mtp_draft_step(void *hs, int tok, int pos) {
    OState *s = (OState *)hs;
    OModel *m = s->m;
    const int d = m->d;
    float *emb = s->t5, *concat = s->x, *mx = s->xb2 + 0;
    float mtp_x[4096];
    if (!m->has_mtp || m->n_draft > 1 || tok < 0 || tok >= m->vocab || pos < 0 || pos >= s->seq_len) return NULL;
    (void)mx;
    embed_row(m, tok, emb);
    o_rmsnorm(concat, emb, m->mtp_pre_e, d, m->eps);
    o_rmsnorm(concat + d, s->mtp_chain, m->mtp_pre_h, d, m->eps);
    o_quantize_q8(concat, 2 * d, s->xq, s->xqs);
    o_matmul_q8g(mtp_x, s->xq, s->xqs, m->mtp_fc.q, m->mtp_fc.s, 2 * d, d, 1, m->mtp_fc.gs, NULL);
    if (m->use_subn) memcpy(s->xb, mtp_x, sizeof(float) * (size_t)d);   /* (:82-88) */
    else o_rmsnorm(s->xb, mtp_x, m->mtp.in_norm, d, m->eps);
    forward_attn(s, &m->mtp, m->n_full, pos, 1, 0, -1);
    for (int i = 0; i < d; i++) mtp_x[i] += s->xb2[i];
    if (m->use_subn) memcpy(s->xb, mtp_x, sizeof(float) * (size_t)d);   /* (:99-105) */
    else o_rmsnorm(s->xb, mtp_x, m->mtp.post_norm, d, m->eps);
    dense_ffn(s, &m->mtp, &m->mtp_gate, &m->mtp_up, &m->mtp_down, 1);
    for (int i = 0; i < d; i++) mtp_x[i] += s->xb2[i];
    o_rmsnorm(s->mtp_chain, mtp_x, m->mtp_norm, d, m->eps);
    o_quantize_q8(s->mtp_chain, d, s->xq, s->xqs);
    o_matmul_q8g(s->mtp_draft, s->xq, s->xqs, m->embed.q, m->embed.s, d, m->vocab, 1, m->embed.gs, NULL);
    return s->mtp_draft;
}

/* lz_mtp_prefill / lz_mtp_catchup, src/forward_mtp.c:561-642.  Only the MTP
 * KV rows are observable afterwards, so the attention runs K/V-only (the
 * reference computes and discards the attention output). */
ORA_API int ora_mtp_prefill(void *hs, const float *h_all, const int *next, int n, int pos0) {
    OState *s = (OState *)hs;
    OModel *m = s->m;
    const int d = m->d;
    int done = 0;
    float *concat = (float *)malloc(sizeof(float) * 2 * (size_t)d);
    float *mx = (float *)malloc(sizeof(float) * (size_t)MAXB * d);
    float emb[4096];
    if (!m->has_mtp || m->n_draft > 1 || !h_all || !next || n < 1) { free(concat); free(mx); return 1; }
    while (done < n) {
        int k = n - done;
        if (k > s->nt_cap) k = s->nt_cap;
        for (int t = 0; t < k; t++) {
            if (next[done + t] < 0 || next[done + t] >= m->vocab) { free(concat); free(mx); return 1; }
            embed_row(m, next[done + t], emb);
            o_rmsnorm(concat, emb, m->mtp_pre_e, d, m->eps);
            o_rmsnorm(concat + d, h_all + (size_t)(done + t) * d, m->mtp_pre_h, d, m->eps);
            o_quantize_q8(concat, 2 * d, s->xq, s->xqs);
            o_matmul_q8g(mx + (size_t)t * d, s->xq, s->xqs, m->mtp_fc.q, m->mtp_fc.s, 2 * d, d, 1, m->mtp_fc.gs, NULL);
        }
        if (m->use_subn)                                 /* (:600-611) */
            memcpy(s->xb, mx, sizeof(float) * (size_t)k * d);
        else
            for (int t = 0; t < k; t++)
                o_rmsnorm(s->xb + (size_t)t * d, mx + (size_t)t * d, m->mtp.in_norm, d, m->eps);
        if (pos0 + done + k > s->seq_len) { free(concat); free(mx); return 1; }
        forward_attn(s, &m->mtp, m->n_full, pos0 + done, k, 1, -1);
        done += k;
    }
    free(concat); free(mx);
    return 0;
}

/* ---------------------------------------------------------------------- */
/* Sampling and acceptance.                                                */
/* ---------------------------------------------------------------------- */

/* xorshift64* (src/sampler.c:112-120). */
static uint32_t rng_u32(uint64_t *st) {
    *st ^= *st >> 12;
    *st ^= *st << 25;
    *st ^= *st >> 27;
    return (uint32_t)((*st * 0x2545F4914F6CDD1Dull) >> 32);
}
ORA_API float o_random_f32(uint64_t *st) {
    return (float)(rng_u32(st) >> 8) / 16777216.0f;
}

/* sample_argmax, src/sampler.c:121-137: order-preserving key, first wins. */
ORA_API int o_argmax(const float *p, int n) {
    int best_i = 0;
    uint32_t best = fkey(p[0]);
    for (int i = 1; i < n; i++) {
        uint32_t k = fkey(p[i]);
        if (k > best) { best_i = i; best = k; }
    }
    return best_i;
}

/* lz_argmax_p1, src/sampler.c:139-155: float '>' argmax with an online
 * softmax for the top-1 probability. */
ORA_API int o_argmax_p1(const float *logits, int n, float *out_p) {
    int best_i = 0;
    float best_v = logits[0], l = 1.0f;
    for (int i = 1; i < n; i++) {
        float v = logits[i];
        if (v > best_v) {
            l = l * o_exp(best_v - v) + 1.0f;
            best_v = v;
            best_i = i;
        } else {
            l += o_exp(v - best_v);
        }
    }
    if (out_p) *out_p = (l > 0.0f) ? 1.0f / l : 1.0f;
    return best_i;
}

/* lz_spec_accept, src/generate.c:232-243. */
ORA_API int o_spec_accept(const int *draft, const int *targ, int n_draft, int bonus, int *out) {
    if (!draft || !targ || !out || n_draft < 0) return 0;
    for (int i = 0; i < n_draft; i++) {
        out[i] = targ[i];
        if (draft[i] != targ[i]) return i;
    }
    out[n_draft] = bonus;
    return n_draft;
}

/* sample_residual + lz_spec_accept_temp, src/generate.c:261-346. */
static int sample_residual(const float *p, const float *q, int vocab, uint64_t *rng) {
    float total = 0.0f, coin, cdf = 0.0f;
    int last_pos = -1;
    for (int i = 0; i < vocab; i++) {
        float dd = p[i] - q[i];
        if (dd > 0.0f) { total += dd; last_pos = i; }
    }
    if (total <= 0.0f) return o_argmax(p, vocab);
    coin = o_random_f32(rng) * total;
    for (int i = 0; i < vocab; i++) {
        float dd = p[i] - q[i];
        if (dd > 0.0f) {
            cdf += dd;
            if (coin < cdf) return i;
        }
    }
    return last_pos;
}
ORA_API int o_spec_accept_temp(const float *p, const float *q, int x, int vocab, float u,
                               uint64_t *rng, int *out_accepted) {
    float qx, ratio;
    if (!p || !q || !rng || vocab <= 0 || x < 0 || x >= vocab) {
        if (out_accepted) *out_accepted = 0;
        return -1;
    }
    qx = q[x];
    if (qx <= 0.0f) ratio = 0.0f;
    else {
        ratio = p[x] / qx;
        if (ratio > 1.0f) ratio = 1.0f;
    }
    if (u < ratio) {
        if (out_accepted) *out_accepted = 1;
        return x;
    }
    if (out_accepted) *out_accepted = 0;
    return sample_residual(p, q, vocab, rng);
}

/* lz_sample_temp_q, src/sampler.c:736-747 (q left in logits). */
static int sample_mult(const float *p, int n, float coin) {
    float cdf = 0.0f;
    for (int i = 0; i < n; i++) {
        cdf += p[i];
        if (coin < cdf) return i;
    }
    return n - 1;
}
ORA_API int o_sample_temp_q(float *logits, int n, float temp, uint64_t *rng) {
    float inv = 1.0f / temp, coin;
    for (int i = 0; i < n; i++) logits[i] *= inv;
    o_softmax(logits, n);
    coin = o_random_f32(rng);
    return sample_mult(logits, n, coin);
}

/* select_all's descending sort by probability.  glibc's qsort is a stable
 * merge sort at these sizes, so equal probabilities keep index order; the
 * restatement sorts stably by (prob desc, index asc). */
typedef struct { float prob; int index; } PI;
static void merge_desc(PI *a, PI *tmp, int n) {
    if (n < 2) return;
    int h = n / 2;
    merge_desc(a, tmp, h);
    merge_desc(a + h, tmp, n - h);
    int i = 0, j = h, k = 0;
    while (i < h && j < n) {
        if (a[j].prob > a[i].prob) tmp[k++] = a[j++];
        else tmp[k++] = a[i++];
    }
    while (i < h) tmp[k++] = a[i++];
    while (j < n) tmp[k++] = a[j++];
    memcpy(a, tmp, sizeof(PI) * (size_t)n);
}

/* lz_target_dist with top-k off and min-p off (src/sampler.c:526-730):
 * /T, softmax, select_all (cutoff (1-topp)/(n-1), sort desc), top-p
 * crossing element kept, renormalized by the kept mass. */
ORA_API void o_target_dist(float *logits, int n, float temp, float topp, float *out_p) {
    float inv;
    if (topp <= 0.0f || topp >= 1.0f) {
        inv = 1.0f / temp;
        for (int i = 0; i < n; i++) logits[i] *= inv;
        o_softmax(logits, n);
        memcpy(out_p, logits, sizeof(float) * (size_t)n);
        return;
    }
    memset(out_p, 0, sizeof(float) * (size_t)n);
    inv = 1.0f / temp;
    for (int i = 0; i < n; i++) logits[i] *= inv;
    o_softmax(logits, n);
    {
        const float cutoff = (n > 1) ? (1.0f - topp) / (float)(n - 1) : 0.0f;
        PI *buf = (PI *)malloc(sizeof(PI) * (size_t)n), *tmp = (PI *)malloc(sizeof(PI) * (size_t)n);
        int n0 = 0, last;
        float mass = 1.0f, limit, cum = 0.0f;
        for (int i = 0; i < n; i++)
            if (logits[i] >= cutoff) { buf[n0].index = i; buf[n0].prob = logits[i]; n0++; }
        if (n0 > 1) merge_desc(buf, tmp, n0);
        if (n0 <= 0) {
            out_p[o_argmax(logits, n)] = 1.0f;
            free(buf); free(tmp);
            return;
        }
        last = n0 - 1;
        limit = topp * mass;
        for (int i = 0; i < n0; i++) {
            cum += buf[i].prob;
            if (cum >= limit) { last = i; break; }
        }
        for (int i = 0; i <= last; i++) out_p[buf[i].index] = buf[i].prob / cum;
        free(buf); free(tmp);
    }
}

/* lz_sample_ex for temperature > 0, top-p on, top-k/min-p off, penalties
 * off (src/sampler.c:794-840): coin first, then the candidate set, then the
 * scan over the sorted candidates scaled by the kept mass. */
ORA_API int o_sample_topp(float *logits, int n, float temp, float topp, uint64_t *rng) {
    float coin, inv;
    if (!(temp > 0.0f)) return o_argmax(logits, n);
    coin = o_random_f32(rng);
    inv = 1.0f / temp;
    if (topp <= 0.0f || topp >= 1.0f) {
        for (int i = 0; i < n; i++) logits[i] *= inv;
        o_softmax(logits, n);
        return sample_mult(logits, n, coin);
    }
    for (int i = 0; i < n; i++) logits[i] *= inv;
    o_softmax(logits, n);
    {
        const float cutoff = (n > 1) ? (1.0f - topp) / (float)(n - 1) : 0.0f;
        PI *buf = (PI *)malloc(sizeof(PI) * (size_t)n), *tmp = (PI *)malloc(sizeof(PI) * (size_t)n);
        int n0 = 0, last, res;
        float limit, cum = 0.0f, r, cdf = 0.0f;
        for (int i = 0; i < n; i++)
            if (logits[i] >= cutoff) { buf[n0].index = i; buf[n0].prob = logits[i]; n0++; }
        if (n0 > 1) merge_desc(buf, tmp, n0);
        if (n0 <= 0) { free(buf); free(tmp); return o_argmax(logits, n); }
        last = n0 - 1;
        limit = topp * 1.0f;
        for (int i = 0; i < n0; i++) {
            cum += buf[i].prob;
            if (cum >= limit) { last = i; break; }
        }
        r = coin * cum;
        res = buf[last].index;
        for (int i = 0; i <= last; i++) {
            cdf += buf[i].prob;
            if (r < cdf) { res = buf[i].index; break; }
        }
        free(buf); free(tmp);
        return res;
    }
}

/* sample_from_dist, src/generate.c:1151-1160. */
static int sample_from_dist(const float *p, int vocab, uint64_t *rng) {
    float coin = o_random_f32(rng), cdf = 0.0f;
    for (int i = 0; i < vocab; i++) {
        cdf += p[i];
        if (coin < cdf) return i;
    }
    return vocab - 1;
}

/* mtp_attn_t1, src/forward_mtp.c:191-376, float arm with Q8 KV: one
 * token at position 0 of the MTP plane with no history.  Softmax over the
 * single score is exactly 1, so K, Q, RoPE and the scores are not
 * computed; V is quantized into the plane's row 0 and read back through
 * wsum_q8_row's arithmetic (src/forward_attn.c:17-21) with weight 1, then
 * gated.  in: s->xb (one row); out: s->xb2. */
static void attn_t1(OState *s, const OLayer *L) {
    const OModel *m = s->m;
    const int d = m->d, hd = m->hd, nh = m->nh, nkv = m->nkv, kvd = m->kv_dim, qd = m->q_dim;
    const int kv_mul = nh / nkv;
    float *qg = s->t0, *vt = s->t2, *ao = s->t4;
    int8_t *vrow = s->vq + (size_t)m->n_full * s->seq_len * kvd;
    float *vsrow = s->vs + (size_t)m->n_full * s->seq_len * kvd / 32;
    if (m->use_subn) {                            /* q and v, each its own norm (:226-235) */
        subn_proj(s, s->xb, L->sn_q, &L->q, qg, 1, 0, s->xb2);
        subn_proj(s, s->xb, L->sn_v, &L->v, vt, 1, 0, s->xb2);
    } else {                                      /* one shared quantization (:236-240) */
        quant_rows(s, s->xb, d, 1);
        mm(s, qg, &L->q, 1);
        mm(s, vt, &L->v, 1);
    }
    o_quantize_q8(vt, kvd, vrow, vsrow);          /* the V write at slot 0 (:250-251) */
    for (int h = 0; h < nh; h++) {
        const int kvh = h / kv_mul;
        const int8_t *vr = vrow + (size_t)kvh * hd;
        const float *vsr = vsrow + (size_t)kvh * hd / 32;
        const float *gate = qg + (size_t)h * 2 * hd + hd;
        float *out = ao + (size_t)h * hd;
        for (int e = 0; e < hd; e++) {
            out[e] = 0.0f;
            out[e] += 1.0f * (float)vr[e] * vsr[e >> 5];
        }
        for (int e = 0; e < hd; e++) out[e] *= o_sigmoid(gate[e]);   /* (:355-356) */
    }
    if (m->use_subn) o_rmsnorm(ao, ao, L->sn_o, qd, m->eps);        /* (:359-362) */
    quant_rows(s, ao, qd, 1);
    mm(s, s->xb2, &L->o, 1);
}

/* lz_mtp_draft_batch, src/forward_mtp.c:385-505: k slots from the same
 * anchor hidden state (s->mtp_chain), each through main_proj over
 * [norm(h) | norm(emb) | depth row], the MTP block at position 0 (attn_t1),
 * the dense FFN, the exit norm and the tied lm_head, into row `slot` of
 * s->mtp_kdraft.  Slot 0's emb is next_token's embedding row, every later
 * slot's the shared mask_embed.  The chain is not changed. */
ORA_API float *ora_mtp_draft_batch(void *hs, int next_token, int k) {
    OState *s = (OState *)hs;
    OModel *m = s->m;
    const int d = m->d;
    float *concat = s->t5, *emb = s->t3, *hn, mtp_x[4096], ex[4096];
    if (!m->has_mtp || m->n_draft <= 1 || next_token < 0 || next_token >= m->vocab || k <= 0 || k > m->n_draft)
        return NULL;
    hn = concat;
    o_rmsnorm(hn, s->mtp_chain, m->mtp_pre_h, d, m->eps);          /* (:404-406) */
    for (int slot = 0; slot < k; slot++) {
        if (slot == 0) embed_row(m, next_token, emb);
        else memcpy(emb, m->mtp_mask, sizeof(float) * (size_t)d);
        o_rmsnorm(concat + d, emb, m->mtp_pre_e, d, m->eps);      /* (:429-431) */
        memcpy(concat + 2 * d, m->mtp_depth + (size_t)slot * d, sizeof(float) * (size_t)d);
        o_quantize_q8(concat, 3 * d, s->xq, s->xqs);               /* lz_matmul_w (:438-439) */
        o_matmul_q8g(mtp_x, s->xq, s->xqs, m->mtp_main.q, m->mtp_main.s, 3 * d, d, 1, m->mtp_main.gs, NULL);
        if (m->use_subn) memcpy(s->xb, mtp_x, sizeof(float) * (size_t)d);
        else o_rmsnorm(s->xb, mtp_x, m->mtp.in_norm, d, m->eps);
        attn_t1(s, &m->mtp);
        for (int i = 0; i < d; i++) mtp_x[i] += s->xb2[i];
        if (m->use_subn) memcpy(s->xb, mtp_x, sizeof(float) * (size_t)d);
        else o_rmsnorm(s->xb, mtp_x, m->mtp.post_norm, d, m->eps);
        dense_ffn(s, &m->mtp, &m->mtp_gate, &m->mtp_up, &m->mtp_down, 1);
        for (int i = 0; i < d; i++) mtp_x[i] += s->xb2[i];
        o_rmsnorm(ex, mtp_x, m->mtp_norm, d, m->eps);               /* (:497-505) */
        o_quantize_q8(ex, d, s->xq, s->xqs);
        o_matmul_q8g(s->mtp_kdraft + (size_t)slot * m->vocab, s->xq, s->xqs, m->embed.q, m->embed.s, d, m->vocab,
                     1, m->embed.gs, NULL);
    }
    return s->mtp_kdraft;
}

/* lz_mtp_markov_correct, src/forward_mtp.c:510-531: logits +=
 * markov_proj(markov_embed[x_prev]).  The rank is 0 for every model.bin
 * (the Markov tensors are [vocab][0]), so the projection is a row of zeros
 * (lz_matmul over no inputs) and the update adds +0 to each entry. */
ORA_API void ora_mtp_markov_correct(void *hs, int x_prev, float *logits) {
    OState *s = (OState *)hs;
    const OModel *m = s->m;
    if (!m->has_mtp || m->n_draft <= 1 || x_prev < 0 || x_prev >= m->vocab) return;
    for (int v = 0; v < m->vocab; v++) logits[v] += 0.0f;
}

/* lz_spec_round_dspark (greedy, no penalties), src/generate.c:1000-1133:
 * one draft batch, each slot corrected and argmax'd in order (p_min cut),
 * the verify, acceptance, ring rollback and the chain reseed; no MTP
 * position advance and no catch-up. */
ORA_API int ora_spec_round_dspark(void *hs, int anchor, int anchor_pos, int k, float p_min, int n_min,
                                  int brk, int *out, int *out_n_accept, int *out_new_pos, int *out_k_eff) {
    OState *s = (OState *)hs;
    const OModel *m = s->m;
    const int V = m->vocab;
    int draft[SPEC_K_EXT], vt[SPEC_K_EXT + 1], targ[SPEC_K_EXT];
    int k_eff = 0, n_accept, bonus, base;
    float *bl;
    if (k < 1 || k > SPEC_K_EXT || k > s->depth - 1 || k > m->n_draft) return -1;
    bl = ora_mtp_draft_batch(s, anchor, k);
    if (!bl) return -2;
    for (int i = 0; i < k; i++) {
        int x_prev = i == 0 ? anchor : draft[i - 1], idx;
        float p1, *row = bl + (size_t)i * V;
        ora_mtp_markov_correct(s, x_prev, row);
        idx = o_argmax_p1(row, V, &p1);
        if (p1 < p_min) break;
        draft[i] = idx;
        k_eff = i + 1;
    }
    if (k_eff < n_min) {
        out[0] = anchor;
        *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
        return 0;
    }
    base = s->ssm_slot;
    vt[0] = anchor;
    for (int i = 0; i < k_eff; i++) vt[i + 1] = draft[i];
    if (ora_forward_verify(s, vt, k_eff + 1, anchor_pos + 1)) return -2;
    for (int i = 0; i < k_eff; i++) targ[i] = o_argmax(s->mtp_logits + (size_t)i * V, V);
    bonus = o_argmax(s->mtp_logits + (size_t)k_eff * V, V);
    n_accept = o_spec_accept(draft, targ, k_eff, bonus, out);
    if (n_accept < k_eff && !brk) s->ssm_slot = (base + n_accept + 1) % s->depth;
    memcpy(s->mtp_chain, s->mtp_hidden + (size_t)n_accept * m->d, sizeof(float) * (size_t)m->d);
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    return n_accept + 1;
}

/* lz_spec_round_dspark_temp (penalties off), src/generate.c:1382-1505. */
ORA_API int ora_spec_round_dspark_temp(void *hs, int anchor, int anchor_pos, int k, float p_min, int n_min,
                                       float temp, float topp, uint64_t *rng, int brk, int *out,
                                       int *out_n_accept, int *out_new_pos, int *out_k_eff) {
    OState *s = (OState *)hs;
    const OModel *m = s->m;
    const int V = m->vocab;
    int draft[SPEC_K_EXT], vt[SPEC_K_EXT + 1];
    int k_eff = 0, n_accept, base;
    float *bl;
    if (k < 1 || k > SPEC_K_EXT || k > s->depth - 1 || k > m->n_draft) return -1;
    bl = ora_mtp_draft_batch(s, anchor, k);
    if (!bl) return -2;
    for (int i = 0; i < k; i++) {
        int x_prev = i == 0 ? anchor : draft[i - 1], idx;
        float *row = bl + (size_t)i * V;
        ora_mtp_markov_correct(s, x_prev, row);
        idx = o_sample_temp_q(row, V, temp, rng);
        if (row[idx] < p_min) break;
        draft[i] = idx;
        memcpy(s->mtp_draft_q + (size_t)i * V, row, sizeof(float) * (size_t)V);
        k_eff = i + 1;
    }
    if (k_eff < n_min) {
        out[0] = anchor;
        *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
        return 0;
    }
    base = s->ssm_slot;
    vt[0] = anchor;
    for (int i = 0; i < k_eff; i++) vt[i + 1] = draft[i];
    if (ora_forward_verify(s, vt, k_eff + 1, anchor_pos + 1)) return -2;
    n_accept = k_eff;
    for (int i = 0; i < k_eff; i++) {
        float *row = s->mtp_logits + (size_t)i * V;
        float u;
        int acc, tok;
        o_target_dist(row, V, temp, topp, s->target_p);
        u = o_random_f32(rng);
        tok = o_spec_accept_temp(s->target_p, s->mtp_draft_q + (size_t)i * V, draft[i], V, u, rng, &acc);
        out[i] = tok;
        if (!acc) { n_accept = i; break; }
    }
    if (n_accept == k_eff) {
        float *row = s->mtp_logits + (size_t)k_eff * V;
        o_target_dist(row, V, temp, topp, s->target_p);
        out[k_eff] = sample_from_dist(s->target_p, V, rng);
    }
    if (n_accept < k_eff && !brk) s->ssm_slot = (base + n_accept + 1) % s->depth;
    memcpy(s->mtp_chain, s->mtp_hidden + (size_t)n_accept * m->d, sizeof(float) * (size_t)m->d);
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    return n_accept + 1;
}

/* lz_spec_round (greedy, no penalties), src/generate.c:694-994. */
ORA_API int ora_spec_round(void *hs, int anchor, int anchor_pos, int k, float p_min, int n_min,
                           int brk, int skipc, int *out, int *out_n_accept, int *out_new_pos,
                           int *out_k_eff) {
    OState *s = (OState *)hs;
    const OModel *m = s->m;
    int draft[SPEC_K_EXT], vt[SPEC_K_EXT + 1], targ[SPEC_K_EXT];
    int k_eff = 0, n_accept, bonus, base;
    if (k < 1 || k > SPEC_K_EXT || k > s->depth - 1) return -1;
    for (int i = 0; i < k; i++) {
        int in_tok = i == 0 ? anchor : draft[i - 1];
        float p1;
        float *lg = ora_mtp_draft_step(s, in_tok, s->mtp_pos + i);
        int idx;
        if (!lg) return -2;
        idx = o_argmax_p1(lg, m->vocab, &p1);
        if (p1 < p_min) break;
        draft[i] = idx;
        k_eff = i + 1;
    }
    if (k_eff < n_min) {
        out[0] = anchor;
        *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
        return 0;
    }
    base = s->ssm_slot;
    vt[0] = anchor;
    for (int i = 0; i < k_eff; i++) vt[i + 1] = draft[i];
    if (ora_forward_verify(s, vt, k_eff + 1, anchor_pos + 1)) return -2;
    for (int i = 0; i < k_eff; i++) targ[i] = o_argmax(s->mtp_logits + (size_t)i * m->vocab, m->vocab);
    bonus = o_argmax(s->mtp_logits + (size_t)k_eff * m->vocab, m->vocab);
    n_accept = o_spec_accept(draft, targ, k_eff, bonus, out);
    if (n_accept < k_eff && !brk) s->ssm_slot = (base + n_accept + 1) % s->depth;
    memcpy(s->mtp_chain, s->mtp_hidden + (size_t)n_accept * m->d, sizeof(float) * (size_t)m->d);
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    if (n_accept > 1 && !skipc)
        if (ora_mtp_prefill(s, s->mtp_hidden, out, n_accept - 1, s->mtp_pos + 1)) return -2;
    s->mtp_pos += n_accept;
    return n_accept + 1;
}

/* lz_spec_round_temp (penalties off), src/generate.c:1234-1377. */
ORA_API int ora_spec_round_temp(void *hs, int anchor, int anchor_pos, int k, float p_min, int n_min,
                                float temp, float topp, uint64_t *rng, int brk, int skipc,
                                int *out, int *out_n_accept, int *out_new_pos, int *out_k_eff) {
    OState *s = (OState *)hs;
    const OModel *m = s->m;
    const int V = m->vocab;
    int draft[SPEC_K_EXT], vt[SPEC_K_EXT + 1];
    int k_eff = 0, n_accept, base;
    if (k < 1 || k > SPEC_K_EXT || k > s->depth - 1) return -1;
    for (int i = 0; i < k; i++) {
        int in_tok = i == 0 ? anchor : draft[i - 1];
        float *lg = ora_mtp_draft_step(s, in_tok, s->mtp_pos + i);
        int idx;
        if (!lg) return -2;
        idx = o_sample_temp_q(lg, V, temp, rng);
        if (lg[idx] < p_min) break;
        draft[i] = idx;
        memcpy(s->mtp_draft_q + (size_t)i * V, lg, sizeof(float) * (size_t)V);
        k_eff = i + 1;
    }
    if (k_eff < n_min) {
        out[0] = anchor;
        *out_n_accept = 0; *out_new_pos = anchor_pos; *out_k_eff = k_eff;
        return 0;
    }
    base = s->ssm_slot;
    vt[0] = anchor;
    for (int i = 0; i < k_eff; i++) vt[i + 1] = draft[i];
    if (ora_forward_verify(s, vt, k_eff + 1, anchor_pos + 1)) return -2;
    n_accept = k_eff;
    for (int i = 0; i < k_eff; i++) {
        float *row = s->mtp_logits + (size_t)i * V;
        float u;
        int acc, tok;
        o_target_dist(row, V, temp, topp, s->target_p);
        u = o_random_f32(rng);
        tok = o_spec_accept_temp(s->target_p, s->mtp_draft_q + (size_t)i * V, draft[i], V, u, rng, &acc);
        out[i] = tok;
        if (!acc) { n_accept = i; break; }
    }
    if (n_accept == k_eff) {
        float *row = s->mtp_logits + (size_t)k_eff * V;
        o_target_dist(row, V, temp, topp, s->target_p);
        out[k_eff] = sample_from_dist(s->target_p, V, rng);
    }
    if (n_accept < k_eff && !brk) s->ssm_slot = (base + n_accept + 1) % s->depth;
    memcpy(s->mtp_chain, s->mtp_hidden + (size_t)n_accept * m->d, sizeof(float) * (size_t)m->d);
    *out_n_accept = n_accept;
    *out_new_pos = anchor_pos + 1 + n_accept;
    *out_k_eff = k_eff;
    if (n_accept > 1 && !skipc)
        if (ora_mtp_prefill(s, s->mtp_hidden, out, n_accept - 1, s->mtp_pos + 1)) return -2;
    s->mtp_pos += n_accept;
    return n_accept + 1;
}

/* Prefill + MTP prefill (src/generate.c:2806-2960). */
ORA_API int ora_session_start(void *hs, const int *prompt, int n_prompt) {
    OState *s = (OState *)hs;
    float *h;
    int rc;
    ora_state_reset(s);
    if (n_prompt < 2) return 1;
    h = (float *)malloc(sizeof(float) * (size_t)(n_prompt - 1) * s->m->d);
    rc = ora_forward_batch_capture(s, prompt, n_prompt - 1, 0, h);
    /* A DSpark head has no fc for lz_mtp_prefill to project through, and no
     * DSpark step reads the MTP KV rows: its session is the body prefill. */
    if (!rc && s->m->has_mtp && s->m->n_draft <= 1) {
        rc = ora_mtp_prefill(s, h, prompt + 1, n_prompt - 1, s->mtp_pos);
        s->mtp_pos = n_prompt - 1;
    }
    free(h);
    return rc;
}

/* The generation loop of lz_generate_spec_round (src/generate.c:1822-2106)
 * with penalties off: tokens[] receives the emitted ids (the whole last
 * round, so up to n_new + k).  p_min / n_min go to every round as the
 * reference harness (oracle/ref_harness.c) passes them; a discarded round
 * records n_accept -1.  Returns the number written or < 0. */
ORA_API int ora_generate_ex(void *hs, const int *prompt, int n_prompt, int k, int n_new,
                            float temp, float topp, uint64_t seed, int brk, int skipc, float p_min,
                            int n_min, int *tokens, int cap, int *k_eff_out, int *n_acc_out,
                            int *n_rounds, uint64_t *rng_out) {
    OState *s = (OState *)hs;
    const OModel *m = s->m;
    uint64_t rng = seed ? seed : 1;
    int n = 0, token, pos, have_seed = 0, rounds = 0;
    if (ora_session_start(s, prompt, n_prompt)) return -1;
    token = prompt[n_prompt - 1];
    pos = n_prompt - 1;
    while (n < n_new) {
        int anchor, anchor_pos, out[SPEC_K_EXT + 1], n_accept = 0, new_pos = 0, k_eff = 0, ne;
        if (have_seed) {
            anchor = token;
            anchor_pos = pos - 1;
        } else {
            float *lg = ora_forward_capture(s, token, pos);
            if (!lg) return -2;
            anchor_pos = pos;
            anchor = temp > 0.0f ? o_sample_topp(lg, m->vocab, temp, topp, &rng)
                                 : o_argmax(lg, m->vocab);
            if (n < cap) tokens[n] = anchor;
            n++;
            if (n >= n_new) break;
        }
        if (m->n_draft > 1 && temp > 0.0f)       /* src/generate.c:1929-1946 */
            ne = ora_spec_round_dspark_temp(s, anchor, anchor_pos, k, p_min, n_min, temp, topp, &rng, brk, out,
                                            &n_accept, &new_pos, &k_eff);
        else if (m->n_draft > 1)
            ne = ora_spec_round_dspark(s, anchor, anchor_pos, k, p_min, n_min, brk, out, &n_accept, &new_pos,
                                       &k_eff);
        else if (temp > 0.0f)
            ne = ora_spec_round_temp(s, anchor, anchor_pos, k, p_min, n_min, temp, topp, &rng, brk,
                                     skipc, out, &n_accept, &new_pos, &k_eff);
        else
            ne = ora_spec_round(s, anchor, anchor_pos, k, p_min, n_min, brk, skipc, out, &n_accept,
                                &new_pos, &k_eff);
        if (ne < 0) return -3;
        if (k_eff_out) k_eff_out[rounds] = k_eff;
        if (n_acc_out) n_acc_out[rounds] = ne > 0 ? n_accept : -1;
        rounds++;
        have_seed = ne > 0;
        if (ne > 0)
            for (int i = 0; i <= n_accept; i++) {
                if (n < cap) tokens[n] = out[i];
                n++;
            }
        pos = new_pos + 1;
        token = out[n_accept];
    }
    if (n_rounds) *n_rounds = rounds;
    if (rng_out) *rng_out = rng;
    return n;
}

ORA_API int ora_generate(void *hs, const int *prompt, int n_prompt, int k, int n_new,
                         float temp, float topp, uint64_t seed, int brk, int skipc,
                         int *tokens, int cap, int *k_eff_out, int *n_acc_out, int *n_rounds,
                         uint64_t *rng_out) {
    return ora_generate_ex(hs, prompt, n_prompt, k, n_new, temp, topp, seed, brk, skipc, 0.0f, 0,
                           tokens, cap, k_eff_out, n_acc_out, n_rounds, rng_out);
}

/* State accessors for the tests. */
ORA_API int ora_state_info(void *hs, int *out) {
    OState *s = (OState *)hs;
    out[0] = s->ssm_slot; out[1] = s->mtp_pos; out[2] = s->depth; out[3] = s->planes;
    out[4] = s->seq_len;
    return 5;
}
ORA_API void ora_set_slot(void *hs, int slot) { ((OState *)hs)->ssm_slot = slot; }
ORA_API const float *ora_kda_state(void *hs, int slot) {
    OState *s = (OState *)hs;
    return s->kda_state + (size_t)slot * kda_slot_floats(s->m);
}
ORA_API const float *ora_conv_state(void *hs, int slot) {
    OState *s = (OState *)hs;
    return s->conv_state + (size_t)slot * conv_slot_floats(s->m);
}
ORA_API const float *ora_mtp_logits(void *hs) { return ((OState *)hs)->mtp_logits; }
ORA_API const float *ora_mtp_hidden(void *hs) { return ((OState *)hs)->mtp_hidden; }
ORA_API const float *ora_mtp_chain(void *hs) { return ((OState *)hs)->mtp_chain; }
ORA_API const float *ora_draft_logits(void *hs) { return ((OState *)hs)->mtp_draft; }
ORA_API const float *ora_kdraft_logits(void *hs) { return ((OState *)hs)->mtp_kdraft; }
ORA_API const float *ora_logits(void *hs) { return ((OState *)hs)->logits; }
ORA_API void ora_kv_plane(void *hs, int plane, int rows, int8_t *kq, float *ks, int8_t *vq, float *vs) {
    OState *s = (OState *)hs;
    int kvd = s->m->kv_dim;
    size_t off = (size_t)plane * s->seq_len * kvd;
    memcpy(kq, s->kq + off, (size_t)rows * kvd);
    memcpy(vq, s->vq + off, (size_t)rows * kvd);
    memcpy(ks, s->ks + off / 32, sizeof(float) * (size_t)rows * kvd / 32);
    memcpy(vs, s->vs + off / 32, sizeof(float) * (size_t)rows * kvd / 32);
}
ORA_API void ora_set_mtp_pos(void *hs, int pos) { ((OState *)hs)->mtp_pos = pos; }

/* Host-side float math for the RoPE cos/sin table.
 *
 * The reference builds its table (src/forward_rope.c:75-210, rope scaling
 * type 0) with its own all-float adaptations of the ARM optimized-routines
 * powf / sinf / cosf (src/lz_mathf.c), which are not correctly rounded: a
 * table of correctly-rounded cos/sin differs from it in most entries.  These
 * functions restate that float algorithm step for step -- table-driven
 * log2 + exp2 for powf, quadrant reduction (fast path below 120, 2/pi bit
 * table above) and the two short polynomials for sin/cos -- so the table is
 * bit-identical.  The constants are the published optimized-routines
 * coefficients rounded to float, as the reference carries them.
 *
 * Plain C, compiled with -ffp-contract=off: every operation rounds once in
 * the written order.
 */
#include <stdint.h>
#include <string.h>

#include "mathf.h"

static uint32_t as_u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float as_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- powf: log2 via a 16-entry (1/c, log2 c) table + degree-5 poly ---- */
static const float PW_INVC[16] = {
    1.39890718460083f, 1.3403141498565674f, 1.2864322662353516f, 1.2367150783538818f,
    1.1906976699829102f, 1.147982120513916f, 1.1082251071929932f, 1.0711297988891602f,
    1.0364372730255127f, 1.0f, 0.9492859840393066f, 0.8951049447059631f,
    0.8476821780204773f, 0.8050314784049988f, 0.7664670944213867f, 0.7314286231994629f,
};
static const float PW_LOGC[16] = {
    -0.4843002259731293f, -0.42257124185562134f, -0.3633754253387451f, -0.30651310086250305f,
    -0.25180721282958984f, -0.19910015165805817f, -0.148251011967659f, -0.09913323819637299f,
    -0.05163281410932541f, 0.0f, 0.07508531957864761f, 0.15987126529216766f,
    0.23840466141700745f, 0.3128829002380371f, 0.38370421528816223f, 0.45121103525161743f,
};
static const float PW_A[5] = {
    0.28845757246017456f, -0.3609260618686676f, 0.4808984696865082f,
    -0.721347451210022f, 1.4426950216293335f,
};
/* exp2: 2^(j/32) mantissas + cubic */
static const uint32_t E2_TAB[32] = {
    0x3f800000, 0x3f82cd87, 0x3f85aac3, 0x3f88980f, 0x3f8b95c2, 0x3f8ea43a, 0x3f91c3d3, 0x3f94f4f0,
    0x3f9837f0, 0x3f9b8d3a, 0x3f9ef532, 0x3fa27043, 0x3fa5fed7, 0x3fa9a15b, 0x3fad583f, 0x3fb123f6,
    0x3fb504f3, 0x3fb8fbaf, 0x3fbd08a4, 0x3fc12c4d, 0x3fc5672a, 0x3fc9b9be, 0x3fce248c, 0x3fd2a81e,
    0x3fd744fd, 0x3fdbfbb8, 0x3fe0ccdf, 0x3fe5b907, 0x3feac0c7, 0x3fefe4ba, 0x3ff5257d, 0x3ffa83b3,
};
static const float E2_C[3] = {0.055503614246845245f, 0.24022845923900604f, 0.6931471824645996f};

static float pw_log2(uint32_t ix) {
    uint32_t tmp = ix - 0x3f330000u;
    int i = (int)((tmp >> 19) % 16u);
    uint32_t top = tmp & 0xff800000u;
    uint32_t iz = ix - top;
    int k = (int32_t)top >> 23;
    float z = as_f(iz);
    float r = z * PW_INVC[i] - 1.0f;
    float yl0 = PW_LOGC[i] + (float)k;
    float r2 = r * r;
    float y = PW_A[0] * r + PW_A[1];
    float p = PW_A[2] * r + PW_A[3];
    float r4 = r2 * r2;
    float q = PW_A[4] * r + yl0;
    q = p * r2 + q;
    y = y * r4 + q;
    return y;
}

static float pw_exp2(float xd) {
    float x32 = xd * 32.0f, frac, r, r2, y, z, s;
    int k = (int)x32, kexp, over = 0;
    frac = x32 - (float)k;
    if (frac > 0.5f || (frac == 0.5f && (k & 1))) k += 1;
    else if (frac < -0.5f || (frac == -0.5f && (k & 1))) k -= 1;
    r = xd - (float)k * 0.03125f;
    uint32_t t = E2_TAB[k & 31];
    kexp = k >> 5;
    if (kexp > 127) { kexp = 127; over = 1; }
    if (kexp >= -126) {
        s = as_f((t & 0x007fffffu) | ((uint32_t)(kexp + 127) << 23));
    } else {
        int shift = kexp + 149;
        s = as_f(t) * as_f(shift > 0 ? 1u << shift : 1u);
    }
    r2 = r * r;
    y = E2_C[0] * r + E2_C[1];
    z = E2_C[2] * r + 1.0f;
    z = y * r2 + z;
    y = z * s;
    if (over) y *= 2.0f;
    return y;
}

/* Positive finite x, finite y: the only domain the table uses (theta > 0,
 * exponent -2i/rot).  y = +-0 gives 1. */
float l98_powf(float x, float y) {
    uint32_t ix = as_u(x), iy = as_u(y);
    if ((iy << 1) == 0) return 1.0f;
    if (ix < 0x00800000u) {                     /* subnormal x */
        ix = as_u(x * 8388608.0f) & 0x7fffffffu;
        ix -= 23u << 23;
    }
    float ylogx = y * pw_log2(ix);
    if (ylogx > 128.0f) return as_f(0x7f800000u);
    if (ylogx <= -150.0f) return 0.0f;
    return pw_exp2(ylogx);
}

/* ---- sinf / cosf ---- */
typedef struct {
    float sign[4], hpi_inv, hpi, c0, c1, c2, c3, c4, s1, s2, s3;
} SC;
static const SC SCT[2] = {
    {{1.0f, -1.0f, -1.0f, 1.0f}, 10680707.0f, 1.5707963705062866f,
     1.0f, -0.5f, 0.04166662320494652f, -0.0013886763481423259f, 2.4390450562350452e-05f,
     -0.16666655242443085f, 0.008332177996635437f, -0.0001951729936990887f},
    {{1.0f, -1.0f, -1.0f, 1.0f}, 10680707.0f, 1.5707963705062866f,
     -1.0f, 0.5f, -0.04166662320494652f, 0.0013886763481423259f, -2.4390450562350452e-05f,
     -0.16666655242443085f, 0.008332177996635437f, -0.0001951729936990887f},
};
static const uint32_t INV_PIO4[24] = {
    0xa2, 0xa2f9, 0xa2f983, 0xa2f9836e, 0xf9836e4e, 0x836e4e44, 0x6e4e4415, 0x4e441529,
    0x441529fc, 0x1529fc27, 0x29fc2757, 0xfc2757d1, 0x2757d1f5, 0x57d1f534, 0xd1f534dd,
    0xf534ddc0, 0x34ddc0db, 0xddc0db62, 0xc0db6295, 0xdb629599, 0x6295993c, 0x95993c43,
    0x993c4390, 0x3c439041,
};
static const float PI63 = 3.4061216748705226e-19f;
static const float PIO4 = 0.7853981852531433f;

static uint32_t top12(float x) { return (as_u(x) >> 20) & 0x7ffu; }

static float reduce_fast(float x, const SC *p, int *np) {
    float r = x * p->hpi_inv;
    int n = ((int32_t)r + 0x800000) >> 24;
    *np = n;
    return x - (float)n * p->hpi;
}

static float reduce_large(uint32_t xi, int *np) {
    const uint32_t *arr = &INV_PIO4[(xi >> 26) & 15];
    int shift = (xi >> 23) & 7;
    uint64_t n, r0, r1, r2;
    xi = (xi & 0xffffffu) | 0x800000u;
    xi <<= shift;
    r0 = (uint32_t)(xi * arr[0]);
    r1 = (uint64_t)xi * arr[4];
    r2 = (uint64_t)xi * arr[8];
    r0 = (r2 >> 32) | (r0 << 32);
    r0 += r1;
    n = (r0 + ((uint64_t)1 << 61)) >> 62;
    r0 -= n << 62;
    *np = (int)n;
    volatile float xf = (float)(int64_t)r0;
    return xf * PI63;
}

static float sc_poly(float x, float x2, const SC *p, int n) {
    if ((n & 1) == 0) {
        float x3 = x * x2;
        float s1 = p->s2 + x2 * p->s3;
        float x7 = x3 * x2;
        float s = x + x3 * p->s1;
        return s + x7 * s1;
    } else {
        float x4 = x2 * x2;
        float c2 = p->c3 + x2 * p->c4;
        float c1 = p->c0 + x2 * p->c1;
        float x6 = x4 * x2;
        float c = c1 + x4 * p->c2;
        return c + x6 * c2;
    }
}

/* Finite arguments only (the table's angles are finite). */
float l98_sinf(float y) {
    float x = y, s;
    int n;
    const SC *p = &SCT[0];
    if (top12(y) < top12(PIO4)) {
        s = x * x;
        if (top12(y) < top12(0.000244140625f)) return y;
        return sc_poly(x, s, p, 0);
    } else if (top12(y) < top12(120.0f)) {
        x = reduce_fast(x, p, &n);
        s = p->sign[n & 3];
        if (n & 2) p = &SCT[1];
        return sc_poly(x * s, x * x, p, n);
    } else {
        uint32_t xi = as_u(y);
        int sign = (int)(xi >> 31);
        x = reduce_large(xi, &n);
        s = p->sign[(n + sign) & 3];
        if ((n + sign) & 2) p = &SCT[1];
        return sc_poly(x * s, x * x, p, n);
    }
}

float l98_cosf(float y) {
    float x = y, s;
    int n;
    const SC *p = &SCT[0];
    if (top12(y) < top12(PIO4)) {
        float x2 = x * x;
        if (top12(y) < top12(0.000244140625f)) return 1.0f;
        return sc_poly(x, x2, p, 1);
    } else if (top12(y) < top12(120.0f)) {
        x = reduce_fast(x, p, &n);
        s = p->sign[n & 3];
        if (n & 2) p = &SCT[1];
        return sc_poly(x * s, x * x, p, n ^ 1);
    } else {
        uint32_t xi = as_u(y);
        int sign = (int)(xi >> 31);
        x = reduce_large(xi, &n);
        s = p->sign[(n + sign) & 3];
        if ((n + sign) & 2) p = &SCT[1];
        return sc_poly(x * s, x * x, p, n ^ 1);
    }
}

/* Rope scaling type 0 (src/forward_rope.c:75-210): freq_i = theta^(-2i/rot),
 * cs[(l*half + i)*2 + {0,1}] = {cos, sin}((float)l * freq_i). */
void l98_rope_table(float *cs, int seq_len, int rot, float theta) {
    int half = rot >> 1;
    for (int i = 0; i < half; i++) {
        float freq = l98_powf(theta, -2.0f * (float)i / (float)rot);
        for (int l = 0; l < seq_len; l++) {
            float ang = (float)l * freq;
            cs[((size_t)l * half + i) * 2] = l98_cosf(ang);
            cs[((size_t)l * half + i) * 2 + 1] = l98_sinf(ang);
        }
    }
}

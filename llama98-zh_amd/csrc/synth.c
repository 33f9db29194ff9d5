/* Seeded random-init KunMoe model.bin writer.  See synth.h for the format
 * contract; every citation below is into the reference tree. */
#define _POSIX_C_SOURCE 200809L
#include "synth.h"

#include <errno.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

/* Format codes of the reference (src/model.h:71-77) and layer kinds
 * (src/model.h:37-39). */
enum { FMT_F32 = 0, FMT_Q8_0 = 1, FMT_BF16 = 6 };
enum { LT_FULL = 1, LT_KDA = 2 };
#define MAX_LAYERS 128
/* The echo variant (config 11): vocabulary and residual-writer std. */
#define ECHO_VOCAB 64
#define ECHO_RESID_STD 0.085f

/* ---------------------------------------------------------------- RNG --- */

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* ln(x) for x > 0 from basic operations: x = m 2^e with m in
 * [sqrt(1/2), sqrt(2)), ln m = 2 atanh((m-1)/(m+1)) by its odd series. */
static double det_log(double x) {
    union { double d; uint64_t u; } b;
    b.d = x;
    int e = (int)((b.u >> 52) & 0x7FF) - 1023;
    b.u = (b.u & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
    double m = b.d;
    if (m > 1.4142135623730951) { m *= 0.5; e += 1; }
    double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double t = 1.0 / 21.0;
    t = t * s2 + 1.0 / 19.0; t = t * s2 + 1.0 / 17.0; t = t * s2 + 1.0 / 15.0;
    t = t * s2 + 1.0 / 13.0; t = t * s2 + 1.0 / 11.0; t = t * s2 + 1.0 / 9.0;
    t = t * s2 + 1.0 / 7.0;  t = t * s2 + 1.0 / 5.0;  t = t * s2 + 1.0 / 3.0;
    t = t * s2 + 1.0;
    return 2.0 * s * t + (double)e * 0.6931471805599453;
}

/* e^x for |x| < 700 from basic operations: x = k ln2 + r, |r| <= ln2/2. */
static double det_exp(double x) {
    double kf = x * 1.4426950408889634;
    long k = (long)(kf < 0 ? kf - 0.5 : kf + 0.5);
    double r = x - (double)k * 0.6931471805599453;
    double t = 1.0, term = 1.0;
    for (int i = 1; i < 20; i++) { term = term * r / (double)i; t += term; }
    union { double d; uint64_t u; } b;
    b.u = (uint64_t)(k + 1023) << 52;
    return t * b.d;
}

/* sin and cos of x in [0, 2pi) by quadrant reduction and Taylor series. */
static void det_sincos(double x, double *sn, double *cs) {
    const double PIO2 = 1.5707963267948966;
    int q = (int)(x / PIO2 + 0.5);
    double r = x - (double)q * PIO2;           /* |r| <= pi/4 (+ulp) */
    double r2 = r * r;
    double s = r, c = 1.0, ts = r, tc = 1.0;
    for (int i = 1; i < 12; i++) {
        ts = -ts * r2 / (double)((2 * i) * (2 * i + 1));
        tc = -tc * r2 / (double)((2 * i - 1) * (2 * i));
        s += ts; c += tc;
    }
    switch (q & 3) {
    case 0: *sn = s;  *cs = c;  break;
    case 1: *sn = c;  *cs = -s; break;
    case 2: *sn = -s; *cs = -c; break;
    default: *sn = -c; *cs = s; break;
    }
}

static double uniform01(uint64_t *st) {        /* [0, 1) */
    return (double)(splitmix64(st) >> 11) * (1.0 / 9007199254740992.0);
}

double l98_synth_normal(uint64_t *st) {
    /* One Box-Muller draw per call (the sine half is discarded) keeps every
     * element a pure function of its own stream position. */
    double u1 = (double)((splitmix64(st) >> 11) + 1) * (1.0 / 9007199254740992.0);
    double u2 = uniform01(st);
    double rad = __builtin_sqrt(-2.0 * det_log(u1));
    double sn, cs;
    det_sincos(6.283185307179586 * u2, &sn, &cs);
    (void)sn;
    return rad * cs;
}

/* ------------------------------------------------------------ configs --- */

int l98_synth_config(int id, L98SynthConfig *c) {
    memset(c, 0, sizeof(*c));
    c->attn_period = 4;
    c->conv_kernel = 4;
    c->w_std = 0.02f;
    c->bias_std = 0.01f;
    switch (id) {
    case 0: case 2: case 4: case 5:
        c->vocab = 8192; c->hidden = 256; c->n_layers = 4; c->seq_len = 512;
        c->n_heads = 4; c->n_kv_heads = 2; c->head_dim = 64;
        c->kda_heads = 4; c->kd = 64; c->vd = 64; c->gate_rank = 64;
        c->n_experts = 16; c->topk = 2; c->latent = 128; c->moe_inter = 256;
        c->shared_w = 256; c->mtp_inter = 256;
        if (id == 4) {
            c->seq_len = 2304;
            c->router_std = 0.0625f;      /* 1/sqrt(256): unit-variance logits */
            c->bias_std = 0.5f;
        }
        if (id == 5) {
            c->use_subn = 1;
            c->hadamard_o = 64;
            c->hadamard_down = 256;
        }
        return 0;
    case 1:
        c->vocab = 65536; c->hidden = 1024; c->n_layers = 24; c->seq_len = 1280;
        c->n_heads = 16; c->n_kv_heads = 4; c->head_dim = 64;
        c->kda_heads = 16; c->kd = 64; c->vd = 64; c->gate_rank = 64;
        c->n_experts = 64; c->topk = 6; c->latent = 256; c->moe_inter = 512;
        c->shared_w = 512; c->mtp_inter = 512;
        return 0;
    case 3:
        c->vocab = 131072; c->hidden = 2048; c->n_layers = 32; c->seq_len = 5200;
        c->n_heads = 16; c->n_kv_heads = 4; c->head_dim = 128;
        c->kda_heads = 16; c->kd = 128; c->vd = 128; c->gate_rank = 128;
        c->n_experts = 128; c->topk = 8; c->latent = 512; c->moe_inter = 768;
        c->shared_w = 768; c->mtp_inter = 768;
        return 0;
    case 13: case 16: case 17:
        if (l98_synth_config(10, c)) return 1;
        c->bin_version = id == 13 ? 9 : id == 16 ? 7 : 8;
        c->gs = id == 16 ? 0 : 32;
        c->scale_layout = id == 13 ? 1 : id == 17 ? 2 : 0;
        c->bf16_small = id == 13 ? 1 : 0;
        return 0;
    case 14: case 15:
        if (l98_synth_config(0, c)) return 1;
        c->bin_version = id == 14 ? 6 : 4;
        c->gs = id == 14 ? 128 : 64;
        c->scale_layout = id == 14 ? 2 : 0;
        c->bf16_small = id == 14 ? 1 : 0;
        return 0;
    case 23:                          /* configs[4]: configs[3]'s model, skewed router */
        if (l98_synth_config(3, c)) return 1;
        c->seq_len = 2304;
        c->router_std = 0.022097087f;     /* 1/sqrt(2048): unit-variance logits */
        c->bias_std = 0.5f;
        return 0;
    case 24: case 25:                 /* the KDA gate's lower-bound arm (K3's -5) */
        if (l98_synth_config(id == 24 ? 0 : 10, c)) return 1;
        c->gate_lb = -5.0f;
        return 0;
    case 22:
        if (l98_synth_config(1, c)) return 1;
        c->bin_version = 6;
        c->mtp_n_draft = 6;
        return 0;
    case 18: case 19: case 20: case 21:
        if (l98_synth_config(id == 18 ? 10 : id == 19 ? 11 : id == 20 ? 0 : 12, c)) return 1;
        c->bin_version = id == 20 ? 7 : 6;
        c->mtp_n_draft = id == 18 ? 4 : id == 19 ? 6 : 3;
        if (id == 20) {
            c->gs = 64;
            c->bf16_small = 1;
        }
        return 0;
    case 10: case 11: case 12:
        c->vocab = 512; c->hidden = 64; c->n_layers = 4; c->seq_len = 160;
        c->n_heads = 2; c->n_kv_heads = 1; c->head_dim = 32;
        c->kda_heads = 2; c->kd = 32; c->vd = 32; c->gate_rank = 32;
        c->n_experts = 8; c->topk = 2; c->latent = 32; c->moe_inter = 64;
        c->shared_w = 64; c->mtp_inter = 64;
        if (id == 11) {
            c->vocab = ECHO_VOCAB;
            c->seq_len = 256;
            c->resid_std = ECHO_RESID_STD;
            c->mtp_echo = 1;
        }
        if (id == 12) {
            c->use_subn = 1;
            c->hadamard_o = 32;
            c->hadamard_down = 64;
        }
        return 0;
    default:
        return 1;
    }
}

/* ------------------------------------------------------------- writer --- */

typedef struct {
    FILE *f;
    uint64_t seed;
    uint32_t tensor_id;         /* position in model_walk order */
    int n_threads;
    int failed;
    int gs, scale_layout, bf16;  /* Q8_0 group size (0: per row), scale plane, BF16 small tensors */
} Writer;

/* IEEE binary16 from binary32, round to nearest even (finite, normal or
 * subnormal results; the scales written here are far inside the range). */
static uint16_t f32_to_f16(float f) {
    union { float f; uint32_t u; } b;
    b.f = f;
    uint32_t sign = (b.u >> 16) & 0x8000u, a = b.u & 0x7FFFFFFFu;
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7BFFu);          /* clamp to the largest finite */
    if (a < 0x33000001u) return (uint16_t)sign;                        /* rounds to zero */
    int e = (int)(a >> 23) - 127;
    uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    int shift = e >= -14 ? 13 : 13 + (-14 - e);                        /* subnormals shift further */
    uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) r++;
    uint32_t h;
    if (e >= -14) h = ((uint32_t)(e + 15) << 10) + (r - 0x400u);       /* a carry into the exponent is fine */
    else h = r;
    return (uint16_t)(sign | h);
}
static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, u;
    if (e == 0) {
        if (m == 0) u = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            u = sign | ((uint32_t)(127 - 14 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else {
        u = sign | ((e + 127u - 15u) << 23) | (m << 13);
    }
    union { uint32_t u; float f; } b;
    b.u = u;
    return b.f;
}
/* bf16 of an f32, round to nearest even (finite inputs). */
static uint16_t f32_to_bf16(float f) {
    union { float f; uint32_t u; } b;
    b.f = f;
    uint32_t r = b.u + 0x7FFFu + ((b.u >> 16) & 1u);
    return (uint16_t)(r >> 16);
}
/* The layout-2 decode the reader applies: base * (u / 255), each step
 * rounded to float. */
static float u8_decode(float base, float u) {
    volatile float levels = 255.0f;
    volatile float q = u / levels;
    volatile float p = base * q;
    return p;
}

static void put_bytes(Writer *w, const void *p, size_t n) {
    if (!w->failed && fwrite(p, 1, n, w->f) != n) w->failed = 1;
}
static void put_u32(Writer *w, uint32_t v) { put_bytes(w, &v, 4); }
static void put_i32(Writer *w, int32_t v) { put_bytes(w, &v, 4); }
static void put_f32(Writer *w, float v) { put_bytes(w, &v, 4); }

typedef enum { INIT_NORMAL, INIT_UNIFORM, INIT_CONST, INIT_ALOG, INIT_DTBIAS, INIT_EYE, INIT_EYE2 } InitKind;

typedef struct {
    uint64_t seed;
    uint32_t tensor_id;
    int rows, cols;
    InitKind kind;
    float a, b;                 /* NORMAL: std, mean; UNIFORM: lo, hi; CONST: value */
    int quantize;
    int gs, layout;             /* Q8: group size, scale plane layout */
    float *f;                   /* rows*cols floats (F32 tensors) */
    int8_t *q;                  /* rows*cols int8 (Q8 tensors) */
    float *scale;               /* rows*cols/gs decoded scales */
    uint16_t *s16;              /* layout 1: binary16 per group; layout 2: binary16 per row */
    uint8_t *u8;                /* layout 2: u8 per group */
    int r0, r1;
} Job;

static uint64_t row_stream(uint64_t seed, uint32_t tensor_id, int row) {
    uint64_t s = seed ^ ((uint64_t)tensor_id * 0xD1B54A32D192ED03ull);
    s ^= (uint64_t)(uint32_t)row * 0x8CB92BA72F3D8DD7ull;
    (void)splitmix64(&s);
    return s;
}

static float init_value(const Job *j, uint64_t *st, int r, int c) {
    switch (j->kind) {
    case INIT_EYE:              /* left square block I, right block N(0, a) */
        if (c >= j->rows) return (float)((double)j->a * l98_synth_normal(st));
        return r == c ? 1.0f : 0.0f;
    case INIT_EYE2:             /* two square blocks I, then N(0, a) */
        if (c >= 2 * j->rows) return (float)((double)j->a * l98_synth_normal(st));
        return r == c % j->rows ? 1.0f : 0.0f;
    case INIT_NORMAL:
        return (float)((double)j->b + (double)j->a * l98_synth_normal(st));
    case INIT_UNIFORM:
        return (float)((double)j->a + ((double)j->b - (double)j->a) * uniform01(st));
    case INIT_ALOG:             /* A_log = ln U(1, 16) */
        return (float)det_log(1.0 + 15.0 * uniform01(st));
    case INIT_DTBIAS: {         /* inverse softplus of dt, dt log-uniform in [1e-3, 1e-1] */
        double lo = det_log(1e-3), hi = det_log(1e-1);
        double dt = det_exp(lo + (hi - lo) * uniform01(st));
        return (float)det_log(det_exp(dt) - 1.0);
    }
    default:
        return j->a;
    }
}

static void *job_run(void *arg) {
    Job *j = (Job *)arg;
    float *row = (float *)malloc(sizeof(float) * (size_t)j->cols);
    if (!row) return NULL;
    for (int r = j->r0; r < j->r1; r++) {
        uint64_t st = row_stream(j->seed, j->tensor_id, r);
        for (int c = 0; c < j->cols; c++) row[c] = init_value(j, &st, r, c);
        if (!j->quantize) {
            memcpy(j->f + (size_t)r * j->cols, row, sizeof(float) * (size_t)j->cols);
            continue;
        }
        /* Symmetric int8 per group of gs: s = amax/127 in the stored form
         * (f32, binary16, or a row's binary16 base times u8/255), then
         * q = rne(w / s) with the scale the reader decodes. */
        const int ng = j->cols / j->gs;
        float sg[4096];
        float base = 0.0f;
        for (int g = 0; g < ng; g++) {
            float amax = 0.0f;
            for (int c = g * j->gs; c < (g + 1) * j->gs; c++) {
                float a = row[c] < 0 ? -row[c] : row[c];
                if (a > amax) amax = a;
            }
            sg[g] = amax > 0.0f ? amax / 127.0f : 1.0f;
            if (sg[g] > base) base = sg[g];
        }
        if (j->layout == 2) {
            const uint16_t b16 = f32_to_f16(base);
            const float bd = f16_to_f32(b16);
            j->s16[r] = b16;
            for (int g = 0; g < ng; g++) {
                int u = (int)__builtin_rintf(255.0f * (sg[g] / bd));
                u = u < 1 ? 1 : u > 255 ? 255 : u;
                j->u8[(size_t)r * ng + g] = (uint8_t)u;
                sg[g] = u8_decode(bd, (float)u);
            }
        } else if (j->layout == 1) {
            for (int g = 0; g < ng; g++) {
                const uint16_t h = f32_to_f16(sg[g]);
                j->s16[(size_t)r * ng + g] = h;
                sg[g] = f16_to_f32(h);
            }
        }
        int8_t *qr = j->q + (size_t)r * j->cols;
        for (int c = 0; c < j->cols; c++) {
            const float s = sg[c / j->gs];
            int qi = (int)__builtin_rintf(row[c] / s);
            if (qi > 127) qi = 127;
            if (qi < -127) qi = -127;
            qr[c] = (int8_t)qi;
        }
        for (int g = 0; g < ng; g++) j->scale[(size_t)r * ng + g] = sg[g];
    }
    free(row);
    return NULL;
}

static void emit_tensor(Writer *w, int rows, int cols, InitKind kind, float a,
                        float b, int quantize) {
    uint32_t tid = w->tensor_id++;
    size_t n = (size_t)rows * cols;
    if (w->failed) return;
    Job base;
    memset(&base, 0, sizeof(base));
    base.seed = w->seed; base.tensor_id = tid; base.rows = rows; base.cols = cols;
    base.kind = kind; base.a = a; base.b = b; base.quantize = quantize;
    base.gs = (w->gs > 0 && cols % w->gs == 0 && cols / w->gs <= 4096) ? w->gs : cols;
    base.layout = w->scale_layout;
    const size_t ngt = n / (size_t)base.gs;
    if (quantize) {
        base.q = (int8_t *)malloc(n);
        base.scale = (float *)malloc(sizeof(float) * ngt);
        base.s16 = (uint16_t *)malloc(sizeof(uint16_t) * (ngt > (size_t)rows ? ngt : (size_t)rows));
        base.u8 = (uint8_t *)malloc(ngt);
    } else {
        base.f = (float *)malloc(sizeof(float) * n);
    }
    if ((quantize && (!base.q || !base.scale || !base.s16 || !base.u8)) || (!quantize && !base.f)) {
        w->failed = 1;
        free(base.q); free(base.scale); free(base.f); free(base.s16); free(base.u8);
        return;
    }
    int nt = w->n_threads;
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    if ((size_t)rows * cols < 65536 || rows < nt) nt = 1;
    Job jobs[64];
    pthread_t th[64];
    for (int t = 0; t < nt; t++) {
        jobs[t] = base;
        jobs[t].r0 = (int)((long)rows * t / nt);
        jobs[t].r1 = (int)((long)rows * (t + 1) / nt);
        if (nt > 1) pthread_create(&th[t], NULL, job_run, &jobs[t]);
        else job_run(&jobs[t]);
    }
    if (nt > 1)
        for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
    /* Record: u8 dtype, u32 n, then Q8_0: u32 gs, int8[n], the scale plane
     * (layout 0: f32[n/gs]; 1: binary16[n/gs]; 2: binary16[rows] row bases,
     * u8[n/gs]); F32: f32[n]; BF16: u16[n]  (reference src/model.c:3424-3812). */
    uint8_t dt = quantize ? FMT_Q8_0 : (w->bf16 ? FMT_BF16 : FMT_F32);
    put_bytes(w, &dt, 1);
    put_u32(w, (uint32_t)n);
    if (quantize) {
        put_u32(w, (uint32_t)base.gs);
        put_bytes(w, base.q, n);
        if (base.layout == 0) put_bytes(w, base.scale, sizeof(float) * ngt);
        else if (base.layout == 1) put_bytes(w, base.s16, sizeof(uint16_t) * ngt);
        else {
            put_bytes(w, base.s16, sizeof(uint16_t) * (size_t)rows);
            put_bytes(w, base.u8, ngt);
        }
    } else if (w->bf16) {
        for (size_t i = 0; i < n; i++) {
            const uint16_t h = f32_to_bf16(base.f[i]);
            put_bytes(w, &h, 2);
        }
    } else {
        put_bytes(w, base.f, sizeof(float) * n);
    }
    free(base.q); free(base.scale); free(base.f); free(base.s16); free(base.u8);
}

/* A tensor of no elements (a [vocab][0] Markov tensor): dtype and count only. */
static void empty_tensor(Writer *w) {
    uint8_t dt = w->bf16 ? FMT_BF16 : FMT_F32;
    w->tensor_id++;
    put_bytes(w, &dt, 1);
    put_u32(w, 0u);
}

static void matrix(Writer *w, int rows, int cols, float std) {
    emit_tensor(w, rows, cols, INIT_NORMAL, std, 0.0f, 1);
}
/* An all-zero int8 matrix (every row scale 1, every code 0). */
static void zero_matrix(Writer *w, int rows, int cols) {
    emit_tensor(w, rows, cols, INIT_CONST, 0.0f, 0.0f, 1);
}
static void vec_norm(Writer *w, int n, float mean, float std) {
    emit_tensor(w, 1, n, INIT_NORMAL, std, mean, 0);
}

int l98_synth_write(const char *dir, const L98SynthConfig *c, uint64_t seed,
                    int n_threads, char *err, int errlen) {
    char path[1024];
    if (!dir || !c) {
        if (err && errlen > 0) snprintf(err, (size_t)errlen, "null argument");
        return 1;
    }
    if (c->n_layers < 1 || c->n_layers > MAX_LAYERS || c->hidden % 32 ||
        c->attn_period < 1) {
        if (err && errlen > 0) snprintf(err, (size_t)errlen, "bad config");
        return 1;
    }
    mkdir(dir, 0755);
    snprintf(path, sizeof(path), "%s/model.bin", dir);
    const int ver = c->bin_version ? c->bin_version : 5;
    if (ver < 4 || ver > 9 || (c->gs && (c->gs % 32)) || c->scale_layout < 0 || c->scale_layout > 2 ||
        (ver < 6 && c->scale_layout != 0) || (ver == 4 && c->use_subn) ||
        (c->mtp_n_draft > 1 && ver < 6) || c->mtp_n_draft > 6) {
        if (err && errlen > 0) snprintf(err, (size_t)errlen, "bad format options");
        return 1;
    }
    Writer w;
    memset(&w, 0, sizeof(w));
    w.seed = seed;
    w.n_threads = n_threads;
    w.gs = c->gs;
    w.scale_layout = c->scale_layout;
    w.bf16 = c->bf16_small;
    w.f = fopen(path, "wb");
    if (!w.f) {
        if (err && errlen > 0)
            snprintf(err, (size_t)errlen, "cannot open %s: %s", path, strerror(errno));
        return 1;
    }
    static char iobuf[1 << 20];
    setvbuf(w.f, iobuf, _IOFBF, sizeof(iobuf));

    const int d = c->hidden, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv_heads;
    const int key = c->kda_heads * c->kd, value = c->kda_heads * c->vd;
    const int q_dim = nh * hd, qgate = 2 * q_dim, kv_dim = nkv * hd;
    int types[MAX_LAYERS];
    int n_full = 0, n_lin = 0;
    memset(types, 0, sizeof(types));
    for (int i = 0; i < c->n_layers; i++) {
        int full = (i % c->attn_period) == c->attn_period - 1;
        types[i] = full ? LT_FULL : LT_KDA;
        if (full) n_full++; else n_lin++;
    }

    /* Header, in lz_open_bin's read order (src/model.c:3993-4460). */
    put_bytes(&w, "L98Z", 4);
    put_u32(&w, (uint32_t)ver);
    put_i32(&w, c->vocab); put_i32(&w, d); put_i32(&w, c->n_layers);
    put_i32(&w, c->seq_len); put_i32(&w, nh); put_i32(&w, nkv); put_i32(&w, hd);
    put_i32(&w, c->shared_w);                          /* intermediate_size (unused: no dense body layer) */
    put_i32(&w, c->kda_heads); put_i32(&w, c->kda_heads);
    put_i32(&w, c->kd); put_i32(&w, c->vd); put_i32(&w, c->conv_kernel);
    put_i32(&w, n_lin); put_i32(&w, n_full); put_i32(&w, c->attn_period);
    put_i32(&w, 1); put_i32(&w, 1);                    /* tie_word_embeddings, attn_output_gate */
    put_f32(&w, 1e-6f); put_f32(&w, 10000.0f); put_f32(&w, 1.0f);
    put_i32(&w, q_dim); put_i32(&w, qgate); put_i32(&w, kv_dim);
    put_i32(&w, key); put_i32(&w, value); put_i32(&w, 2 * key + value);
    put_i32(&w, hd);                                   /* rotary_dim */
    for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, types[i]);
    put_i32(&w, c->gate_rank); put_i32(&w, c->gate_lb != 0.0f); put_f32(&w, c->gate_lb);
    put_i32(&w, c->n_experts); put_i32(&w, c->topk); put_i32(&w, 1);
    put_i32(&w, c->moe_inter); put_i32(&w, c->latent);
    put_i32(&w, 0);                                    /* first_k_dense_replace */
    put_i32(&w, 1); put_i32(&w, 1); put_i32(&w, 0);    /* renormalize, sigmoid, latent_use_norm */
    put_i32(&w, c->shared_w);
    if (ver >= 5) {
    /* version-5 tail */
    put_i32(&w, 1); put_i32(&w, c->mtp_inter);         /* mtp_n_layers, mtp_intermediate_size */
    put_i32(&w, 0); put_f32(&w, 1.0f); put_f32(&w, 4096.0f);
    put_f32(&w, 32.0f); put_f32(&w, 1.0f);             /* rope scaling: none */
    put_i32(&w, c->use_subn); put_i32(&w, c->hadamard_o); put_i32(&w, c->hadamard_down);
    put_i32(&w, 0); put_i32(&w, 0); put_i32(&w, 0);    /* mla_q, mla_o, attn_kv_share */
    put_i32(&w, 0); put_i32(&w, 0); put_i32(&w, 0); put_i32(&w, 0); /* sink, gated_residual, ced_split, ced_kv */
    for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, 0);   /* csa2_on */
    for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, 0);   /* csa2_mode */
    for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, -1);  /* csa2_source */
    put_i32(&w, 0);                                    /* ced_replay_w */
    put_i32(&w, 4); put_i32(&w, 64); put_i32(&w, 1);   /* csa2_compress_m, topk, indexer_heads */
    put_i32(&w, hd); put_i32(&w, 1);                   /* indexer_head_dim, indexer_q_lora_rank */
    for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, 0);   /* csa2_compress_m_layer */
    }
    if (ver >= 6) {                                    /* the identity application table, ... */
        put_i32(&w, c->n_layers);
        for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, i < c->n_layers ? i : 0);   /* app_layer */
        for (int i = 0; i < MAX_LAYERS; i++) put_i32(&w, 0);                        /* app_loop */
        put_i32(&w, c->mtp_n_draft > 1 ? c->mtp_n_draft : 1);   /* mtp_n_draft */
        put_i32(&w, 0); put_i32(&w, 0);                /* embed_hadamard, embed_signs_seed */
        put_i32(&w, c->scale_layout);
    }
    if (ver >= 7) put_i32(&w, 0);                      /* loop_input_mix */
    if (ver >= 8) put_i32(&w, 0);                      /* ced_local */
    if (ver >= 9) put_i32(&w, 2);                      /* loop_input_mix_from */

    const float ws = c->w_std;
    const float rs = c->router_std > 0.0f ? c->router_std : ws;
    const float os = c->resid_std > 0.0f ? c->resid_std : ws;   /* residual writers */
    /* Tensors in model_walk order (src/model.c:2240-2625). */
    matrix(&w, c->vocab, d, ws);                       /* embed_tokens (tied lm_head) */
    vec_norm(&w, d, 0.0f, ws);                         /* norm */
    for (int li = 0; li < c->n_layers; li++) {
        vec_norm(&w, d, 0.0f, ws);                     /* input_layernorm */
        vec_norm(&w, d, 0.0f, ws);                     /* post_attention_layernorm */
        if (types[li] == LT_FULL) {
            matrix(&w, qgate, d, ws);                  /* q_proj ([q|gate] per head) */
            matrix(&w, kv_dim, d, ws);                 /* k_proj */
            matrix(&w, kv_dim, d, ws);                 /* v_proj */
            matrix(&w, d, q_dim, os);                  /* o_proj */
            vec_norm(&w, hd, 0.0f, ws);                /* q_norm */
            vec_norm(&w, hd, 0.0f, ws);                /* k_norm */
            if (c->use_subn) {                         /* q/k/v/o_proj.norm */
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, q_dim, 0.0f, ws);
            }
        } else {
            matrix(&w, key, d, ws);                    /* q_proj */
            matrix(&w, key, d, ws);                    /* k_proj */
            matrix(&w, value, d, ws);                  /* v_proj */
            emit_tensor(&w, key, c->conv_kernel, INIT_UNIFORM, -0.5f, 0.5f, 0);
            emit_tensor(&w, key, c->conv_kernel, INIT_UNIFORM, -0.5f, 0.5f, 0);
            emit_tensor(&w, value, c->conv_kernel, INIT_UNIFORM, -0.5f, 0.5f, 0);
            emit_tensor(&w, 1, c->kda_heads, INIT_ALOG, 0, 0, 0);       /* A_log */
            matrix(&w, c->gate_rank, d, ws);           /* f_a_proj */
            matrix(&w, c->kda_heads * c->kd, c->gate_rank, ws);  /* f_b_proj */
            emit_tensor(&w, 1, c->kda_heads * c->kd, INIT_DTBIAS, 0, 0, 0);  /* dt_bias */
            matrix(&w, c->kda_heads, d, ws);           /* b_proj */
            matrix(&w, value, d, ws);                  /* g_proj */
            vec_norm(&w, c->vd, 1.0f, ws);             /* o_norm (gain w, not 1+w) */
            matrix(&w, d, value, os);                  /* o_proj */
            if (c->use_subn) {                         /* q/k/v/g/o_proj.norm */
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, d, 0.0f, ws);
                vec_norm(&w, value, 0.0f, ws);
            }
        }
        matrix(&w, c->n_experts, d, rs);               /* mlp.gate (router) */
        emit_tensor(&w, 1, c->n_experts, INIT_NORMAL, c->bias_std, 0.0f, 0);
        matrix(&w, c->latent, d, ws);                  /* routed_expert_down_proj */
        matrix(&w, d, c->latent, os);                  /* routed_expert_up_proj */
        matrix(&w, c->shared_w, d, ws);                /* shared gate_proj */
        matrix(&w, c->shared_w, d, ws);                /* shared up_proj */
        matrix(&w, d, c->shared_w, os);                /* shared down_proj */
        if (c->use_subn) {          /* gate, routed down/up, shared gate/up/down .norm */
            vec_norm(&w, d, 0.0f, ws);
            vec_norm(&w, d, 0.0f, ws);
            vec_norm(&w, c->latent, 0.0f, ws);
            vec_norm(&w, d, 0.0f, ws);
            vec_norm(&w, d, 0.0f, ws);
            vec_norm(&w, c->shared_w, 0.0f, ws);
        }
        for (int e = 0; e < c->n_experts; e++) {
            matrix(&w, c->moe_inter, c->latent, ws);   /* w1 */
            matrix(&w, c->latent, c->moe_inter, ws);   /* w2 */
            matrix(&w, c->moe_inter, c->latent, ws);   /* w3 */
        }
    }
    /* MTP block (none in a version-4 file): full-attention rows, dense FFN,
     * then the head's own.  The
     * echo head keeps the block's K/V rows (the MTP KV plane still fills)
     * but zeroes what it adds to its residual, and its fc passes the
     * normalized embedding half through (the hidden half adds a little
     * noise, so the chain moves a step's top-1 probability), so its logits
     * are about E . norm(E[tok]) and the draft is the input token. */
    if (ver >= 5) {
    vec_norm(&w, d, 0.0f, ws);
    vec_norm(&w, d, 0.0f, ws);
    if (c->use_subn) {                                 /* mlp.gate/up_proj.norm */
        vec_norm(&w, d, 0.0f, ws);
        vec_norm(&w, d, 0.0f, ws);
    }
    matrix(&w, qgate, d, ws);
    matrix(&w, kv_dim, d, ws);
    matrix(&w, kv_dim, d, ws);
    if (c->mtp_echo) zero_matrix(&w, d, q_dim);
    else matrix(&w, d, q_dim, ws);
    vec_norm(&w, hd, 0.0f, ws);
    vec_norm(&w, hd, 0.0f, ws);
    if (c->use_subn) {                                 /* self_attn.q/k/v/o_proj.norm */
        vec_norm(&w, d, 0.0f, ws);
        vec_norm(&w, d, 0.0f, ws);
        vec_norm(&w, d, 0.0f, ws);
        vec_norm(&w, q_dim, 0.0f, ws);
    }
    matrix(&w, c->mtp_inter, d, ws);                   /* gate_proj */
    matrix(&w, c->mtp_inter, d, ws);                   /* up_proj */
    if (c->mtp_echo) zero_matrix(&w, d, c->mtp_inter); /* down_proj */
    else matrix(&w, d, c->mtp_inter, ws);
    if (c->use_subn) vec_norm(&w, c->mtp_inter, 0.0f, ws);   /* down_proj.norm */
    const int dspark = c->mtp_n_draft > 1;
    if (!dspark) {
        if (c->mtp_echo) emit_tensor(&w, d, 2 * d, INIT_EYE, ws, 0.0f, 1);   /* mtp.fc = [I | N(0, ws)] */
        else matrix(&w, d, 2 * d, ws);                 /* mtp.fc */
    }
    vec_norm(&w, d, 0.0f, ws);                         /* mtp.norm */
    vec_norm(&w, d, 0.0f, ws);                         /* pre_fc_norm_hidden */
    vec_norm(&w, d, 0.0f, ws);                         /* pre_fc_norm_embedding */
    if (dspark) {
        /* main_proj over [norm(h) | norm(emb or mask) | depth row] */
        if (c->mtp_echo) emit_tensor(&w, d, 3 * d, INIT_EYE2, ws, 0.0f, 1);
        else matrix(&w, d, 3 * d, ws);
        matrix(&w, c->mtp_n_draft, d, 1.0f);           /* depth_embed */
        emit_tensor(&w, 1, d, INIT_NORMAL, 1.0f, 0.0f, 0);   /* mask_embed */
        empty_tensor(&w);                              /* markov_embed [vocab][0] */
        empty_tensor(&w);                              /* markov_proj [vocab][0] */
    }
    }

    if (fclose(w.f) != 0) w.failed = 1;
    if (w.failed) {
        if (err && errlen > 0) snprintf(err, (size_t)errlen, "write failed: %s", path);
        return 1;
    }
    return 0;
}

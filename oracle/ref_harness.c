/* Test-infrastructure driver for the REFERENCE engine built by oracle/ref.mk.
 * It links the reference's own objects and calls the reference API; it is
 * the checker and the CPU baseline, never part of the product.
 *
 * The session is set up the way lz_generate_call does it
 * (reference src/generate.c:2806-2960 and the spec round driver
 * src/generate.c:1822-2106):
 *   lz_forward_batch_capture(prompt[0..n-2]) -> lz_mtp_prefill -> mtp_pos=n-1
 *   lz_forward_capture(prompt[n-1]) -> anchor = sample(logits)
 *   loop lz_spec_round / lz_spec_round_temp.
 * A DSpark model (config.mtp_n_draft > 1) runs lz_spec_round_dspark /
 * lz_spec_round_dspark_temp, as the driver dispatches (src/generate.c:
 * 1929-1946), and its session start skips lz_mtp_prefill: that function
 * projects through mtp.fc (src/forward_mtp.c:590), which a DSpark head does
 * not bind (src/model.c:2531-2532), so the driver's default prompt pass
 * faults on such a model; its MTP-prefill skip knob gives the body-only
 * prefill used here, and no DSpark step reads the MTP KV rows.
 *
 * Usage:
 *   l98ref_* gen MODEL_DIR PROMPT_FILE K N_NEW TEMP TOPP SEED OUT_PREFIX [opts]
 *       opts: --dump-rounds N   write logits/hidden of the first N rounds
 *             --break-rollback  --skip-catchup  --pmin P  --nmin N
 *             --timing          per-round wall times
 *             --verify-iters N  after the run, time N lz_forward_verify
 *                               calls of M = K+1 tokens at the final
 *                               position (ring slot restored between calls)
 *   l98ref_* capture MODEL_DIR PROMPT_FILE OUT_PREFIX
 *       a prefill and one capture, logits and hidden rows dumped
 *   l98ref_* verify MODEL_DIR PROMPT_FILE K ITERS OUT_PREFIX
 *       times lz_forward_verify of M=K+1 tokens in isolation (the ring slot
 *       is restored between calls, so every call reads the same state)
 * PROMPT_FILE is raw little-endian int32 token ids.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "forward.h"
#include "generate.h"
#include "llama_zh.h"
#include "model.h"
#include "ops.h"
#include "sampler.h"

#if HARNESS_TAP
/* Appends (tag[8], layer, n, n floats) records to $L98_TAP_FILE. */
void l98_tap(const char *tag, int layer, const float *p, int n) {
    static FILE *f;
    char t[8];
    if (!f) {
        const char *path = getenv("L98_TAP_FILE");
        if (!path) return;
        f = fopen(path, "wb");
        if (!f) return;
    }
    memset(t, 0, sizeof t);
    strncpy(t, tag, sizeof t);
    fwrite(t, 1, 8, f);
    fwrite(&layer, 4, 1, f);
    fwrite(&n, 4, 1, f);
    fwrite(p, 4, (size_t)n, f);
    fflush(f);
}
#endif

static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e6 + (double)ts.tv_nsec * 1e-3;
}

static int *read_prompt(const char *path, int *n) {
    FILE *f = fopen(path, "rb");
    long sz;
    int *p;
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    p = (int *)malloc((size_t)sz);
    if (!p || fread(p, 1, (size_t)sz, f) != (size_t)sz) { fclose(f); free(p); return NULL; }
    fclose(f);
    *n = (int)(sz / 4);
    return p;
}

static void dump(const char *prefix, const char *tag, const void *p, size_t bytes) {
    char path[1024];
    FILE *f;
    snprintf(path, sizeof path, "%s.%s.bin", prefix, tag);
    f = fopen(path, "wb");
    if (!f) return;
    fwrite(p, 1, bytes, f);
    fclose(f);
}

static void select_mode(void) {
#if HARNESS_ORACLE
    lz_float_ref_select("off");
    lz_fastfp_select("off");
#endif
    lz_attn_window = 0;
    lz_attn_sink = 0;
    lz_kv_kfmt = LZ_KVF_Q8;
    lz_kv_vfmt = LZ_KVF_Q8;
    lz_kernel_select(LZ_KERNEL_AUTO);
}

/* Prefill + MTP prefill exactly as the generation driver does. Leaves
 * *token = prompt[n-1], *pos = n-1 (have_seed = 0). */
static int session_start(const LZModel *m, LZRunState *s, const int *prompt,
                         int n_prompt, double *t_prefill_us) {
    const int dspark = m->config.mtp_n_draft > 1;
    int dim = m->config.hidden_size;
    float *h_all;
    double t0 = now_us();
    lz_state_reset(s, m);
    if (n_prompt < 2) return 1;
    h_all = (float *)malloc(sizeof(float) * (size_t)(n_prompt - 1) * dim);
    if (!h_all) return 1;
    if (!lz_forward_batch_capture(m, s, prompt, n_prompt - 1, 0, h_all)) { free(h_all); return 1; }
    if (!dspark) {
        if (lz_mtp_prefill(m, s, h_all, prompt + 1, n_prompt - 1, s->mtp_pos) != 0) { free(h_all); return 1; }
        s->mtp_pos = n_prompt - 1;
    }
    free(h_all);
    if (t_prefill_us) *t_prefill_us = now_us() - t0;
    return 0;
}

static void dump_state(const char *prefix, const LZModel *m, const LZRunState *s, int pos) {
    const LZModelConfig *c = &m->config;
#if LZ_GDN_STATE_F32
    size_t per_slot = (size_t)s->n_linear_apps * c->lin_n_v_heads * c->lin_k_head_dim *
                      c->lin_v_head_dim;
    dump(prefix, "kda_state", s->ssm_state_f32 + (size_t)s->ssm_slot * per_slot,
         per_slot * sizeof(float));
#endif
    {
        size_t conv_slot = (size_t)s->n_linear_apps * c->lin_conv_dim * (c->conv_kernel - 1);
        dump(prefix, "conv_state", s->conv_state + (size_t)s->ssm_slot * conv_slot,
             conv_slot * sizeof(float));
    }
    {
        /* KV planes: every dense plane plus the MTP plane, rows < pos. */
        int planes = lz_n_dense_kv_apps(m) + (m->mtp ? 1 : 0);
        int kvd = c->attn_kv_dim, pl;
        size_t rows = (size_t)pos;
        FILE *f;
        char path[1024];
        snprintf(path, sizeof path, "%s.kv.bin", prefix);
        f = fopen(path, "wb");
        if (f) {
            for (pl = 0; pl < planes; pl++) {
                size_t off = (size_t)pl * s->kv_slots * kvd;
                fwrite(s->kq8 + off, 1, rows * kvd, f);
                fwrite(s->ksq + off / 32, sizeof(float), rows * kvd / 32, f);
                fwrite(s->vq8 + off, 1, rows * kvd, f);
                fwrite(s->vsq + off / 32, sizeof(float), rows * kvd / 32, f);
            }
            fclose(f);
        }
    }
    dump(prefix, "mtp_chain", s->mtp_chain, sizeof(float) * (size_t)c->hidden_size);
    dump(prefix, "rope_cs", s->rope_cs, sizeof(float) * (size_t)s->seq_len * c->rotary_dim);
}

static int cmp_d(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : x > y;
}

static int cmd_gen(int argc, char **argv) {
    const char *dir = argv[2], *pf = argv[3];
    int k = atoi(argv[4]), n_new = atoi(argv[5]);
    float temp = (float)atof(argv[6]), topp = (float)atof(argv[7]);
    unsigned long long seed = strtoull(argv[8], NULL, 10);
    const char *prefix = argv[9];
    int dump_rounds = 0, brk = 0, skipc = 0, n_min = 0, timing = 0, verify_iters = 0;
    double verify_med = 0.0, verify_min = 0.0;
    float p_min = 0.0f;
    int i, n_prompt, rc;
    char err[512];
    LZModel m;
    LZRunState s;
    LZSampler samp;
    LZSampleParams sp;
    int *prompt, *toks;
    int n_tok = 0, token, pos, have_seed = 0, rounds = 0;
    int *rk, *ra;
    double *rt;
    double t_prefill = 0, t_loop0, t_loop;
    FILE *out;
    char path[1024];

    for (i = 10; i < argc; i++) {
        if (!strcmp(argv[i], "--dump-rounds") && i + 1 < argc) dump_rounds = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--break-rollback")) brk = 1;
        else if (!strcmp(argv[i], "--skip-catchup")) skipc = 1;
        else if (!strcmp(argv[i], "--pmin") && i + 1 < argc) p_min = (float)atof(argv[++i]);
        else if (!strcmp(argv[i], "--nmin") && i + 1 < argc) n_min = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--timing")) timing = 1;
        else if (!strcmp(argv[i], "--verify-iters") && i + 1 < argc) verify_iters = atoi(argv[++i]);
    }
    select_mode();
    prompt = read_prompt(pf, &n_prompt);
    if (!prompt) { fprintf(stderr, "bad prompt file\n"); return 2; }
    if (lz_open(&m, dir, err, sizeof err) != 0) { fprintf(stderr, "lz_open: %s\n", err); return 2; }
    if (lz_state_alloc(&s, &m, m.config.seq_len, LZ_SPEC_K_MAX, err, sizeof err) != 0) {
        fprintf(stderr, "lz_state_alloc: %s\n", err);
        return 2;
    }
    memset(&sp, 0, sizeof sp);
    lz_sample_defaults(&sp);
    sp.temperature = temp;
    sp.topp = topp;
    sp.topk = 0;
    sp.minp = 0.0f;
    sp.presence_penalty = 0.0f;
    sp.frequency_penalty = 0.0f;
    sp.repetition_penalty = 1.0f;
    sp.repeat_last_n = 0;
    if (lz_sampler_init(&samp, m.config.vocab_size, &sp, (lz_u64)seed) != 0) return 2;

    if (session_start(&m, &s, prompt, n_prompt, &t_prefill) != 0) { fprintf(stderr, "prefill failed\n"); return 3; }
    token = prompt[n_prompt - 1];
    pos = n_prompt - 1;
    toks = (int *)malloc(sizeof(int) * (size_t)(n_new + 16));
    rk = (int *)malloc(sizeof(int) * (size_t)(2 * n_new + 16));
    ra = (int *)malloc(sizeof(int) * (size_t)(2 * n_new + 16));
    rt = (double *)malloc(sizeof(double) * (size_t)(2 * n_new + 16));
    t_loop0 = now_us();
    while (n_tok < n_new) {
        int anchor, anchor_pos, out_t[LZ_SPEC_K_MAX + 1];
        int n_accept = 0, new_pos = 0, k_eff = 0, n_emit;
        double t0 = now_us();
        if (have_seed) {
            anchor = token;
            anchor_pos = pos - 1;
        } else {
            float *lg = lz_forward_capture(&m, &s, token, pos);
            if (!lg) { fprintf(stderr, "capture failed\n"); return 3; }
            if (rounds < dump_rounds) {
                char tag[64];
                snprintf(tag, sizeof tag, "capture%d", rounds);
                dump(prefix, tag, lg, sizeof(float) * (size_t)m.config.vocab_size);
            }
            anchor_pos = pos;
            anchor = lz_sample_ex(&samp, lg, NULL, 0);
            lz_sampler_observe(&samp, anchor);
            toks[n_tok++] = anchor;
            if (n_tok >= n_new) break;
        }
        if (m.config.mtp_n_draft > 1 && temp > 0.0f)
            n_emit = lz_spec_round_dspark_temp(&m, &s, anchor, anchor_pos, k, p_min, n_min, &samp,
                                               brk, out_t, &n_accept, &new_pos, &k_eff, err, sizeof err);
        else if (m.config.mtp_n_draft > 1)
            n_emit = lz_spec_round_dspark(&m, &s, anchor, anchor_pos, k, p_min, n_min, &samp,
                                          brk, out_t, &n_accept, &new_pos, &k_eff, err, sizeof err);
        else if (temp > 0.0f)
            n_emit = lz_spec_round_temp(&m, &s, anchor, anchor_pos, k, p_min, n_min, &samp,
                                        brk, skipc, out_t, &n_accept, &new_pos, &k_eff,
                                        err, sizeof err);
        else
            n_emit = lz_spec_round(&m, &s, anchor, anchor_pos, k, p_min, n_min, &samp,
                                   brk, skipc, out_t, &n_accept, &new_pos, &k_eff,
                                   err, sizeof err);
        if (n_emit < 0) { fprintf(stderr, "spec round: %s\n", err); return 3; }
        rt[rounds] = now_us() - t0;
        rk[rounds] = k_eff;
        ra[rounds] = n_emit > 0 ? n_accept : -1;
        if (rounds < dump_rounds && temp <= 0.0f && n_emit > 0) {
            char tag[64];
            snprintf(tag, sizeof tag, "verify%d", rounds);
            dump(prefix, tag, s.mtp_logits,
                 sizeof(float) * (size_t)(k_eff + 1) * m.config.vocab_size);
            snprintf(tag, sizeof tag, "vhidden%d", rounds);
            dump(prefix, tag, s.mtp_verify_hidden,
                 sizeof(float) * (size_t)(k_eff + 1) * m.config.hidden_size);
            snprintf(tag, sizeof tag, "draft%d", rounds);
            if (m.config.mtp_n_draft > 1)       /* every slot's (corrected) logits */
                dump(prefix, tag, s.mtp_kdraft_logits, sizeof(float) * (size_t)k * m.config.vocab_size);
            else
                dump(prefix, tag, s.mtp_draft_logits, sizeof(float) * (size_t)m.config.vocab_size);
        }
        rounds++;
        have_seed = (n_emit > 0);
        if (n_emit > 0)
            for (i = 0; i <= n_accept; i++) {
                lz_sampler_observe(&samp, out_t[i]);
                if (n_tok < n_new + 8) toks[n_tok++] = out_t[i];
            }
        pos = new_pos + 1;
        token = out_t[n_accept];
    }
    t_loop = now_us() - t_loop0;
    dump_state(prefix, &m, &s, pos);
    if (verify_iters > 0 && pos + k + 1 < s.seq_len) {
        /* the verify forward alone at the run's final position: the same
           M = k+1 tokens each time, from the same ring slot */
        int vt[LZ_SPEC_K_MAX + 1], base_slot = s.ssm_slot;
        double *tv = (double *)malloc(sizeof(double) * (size_t)verify_iters);
        for (i = 0; i <= k; i++) vt[i] = toks[(n_tok - 1 - i + n_tok) % n_tok];
        for (i = 0; i < verify_iters; i++) {
            double t0 = now_us();
            s.ssm_slot = base_slot;
            if (lz_forward_verify(&m, &s, vt, k + 1, pos) != 0) { fprintf(stderr, "verify failed\n"); return 3; }
            tv[i] = now_us() - t0;
        }
        s.ssm_slot = base_slot;
        qsort(tv, (size_t)verify_iters, sizeof(double), cmp_d);
        verify_med = tv[verify_iters / 2];
        verify_min = tv[0];
        free(tv);
    }

    snprintf(path, sizeof path, "%s.txt", prefix);
    out = fopen(path, "w");
    if (!out) return 4;
    fprintf(out, "kernel %s\n", lz_kernel_name());
    fprintf(out, "mode %s\n", HARNESS_ORACLE ? "oracle" : "ship");
    fprintf(out, "n_prompt %d\nn_tokens %d\nrounds %d\n", n_prompt, n_tok, rounds);
    fprintf(out, "final_pos %d\nmtp_pos %d\nssm_slot %d\nrng %llu\n", pos, s.mtp_pos, s.ssm_slot,
            (unsigned long long)samp.rng_state);
    fprintf(out, "prefill_us %.1f\nloop_us %.1f\n", t_prefill, t_loop);
    if (verify_iters > 0) fprintf(out, "verify_M %d\nverify_us_median %.1f\nverify_us_min %.1f\n", k + 1, verify_med, verify_min);
    fprintf(out, "tokens");
    for (i = 0; i < n_tok; i++) fprintf(out, " %d", toks[i]);
    fprintf(out, "\nk_eff");
    for (i = 0; i < rounds; i++) fprintf(out, " %d", rk[i]);
    fprintf(out, "\nn_accept");
    for (i = 0; i < rounds; i++) fprintf(out, " %d", ra[i]);
    fprintf(out, "\n");
    if (timing) {
        fprintf(out, "round_us");
        for (i = 0; i < rounds; i++) fprintf(out, " %.1f", rt[i]);
        fprintf(out, "\n");
    }
    fclose(out);
    rc = 0;
    lz_sampler_free(&samp);
    lz_state_free(&s);
    lz_free(&m);
    free(prompt); free(toks); free(rk); free(ra); free(rt);
    return rc;
}

static int cmd_verify(int argc, char **argv) {
    const char *dir = argv[2], *pf = argv[3];
    int k = atoi(argv[4]), iters = atoi(argv[5]);
    const char *prefix = argv[6];
    int n_prompt, i, base_slot, toks[LZ_SPEC_K_MAX + 1];
    char err[512], path[1024];
    LZModel m;
    LZRunState s;
    int *prompt;
    double *t;
    FILE *out;
    (void)argc;
    select_mode();
    prompt = read_prompt(pf, &n_prompt);
    if (!prompt || lz_open(&m, dir, err, sizeof err) != 0) { fprintf(stderr, "open: %s\n", err); return 2; }
    if (lz_state_alloc(&s, &m, m.config.seq_len, LZ_SPEC_K_MAX, err, sizeof err) != 0) return 2;
    if (session_start(&m, &s, prompt, n_prompt, NULL) != 0) return 3;
    for (i = 0; i <= k; i++) toks[i] = prompt[(n_prompt - 1 + i) % n_prompt];
    base_slot = s.ssm_slot;
    t = (double *)malloc(sizeof(double) * (size_t)(iters + 1));
    for (i = 0; i <= iters; i++) {
        double t0 = now_us();
        s.ssm_slot = base_slot;
        if (lz_forward_verify(&m, &s, toks, k + 1, n_prompt - 1) != 0) return 3;
        t[i] = now_us() - t0;
    }
    qsort(t + 1, (size_t)iters, sizeof(double), cmp_d);
    snprintf(path, sizeof path, "%s.txt", prefix);
    out = fopen(path, "w");
    if (!out) return 4;
    fprintf(out, "kernel %s\nmode %s\nM %d\niters %d\nverify_us_median %.1f\nverify_us_min %.1f\n",
            lz_kernel_name(), HARNESS_ORACLE ? "oracle" : "ship", k + 1, iters,
            t[1 + iters / 2], t[1]);
    fclose(out);
    dump(prefix, "verify_logits", s.mtp_logits,
         sizeof(float) * (size_t)(k + 1) * m.config.vocab_size);
    return 0;
}

/* l98ref_* capture MODEL_DIR PROMPT_FILE OUT_PREFIX
 *   lz_forward_batch_capture of prompt[0..n-2] at 0, then
 *   lz_forward_capture(prompt[n-1], n-1): dumps its logits ("capture") and
 *   the final-normed hidden rows of the prefill ("hidden") and of the last
 *   token ("chain").  Needs no MTP head (a version-4 model has none). */
static int cmd_capture(int argc, char **argv) {
    const char *dir = argv[2], *pf = argv[3], *prefix = argv[4];
    int n_prompt;
    char err[512];
    LZModel m;
    LZRunState s;
    int *prompt;
    float *h_all, *lg;
    (void)argc;
    select_mode();
    prompt = read_prompt(pf, &n_prompt);
    if (!prompt || n_prompt < 2 || lz_open(&m, dir, err, sizeof err) != 0) {
        fprintf(stderr, "open: %s\n", err);
        return 2;
    }
    if (lz_state_alloc(&s, &m, m.config.seq_len, LZ_SPEC_K_MAX, err, sizeof err) != 0) {
        fprintf(stderr, "lz_state_alloc: %s\n", err);
        return 2;
    }
    h_all = (float *)malloc(sizeof(float) * (size_t)(n_prompt - 1) * m.config.hidden_size);
    if (!h_all) return 2;
    if (!lz_forward_batch_capture(&m, &s, prompt, n_prompt - 1, 0, h_all)) return 3;
    lg = lz_forward_capture(&m, &s, prompt[n_prompt - 1], n_prompt - 1);
    if (!lg) return 3;
    dump(prefix, "capture", lg, sizeof(float) * (size_t)m.config.vocab_size);
    dump(prefix, "hidden", h_all, sizeof(float) * (size_t)(n_prompt - 1) * m.config.hidden_size);
    if (s.mtp_chain)   /* no MTP head, no chain (src/forward.c:1623-1629) */
        dump(prefix, "chain", s.mtp_chain, sizeof(float) * (size_t)m.config.hidden_size);
    free(h_all);
    free(prompt);
    lz_state_free(&s);
    lz_free(&m);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 5 && !strcmp(argv[1], "capture")) return cmd_capture(argc, argv);
    if (argc >= 10 && !strcmp(argv[1], "gen")) return cmd_gen(argc, argv);
    if (argc >= 7 && !strcmp(argv[1], "verify")) return cmd_verify(argc, argv);
    fprintf(stderr, "usage: see oracle/ref_harness.c\n");
    return 1;
}

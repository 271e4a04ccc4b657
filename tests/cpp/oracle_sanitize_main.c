/* Drives every function of the oracle (oracle/pk_oracle.c) on seeded random
 * decoders, for builds with AddressSanitizer + UndefinedBehaviorSanitizer and
 * with ThreadSanitizer (the batch driver's worker threads).  Test
 * infrastructure only.
 *
 * Covered: dequantisation of every block type on random blocks; TDT (2 layers,
 * durations {0..4}) and EOU (1 layer, special pieces) greedy windows of
 * 0 .. 40 frames with state carried across windows; the teacher-forced replay
 * of each window's own trace, which must find no mismatch (a self-check that
 * also runs the classifier); windows whose output arrays are too small (the
 * bounded-output path returns rc 11); a batch over 3 worker threads that must
 * match one-at-a-time windows.  Prints "ok" and exits 0, or names the failed
 * check and exits 1. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pk_oracle.h"

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    rs ^= rs << 13;
    rs ^= rs >> 7;
    rs ^= rs << 17;
    return (uint32_t)(rs >> 16);
}
static float frand(float scale) { return scale * ((float)(rnd() % 20001) / 10000.0f - 1.0f); }

static float *fill(size_t n, float scale) {
    float *p = malloc(n * sizeof *p);
    for (size_t i = 0; i < n; ++i) p[i] = frand(scale);
    return p;
}

#define CHECK(c, what)                                   \
    do {                                                 \
        if (!(c)) {                                      \
            fprintf(stderr, "check failed: %s\n", what); \
            return 1;                                    \
        }                                                \
    } while (0)

typedef struct {
    ora_model m;
    float *bufs[32];
    int nb;
    uint8_t special[64];
} model_t;

static const float *keep(model_t *t, float *p) {
    t->bufs[t->nb++] = p;
    return p;
}

static void make_model(model_t *t, int kind) {
    memset(t, 0, sizeof *t);
    ora_model *m = &t->m;
    m->kind = kind;
    m->H = 24;
    m->L = kind == ORA_TDT ? 2 : 1;
    m->J = 32;
    m->D = 16;
    const int vocab = kind == ORA_TDT ? 29 : 35;
    m->V1 = vocab + 1;
    m->blank = vocab;
    m->Dn = kind == ORA_TDT ? 5 : 0;
    m->Vo = m->V1 + m->Dn;
    m->n_dur = m->Dn;
    for (int i = 0; i < m->Dn; ++i) m->durations[i] = i;
    if (kind == ORA_EOU) {
        m->eou = vocab - 2;
        m->eob = vocab - 1;
        for (int i = 0; i < vocab; ++i) t->special[i] = (i == 0 || i >= vocab - 2);
        m->special = t->special;
        m->n_special = vocab;
    }
    const float s = 0.4f;
    m->embed = keep(t, fill((size_t)m->V1 * m->H, s));
    for (int l = 0; l < m->L; ++l) {
        m->w_ih[l] = keep(t, fill((size_t)4 * m->H * m->H, s));
        m->w_hh[l] = keep(t, fill((size_t)4 * m->H * m->H, s));
        m->b_ih[l] = keep(t, fill((size_t)4 * m->H, s));
        m->b_hh[l] = keep(t, fill((size_t)4 * m->H, s));
    }
    m->enc_w = keep(t, fill((size_t)m->J * m->D, s));
    m->enc_b = keep(t, fill((size_t)m->J, s));
    m->pred_w = keep(t, fill((size_t)m->J * m->H, s));
    m->pred_b = keep(t, fill((size_t)m->J, s));
    m->out_w = keep(t, fill((size_t)m->Vo * m->J, 1.5f));
    m->out_b = keep(t, fill((size_t)m->Vo, 1.0f));
}

static void free_model(model_t *t) {
    for (int i = 0; i < t->nb; ++i) free(t->bufs[i]);
}

typedef struct {
    float *h, *c, *pred;
    ora_state st;
} state_t;

static void new_state(const ora_model *m, state_t *s) {
    s->h = calloc((size_t)m->L * m->H, sizeof(float));
    s->c = calloc((size_t)m->L * m->H, sizeof(float));
    s->pred = calloc((size_t)m->H, sizeof(float));
    memset(&s->st, 0, sizeof s->st);
    s->st.h = s->h;
    s->st.c = s->c;
    s->st.pred = s->pred;
}

static void copy_state(const ora_model *m, state_t *dst, const state_t *src) {
    memcpy(dst->h, src->h, (size_t)m->L * m->H * sizeof(float));
    memcpy(dst->c, src->c, (size_t)m->L * m->H * sizeof(float));
    memcpy(dst->pred, src->pred, (size_t)m->H * sizeof(float));
    float *h = dst->h, *c = dst->c, *p = dst->pred;
    dst->st = src->st;
    dst->st.h = h;
    dst->st.c = c;
    dst->st.pred = p;
}

static void free_state(state_t *s) {
    free(s->h);
    free(s->c);
    free(s->pred);
}

static int window(const ora_model *m, const float *enc, int T, int ms, state_t *s, int32_t *tok, int cap, int *n,
                  int32_t *seg, int *nseg, int *steps, int32_t *trace, int tcap) {
    if (m->kind == ORA_TDT) return ora_tdt_decode_window(m, enc, T, m->D, ms, 0.0f, &s->st, tok, cap, n, steps, trace, tcap);
    return ora_eou_decode_window(m, enc, T, m->D, ms, 0.0f, &s->st, tok, cap, n, seg, 64, nseg, steps, trace, tcap);
}

static int run_model(int kind) {
    model_t t;
    make_model(&t, kind);
    const ora_model *m = &t.m;
    const int ms = kind == ORA_TDT ? 10 : 5;
    static const int lens[] = {0, 1, 3, 7, 40};
    for (int li = 0; li < 5; ++li) {
        const int T = lens[li];
        float *enc = fill((size_t)(T ? T : 1) * m->D, 1.0f);
        const int cap = T * ms + 1, tcap = T * (ms + 1) + 1;
        int32_t *tok = malloc((size_t)cap * sizeof *tok), *trace = malloc((size_t)2 * tcap * sizeof *trace);
        int32_t seg[64];
        int n = 0, nseg = 0, steps = 0;
        state_t s, s0, r;
        new_state(m, &s);
        new_state(m, &s0);
        new_state(m, &r);
        ora_init_state(m, &s.st);
        copy_state(m, &s0, &s);
        CHECK(window(m, enc, T, ms, &s, tok, cap, &n, seg, &nseg, &steps, trace, tcap) == 0, "window rc");
        CHECK(steps <= tcap, "steps within the trace");
        /* replay the window's own decisions from the same start state */
        copy_state(m, &r, &s0);
        int32_t *rtok = malloc((size_t)cap * sizeof *rtok), rseg[64];
        int rn = 0, rnseg = 0;
        const int ntap = steps < 3 ? steps : 3;
        float *tap = malloc((size_t)(ntap ? ntap : 1) * m->Vo * sizeof(float));
        ora_replay_stats st;
        CHECK(ora_replay_window(m, enc, T, m->D, ms, 0.0f, &r.st, trace, steps, 1e-4f, rtok, cap, &rn, rseg, 64, &rnseg,
                                tap, ntap, &st) == 0, "replay rc");
        CHECK(st.unexplained == 0 && st.tok_mismatch == 0 && st.structure_error == 0, "self replay is exact");
        CHECK(rn == n && memcmp(rtok, tok, (size_t)n * sizeof *tok) == 0, "replay tokens");
        CHECK(memcmp(r.h, s.h, (size_t)m->L * m->H * sizeof(float)) == 0, "replay state");
        /* too-small output arrays: rc 11, never a write past them */
        if (n > 1) {
            state_t o;
            new_state(m, &o);
            copy_state(m, &o, &s0);
            int32_t *small = malloc((size_t)(n - 1) * sizeof *small);
            int on = 0, onseg = 0, osteps = 0;
            CHECK(window(m, enc, T, ms, &o, small, n - 1, &on, seg, &onseg, &osteps, NULL, 0) == 11, "overflow rc");
            free(small);
            free_state(&o);
        }
        /* a second window carries the state on */
        n = 0;
        nseg = 0;
        CHECK(window(m, enc, T, ms, &s, tok, cap, &n, seg, &nseg, &steps, NULL, 0) == 0, "second window");
        free(tap);
        free(rtok);
        free(tok);
        free(trace);
        free(enc);
        free_state(&s);
        free_state(&s0);
        free_state(&r);
    }
    /* the batch driver over 3 threads equals one-at-a-time windows */
    enum { NU = 5, T = 12 };
    const float *encs[NU];
    int nf[NU];
    float bias[NU];
    float *bufs[NU];
    const int cap = T * ms + 1;
    int32_t *tokens = calloc((size_t)NU * cap, sizeof *tokens), ntok[NU], steps[NU];
    for (int u = 0; u < NU; ++u) {
        bufs[u] = fill((size_t)T * m->D, 1.0f);
        encs[u] = bufs[u];
        nf[u] = T - u;
        bias[u] = 0.0f;
    }
    CHECK(ora_decode_batch(m, NU, encs, nf, bias, ms, 3, tokens, cap, ntok, steps) == 0, "batch rc");
    for (int u = 0; u < NU; ++u) {
        state_t s;
        new_state(m, &s);
        int32_t *tok = malloc((size_t)cap * sizeof *tok), seg[64];
        int n = 0, nseg = 0, st = 0;
        CHECK(window(m, encs[u], nf[u], ms, &s, tok, cap, &n, seg, &nseg, &st, NULL, 0) == 0, "single rc");
        CHECK(n == ntok[u] && st == steps[u] && memcmp(tok, tokens + (size_t)u * cap, (size_t)n * sizeof *tok) == 0,
              "batch equals single");
        free(tok);
        free_state(&s);
        free(bufs[u]);
    }
    free(tokens);
    free_model(&t);
    return 0;
}

static int dequant_all(void) {
    static const int types[] = {0, 1, 2, 6, 8};
    static const int bytes_per_32[] = {128, 64, 18, 22, 34};
    for (int k = 0; k < 5; ++k) {
        const int n = 32 * 7;
        const size_t nb = (size_t)bytes_per_32[k] * 7;
        uint8_t *src = malloc(nb);
        for (size_t i = 0; i < nb; ++i) src[i] = (uint8_t)rnd();
        if (types[k] >= 2 || types[k] == 1) {   /* finite f16 scales / values: clear the top exponent bit */
            const int stride = types[k] == 1 ? 2 : bytes_per_32[k];
            for (size_t i = 0; i + 1 < nb; i += (size_t)stride) src[i + 1] &= 0x3F;
        }
        if (types[k] == 0)
            for (int i = 0; i < n; ++i) ((float *)src)[i] = frand(4.0f);
        float *dst = malloc((size_t)n * sizeof *dst);
        ora_dequant(src, types[k], n, dst);
        for (int i = 0; i < n; ++i) CHECK(isfinite(dst[i]), "finite dequant");
        free(dst);
        free(src);
    }
    return 0;
}

int main(void) {
    if (dequant_all()) return 1;
    if (run_model(ORA_TDT)) return 1;
    if (run_model(ORA_EOU)) return 1;
    printf("ok\n");
    return 0;
}

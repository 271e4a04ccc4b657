/*
 * pk_oracle.c -- CPU restatement of parakeet.cpp's transducer greedy decoder.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle + CPU baseline); see pk_oracle.h.
 * Each function cites the reference function it restates.  The arithmetic is
 * the reference's: f32 GEMV rows accumulated from the bias, libm exp/tanh,
 * first-index argmax, the same statement order in the control flow.
 */
#include "pk_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* src/parakeet_tdt.cpp:25-32: first index of the maximum (strict '>'). */
int ora_argmax(const float *data, int n) {
    int best = 0;
    float best_val = data[0];
    for (int i = 1; i < n; ++i) {
        if (data[i] > best_val) { best_val = data[i]; best = i; }
    }
    return best;
}

/* src/parakeet_tdt.cpp:34 */
static inline float ora_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* src/parakeet_tdt.cpp:47-57: y[i] = (b ? b[i] : 0) + sum_j W[i,j] x[j]. */
void ora_gemv(const float *__restrict W, const float *__restrict x,
              const float *__restrict b, float *__restrict y, int out_dim, int in_dim) {
    for (int i = 0; i < out_dim; ++i) {
        const float *__restrict row = W + (size_t)i * in_dim;
        float acc = b ? b[i] : 0.0f;
        for (int j = 0; j < in_dim; ++j) acc += row[j] * x[j];
        y[i] = acc;
    }
}

/* src/parakeet_tdt.cpp:59-68: y[i] += sum_j W[i,j] x[j]. */
void ora_gemv_add(const float *__restrict W, const float *__restrict x,
                  float *__restrict y, int out_dim, int in_dim) {
    for (int i = 0; i < out_dim; ++i) {
        const float *__restrict row = W + (size_t)i * in_dim;
        float acc = 0.0f;
        for (int j = 0; j < in_dim; ++j) acc += row[j] * x[j];
        y[i] += acc;
    }
}

/* IEEE binary16 -> binary32, exact (normal, subnormal, inf, nan). */
float ora_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {               /* subnormal: renormalise */
            int e = -1;
            do { ++e; mant <<= 1; } while ((mant & 0x400u) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* ggml to_float as used by dequantize_to_f32 (src/parakeet_tdt.cpp:78-95).
 * ggml is not vendored in the reference (scripts/setup-ggml.sh:32 pins upstream
 * commit 58c38058); its published block formats, 32 weights per block:
 *   type 0 = f32 copy, 1 = f16,
 *   8 = q8_0 {f16 d; int8 q[32]}              -> q*d,
 *   6 = q5_0 {f16 d; u8 qh[4]; u8 qs[16]}     -> ((nibble | bit << 4) - 16)*d,
 *   2 = q4_0 {f16 d; u8 qs[16]}               -> (nibble - 8)*d,
 * where weight j (< 16) takes the low nibble of qs[j] and bit j of qh, and
 * weight j + 16 the high nibble of qs[j] and bit j + 16 of qh (little endian). */
void ora_dequant(const void *src, int ggml_type, int64_t n, float *dst) {
    if (ggml_type == 0) {
        memcpy(dst, src, (size_t)n * sizeof(float));
    } else if (ggml_type == 1) {
        const uint16_t *s = (const uint16_t *)src;
        for (int64_t i = 0; i < n; ++i) dst[i] = ora_f16_to_f32(s[i]);
    } else if (ggml_type == 8) {
        const uint8_t *s = (const uint8_t *)src;
        for (int64_t b = 0; b < n / 32; ++b) {
            uint16_t dh;
            memcpy(&dh, s + 34 * b, 2);
            const float d = ora_f16_to_f32(dh);
            const int8_t *q = (const int8_t *)(s + 34 * b + 2);
            for (int j = 0; j < 32; ++j) dst[32 * b + j] = q[j] * d;
        }
    } else if (ggml_type == 6 || ggml_type == 2) {
        const int five = ggml_type == 6, bytes = five ? 22 : 18;
        const uint8_t *s = (const uint8_t *)src;
        for (int64_t b = 0; b < n / 32; ++b) {
            const uint8_t *blk = s + (size_t)bytes * b;
            uint16_t dh;
            memcpy(&dh, blk, 2);
            const float d = ora_f16_to_f32(dh);
            uint32_t qh = 0;
            const uint8_t *qs = blk + 2;
            if (five) {
                qh = (uint32_t)blk[2] | (uint32_t)blk[3] << 8 | (uint32_t)blk[4] << 16 | (uint32_t)blk[5] << 24;
                qs = blk + 6;
            }
            for (int j = 0; j < 16; ++j) {
                const int lo = (qs[j] & 15) | (int)((qh >> j) & 1u) << 4;
                const int hi = (qs[j] >> 4) | (int)((qh >> (j + 16)) & 1u) << 4;
                dst[32 * b + j] = (float)(lo - (five ? 16 : 8)) * d;
                dst[32 * b + j + 16] = (float)(hi - (five ? 16 : 8)) * d;
            }
        }
    }
}

/* src/parakeet_tdt.cpp:106-142 (== src/parakeet_eou.cpp:78-116).
 * gates = ((b_ih + W_ih x) + b_hh) + W_hh h; order i, f, g, o;
 * c = f c + i g; h = o tanh(c); the next layer's input is this layer's h. */
void ora_lstm_step(const ora_model *m, const float *x_input, float *h_state, float *c_state,
                   float *scratch, float *layer_input) {
    const int H = m->H, L = m->L, G = 4 * H;
    const float *x = x_input;
    for (int layer = 0; layer < L; ++layer) {
        const float *h_l = h_state + (size_t)layer * H;
        float *c_l = c_state + (size_t)layer * H;
        ora_gemv(m->w_ih[layer], x, m->b_ih[layer], scratch, G, H);
        for (int i = 0; i < G; ++i) scratch[i] += m->b_hh[layer][i];
        ora_gemv_add(m->w_hh[layer], h_l, scratch, G, H);
        float *h_new = h_state + (size_t)layer * H;
        for (int i = 0; i < H; ++i) {
            const float i_g = ora_sigmoid(scratch[0 * H + i]);
            const float f_g = ora_sigmoid(scratch[1 * H + i]);
            const float g_g = tanhf(scratch[2 * H + i]);
            const float o_g = ora_sigmoid(scratch[3 * H + i]);
            const float c_new = f_g * c_l[i] + i_g * g_g;
            c_l[i] = c_new;
            h_new[i] = o_g * tanhf(c_new);
        }
        memcpy(layer_input, h_new, (size_t)H * sizeof(float));
        x = layer_input;
    }
}

/* src/parakeet_tdt.cpp:154-177 (TDT, logits over Vo) and
 * src/parakeet_eou.cpp:123-143 (EOU, Vo == V1):
 * hidden = relu((b_e + W_e enc) + (b_p + W_p pred)); logits = b_o + W_o hidden. */
void ora_joint_step(const ora_model *m, const float *enc, const float *pred,
                    float *hidden, float *logits, float *tmp) {
    const int J = m->J;
    ora_gemv(m->enc_w, enc, m->enc_b, hidden, J, m->D);
    ora_gemv(m->pred_w, pred, m->pred_b, tmp, J, m->H);
    for (int i = 0; i < J; ++i) hidden[i] += tmp[i];
    for (int i = 0; i < J; ++i) hidden[i] = (0.0f < hidden[i]) ? hidden[i] : 0.0f; /* std::max(0.0f, x) */
    ora_gemv(m->out_w, hidden, m->out_b, logits, m->Vo, J);
}

static void lstm_from_token(const ora_model *m, ora_state *st, int token) {
    float *scratch = (float *)malloc(sizeof(float) * 4 * (size_t)m->H);
    float *layer_in = (float *)malloc(sizeof(float) * (size_t)m->H);
    ora_lstm_step(m, m->embed + (size_t)token * m->H, st->h, st->c, scratch, layer_in);
    memcpy(st->pred, st->h + (size_t)(m->L - 1) * m->H, sizeof(float) * (size_t)m->H);
    free(scratch);
    free(layer_in);
}

/* src/parakeet_tdt.cpp:813-863 (CPU branch) and src/parakeet_eou.cpp:206-230:
 * zero h, c; one LSTM step on embed[blank]; pred = h[L-1]. */
void ora_init_state(const ora_model *m, ora_state *st) {
    const size_t n = (size_t)m->L * m->H;
    memset(st->h, 0, n * sizeof(float));
    memset(st->c, 0, n * sizeof(float));
    memset(st->pred, 0, (size_t)m->H * sizeof(float));
    st->symbols_this_step = 0;
    st->carry_frames = 0;
    st->last_token = -1;
    st->segment_start_token = 0;
    lstm_from_token(m, st, m->blank);
    st->initialized = 1;
}

typedef struct scratch_t {
    float *hidden, *tmp, *logits, *lstm_g, *lstm_h;
} scratch_t;

static int scratch_alloc(const ora_model *m, scratch_t *s) {
    s->hidden = (float *)malloc(sizeof(float) * (size_t)m->J);
    s->tmp = (float *)malloc(sizeof(float) * (size_t)m->J);
    s->logits = (float *)malloc(sizeof(float) * (size_t)m->Vo);
    s->lstm_g = (float *)malloc(sizeof(float) * 4 * (size_t)m->H);
    s->lstm_h = (float *)malloc(sizeof(float) * (size_t)m->H);
    return s->hidden && s->tmp && s->logits && s->lstm_g && s->lstm_h;
}

static void scratch_free(scratch_t *s) {
    free(s->hidden); free(s->tmp); free(s->logits); free(s->lstm_g); free(s->lstm_h);
}

static void lstm_emit(const ora_model *m, ora_state *st, scratch_t *s, int token) {
    ora_lstm_step(m, m->embed + (size_t)token * m->H, st->h, st->c, s->lstm_g, s->lstm_h);
    memcpy(st->pred, st->h + (size_t)(m->L - 1) * m->H, sizeof(float) * (size_t)m->H);
}

static inline int dur_value(const ora_model *m, int idx) {
    return m->n_dur > 0 ? m->durations[idx] : idx;
}

/* One joint evaluation + argmaxes (src/parakeet_tdt.cpp:930-934). */
static void joint_argmax(const ora_model *m, const float *enc_frame, const ora_state *st,
                         scratch_t *s, float blank_bias, int *tok, int *dur_idx) {
    ora_joint_step(m, enc_frame, st->pred, s->hidden, s->logits, s->tmp);
    if (blank_bias != 0.0f) s->logits[m->blank] += blank_bias;   /* build addition, 0 = reference */
    *tok = ora_argmax(s->logits, m->V1);
    *dur_idx = m->Dn > 0 ? ora_argmax(s->logits + m->V1, m->Dn) : -1;
}

/* src/parakeet_tdt.cpp:865-981 (CPU branch). */
int ora_tdt_decode_window(const ora_model *m, const float *enc, int n_frames, int D_enc,
                          int max_symbols, float blank_bias, ora_state *st,
                          int32_t *out_tokens, int token_cap, int *n_out, int *out_steps,
                          int32_t *trace, int trace_cap) {
    *out_steps = 0;
    if (D_enc != m->D) return 1;
    if (n_frames <= 0) return 0;
    if (!st->initialized) ora_init_state(m, st);

    scratch_t s;
    if (!scratch_alloc(m, &s)) { scratch_free(&s); return 12; }
    int rc = 0;
    int t = 0;
    if (st->carry_frames > 0) {
        t = st->carry_frames < n_frames ? st->carry_frames : n_frames;
        st->carry_frames -= t;
    }
    while (t < n_frames) {
        int tok, di;
        joint_argmax(m, enc + (size_t)t * D_enc, st, &s, blank_bias, &tok, &di);
        if (trace && *out_steps < trace_cap) {
            trace[2 * *out_steps] = tok;
            trace[2 * *out_steps + 1] = di;
        }
        ++*out_steps;
        const int dur = dur_value(m, di);
        if (tok == m->blank) {
            t += dur > 1 ? dur : 1;
            st->symbols_this_step = 0;
            continue;
        }
        if (*n_out >= token_cap) { rc = 11; break; }
        out_tokens[(*n_out)++] = tok;
        lstm_emit(m, st, &s, tok);
        ++st->symbols_this_step;
        if (dur > 0 || st->symbols_this_step >= max_symbols) {
            t += dur > 1 ? dur : 1;
            st->symbols_this_step = 0;
        }
    }
    st->carry_frames = t - n_frames > 0 ? t - n_frames : 0;
    scratch_free(&s);
    return rc;
}

static inline int is_special(const ora_model *m, int tok) {
    return tok >= 0 && tok < m->n_special && m->special && m->special[tok];
}

/* src/parakeet_eou.cpp:232-336. */
int ora_eou_decode_window(const ora_model *m, const float *enc, int n_frames, int D_enc,
                          int max_symbols, float blank_bias, ora_state *st,
                          int32_t *out_tokens, int token_cap, int *n_out,
                          int32_t *out_segments, int seg_cap, int *n_seg,
                          int *out_steps, int32_t *trace, int trace_cap) {
    if (D_enc != m->D) return 1;
    if (!st->initialized) ora_init_state(m, st);
    const int max_syms = max_symbols > 1 ? max_symbols : 1;
    scratch_t s;
    if (!scratch_alloc(m, &s)) { scratch_free(&s); return 12; }
    int rc = 0;
    *out_steps = 0;
    for (int t = 0; t < n_frames && rc == 0; ++t) {
        const float *enc_frame = enc + (size_t)t * D_enc;
        st->symbols_this_step = 0;
        while (st->symbols_this_step < max_syms) {
            int best, di;
            joint_argmax(m, enc_frame, st, &s, blank_bias, &best, &di);
            if (trace && *out_steps < trace_cap) {
                trace[2 * *out_steps] = best;
                trace[2 * *out_steps + 1] = -1;
            }
            ++*out_steps;
            if (best == m->blank) break;
            if (best == m->eob) break;
            if (best == m->eou) {
                if (*n_out > st->segment_start_token) {
                    if (*n_seg >= seg_cap) { rc = 11; break; }
                    out_segments[(*n_seg)++] = *n_out;
                    st->segment_start_token = *n_out;
                }
                memset(st->h, 0, sizeof(float) * (size_t)m->L * m->H);
                memset(st->c, 0, sizeof(float) * (size_t)m->L * m->H);
                st->last_token = m->blank;
                lstm_emit(m, st, &s, m->blank);
                break;
            }
            if (is_special(m, best)) break;
            if (*n_out >= token_cap) { rc = 11; break; }
            out_tokens[(*n_out)++] = best;
            lstm_emit(m, st, &s, best);
            st->last_token = best;
            ++st->symbols_this_step;
        }
    }
    scratch_free(&s);
    return rc;
}

/* Compare one decision of another decoder with the oracle logits. */
static void classify(const ora_model *m, const float *lg, int tok_o, int di_o, int tok_d, int di_d,
                     float eps, int step, ora_replay_stats *st) {
    /* top-1 minus top-2 over the token logits */
    float second = -FLT_MAX;
    for (int i = 0; i < m->V1; ++i)
        if (i != tok_o && lg[i] > second) second = lg[i];
    const float top2 = lg[tok_o] - second;
    if (top2 < st->min_top2) st->min_top2 = top2;

    if (tok_d != tok_o) {
        st->tok_mismatch++;
        const float margin = (tok_d >= 0 && tok_d < m->V1) ? lg[tok_o] - lg[tok_d] : FLT_MAX;
        if (margin > st->worst_margin) st->worst_margin = margin;
        if (margin < eps) st->near_ties++;
        else { st->unexplained++; if (st->first_unexplained < 0) st->first_unexplained = step; }
    }
    if (m->Dn > 0 && di_d != di_o) {
        st->dur_mismatch++;
        const float margin = (di_d >= 0 && di_d < m->Dn) ? lg[m->V1 + di_o] - lg[m->V1 + di_d] : FLT_MAX;
        if (margin > st->worst_margin) st->worst_margin = margin;
        if (margin < eps) st->near_ties++;
        else { st->unexplained++; if (st->first_unexplained < 0) st->first_unexplained = step; }
    }
}

int ora_replay_window(const ora_model *m, const float *enc, int n_frames, int D_enc,
                      int max_symbols, float blank_bias, ora_state *st,
                      const int32_t *trace, int n_trace, float tie_eps,
                      int32_t *out_tokens, int token_cap, int *n_out,
                      int32_t *out_segments, int seg_cap, int *n_seg,
                      float *logit_tap, int n_tap, ora_replay_stats *stats) {
    memset(stats, 0, sizeof *stats);
    stats->first_unexplained = -1;
    stats->min_top2 = FLT_MAX;
    if (D_enc != m->D) return 1;
    if (m->kind == ORA_TDT && n_frames <= 0) {
        stats->structure_error = n_trace != 0;
        return 0;
    }
    if (!st->initialized) ora_init_state(m, st);
    scratch_t s;
    if (!scratch_alloc(m, &s)) { scratch_free(&s); return 12; }
    int rc = 0, step = 0;

#define REPLAY_STEP(FRAME)                                                         \
    int tok_o, di_o;                                                               \
    joint_argmax(m, (FRAME), st, &s, blank_bias, &tok_o, &di_o);                   \
    if (logit_tap && step < n_tap)                                                 \
        memcpy(logit_tap + (size_t)step * m->Vo, s.logits, sizeof(float) * m->Vo); \
    if (step >= n_trace) { stats->structure_error = 1; goto done; }                \
    const int tok = trace[2 * step], di = trace[2 * step + 1];                     \
    classify(m, s.logits, tok_o, di_o, tok, di, tie_eps, step, stats);             \
    if (tok < 0 || tok >= m->V1 || (m->Dn > 0 && (di < 0 || di >= m->Dn))) {       \
        stats->structure_error = 1; goto done;                                     \
    }                                                                              \
    ++step;

    if (m->kind == ORA_TDT) {
        int t = 0;
        if (st->carry_frames > 0) {
            t = st->carry_frames < n_frames ? st->carry_frames : n_frames;
            st->carry_frames -= t;
        }
        while (t < n_frames) {
            REPLAY_STEP(enc + (size_t)t * D_enc)
            const int dur = dur_value(m, di);
            if (tok == m->blank) {
                t += dur > 1 ? dur : 1;
                st->symbols_this_step = 0;
                continue;
            }
            if (*n_out >= token_cap) { rc = 11; goto done; }
            out_tokens[(*n_out)++] = tok;
            lstm_emit(m, st, &s, tok);
            ++st->symbols_this_step;
            if (dur > 0 || st->symbols_this_step >= max_symbols) {
                t += dur > 1 ? dur : 1;
                st->symbols_this_step = 0;
            }
        }
        st->carry_frames = t - n_frames > 0 ? t - n_frames : 0;
    } else {
        const int max_syms = max_symbols > 1 ? max_symbols : 1;
        for (int t = 0; t < n_frames; ++t) {
            st->symbols_this_step = 0;
            while (st->symbols_this_step < max_syms) {
                REPLAY_STEP(enc + (size_t)t * D_enc)
                (void)di;
                if (tok == m->blank || tok == m->eob) break;
                if (tok == m->eou) {
                    if (*n_out > st->segment_start_token) {
                        if (*n_seg >= seg_cap) { rc = 11; goto done; }
                        out_segments[(*n_seg)++] = *n_out;
                        st->segment_start_token = *n_out;
                    }
                    memset(st->h, 0, sizeof(float) * (size_t)m->L * m->H);
                    memset(st->c, 0, sizeof(float) * (size_t)m->L * m->H);
                    st->last_token = m->blank;
                    lstm_emit(m, st, &s, m->blank);
                    break;
                }
                if (is_special(m, tok)) break;
                if (*n_out >= token_cap) { rc = 11; goto done; }
                out_tokens[(*n_out)++] = tok;
                lstm_emit(m, st, &s, tok);
                st->last_token = tok;
                ++st->symbols_this_step;
            }
        }
    }
#undef REPLAY_STEP
    if (step != n_trace) stats->structure_error = 1;
done:
    stats->steps = step;
    scratch_free(&s);
    return rc;
}

/* ---- thread-pool batch driver (CPU baseline) ---- */

typedef struct batch_ctx {
    const ora_model *m;
    int n_utts;
    const float *const *enc;
    const int *n_frames;
    const float *blank_bias;
    int max_symbols;
    int32_t *tokens;
    int token_cap;
    int32_t *n_tokens, *steps;
    int next;      /* work counter */
    int rc;
} batch_ctx;

static void *batch_worker(void *arg) {
    batch_ctx *b = (batch_ctx *)arg;
    const ora_model *m = b->m;
    float *h = (float *)malloc(sizeof(float) * (size_t)m->L * m->H);
    float *c = (float *)malloc(sizeof(float) * (size_t)m->L * m->H);
    float *pred = (float *)malloc(sizeof(float) * (size_t)m->H);
    int32_t *seg = (int32_t *)malloc(sizeof(int32_t) * ((size_t)b->token_cap + 1));
    for (;;) {
        const int u = __atomic_fetch_add(&b->next, 1, __ATOMIC_RELAXED);
        if (u >= b->n_utts) break;
        ora_state st;
        memset(&st, 0, sizeof st);
        st.h = h; st.c = c; st.pred = pred;
        int n_out = 0, steps = 0, rc;
        const float bias = b->blank_bias ? b->blank_bias[u] : 0.0f;
        int32_t *out = b->tokens + (size_t)u * b->token_cap;
        if (m->kind == ORA_TDT) {
            rc = ora_tdt_decode_window(m, b->enc[u], b->n_frames[u], m->D, b->max_symbols, bias,
                                       &st, out, b->token_cap, &n_out, &steps, NULL, 0);
        } else {
            int n_seg = 0;
            rc = ora_eou_decode_window(m, b->enc[u], b->n_frames[u], m->D, b->max_symbols, bias,
                                       &st, out, b->token_cap, &n_out, seg, b->token_cap + 1,
                                       &n_seg, &steps, NULL, 0);
        }
        b->n_tokens[u] = n_out;
        b->steps[u] = steps;
        if (rc) __atomic_store_n(&b->rc, rc, __ATOMIC_RELAXED);
    }
    free(h); free(c); free(pred); free(seg);
    return NULL;
}

int ora_decode_batch(const ora_model *m, int n_utts, const float *const *enc,
                     const int *n_frames, const float *blank_bias, int max_symbols,
                     int n_threads, int32_t *tokens, int token_cap, int32_t *n_tokens,
                     int32_t *steps) {
    batch_ctx b = {m, n_utts, enc, n_frames, blank_bias, max_symbols,
                   tokens, token_cap, n_tokens, steps, 0, 0};
    if (n_threads < 1) n_threads = 1;
    if (n_threads > n_utts) n_threads = n_utts > 0 ? n_utts : 1;
    if (n_threads == 1) {
        batch_worker(&b);
        return b.rc;
    }
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
    for (int i = 0; i < n_threads; ++i) pthread_create(&th[i], NULL, batch_worker, &b);
    for (int i = 0; i < n_threads; ++i) pthread_join(th[i], NULL);
    free(th);
    return b.rc;
}

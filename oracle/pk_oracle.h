/*
 * pk_oracle.h -- CPU restatement of parakeet.cpp's transducer greedy decoder.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity oracle and the same-box CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product path (parakeet.cpp_amd/) never links it.
 *
 * Every function restates one function of the reference's scalar CPU decoder
 * (src/parakeet_tdt.cpp, src/parakeet_eou.cpp) on host-dequantised f32
 * weights, compiled with the reference's release flags
 * (-O3 -ffast-math -funroll-loops, CMakeLists.txt:327-335).
 *
 * Additions that the reference does not have, each marked where defined:
 *   - per-utterance blank-logit offset (blank_bias), 0 reproduces the reference;
 *   - bounded output arrays instead of std::vector (overflow -> rc 11);
 *   - a per-step decision trace (token, duration index) and a teacher-forced
 *     replay that follows another decoder's decisions and classifies every
 *     disagreement as a near-tie or not;
 *   - a thread-pool batch driver (one utterance per task) for the CPU baseline.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORA_MAX_L 8
#define ORA_MAX_DUR 16

enum { ORA_TDT = 0, ORA_EOU = 1 };

typedef struct ora_model {
    int kind;       /* ORA_TDT or ORA_EOU */
    int H;          /* prediction-net hidden (pred_hidden) */
    int L;          /* LSTM layers */
    int J;          /* joint hidden */
    int D;          /* encoder dim */
    int V1;         /* vocab + blank: token logits */
    int Dn;         /* duration logits (0 for EOU) */
    int Vo;         /* V1 + Dn */
    int blank;
    int eou, eob;   /* EOU only */
    int n_dur;      /* entries in durations[]; 0 -> duration = index */
    int durations[ORA_MAX_DUR];
    const float *embed;                        /* [V1][H] */
    const float *w_ih[ORA_MAX_L];              /* [4H][H_in] */
    const float *w_hh[ORA_MAX_L];              /* [4H][H] */
    const float *b_ih[ORA_MAX_L], *b_hh[ORA_MAX_L];
    const float *enc_w, *enc_b;                /* [J][D], [J] */
    const float *pred_w, *pred_b;              /* [J][H], [J] */
    const float *out_w, *out_b;                /* [Vo][J], [Vo] */
    const uint8_t *special;                    /* EOU: 1 where vocab piece is "<...>" */
    int n_special;                             /* number of vocab pieces (0: none) */
} ora_model;

typedef struct ora_state {
    float *h;        /* [L*H], caller-allocated */
    float *c;        /* [L*H] */
    float *pred;     /* [H]   */
    int symbols_this_step;
    int initialized;
    int carry_frames;          /* TDT */
    int last_token;            /* EOU */
    int segment_start_token;   /* EOU */
} ora_state;

typedef struct ora_replay_stats {
    int steps;              /* joint evaluations replayed */
    int tok_mismatch;       /* steps where the other decoder's token != oracle argmax */
    int dur_mismatch;       /* same for the duration head */
    int near_ties;          /* mismatches whose oracle margin is below tie_eps */
    int unexplained;        /* mismatches at or above tie_eps */
    int structure_error;    /* trace shorter/longer than the control flow implies */
    int first_unexplained;  /* step index, -1 if none */
    float worst_margin;     /* largest margin among mismatches */
    float min_top2;         /* smallest oracle top-1 minus top-2 token margin seen */
} ora_replay_stats;

/* src/parakeet_tdt.cpp:25-32 */
int  ora_argmax(const float *data, int n);
/* src/parakeet_tdt.cpp:47-68 */
void ora_gemv(const float *W, const float *x, const float *b, float *y, int out_dim, int in_dim);
void ora_gemv_add(const float *W, const float *x, float *y, int out_dim, int in_dim);
/* ggml to_float for f16, q8_0, q5_0 and q4_0, as called at src/parakeet_tdt.cpp:86-94 */
float ora_f16_to_f32(uint16_t h);
void ora_dequant(const void *src, int ggml_type, int64_t n, float *dst);
/* src/parakeet_tdt.cpp:106-142 (TDT) == src/parakeet_eou.cpp:78-116 (EOU) */
void ora_lstm_step(const ora_model *m, const float *x, float *h, float *c,
                   float *scratch_g, float *scratch_h);
/* src/parakeet_tdt.cpp:154-177; EOU src/parakeet_eou.cpp:123-143 (logits over V1 only) */
void ora_joint_step(const ora_model *m, const float *enc, const float *pred,
                    float *hidden, float *logits, float *tmp);
/* src/parakeet_tdt.cpp:813-863 / src/parakeet_eou.cpp:206-230 */
void ora_init_state(const ora_model *m, ora_state *st);

/* src/parakeet_tdt.cpp:865-981.  Tokens are appended at out_tokens[*n_out].
 * trace (nullable) receives (token, duration index) per step. */
int ora_tdt_decode_window(const ora_model *m, const float *enc, int n_frames, int D_enc,
                          int max_symbols, float blank_bias, ora_state *st,
                          int32_t *out_tokens, int token_cap, int *n_out, int *out_steps,
                          int32_t *trace, int trace_cap);

/* src/parakeet_eou.cpp:232-336.  *n_out is the caller's token count before the
 * call (the reference compares segment starts against out_tokens.size()). */
int ora_eou_decode_window(const ora_model *m, const float *enc, int n_frames, int D_enc,
                          int max_symbols, float blank_bias, ora_state *st,
                          int32_t *out_tokens, int token_cap, int *n_out,
                          int32_t *out_segments, int seg_cap, int *n_seg,
                          int *out_steps, int32_t *trace, int trace_cap);

/* Teacher-forced replay: run the control flow of the window, but at every step
 * follow trace[2*s] (token) and trace[2*s+1] (duration index) instead of the
 * oracle argmax.  Disagreements are classified with tie_eps.  logit_tap
 * (nullable) receives the oracle logits of the first n_tap steps ([n_tap][Vo]). */
int ora_replay_window(const ora_model *m, const float *enc, int n_frames, int D_enc,
                      int max_symbols, float blank_bias, ora_state *st,
                      const int32_t *trace, int n_trace, float tie_eps,
                      int32_t *out_tokens, int token_cap, int *n_out,
                      int32_t *out_segments, int seg_cap, int *n_seg,
                      float *logit_tap, int n_tap, ora_replay_stats *stats);

/* CPU baseline: n_utts independent greedy decodes (fresh state each) over
 * n_threads worker threads, one utterance per task.  enc[u] points at
 * [n_frames[u]][D] f32.  Outputs are [n_utts][token_cap]. */
int ora_decode_batch(const ora_model *m, int n_utts, const float *const *enc,
                     const int *n_frames, const float *blank_bias, int max_symbols,
                     int n_threads, int32_t *tokens, int token_cap, int32_t *n_tokens,
                     int32_t *steps);

#ifdef __cplusplus
}
#endif
#endif

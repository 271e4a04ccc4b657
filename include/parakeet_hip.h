/*
 * parakeet_hip.h -- C ABI of the MI355X transducer greedy-decode library
 * (libparakeet_hip.so).
 *
 * The ABI replaces the device side of parakeet.cpp's decoder runtime:
 *
 *   pk_decoder_create   <- tdt_prepare_runtime (src/parakeet_tdt.cpp:585-718)
 *                          and eou_prepare_runtime (src/parakeet_eou.cpp:172-204):
 *                          uploads the GGUF decoder tensors once, q8_0/f16 kept
 *                          at their stored precision (q4_0 / q5_0 blocks become
 *                          q8_0 blocks with the same scale: their weights are
 *                          exact int8 values).
 *   pk_decoder_destroy  <- ~TdtRuntimeWeights (src/parakeet_tdt.cpp:560-583)
 *   pk_slot_init        <- tdt_init_state (src/parakeet_tdt.cpp:813-863),
 *                          eou_init_state (src/parakeet_eou.cpp:206-230)
 *   pk_decode           <- tdt_decode_window (src/parakeet_tdt.cpp:865-981) and
 *                          eou_decode_window (src/parakeet_eou.cpp:232-336),
 *                          batched over utterances; one call decodes a window
 *                          for every utterance in the batch.
 *   pk_slot_read        <- the host-visible TdtDecodeState / EouDecodeState
 *                          (src/parakeet_tdt.h:175-183, src/parakeet_eou.h:53-66)
 *
 * Decoder state (the reference's *DecodeState) lives on the device in
 * numbered slots owned by the handle; callers keep slot ids, as a streaming
 * session keeps its state object.  Plain C types only; every entry point
 * returns an int status (0 = ok) and never throws.  Status values keep the
 * reference's meanings where one exists (1 = encoder dim mismatch, as
 * tdt_decode_window / eou_decode_window return; 2 = missing/invalid decoder
 * tensor, as tdt_prepare_runtime returns).
 *
 * Threading: one call at a time per handle (the reference Engine's contract,
 * include/parakeet/engine.h:35-63).  Work runs on one HIP stream owned by the
 * handle; pk_decode returns when the batch is decoded.
 */
#ifndef PARAKEET_HIP_H
#define PARAKEET_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_API __attribute__((visibility("default")))

#define PK_MAX_LAYERS 8
#define PK_MAX_DURATIONS 16
#define PK_MAX_BATCH 512   /* utterances per pk_decode call */

enum { PK_KIND_TDT = 0, PK_KIND_EOU = 1 };
enum { PK_TYPE_F32 = 0, PK_TYPE_F16 = 1, PK_TYPE_Q4_0 = 2, PK_TYPE_Q5_0 = 6, PK_TYPE_Q8_0 = 8 };   /* ggml type ids */
/* pk_batch.mem: where the frames and the outputs live.
 *   PK_MEM_HOST           frames and outputs in host memory (frames uploaded per call)
 *   PK_MEM_DEVICE         frames and outputs in device memory
 *   PK_MEM_DEVICE_FRAMES  frames in device memory, read in place (an encoder output
 *                         that stays on the device, instead of the host copy of
 *                         src/parakeet_ctc.cpp:1660-1667); outputs in host memory
 * Device frames must be complete before the call: the decoder runs on its own
 * stream, so the caller synchronises the stream that produced them. */
enum { PK_MEM_HOST = 0, PK_MEM_DEVICE = 1, PK_MEM_DEVICE_FRAMES = 2 };

enum {
    PK_OK = 0,
    PK_ERR_D_ENC = 1,        /* encoder dim mismatch (reference rc 1) */
    PK_ERR_TENSOR = 2,       /* missing / mis-shaped decoder tensor (reference prepare rc 2) */
    PK_ERR_ARG = 3,          /* invalid argument */
    PK_ERR_NOMEM = 4,        /* device allocation failed */
    PK_ERR_UNSUPPORTED = 5,  /* shape outside what the kernels handle */
    PK_ERR_DEVICE = 6,       /* HIP runtime error (reference rc 6-9 are GPU-path failures) */
    PK_ERR_TIMEOUT = 7,      /* device-side iteration cap or barrier time-out hit */
    PK_ERR_OVERFLOW = 11     /* token / segment output capacity exceeded */
};

/* One GGUF tensor as stored: ne0 = innermost (in) length, ne1 = rows (out). */
typedef struct pk_tensor {
    const void *data;   /* host pointer to the stored bytes */
    int32_t type;       /* PK_TYPE_*: f32 / f16 / q4_0 / q5_0 / q8_0 (biases f32 / f16) */
    int64_t ne0;
    int64_t ne1;        /* 1 for vectors */
} pk_tensor;

/* Decoder description: the metadata src/parakeet_ctc.cpp:418-458 reads and the
 * tensors bound at src/parakeet_ctc.cpp:603-665. */
typedef struct pk_decoder_desc {
    int32_t kind;             /* PK_KIND_TDT / PK_KIND_EOU */
    int32_t pred_hidden;      /* H */
    int32_t pred_rnn_layers;  /* L */
    int32_t joint_hidden;     /* J */
    int32_t d_enc;            /* encoder d_model */
    int32_t vocab_size;       /* labels without blank; token logits = vocab_size + 1 */
    int32_t blank_id;
    int32_t num_durations;    /* TDT duration logits (0 for EOU) */
    int32_t n_duration_values;/* entries of durations[]; 0 -> duration = index */
    int32_t durations[PK_MAX_DURATIONS];
    int32_t eou_id, eob_id;   /* EOU */
    const uint8_t *special;   /* EOU: [n_special] 1 where the vocab piece is "<...>" (nullable) */
    int32_t n_special;
    pk_tensor embed;                          /* [V+1 rows][H] */
    pk_tensor w_ih[PK_MAX_LAYERS], w_hh[PK_MAX_LAYERS];   /* [4H][H] */
    pk_tensor b_ih[PK_MAX_LAYERS], b_hh[PK_MAX_LAYERS];   /* [4H] f32 */
    pk_tensor joint_enc_w, joint_enc_b;       /* [J][D], [J] */
    pk_tensor joint_pred_w, joint_pred_b;     /* [J][H], [J] */
    pk_tensor joint_out_w, joint_out_b;       /* [V+1+num_durations][J], [...] */
} pk_decoder_desc;

typedef struct pk_decoder pk_decoder;

/* One batched decode call: utterance u decodes frames
 * enc[enc_row[u] .. enc_row[u] + n_frames[u]) with the state in slot[u].
 * Descriptor arrays (enc_row .. tokens_base) are host arrays.  enc is a
 * device pointer for PK_MEM_DEVICE and PK_MEM_DEVICE_FRAMES; the output
 * arrays are device pointers for PK_MEM_DEVICE only. */
typedef struct pk_batch {
    int32_t n_utts;
    int32_t mem;
    int32_t d_enc;
    int32_t max_symbols;        /* TdtDecodeOptions / EouDecodeOptions::max_symbols_per_step */
    const float *enc;           /* [rows][d_enc] f32 */
    const int64_t *enc_row;     /* [n_utts] */
    const int32_t *n_frames;    /* [n_utts] */
    const int32_t *slot;        /* [n_utts], distinct */
    const float *blank_bias;    /* [n_utts] additive offset on the blank logit, nullable */
    const int32_t *tokens_base; /* [n_utts] caller's token count before the call (EOU segment
                                   indices count from it), nullable = 0 */
    int32_t *tokens;            /* out [n_utts][token_cap] emitted token ids */
    int32_t token_cap;
    int32_t *n_tokens;          /* out [n_utts] */
    int32_t *steps;             /* out [n_utts] joint evaluations (the reference's out_steps) */
    int32_t *segments;          /* EOU out [n_utts][seg_cap] boundary token indices, nullable */
    int32_t seg_cap;
    int32_t *n_segments;        /* EOU out [n_utts], nullable */
    int32_t *trace;             /* out [n_utts][trace_cap][2] (token, duration index) per step, nullable */
    int32_t trace_cap;
    /* Debug tap, nullable: out [n_utts][logit_steps][V+1+num_durations] f32, the joint
     * logits (bias and blank offset included) of each utterance's first logit_steps
     * steps -- the values src/parakeet_tdt.cpp:154-177 produces before the argmax.
     * Rows of steps an utterance does not reach are left untouched.  Parity tests
     * only; a timed call passes NULL. */
    float *logits;
    int32_t logit_steps;
    /* [n_utts], nullable: 1 = start utterance u from a fresh state (zero h, c, one
     * LSTM step on embed[blank], counters reset -- what tdt_init_state /
     * eou_init_state do, src/parakeet_tdt.cpp:813-863) whatever its slot holds;
     * the initial step runs inside the same launch.  A TDT window of 0 frames does
     * not run at all (src/parakeet_tdt.cpp:879 returns before initialising): its
     * slot keeps what it held, reset or not, its outputs are 0 and its ctrl_out
     * reads as fresh when reset, so a caller passes the reset again with the slot's
     * next window.  PK_MEM_DEVICE batches must not hold such windows (PK_ERR_ARG). */
    const uint8_t *reset;
    /* out [n_utts][PK_CTRL_N], nullable: each utterance's slot control words after
     * the call (as pk_slot_read returns them), copied back with the other outputs. */
    int32_t *ctrl_out;
} pk_batch;

/* Slot control words (pk_slot_read ctrl[]): */
enum { PK_CTRL_INIT = 0, PK_CTRL_SYM, PK_CTRL_CARRY, PK_CTRL_LAST, PK_CTRL_SEGSTART,
       PK_CTRL_CUR, PK_CTRL_N = 8 };

/* Upload the decoder and allocate n_slots state slots on the current device.
 * Shapes: pred_hidden, joint_hidden and d_enc multiples of 32; 1 .. PK_MAX_LAYERS
 * LSTM layers; vocab_size + 1 below 16383; 1 .. PK_MAX_DURATIONS TDT durations.
 * The wider of pred_hidden and joint_hidden is staged as 16 rows of f16 hi + lo
 * in one workgroup's LDS with the loop's other buffers, about 2,400 at most on
 * gfx950; a wider decoder returns PK_ERR_UNSUPPORTED with the LDS figures. */
PK_API int pk_decoder_create(const pk_decoder_desc *desc, int32_t n_slots, pk_decoder **out);
PK_API int pk_decoder_destroy(pk_decoder *dec);
/* tdt_init_state / eou_init_state: zero h, c, run the LSTM on embed[blank]. */
PK_API int pk_slot_init(pk_decoder *dec, int32_t slot);
/* Mark a slot uninitialised (TdtDecodeState{} / EouDecodeState{}): the next
 * decode of the slot initialises it first, as *_decode_window does. */
PK_API int pk_slot_reset(pk_decoder *dec, int32_t slot);
/* Copy a slot's state to host arrays (each nullable): h, c [L*H], pred [H],
 * ctrl [PK_CTRL_N]. */
PK_API int pk_slot_read(pk_decoder *dec, int32_t slot, float *h, float *c, float *pred, int32_t *ctrl);
/* Copy the whole state of slot src into slot dst (device to device): a copy of a
 * TdtDecodeState / EouDecodeState value (src/parakeet_tdt.h:175-183) that then
 * decodes independently of the original. */
PK_API int pk_slot_copy(pk_decoder *dec, int32_t src, int32_t dst);
/* Decode one window for every utterance of the batch.  Windows of any length: a
 * window one launch of the decode loop cannot take (see pk_window_split) is decoded
 * in several launches, its state carried from piece to piece, with the same results
 * as one launch (the reference's loop, src/parakeet_tdt.cpp:917-967, has no length
 * limit).  The logit tap takes windows of one launch only. */
PK_API int pk_decode(pk_decoder *dec, const pk_batch *batch);
/* How pk_decode splits windows.  One launch takes at most 2^18 - 1 lockstep
 * iterations (the 18-bit stamp of its argmax keys; a window of T frames may take
 * T * (max_symbols + 1) + 4) and at most (2^31 - 1) / (4 * joint_hidden) frames in
 * all (32-bit offsets of its enc_proj rows).  When a batch exceeds either, utterance
 * u is decoded as launches[u] consecutive pieces of nearly equal length (the first
 * n_frames[u] % launches[u] pieces one frame longer than n_frames[u] / launches[u]),
 * at most *piece_frames frames each, and launch j takes piece j of every utterance
 * that has one.  Every piece is longer than the largest carry a TDT duration can
 * leave (max_duration - 1, where max_duration is the largest value of the duration
 * table), which makes the split decode equal to one launch over each window.
 * launches[u] is 1 for every non-empty window when no split is needed (0 for an
 * empty one).  Returns PK_ERR_UNSUPPORTED when no piece length satisfies the bounds.
 * Host arithmetic only: needs no device. */
PK_API int pk_window_split(int32_t n_utts, const int32_t *n_frames, int32_t max_symbols, int32_t joint_hidden,
                           int32_t max_duration, int32_t *piece_frames, int32_t *launches);
/* pk_decode without any device allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  batch->mem must be
 * PK_MEM_DEVICE (frames and outputs already in device memory).  Every device
 * buffer of the call beyond its inputs and outputs (descriptors, enc_proj rows,
 * barrier flags, argmax keys, exchange buffers) comes from one fixed 32 MiB
 * array per device, held until the process ends; a batch that needs more is
 * refused with PK_ERR_UNSUPPORTED (about 16,000 frames x 640 joint units at
 * 64 utterances).  All calls on one device share that array: two calls that
 * overlap in time on the same device race. */
PK_API int pk_decode_noalloc(pk_decoder *dec, const pk_batch *batch);
/* Time, with HIP events on the handle's stream, the last pk_decode's
 * kernels: enc_proj GEMM and the decode loop (milliseconds), and its lockstep
 * iterations; summed over the launches of a call decoded in several.  The
 * times are -1 when the handle's timing was off for that call (the iterations
 * are always given).  The reference times its decode on the host clock
 * (src/parakeet_tdt.cpp:983-1005, decode_ms). */
PK_API int pk_last_timing(pk_decoder *dec, float *enc_proj_ms, float *loop_ms, int32_t *iterations);
/* Record the timing events of pk_last_timing in this handle's calls (on: 1,
 * the default) or not (0).  No counterpart in the reference: the three event
 * records add a few microseconds to every call, which latency-bound callers
 * that never read the times (the drop-in and C++ runtimes) leave out. */
PK_API int pk_decoder_set_timing(pk_decoder *dec, int32_t on);
/* Message of the last failure on this thread ("" if none). */
PK_API const char *pk_last_error(void);
/* Device facts used for launches: compute units, LDS bytes per block, wave size. */
PK_API int pk_device_info(int32_t *n_cu, int32_t *lds_per_block, int32_t *wave_size);

#ifdef __cplusplus
}
#endif
#endif

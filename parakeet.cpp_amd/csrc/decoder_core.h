// decoder_core.h -- the host pieces shared by the standalone C++ decoder API
// (include/parakeet_decoder.h) and the drop-in for parakeet.cpp's decoder
// headers (include/dropin/): the pool of device state slots of one decoder,
// the frame sources of a batch, and one batched decode through the C ABI.
#pragma once

#include <array>
#include <cstdio>
#include <exception>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "parakeet_hip.h"
#include "parakeet_slot.h"

namespace parakeet_hip {

// The device decoder of one runtime and its free state slots.
struct SlotPool {
    pk_decoder *dec = nullptr;
    std::mutex mu;
    std::vector<int> free_slots;
    ~SlotPool();
    int acquire();            // -1 when every slot is leased
    void release(int slot);
};

namespace core {

// Upload a decoder (pk_decoder_create) and give it n_slots free slots.
// Returns the C ABI status (2 for a missing / mis-shaped tensor).
int make_pool(const pk_decoder_desc &desc, int n_slots, std::shared_ptr<SlotPool> &out);

// Encoder frames of a batch: one host window per utterance (packed into one
// upload per call), or rows of an encoder output resident in device memory,
// read in place by the enc_proj kernel.
struct Frames {
    bool device = false;
    std::vector<const float *> host;   // host window of each utterance
    const float *dev = nullptr;        // device encoder output
    std::vector<int64_t> dev_row;      // first row of each utterance in it
    Frames pick(const std::vector<int> &idx, size_t i, size_t j) const;
};

// Frames of a device-resident encoder output [n_rows][d_model], checked
// against its extent.  Returns 0, 1 (d_model mismatch, the reference's rc) or
// 3 (a window outside the rows).
int device_frames(const float *data, int64_t n_rows, int d_model, const std::vector<int64_t> &row_offset,
                  const std::vector<int> &n_frames, int D_expected, const char *who, Frames &fr);

struct BatchOut {
    std::vector<std::vector<int32_t>> tokens;
    std::vector<std::vector<int32_t>> segments;   // EOU boundary token indices
    std::vector<int> steps;
    std::vector<std::array<int32_t, PK_CTRL_N>> ctrl;   // slot control words after the call
};

// Decode utterance u = 0 .. n-1 with the state in slots[u] (every handle
// leased from `pool`); handles marked fresh start from a fresh state inside
// the launch and are marked initialised once their window runs (TDT windows
// with no frames do not run, src/parakeet_tdt.cpp:879).  Batches larger than
// PK_MAX_BATCH are split into several launches.  Returns the C ABI status.
int decode(SlotPool &pool, int D_enc, int max_symbols, const Frames &fr, const std::vector<int> &n_frames,
           const std::vector<SlotHandle *> &slots, const std::vector<int> &tokens_base, bool tdt, BatchOut &out);

// src/sentencepiece_bpe.cpp:9-38: pieces joined (blank / bos / eos / pad ids
// skipped), U+2581 -> ' ', leading spaces trimmed.
std::string detokenize(const std::vector<std::string> &pieces, int32_t blank_id, int32_t bos_id, int32_t eos_id,
                       int32_t pad_id, const std::vector<int32_t> &ids);
// src/parakeet_eou.cpp:359-382: each segment detokenized and trimmed, the
// non-empty ones joined with '\n'.
std::string eou_text(const std::vector<std::string> &pieces, int32_t blank_id, int32_t bos_id, int32_t eos_id,
                     int32_t pad_id, const std::vector<int32_t> &ids, const std::vector<int32_t> &boundaries);

// Runs f() and returns its status; an exception (a state slot that cannot be
// leased, or a failed device copy of a state) becomes PK_ERR_NOMEM with the
// message on stderr, so the decoder entry points return status codes and never
// throw, as the reference's do.
template <class F>
int no_throw(const char *who, F &&f) {
    try {
        return f();
    } catch (const std::exception &e) {
        std::fprintf(stderr, "%s: %s\n", who, e.what());
        return PK_ERR_NOMEM;
    }
}

// 1 where the vocabulary piece is "<...>" (the EOU loop's special pieces).
std::vector<uint8_t> special_pieces(const std::vector<std::string> &pieces);

// ---- decode-state handling shared by both C++ front ends ----
//
// State is a TdtDecodeState / EouDecodeState of either front end (the same
// fields as the reference's, src/parakeet_tdt.h:175-183, src/parakeet_eou.h:
// 53-66, plus the SlotHandle `slot`).

// src/parakeet_tdt.cpp:813-863: a fresh state.  The slot is leased and
// marked fresh; the zero state and the LSTM step on embed[blank] run at the
// start of the state's next decode, inside that decode's launch.
template <class State>
void tdt_fresh(const std::shared_ptr<SlotPool> &pool, State &st) {
    st.slot.reset(pool);
    st.symbols_this_step = 0;
    st.carry_frames = 0;
    st.h_state.clear();
    st.c_state.clear();
    st.pred_out.clear();
    st.initialized = true;
}

// src/parakeet_eou.cpp:206-230, deferred the same way.
template <class State>
void eou_fresh(const std::shared_ptr<SlotPool> &pool, State &st) {
    st.slot.reset(pool);
    st.h_state.clear();
    st.c_state.clear();
    st.pred_out.clear();
    st.last_token = -1;
    st.symbols_this_step = 0;
    st.segment_start_token = 0;
    st.initialized = true;
}

// tdt_decode_window for every state of a batch in one launch: an
// uninitialised state (or one of another runtime) starts fresh, except in a
// window with no frames, which returns before initialising
// (src/parakeet_tdt.cpp:879-881); the control words come back with the outputs.
template <class State>
int tdt_run(const std::shared_ptr<SlotPool> &pool, int D_enc, int max_symbols, const Frames &fr,
            const std::vector<int> &n_frames, const std::vector<State *> &states,
            std::vector<std::vector<int32_t>> &out_tokens, std::vector<int> &out_steps) {
    const size_t n = n_frames.size();
    std::vector<SlotHandle *> slots(n);
    for (size_t u = 0; u < n; ++u) {
        State &st = *states[u];
        if (n_frames[u] > 0 && (!st.initialized || st.slot.pool() != pool)) tdt_fresh(pool, st);
        if (!st.slot.valid() || st.slot.pool() != pool) st.slot.reset(pool);   // a slot id for a window that does not run
        slots[u] = &st.slot;
    }
    BatchOut out;
    if (int rc = decode(*pool, D_enc, max_symbols, fr, n_frames, slots, {}, true, out)) return rc;
    for (size_t u = 0; u < n; ++u) {
        out_tokens[u] = std::move(out.tokens[u]);
        out_steps[u] = out.steps[u];
        if (n_frames[u] <= 0) continue;
        states[u]->symbols_this_step = out.ctrl[u][PK_CTRL_SYM];
        states[u]->carry_frames = out.ctrl[u][PK_CTRL_CARRY];
    }
    return 0;
}

// eou_decode_window for every state of a batch in one launch; tokens_base
// (empty: 0) is each caller's token count before the call, from which
// segment boundaries count (src/parakeet_eou.cpp:293-298).  Boundaries go to
// out_boundaries[u] as token indices.
template <class State>
int eou_run(const std::shared_ptr<SlotPool> &pool, int D_enc, int max_symbols, const Frames &fr,
            const std::vector<int> &n_frames, const std::vector<State *> &states, const std::vector<int> &tokens_base,
            std::vector<std::vector<int32_t>> &out_tokens, std::vector<std::vector<int32_t>> &out_boundaries,
            std::vector<int> &out_steps) {
    const size_t n = n_frames.size();
    std::vector<SlotHandle *> slots(n);
    for (size_t u = 0; u < n; ++u) {
        State &st = *states[u];
        if (!st.initialized || st.slot.pool() != pool) eou_fresh(pool, st);
        slots[u] = &st.slot;
    }
    BatchOut out;
    if (int rc = decode(*pool, D_enc, max_symbols, fr, n_frames, slots, tokens_base, false, out)) return rc;
    for (size_t u = 0; u < n; ++u) {
        out_tokens[u] = std::move(out.tokens[u]);
        out_boundaries[u] = std::move(out.segments[u]);
        out_steps[u] = out.steps[u];
        states[u]->symbols_this_step = out.ctrl[u][PK_CTRL_SYM];
        states[u]->last_token = out.ctrl[u][PK_CTRL_LAST];
        states[u]->segment_start_token = out.ctrl[u][PK_CTRL_SEGSTART];
    }
    return 0;
}

}  // namespace core
}  // namespace parakeet_hip

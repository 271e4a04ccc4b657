// parakeet_tdt.h (drop-in) -- parakeet.cpp's TDT decoder interface on the
// MI355X kernels.
//
// Replaces the reference's src/parakeet_tdt.h: same types, fields, function
// names, signatures and status codes (src/parakeet_tdt.h:51-205), so the
// Engine and CLI call sites (src/parakeet_engine.cpp:155-166, 273-297,
// 407-452, 726-838, 1045-1059; src/main.cpp:745-777) compile unchanged.  The
// model is the reference's own ParakeetCtcModel (src/parakeet_ctc.h, included
// from the reference's source directory), loaded by its load_from_gguf;
// tdt_prepare_runtime reads the TdtWeights tensors once
// (ggml_backend_tensor_get, as src/parakeet_tdt.cpp:78-95 does) and uploads
// them to the device decoder at their stored precision.
//
// Differences, on purpose:
//   - decode state lives in a device slot: TdtDecodeState carries a
//     parakeet_hip::SlotHandle beside the reference's fields (a copy of a
//     state leases a new slot and copies the state); h_state / c_state /
//     pred_out stay empty, as on the reference GPU path;
//   - TdtRuntimeWeights holds the device decoder instead of host f32 copies
//     and ggml graphs, and is movable (the reference's is move-only);
//   - tdt_decode_batch decodes many states in one lockstep launch.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "parakeet_ctc.h"
#include "parakeet_slot.h"

namespace parakeet {

struct TdtRuntimeWeights {
    int H_pred = 640;
    int H_joint = 640;
    int D_enc = 1024;
    int V_plus_1 = 8193;
    int V_out = 8198;
    int L = 2;
    int num_durations = 5;

    const TdtWeights *weights = nullptr;
    std::shared_ptr<parakeet_hip::SlotPool> pool;   // the device decoder and its state slots

    bool ready() const { return weights != nullptr && pool != nullptr; }
};

struct TdtDecodeOptions {
    int max_symbols_per_step = 10;
};

struct TdtDecodeResult {
    std::vector<int32_t> token_ids;
    std::string text;
    int steps = 0;
    double decode_ms = 0.0;
};

struct TdtDecodeState {
    std::vector<float> h_state;
    std::vector<float> c_state;
    std::vector<float> pred_out;

    int symbols_this_step = 0;
    bool initialized = false;
    int carry_frames = 0;

    parakeet_hip::SlotHandle slot;   // the device slot holding h, c, pred and the control words
};

int tdt_prepare_runtime(const ParakeetCtcModel &model, TdtRuntimeWeights &out);

void tdt_init_state(TdtRuntimeWeights &W, int blank_id, TdtDecodeState &state);

int tdt_decode_window(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const TdtDecodeOptions &opts, TdtDecodeState &state,
                      std::vector<int32_t> &out_tokens, int &out_steps);

int tdt_greedy_decode(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const float *encoder_out, int T_enc,
                      int D_enc, const TdtDecodeOptions &opts, TdtDecodeResult &result);

// Addition: tdt_decode_window for many states in one launch (utterance u
// decodes enc[u][0 .. n_frames[u]) with states[u]; tokens go to out_tokens[u]).
int tdt_decode_batch(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const TdtDecodeOptions &opts,
                     const std::vector<TdtDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<int> &out_steps);

}  // namespace parakeet

// parakeet_eou.h (drop-in) -- parakeet.cpp's EOU RNN-T decoder interface on
// the MI355X kernels.
//
// Replaces the reference's src/parakeet_eou.h: same types, fields, function
// names, signatures and status codes (src/parakeet_eou.h:20-107), so the
// Engine's Mode 1 / 2 / 3 call sites (src/parakeet_engine.cpp:162-166,
// 286-297, 438-452, 822-838, 1058) compile unchanged.  See the drop-in
// parakeet_tdt.h for how the runtime and the state differ.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "parakeet_ctc.h"
#include "parakeet_slot.h"
#include "parakeet_tdt.h"

namespace parakeet {

struct EouRuntimeWeights {
    int H_pred = 640;
    int H_joint = 640;
    int D_enc = 512;
    int V_plus_1 = 1027;
    int L = 1;

    int blank_id = 1026;
    int eou_id = 1024;
    int eob_id = 1025;

    std::shared_ptr<parakeet_hip::SlotPool> pool;   // the device decoder and its state slots
};

struct EouDecodeOptions {
    int max_symbols_per_step = 5;
};

struct EouDecodeState {
    std::vector<float> h_state;
    std::vector<float> c_state;
    std::vector<float> pred_out;

    int32_t last_token = -1;
    int symbols_this_step = 0;
    bool initialized = false;

    int segment_start_token = 0;

    parakeet_hip::SlotHandle slot;   // the device slot holding h, c, pred and the control words
};

struct EouSegmentBoundary {
    int token_index = 0;
    bool is_eou_flush = true;
};

struct EouDecodeResult {
    std::vector<int32_t> token_ids;
    std::vector<EouSegmentBoundary> segments;
    std::string text;
    int steps = 0;
    int eou_count = 0;
    double decode_ms = 0.0;
};

int eou_prepare_runtime(const ParakeetCtcModel &model, EouRuntimeWeights &out);

void eou_init_state(const EouRuntimeWeights &W, EouDecodeState &state);

int eou_decode_window(const ParakeetCtcModel &model, const EouRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const EouDecodeOptions &opts, EouDecodeState &state,
                      std::vector<int32_t> &out_tokens, std::vector<EouSegmentBoundary> &out_segments,
                      int &out_steps);

int eou_greedy_decode(const ParakeetCtcModel &model, const EouRuntimeWeights &W, const float *encoder_out,
                      int T_enc, int D_enc, const EouDecodeOptions &opts, EouDecodeResult &result);

// Addition: eou_decode_window for many states in one launch.
int eou_decode_batch(const ParakeetCtcModel &model, const EouRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const EouDecodeOptions &opts,
                     const std::vector<EouDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps);

}  // namespace parakeet

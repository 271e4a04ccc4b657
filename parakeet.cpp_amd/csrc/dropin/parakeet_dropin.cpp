// parakeet_dropin.cpp -- the drop-in decoder interface (include/dropin/
// parakeet_tdt.h, parakeet_eou.h) over the MI355X kernels: parakeet.cpp's
// ParakeetCtcModel in, the shared host core (decoder_core.h) and the C ABI
// underneath.  Built inside parakeet.cpp's build with dropin/
// ggml_tensor_bytes.cpp, in place of src/parakeet_tdt.cpp and
// src/parakeet_eou.cpp.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <stdexcept>

#include "decoder_core.h"
#include "dropin_tensor.h"
#include "parakeet_eou.h"
#include "parakeet_tdt.h"

namespace parakeet {

namespace {

namespace core = parakeet_hip::core;

// State slots of a drop-in runtime: the reference's prepare functions take
// no slot count, so every runtime holds this many concurrent states.
constexpr int kDropinSlots = 1024;

// The device decoder of a TdtWeights / EouWeights set (bound at
// src/parakeet_ctc.cpp:603-619, 648-665) with the metadata the reference reads
// at src/parakeet_ctc.cpp:418-458.  Tensor bytes are read once, here.
template <class Weights>
int make_pool(const ParakeetCtcModel &m, const Weights &w, bool eou, std::shared_ptr<parakeet_hip::SlotPool> &out) {
    pk_decoder_desc d{};
    const EncoderConfig &c = m.encoder_cfg;
    d.kind = eou ? PK_KIND_EOU : PK_KIND_TDT;
    d.pred_hidden = eou ? c.eou_pred_hidden : c.tdt_pred_hidden;
    d.pred_rnn_layers = eou ? c.eou_pred_rnn_layers : c.tdt_pred_rnn_layers;
    d.joint_hidden = eou ? c.eou_joint_hidden : c.tdt_joint_hidden;
    d.d_enc = c.d_model;
    d.vocab_size = m.vocab_size;
    d.blank_id = m.blank_id;
    d.num_durations = eou ? 0 : c.tdt_num_durations;
    d.n_duration_values = eou ? 0 : (int32_t)std::min<size_t>(m.tdt_durations.size(), PK_MAX_DURATIONS);
    for (int i = 0; i < d.n_duration_values; ++i) d.durations[i] = m.tdt_durations[i];
    d.eou_id = m.eou_id;
    d.eob_id = m.eob_id;
    const std::vector<uint8_t> special = core::special_pieces(m.vocab.pieces);
    d.special = special.empty() ? nullptr : special.data();
    d.n_special = (int32_t)special.size();
    if (d.pred_rnn_layers > PK_MAX_LAYERS || (int)w.lstm.size() < d.pred_rnn_layers) return 2;
    std::vector<std::vector<uint8_t>> bytes(7 + 4 * (size_t)d.pred_rnn_layers);   // one per tensor below
    size_t k = 0;
    int rc = 0;
    auto take = [&](const ggml_tensor *t, pk_tensor &dst) {
        if (rc == 0) rc = parakeet_hip::dropin::tensor_bytes(t, &dst, &bytes[k]);
        ++k;
    };
    take(w.predict_embed, d.embed);
    for (int l = 0; l < d.pred_rnn_layers; ++l) {
        take(w.lstm[l].w_ih, d.w_ih[l]);
        take(w.lstm[l].w_hh, d.w_hh[l]);
        take(w.lstm[l].b_ih, d.b_ih[l]);
        take(w.lstm[l].b_hh, d.b_hh[l]);
    }
    take(w.joint_enc_w, d.joint_enc_w);
    take(w.joint_enc_b, d.joint_enc_b);
    take(w.joint_pred_w, d.joint_pred_w);
    take(w.joint_pred_b, d.joint_pred_b);
    take(w.joint_out_w, d.joint_out_w);
    take(w.joint_out_b, d.joint_out_b);
    if (rc) return rc;
    return core::make_pool(d, kDropinSlots, out);
}

}  // namespace

// ------------------------------------------------------------------ TDT

int tdt_prepare_runtime(const ParakeetCtcModel &model, TdtRuntimeWeights &W) {
    W = TdtRuntimeWeights{};
    if (model.model_type != ParakeetModelType::TDT) return 2;
    const EncoderConfig &c = model.encoder_cfg;
    W.H_pred = c.tdt_pred_hidden;
    W.H_joint = c.tdt_joint_hidden;
    W.D_enc = c.d_model;
    W.L = c.tdt_pred_rnn_layers;
    W.num_durations = c.tdt_num_durations;
    W.V_plus_1 = model.vocab_size + 1;
    W.V_out = W.V_plus_1 + W.num_durations;
    if (int rc = make_pool(model, model.tdt, false, W.pool)) return rc;
    W.weights = &model.tdt;
    return 0;
}

void tdt_init_state(TdtRuntimeWeights &W, int, TdtDecodeState &state) {
    // a state that gets no slot stays uninitialised; its next window tries again and returns a status
    if (core::no_throw("tdt_init_state", [&] { core::tdt_fresh(W.pool, state); return 0; })) state.initialized = false;
}

int tdt_decode_batch(const ParakeetCtcModel &, TdtRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const TdtDecodeOptions &opts,
                     const std::vector<TdtDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<int> &out_steps) {
    const int n = (int)enc.size();
    out_steps.assign(n, 0);
    out_tokens.assign(n, {});
    if (D_enc != W.D_enc) {   // src/parakeet_tdt.cpp:874-877
        std::fprintf(stderr, "tdt_decode_window: encoder d_model mismatch (%d vs %d)\n", D_enc, W.D_enc);
        return 1;
    }
    if ((int)n_frames.size() != n || (int)states.size() != n || !W.pool) return 3;
    core::Frames fr;
    fr.host = enc;
    return core::no_throw("tdt_decode_window", [&] {
        return core::tdt_run(W.pool, D_enc, opts.max_symbols_per_step, fr, n_frames, states, out_tokens, out_steps);
    });
}

int tdt_decode_window(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const TdtDecodeOptions &opts, TdtDecodeState &state,
                      std::vector<int32_t> &out_tokens, int &out_steps) {
    std::vector<std::vector<int32_t>> toks;
    std::vector<int> steps;
    const int rc = tdt_decode_batch(model, W, {encoder_out_window}, {n_frames}, D_enc, opts, {&state}, toks, steps);
    out_steps = steps.empty() ? 0 : steps[0];
    if (rc == 0) out_tokens.insert(out_tokens.end(), toks[0].begin(), toks[0].end());
    return rc;
}

int tdt_greedy_decode(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const float *encoder_out, int T_enc,
                      int D_enc, const TdtDecodeOptions &opts, TdtDecodeResult &result) {
    const auto t0 = std::chrono::steady_clock::now();
    TdtDecodeState state;
    result.token_ids.clear();
    result.token_ids.reserve(T_enc);
    if (int rc = tdt_decode_window(model, W, encoder_out, T_enc, D_enc, opts, state, result.token_ids, result.steps))
        return rc;
    const BpeVocab &v = model.vocab;
    result.text = core::detokenize(v.pieces, v.blank_id, v.bos_id, v.eos_id, v.pad_id, result.token_ids);
    result.decode_ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    return 0;
}

// ------------------------------------------------------------------ EOU

int eou_prepare_runtime(const ParakeetCtcModel &model, EouRuntimeWeights &W) {
    if (model.model_type != ParakeetModelType::EOU) return 1;   // src/parakeet_eou.cpp:173-175
    const EncoderConfig &c = model.encoder_cfg;
    W = EouRuntimeWeights{};
    W.H_pred = c.eou_pred_hidden;
    W.H_joint = c.eou_joint_hidden;
    W.D_enc = c.d_model;
    W.L = c.eou_pred_rnn_layers;
    W.V_plus_1 = model.vocab_size + 1;
    W.blank_id = model.blank_id;
    W.eou_id = model.eou_id >= 0 ? model.eou_id : model.vocab_size - 2;   // src/parakeet_eou.cpp:182-183
    W.eob_id = model.eob_id >= 0 ? model.eob_id : model.vocab_size - 1;
    return make_pool(model, model.eou, true, W.pool);
}

void eou_init_state(const EouRuntimeWeights &W, EouDecodeState &state) {
    if (core::no_throw("eou_init_state", [&] { core::eou_fresh(W.pool, state); return 0; })) state.initialized = false;
}

namespace {

int eou_batch(const EouRuntimeWeights &W, const std::vector<const float *> &enc, const std::vector<int> &n_frames,
              int D_enc, const EouDecodeOptions &opts, const std::vector<EouDecodeState *> &states,
              const std::vector<int> &tokens_base, std::vector<std::vector<int32_t>> &out_tokens,
              std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps) {
    core::Frames fr;
    fr.host = enc;
    std::vector<std::vector<int32_t>> bounds(n_frames.size());
    if (int rc = core::no_throw("eou_decode_window", [&] {
            return core::eou_run(W.pool, D_enc, opts.max_symbols_per_step, fr, n_frames, states, tokens_base,
                                 out_tokens, bounds, out_steps);
        }))
        return rc;
    for (size_t u = 0; u < n_frames.size(); ++u)
        for (int32_t b : bounds[u]) out_segments[u].push_back(EouSegmentBoundary{b, true});
    return 0;
}

}  // namespace

int eou_decode_batch(const ParakeetCtcModel &, const EouRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const EouDecodeOptions &opts,
                     const std::vector<EouDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps) {
    const int n = (int)enc.size();
    out_tokens.assign(n, {});
    out_segments.assign(n, {});
    out_steps.assign(n, 0);
    if (D_enc != W.D_enc) {
        std::fprintf(stderr, "eou_decode_window: encoder d_model mismatch (%d vs %d)\n", D_enc, W.D_enc);
        return 1;
    }
    if ((int)n_frames.size() != n || (int)states.size() != n || !W.pool) return 3;
    return eou_batch(W, enc, n_frames, D_enc, opts, states, {}, out_tokens, out_segments, out_steps);
}

int eou_decode_window(const ParakeetCtcModel &, const EouRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const EouDecodeOptions &opts, EouDecodeState &state,
                      std::vector<int32_t> &out_tokens, std::vector<EouSegmentBoundary> &out_segments,
                      int &out_steps) {
    if (D_enc != W.D_enc) {   // src/parakeet_eou.cpp:241-245
        std::fprintf(stderr, "eou_decode_window: encoder d_model mismatch (%d vs %d)\n", D_enc, W.D_enc);
        return 1;
    }
    if (!W.pool) return 3;
    // segment indices count from the caller's token vector (src/parakeet_eou.cpp:293-298)
    std::vector<std::vector<int32_t>> tv(1);
    std::vector<std::vector<EouSegmentBoundary>> sv(1);
    std::vector<int> steps(1, 0);
    if (int rc = eou_batch(W, {encoder_out_window}, {std::max(0, n_frames)}, D_enc, opts, {&state},
                           {(int)out_tokens.size()}, tv, sv, steps))
        return rc;
    out_steps = steps[0];
    out_tokens.insert(out_tokens.end(), tv[0].begin(), tv[0].end());
    out_segments.insert(out_segments.end(), sv[0].begin(), sv[0].end());
    return 0;
}

int eou_greedy_decode(const ParakeetCtcModel &model, const EouRuntimeWeights &W, const float *encoder_out,
                      int T_enc, int D_enc, const EouDecodeOptions &opts, EouDecodeResult &result) {
    const auto t0 = std::chrono::steady_clock::now();
    EouDecodeState state;
    result.token_ids.clear();
    result.segments.clear();
    result.token_ids.reserve(T_enc);
    if (int rc = eou_decode_window(model, W, encoder_out, T_enc, D_enc, opts, state, result.token_ids,
                                   result.segments, result.steps))
        return rc;
    result.eou_count = (int)result.segments.size();
    std::vector<int32_t> bounds;
    for (const auto &b : result.segments) bounds.push_back(b.token_index);
    const BpeVocab &v = model.vocab;
    result.text = core::eou_text(v.pieces, v.blank_id, v.bos_id, v.eos_id, v.pad_id, result.token_ids, bounds);
    result.decode_ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    return 0;
}

}  // namespace parakeet

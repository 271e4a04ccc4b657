// parakeet_decoder.cpp -- the standalone reference-shaped C++ decoder API on
// top of the C ABI (parakeet_hip.h).  See include/parakeet_decoder.h.
#include "parakeet_decoder.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <stdexcept>

#include "decoder_core.h"
#include "gguf_reader.h"
#include "parakeet_hip.h"

namespace parakeet_hip {

struct DecoderModel::Impl {
    gguf::File file;
};

namespace {

using core::BatchOut;
using core::Frames;

const char *prefix(ParakeetModelType t) { return t == ParakeetModelType::EOU ? "eou." : "tdt."; }

pk_tensor tensor_of(const DecoderModel &m, const std::string &name) {
    pk_tensor t{};
    const gguf::Tensor *g = m.impl ? m.impl->file.tensor(name) : nullptr;
    if (!g) return t;
    t.data = g->data;
    t.type = (int32_t)g->type;
    t.ne0 = g->ne.empty() ? 0 : g->ne[0];
    t.ne1 = g->ne.size() > 1 ? g->ne[1] : 1;
    return t;
}

// Decoder description from the loaded model (the tensors bound at
// src/parakeet_ctc.cpp:603-665 and the metadata read at :418-458).
int make_pool(const DecoderModel &m, int n_slots, std::shared_ptr<SlotPool> &out) {
    pk_decoder_desc d{};
    const bool eou = m.model_type == ParakeetModelType::EOU;
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
    const std::string p = prefix(m.model_type);
    d.embed = tensor_of(m, p + "predict.embed.weight");
    if (d.pred_rnn_layers > PK_MAX_LAYERS) return 2;
    for (int l = 0; l < d.pred_rnn_layers; ++l) {
        const std::string pl = p + "predict.lstm." + std::to_string(l) + ".";
        d.w_ih[l] = tensor_of(m, pl + "w_ih");
        d.w_hh[l] = tensor_of(m, pl + "w_hh");
        d.b_ih[l] = tensor_of(m, pl + "b_ih");
        d.b_hh[l] = tensor_of(m, pl + "b_hh");
    }
    d.joint_enc_w = tensor_of(m, p + "joint.enc.weight");
    d.joint_enc_b = tensor_of(m, p + "joint.enc.bias");
    d.joint_pred_w = tensor_of(m, p + "joint.pred.weight");
    d.joint_pred_b = tensor_of(m, p + "joint.pred.bias");
    d.joint_out_w = tensor_of(m, p + "joint.out.weight");
    d.joint_out_b = tensor_of(m, p + "joint.out.bias");
    return core::make_pool(d, n_slots, out);
}

int device_frames(const DeviceEncoderOutput &enc, const std::vector<int64_t> &row_offset,
                  const std::vector<int> &n_frames, int D_expected, const char *who, Frames &fr) {
    return core::device_frames(enc.data, enc.n_rows, enc.d_model, row_offset, n_frames, D_expected, who, fr);
}

}  // namespace

// ------------------------------------------------------------------ loading

int load_from_gguf(const std::string &gguf_path, DecoderModel &out, int, int, bool verbose) {
    auto impl = std::make_shared<DecoderModel::Impl>();
    std::string err;
    if (impl->file.open(gguf_path, err)) {
        std::fprintf(stderr, "gguf: %s\n", err.c_str());
        return 1;
    }
    const gguf::File &g = impl->file;
    if (g.get_str("general.architecture", "") != "parakeet-ctc") {
        std::fprintf(stderr, "gguf: expected arch=parakeet-ctc\n");
        return 2;
    }
    out = DecoderModel{};
    out.encoder_cfg.d_model = (int)g.get_u32("parakeet.encoder.d_model", 1024);
    out.encoder_cfg.subsampling_factor = (int)g.get_u32("parakeet.encoder.subsampling_factor", 8);
    out.mel_cfg.sample_rate = (int)g.get_u32("parakeet.preproc.sample_rate", 16000);
    out.mel_cfg.hop_length = (int)g.get_u32("parakeet.preproc.hop_length", 160);
    const std::string mt = g.get_str("parakeet.model.type", "ctc");
    out.model_type = mt == "tdt" ? ParakeetModelType::TDT
                   : mt == "eou" ? ParakeetModelType::EOU
                   : mt == "sortformer" ? ParakeetModelType::SORTFORMER : ParakeetModelType::CTC;
    EncoderConfig &c = out.encoder_cfg;
    if (out.model_type == ParakeetModelType::TDT) {
        c.tdt_pred_hidden = (int)g.get_u32("parakeet.tdt.pred_hidden", 640);
        c.tdt_pred_rnn_layers = (int)g.get_u32("parakeet.tdt.pred_rnn_layers", 2);
        c.tdt_joint_hidden = (int)g.get_u32("parakeet.tdt.joint_hidden", 640);
        c.tdt_num_durations = (int)g.get_u32("parakeet.tdt.num_durations", 5);
        out.vocab_size = (int32_t)g.get_u32("parakeet.tdt.vocab_size", 8192);
        out.blank_id = (int32_t)g.get_u32("parakeet.tdt.blank_id", (uint32_t)out.vocab_size);
        if (const gguf::Value *v = g.find("parakeet.tdt.durations"))
            out.tdt_durations.assign(v->arr_i.begin(), v->arr_i.end());
        else
            out.tdt_durations = {0, 1, 2, 3, 4};
    } else if (out.model_type == ParakeetModelType::EOU) {
        c.eou_pred_hidden = (int)g.get_u32("parakeet.eou.pred_hidden", 640);
        c.eou_pred_rnn_layers = (int)g.get_u32("parakeet.eou.pred_rnn_layers", 1);
        c.eou_joint_hidden = (int)g.get_u32("parakeet.eou.joint_hidden", 640);
        c.eou_max_symbols_per_step = (int)g.get_u32("parakeet.eou.max_symbols_per_step", 5);
        out.vocab_size = (int32_t)g.get_u32("parakeet.eou.vocab_size", 1026);
        out.blank_id = (int32_t)g.get_u32("parakeet.eou.blank_id", (uint32_t)out.vocab_size);
        out.eou_id = g.find("parakeet.eou.eou_id") ? g.get_i32("parakeet.eou.eou_id", -1) : -1;
        out.eob_id = g.find("parakeet.eou.eob_id") ? g.get_i32("parakeet.eou.eob_id", -1) : -1;
    }
    // sizes the decoder can hold; a corrupt file asking for more is refused here,
    // before anything is sized from it
    {
        const bool tdt = out.model_type == ParakeetModelType::TDT;
        const int L = tdt ? c.tdt_pred_rnn_layers : c.eou_pred_rnn_layers;
        const int H = tdt ? c.tdt_pred_hidden : c.eou_pred_hidden;
        const int J = tdt ? c.tdt_joint_hidden : c.eou_joint_hidden;
        const bool dec = tdt || out.model_type == ParakeetModelType::EOU;
        if (dec && (L < 1 || L > PK_MAX_LAYERS || H < 1 || H > (1 << 16) || J < 1 || J > (1 << 16) ||
                    c.d_model < 1 || c.d_model > (1 << 16) || out.vocab_size < 1 || out.vocab_size > (1 << 20) ||
                    (tdt && (c.tdt_num_durations < 0 || c.tdt_num_durations > PK_MAX_DURATIONS ||
                             out.tdt_durations.size() > (size_t)PK_MAX_DURATIONS)))) {
            std::fprintf(stderr, "gguf: decoder sizes out of range\n");
            return 2;
        }
    }
    out.vocab.blank_id = out.blank_id;
    if (const gguf::Value *v = g.find("tokenizer.ggml.tokens")) out.vocab.pieces = v->arr_s;
    out.vocab.unk_id = (int32_t)g.get_u32("tokenizer.ggml.unk_token_id", (uint32_t)-1);
    out.vocab.bos_id = (int32_t)g.get_u32("tokenizer.ggml.bos_token_id", (uint32_t)-1);
    out.vocab.eos_id = (int32_t)g.get_u32("tokenizer.ggml.eos_token_id", (uint32_t)-1);
    out.vocab.pad_id = (int32_t)g.get_u32("tokenizer.ggml.pad_token_id", (uint32_t)-1);
    out.impl = impl;
    if (out.model_type == ParakeetModelType::TDT || out.model_type == ParakeetModelType::EOU) {
        const std::string p = prefix(out.model_type);
        const int L = out.model_type == ParakeetModelType::TDT ? c.tdt_pred_rnn_layers : c.eou_pred_rnn_layers;
        std::vector<std::string> need = {p + "predict.embed.weight", p + "joint.enc.weight", p + "joint.enc.bias",
                                         p + "joint.pred.weight", p + "joint.pred.bias", p + "joint.out.weight",
                                         p + "joint.out.bias"};
        for (int l = 0; l < L; ++l)
            for (const char *n : {"w_ih", "w_hh", "b_ih", "b_hh"})
                need.push_back(p + "predict.lstm." + std::to_string(l) + "." + n);
        for (const auto &n : need)
            if (!g.tensor(n)) {
                std::fprintf(stderr, "gguf: missing tensor %s\n", n.c_str());
                return 2;
            }
    }
    if (verbose)
        std::fprintf(stderr, "gguf: %s type=%s vocab=%d blank=%d\n", gguf_path.c_str(), mt.c_str(), out.vocab_size,
                     out.blank_id);
    return 0;
}

std::string detokenize(const BpeVocab &vocab, const std::vector<int32_t> &ids) {
    return core::detokenize(vocab.pieces, vocab.blank_id, vocab.bos_id, vocab.eos_id, vocab.pad_id, ids);
}

// ------------------------------------------------------------------ TDT

int tdt_prepare_runtime(const DecoderModel &model, TdtRuntimeWeights &W, int n_slots) {
    W = TdtRuntimeWeights{};
    if (model.model_type != ParakeetModelType::TDT || !model.impl) return 2;
    const EncoderConfig &c = model.encoder_cfg;
    W.H_pred = c.tdt_pred_hidden;
    W.H_joint = c.tdt_joint_hidden;
    W.D_enc = c.d_model;
    W.L = c.tdt_pred_rnn_layers;
    W.num_durations = c.tdt_num_durations;
    W.V_plus_1 = model.vocab_size + 1;
    W.V_out = W.V_plus_1 + W.num_durations;
    W.weights_model = &model;
    return make_pool(model, n_slots, W.pool);
}

// src/parakeet_tdt.cpp:813-863 (see core::tdt_fresh: the device work runs in
// the state's next decode launch).
void tdt_init_state(TdtRuntimeWeights &W, int, TdtDecodeState &state) {
    // a state that gets no slot stays uninitialised; its next window tries again and returns a status
    if (core::no_throw("tdt_init_state", [&] { core::tdt_fresh(W.pool, state); return 0; })) state.initialized = false;
}

namespace {

int tdt_batch(TdtRuntimeWeights &W, const Frames &fr, const std::vector<int> &n_frames, int D_enc,
              const TdtDecodeOptions &opts, const std::vector<TdtDecodeState *> &states,
              std::vector<std::vector<int32_t>> &out_tokens, std::vector<int> &out_steps) {
    return core::no_throw("tdt_decode_window", [&] {
        return core::tdt_run(W.pool, D_enc, opts.max_symbols_per_step, fr, n_frames, states, out_tokens, out_steps);
    });
}

}  // namespace

int tdt_decode_batch(const DecoderModel &, TdtRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const TdtDecodeOptions &opts,
                     const std::vector<TdtDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<int> &out_steps) {
    const int n = (int)enc.size();
    out_steps.assign(n, 0);
    out_tokens.assign(n, {});
    if (D_enc != W.D_enc) {
        std::fprintf(stderr, "tdt_decode_window: encoder d_model mismatch (%d vs %d)\n", D_enc, W.D_enc);
        return 1;
    }
    if ((int)n_frames.size() != n || (int)states.size() != n) return 3;
    Frames fr;
    fr.host = enc;
    return tdt_batch(W, fr, n_frames, D_enc, opts, states, out_tokens, out_steps);
}

int tdt_decode_batch_device(const DecoderModel &, TdtRuntimeWeights &W, const DeviceEncoderOutput &enc,
                            const std::vector<int64_t> &row_offset, const std::vector<int> &n_frames,
                            const TdtDecodeOptions &opts, const std::vector<TdtDecodeState *> &states,
                            std::vector<std::vector<int32_t>> &out_tokens, std::vector<int> &out_steps) {
    const int n = (int)n_frames.size();
    out_steps.assign(n, 0);
    out_tokens.assign(n, {});
    if ((int)states.size() != n) return 3;
    Frames fr;
    if (int rc = device_frames(enc, row_offset, n_frames, W.D_enc, "tdt_decode_batch_device", fr)) return rc;
    return tdt_batch(W, fr, n_frames, W.D_enc, opts, states, out_tokens, out_steps);
}

int tdt_decode_window(const DecoderModel &model, TdtRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const TdtDecodeOptions &opts, TdtDecodeState &state,
                      std::vector<int32_t> &out_tokens, int &out_steps) {
    std::vector<std::vector<int32_t>> toks;
    std::vector<int> steps;
    const int rc = tdt_decode_batch(model, W, {encoder_out_window}, {n_frames}, D_enc, opts, {&state}, toks, steps);
    out_steps = steps.empty() ? 0 : steps[0];
    if (rc == 0) out_tokens.insert(out_tokens.end(), toks[0].begin(), toks[0].end());
    return rc;
}

int tdt_greedy_decode(const DecoderModel &model, TdtRuntimeWeights &W, const float *encoder_out, int T_enc,
                      int D_enc, const TdtDecodeOptions &opts, TdtDecodeResult &result) {
    const auto t0 = std::chrono::steady_clock::now();
    TdtDecodeState state;
    result.token_ids.clear();
    result.token_ids.reserve(T_enc);
    if (int rc = tdt_decode_window(model, W, encoder_out, T_enc, D_enc, opts, state, result.token_ids, result.steps))
        return rc;
    result.text = detokenize(model.vocab, result.token_ids);
    result.decode_ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    return 0;
}

// ------------------------------------------------------------------ EOU

int eou_prepare_runtime(const DecoderModel &model, EouRuntimeWeights &W, int n_slots) {
    if (model.model_type != ParakeetModelType::EOU) return 1;   // src/parakeet_eou.cpp:173-175
    const EncoderConfig &c = model.encoder_cfg;
    W = EouRuntimeWeights{};
    W.H_pred = c.eou_pred_hidden;
    W.H_joint = c.eou_joint_hidden;
    W.D_enc = c.d_model;
    W.L = c.eou_pred_rnn_layers;
    W.V_plus_1 = model.vocab_size + 1;
    W.blank_id = model.blank_id;
    W.eou_id = model.eou_id >= 0 ? model.eou_id : model.vocab_size - 2;
    W.eob_id = model.eob_id >= 0 ? model.eob_id : model.vocab_size - 1;
    return make_pool(model, n_slots, W.pool);
}

// src/parakeet_eou.cpp:206-230 (see core::eou_fresh).
void eou_init_state(const EouRuntimeWeights &W, EouDecodeState &state) {
    if (core::no_throw("eou_init_state", [&] { core::eou_fresh(W.pool, state); return 0; })) state.initialized = false;
}

namespace {

int eou_batch(const EouRuntimeWeights &W, const Frames &fr, const std::vector<int> &n_frames, int D_enc,
              const EouDecodeOptions &opts, const std::vector<EouDecodeState *> &states,
              const std::vector<int> &tokens_base, std::vector<std::vector<int32_t>> &out_tokens,
              std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps) {
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

int eou_decode_batch(const DecoderModel &, const EouRuntimeWeights &W, const std::vector<const float *> &enc,
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
    if ((int)n_frames.size() != n || (int)states.size() != n) return 3;
    Frames fr;
    fr.host = enc;
    return eou_batch(W, fr, n_frames, D_enc, opts, states, {}, out_tokens, out_segments, out_steps);
}

int eou_decode_batch_device(const DecoderModel &, const EouRuntimeWeights &W, const DeviceEncoderOutput &enc,
                            const std::vector<int64_t> &row_offset, const std::vector<int> &n_frames,
                            const EouDecodeOptions &opts, const std::vector<EouDecodeState *> &states,
                            std::vector<std::vector<int32_t>> &out_tokens,
                            std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps) {
    const int n = (int)n_frames.size();
    out_tokens.assign(n, {});
    out_segments.assign(n, {});
    out_steps.assign(n, 0);
    if ((int)states.size() != n) return 3;
    Frames fr;
    if (int rc = device_frames(enc, row_offset, n_frames, W.D_enc, "eou_decode_batch_device", fr)) return rc;
    return eou_batch(W, fr, n_frames, W.D_enc, opts, states, {}, out_tokens, out_segments, out_steps);
}

int eou_decode_window(const DecoderModel &, const EouRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const EouDecodeOptions &opts, EouDecodeState &state,
                      std::vector<int32_t> &out_tokens, std::vector<EouSegmentBoundary> &out_segments,
                      int &out_steps) {
    if (D_enc != W.D_enc) {
        std::fprintf(stderr, "eou_decode_window: encoder d_model mismatch (%d vs %d)\n", D_enc, W.D_enc);
        return 1;
    }
    // segment indices count from the caller's token vector (src/parakeet_eou.cpp:293-298)
    std::vector<std::vector<int32_t>> tv;
    std::vector<std::vector<EouSegmentBoundary>> sv(1);
    std::vector<int> steps(1, 0);
    tv.assign(1, {});
    Frames fr;
    fr.host = {encoder_out_window};
    if (int rc = eou_batch(W, fr, {std::max(0, n_frames)}, D_enc, opts, {&state}, {(int)out_tokens.size()}, tv, sv,
                           steps))
        return rc;
    out_steps = steps[0];
    out_tokens.insert(out_tokens.end(), tv[0].begin(), tv[0].end());
    out_segments.insert(out_segments.end(), sv[0].begin(), sv[0].end());
    return 0;
}

int eou_greedy_decode(const DecoderModel &model, const EouRuntimeWeights &W, const float *encoder_out, int T_enc,
                      int D_enc, const EouDecodeOptions &opts, EouDecodeResult &result) {
    const auto t0 = std::chrono::steady_clock::now();
    EouDecodeState state;
    result.token_ids.clear();
    result.segments.clear();
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

// ------------------------------------------------------------------ Engine

struct Engine::Impl {
    EngineOptions opts;
    DecoderModel model;
    TdtRuntimeWeights tdt;
    EouRuntimeWeights eou;
};

Engine::Engine(const EngineOptions &opts) : pimpl_(std::make_unique<Impl>()) {
    pimpl_->opts = opts;
    if (int rc = load_from_gguf(opts.model_gguf_path, pimpl_->model))
        throw std::runtime_error("parakeet::Engine: failed to load GGUF '" + opts.model_gguf_path +
                                 "' (rc=" + std::to_string(rc) + ")");
    if (pimpl_->model.model_type == ParakeetModelType::TDT) {
        if (tdt_prepare_runtime(pimpl_->model, pimpl_->tdt, opts.n_slots) != 0)
            throw std::runtime_error("Engine: tdt_prepare_runtime failed");
    } else if (pimpl_->model.model_type == ParakeetModelType::EOU) {
        if (eou_prepare_runtime(pimpl_->model, pimpl_->eou, opts.n_slots) != 0)
            throw std::runtime_error("Engine: eou_prepare_runtime failed");
    } else {
        throw std::runtime_error("parakeet::Engine: loaded GGUF has no transducer decoder");
    }
}

Engine::~Engine() = default;

const DecoderModel &Engine::model() const { return pimpl_->model; }

EngineResult Engine::transcribe_features(const float *enc, int T_enc, int D_enc) {
    return transcribe_features_batch({enc}, {T_enc}, D_enc)[0];
}

namespace {

// The Engine's batch decode over either frame source: fresh states, one result per utterance.
std::vector<EngineResult> engine_decode(Engine::Impl &E, const Frames &fr, const std::vector<int> &T_enc, int D_enc) {
    const auto t0 = std::chrono::steady_clock::now();
    const int n = (int)T_enc.size();
    std::vector<EngineResult> out(n);
    const DecoderModel &m = E.model;
    if (m.model_type == ParakeetModelType::TDT) {
        std::vector<TdtDecodeState> states(n);
        std::vector<TdtDecodeState *> sp(n);
        for (int u = 0; u < n; ++u) sp[u] = &states[u];
        std::vector<std::vector<int32_t>> toks(n);
        std::vector<int> steps(n, 0);
        int rc = D_enc != E.tdt.D_enc ? 1 : 0;
        if (rc == 0) rc = tdt_batch(E.tdt, fr, T_enc, D_enc, TdtDecodeOptions{}, sp, toks, steps);
        if (rc) throw std::runtime_error("parakeet::Engine: tdt decode failed (rc=" + std::to_string(rc) + ")");
        for (int u = 0; u < n; ++u) {
            out[u].token_ids = std::move(toks[u]);
            out[u].text = detokenize(m.vocab, out[u].token_ids);
            out[u].steps = steps[u];
        }
    } else {
        EouDecodeOptions o;
        o.max_symbols_per_step = m.encoder_cfg.eou_max_symbols_per_step;
        std::vector<EouDecodeState> states(n);
        std::vector<EouDecodeState *> sp(n);
        for (int u = 0; u < n; ++u) sp[u] = &states[u];
        std::vector<std::vector<int32_t>> toks(n);
        std::vector<std::vector<EouSegmentBoundary>> segs(n);
        std::vector<int> steps(n, 0);
        int rc = D_enc != E.eou.D_enc ? 1 : 0;
        if (rc == 0) rc = eou_batch(E.eou, fr, T_enc, D_enc, o, sp, {}, toks, segs, steps);
        if (rc) throw std::runtime_error("parakeet::Engine: eou decode failed (rc=" + std::to_string(rc) + ")");
        for (int u = 0; u < n; ++u) {
            out[u].token_ids = std::move(toks[u]);
            out[u].steps = steps[u];
            std::vector<int32_t> bounds;
            for (const auto &b : segs[u]) bounds.push_back(b.token_index);
            const BpeVocab &v = m.vocab;
            out[u].text = core::eou_text(v.pieces, v.blank_id, v.bos_id, v.eos_id, v.pad_id, out[u].token_ids, bounds);
        }
    }
    const double ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    for (int u = 0; u < n; ++u) {
        out[u].decode_ms = ms;
        out[u].encoder_frames = T_enc[u];
    }
    return out;
}

}  // namespace

std::vector<EngineResult> Engine::transcribe_features_batch(const std::vector<const float *> &enc,
                                                            const std::vector<int> &T_enc, int D_enc) {
    if (enc.size() != T_enc.size())
        throw std::invalid_argument("parakeet::Engine::transcribe_features_batch: size mismatch");
    Frames fr;
    fr.host = enc;
    return engine_decode(*pimpl_, fr, T_enc, D_enc);
}

std::vector<EngineResult> Engine::transcribe_device_batch(const DeviceEncoderOutput &enc,
                                                          const std::vector<int64_t> &row_offset,
                                                          const std::vector<int> &T_enc) {
    const DecoderModel &m = pimpl_->model;
    const int D = m.model_type == ParakeetModelType::TDT ? pimpl_->tdt.D_enc : pimpl_->eou.D_enc;
    Frames fr;
    if (int rc = device_frames(enc, row_offset, T_enc, D, "parakeet_hip::Engine::transcribe_device_batch", fr))
        throw std::runtime_error("parakeet::Engine: device frames rejected (rc=" + std::to_string(rc) + ")");
    return engine_decode(*pimpl_, fr, T_enc, D);
}

// ------------------------------------------------------------------ streaming over features

double encoder_frame_stride_ms(const DecoderModel &m) {
    const int sub = m.encoder_cfg.subsampling_factor > 0 ? m.encoder_cfg.subsampling_factor : 8;
    const int sr = m.mel_cfg.sample_rate > 0 ? m.mel_cfg.sample_rate : 16000;
    return 1000.0 * (double)(m.mel_cfg.hop_length * sub) / (double)sr;
}

struct FeatureStreamSession::Impl {
    Engine::Impl *engine = nullptr;
    FeatureStreamOptions opts;
    StreamingCallback on_segment;
    double stride_ms = 80.0;
    TdtDecodeState tdt;
    EouDecodeState eou;
    std::vector<int32_t> cum_ids;     // every token of the session so far
    std::string cum_text;             // detokenize(cum_ids)
    long long emitted_frames = 0;
    int chunk_index = 0;
    int steps = 0;
    bool cancelled = false, finalized = false;

    // Segment and events of one decoded chunk (src/parakeet_engine.cpp:838-864).
    void emit(const std::vector<int32_t> &win_tokens, int n_boundaries, int n_frames, double decode_ms);
};

FeatureStreamSession::FeatureStreamSession(std::unique_ptr<Impl> impl) : pimpl_(std::move(impl)) {}
FeatureStreamSession::~FeatureStreamSession() = default;
const FeatureStreamOptions &FeatureStreamSession::options() const { return pimpl_->opts; }
int FeatureStreamSession::chunks_emitted() const { return pimpl_->chunk_index; }
const std::vector<int32_t> &FeatureStreamSession::token_ids() const { return pimpl_->cum_ids; }
const std::string &FeatureStreamSession::text() const { return pimpl_->cum_text; }
int FeatureStreamSession::steps() const { return pimpl_->steps; }
void FeatureStreamSession::cancel() { pimpl_->cancelled = true; }
void FeatureStreamSession::finalize() { pimpl_->finalized = true; }

void FeatureStreamSession::Impl::emit(const std::vector<int32_t> &win_tokens, int n_boundaries, int n_frames,
                                      double decode_ms) {
    const DecoderModel &m = engine->model;
    const size_t prev = cum_text.size();
    cum_ids.insert(cum_ids.end(), win_tokens.begin(), win_tokens.end());
    cum_text = detokenize(m.vocab, cum_ids);
    const double start_s = (double)emitted_frames * stride_ms / 1000.0;
    const double end_s = (double)(emitted_frames + n_frames) * stride_ms / 1000.0;
    if (on_segment) {
        StreamingSegment seg;
        seg.text = cum_text.substr(prev);
        seg.token_ids = win_tokens;
        seg.start_s = start_s;
        seg.end_s = end_s;
        seg.chunk_index = chunk_index;
        seg.is_final = true;
        seg.is_eou_boundary = n_boundaries > 0;
        seg.decode_ms = decode_ms;
        on_segment(seg);
    }
    if (opts.on_event && n_boundaries > 0) {   // one EndOfTurn per boundary, confidence 1
        StreamEvent ev;
        ev.type = StreamEventType::EndOfTurn;
        ev.timestamp_s = end_s;
        ev.chunk_index = chunk_index;
        ev.eot_confidence = 1.0f;
        for (int i = 0; i < n_boundaries; ++i) opts.on_event(ev);
    }
    emitted_frames += n_frames;
    ++chunk_index;
}

void FeatureStreamSession::feed_frames(const float *enc, int n_frames, int D_enc) {
    feed_frames_batch({this}, {enc}, {n_frames}, D_enc);
}

void FeatureStreamSession::feed_frames_batch(const std::vector<FeatureStreamSession *> &sessions,
                                             const std::vector<const float *> &enc, const std::vector<int> &n_frames,
                                             int D_enc) {
    if (enc.size() != sessions.size() || n_frames.size() != sessions.size())
        throw std::invalid_argument("FeatureStreamSession::feed_frames_batch: size mismatch");
    std::vector<Impl *> live;
    std::vector<const float *> e;
    std::vector<int> nf;
    for (size_t i = 0; i < sessions.size(); ++i) {
        Impl *s = sessions[i]->pimpl_.get();
        if (s->cancelled) continue;
        if (s->finalized) throw std::logic_error("FeatureStreamSession: feed after finalize()");
        if (!live.empty() && s->engine != live[0]->engine)
            throw std::invalid_argument("FeatureStreamSession::feed_frames_batch: sessions of different engines");
        if (n_frames[i] < 0) throw std::invalid_argument("FeatureStreamSession: negative n_frames");
        for (Impl *o : live)
            if (o == s) throw std::invalid_argument("FeatureStreamSession::feed_frames_batch: repeated session");
        live.push_back(s);
        e.push_back(enc[i]);
        nf.push_back(n_frames[i]);
    }
    if (live.empty()) return;
    Engine::Impl &E = *live[0]->engine;
    const DecoderModel &m = E.model;
    const int n = (int)live.size();
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::vector<int32_t>> toks;
    std::vector<int> steps, nb(n, 0);
    if (m.model_type == ParakeetModelType::TDT) {
        std::vector<TdtDecodeState *> st(n);
        for (int i = 0; i < n; ++i) st[i] = &live[i]->tdt;
        if (int rc = tdt_decode_batch(m, E.tdt, e, nf, D_enc, TdtDecodeOptions{}, st, toks, steps))
            throw std::runtime_error("FeatureStreamSession: tdt_decode_window failed (rc=" + std::to_string(rc) + ")");
    } else {
        EouDecodeOptions o;
        o.max_symbols_per_step = m.encoder_cfg.eou_max_symbols_per_step;
        std::vector<EouDecodeState *> st(n);
        for (int i = 0; i < n; ++i) st[i] = &live[i]->eou;
        std::vector<std::vector<EouSegmentBoundary>> segs;
        if (int rc = eou_decode_batch(m, E.eou, e, nf, D_enc, o, st, toks, segs, steps))
            throw std::runtime_error("FeatureStreamSession: eou_decode_window failed (rc=" + std::to_string(rc) + ")");
        for (int i = 0; i < n; ++i) nb[i] = (int)segs[i].size();
    }
    const double ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    for (int i = 0; i < n; ++i) {
        live[i]->steps += steps[i];
        live[i]->emit(toks[i], nb[i], nf[i], ms);
    }
}

std::unique_ptr<FeatureStreamSession> Engine::stream_start(const FeatureStreamOptions &opts,
                                                           StreamingCallback on_segment) {
    if (opts.chunk_ms <= 0 && opts.chunk_frames <= 0)
        throw std::runtime_error("Engine::stream_start: chunk_ms must be > 0");
    auto impl = std::make_unique<FeatureStreamSession::Impl>();
    impl->engine = pimpl_.get();
    impl->opts = opts;
    impl->on_segment = std::move(on_segment);
    impl->stride_ms = encoder_frame_stride_ms(pimpl_->model);
    if (pimpl_->model.model_type == ParakeetModelType::TDT)
        tdt_init_state(pimpl_->tdt, pimpl_->model.blank_id, impl->tdt);
    else
        eou_init_state(pimpl_->eou, impl->eou);
    return std::make_unique<FeatureStreamSession>(std::move(impl));
}

EngineResult Engine::transcribe_features_stream(const float *enc, int T_enc, int D_enc,
                                                const FeatureStreamOptions &opts, StreamingCallback on_segment) {
    if (!enc || T_enc <= 0) throw std::runtime_error("parakeet::Engine::transcribe_features_stream: empty input");
    const auto t0 = std::chrono::steady_clock::now();
    const double stride = encoder_frame_stride_ms(pimpl_->model);
    int fpw = opts.chunk_frames > 0 ? opts.chunk_frames : (int)std::floor(opts.chunk_ms / stride);
    if (fpw < 1) fpw = 1;
    auto session = stream_start(opts, std::move(on_segment));
    EngineResult result;
    result.encoder_frames = T_enc;
    for (int start = 0; start < T_enc; start += fpw) {
        const int end = std::min(T_enc, start + fpw);
        session->feed_frames(enc + (size_t)start * D_enc, end - start, D_enc);
    }
    session->finalize();
    result.token_ids = session->token_ids();
    result.text = session->text();
    result.steps = session->steps();
    result.decode_ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    return result;
}

}  // namespace parakeet_hip

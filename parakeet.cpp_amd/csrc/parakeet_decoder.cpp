// parakeet_decoder.cpp -- the reference-shaped C++ decoder API on top of the
// C ABI (parakeet_hip.h).  See include/parakeet_decoder.h.
#include "parakeet_decoder.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <stdexcept>

#include "gguf_reader.h"
#include "parakeet_hip.h"

namespace parakeet {

struct ParakeetCtcModel::Impl {
    gguf::File file;
};

namespace detail {

// The device decoder of one runtime and its pool of state slots.
struct SlotPool {
    pk_decoder *dec = nullptr;
    std::mutex mu;
    std::vector<int> free_slots;
    ~SlotPool() { if (dec) pk_decoder_destroy(dec); }
    int acquire() {
        std::lock_guard<std::mutex> lk(mu);
        if (free_slots.empty()) return -1;
        const int s = free_slots.back();
        free_slots.pop_back();
        return s;
    }
    void release(int s) {
        std::lock_guard<std::mutex> lk(mu);
        free_slots.push_back(s);
    }
};

// A state's claim on one slot, returned to the pool when the state goes away.
struct SlotLease {
    std::shared_ptr<SlotPool> pool;
    int slot = -1;
    ~SlotLease() { if (pool && slot >= 0) pool->release(slot); }
};

}  // namespace detail

namespace {

const char *prefix(ParakeetModelType t) { return t == ParakeetModelType::EOU ? "eou." : "tdt."; }

pk_tensor tensor_of(const ParakeetCtcModel &m, const std::string &name) {
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
int make_pool(const ParakeetCtcModel &m, int n_slots, std::shared_ptr<detail::SlotPool> &out) {
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
    std::vector<uint8_t> special(m.vocab.pieces.size());
    for (size_t i = 0; i < special.size(); ++i) {
        const std::string &p = m.vocab.pieces[i];
        special[i] = (!p.empty() && p.front() == '<' && p.back() == '>') ? 1 : 0;
    }
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
    auto pool = std::make_shared<detail::SlotPool>();
    if (int rc = pk_decoder_create(&d, n_slots, &pool->dec)) {
        std::fprintf(stderr, "prepare_runtime: %s\n", pk_last_error());
        return rc;
    }
    for (int s = n_slots - 1; s >= 0; --s) pool->free_slots.push_back(s);
    out = std::move(pool);
    return 0;
}

std::shared_ptr<detail::SlotLease> lease(const std::shared_ptr<detail::SlotPool> &pool) {
    const int s = pool->acquire();
    if (s < 0) throw std::runtime_error("parakeet: no free decoder state slot");
    auto l = std::make_shared<detail::SlotLease>();
    l->pool = pool;
    l->slot = s;
    return l;
}

// Encoder frames of a batch: one host window per utterance (packed into one
// upload per call), or rows of an encoder output resident in device memory,
// read in place by the enc_proj kernel.
struct Frames {
    bool device = false;
    std::vector<const float *> host;   // host window of each utterance
    const float *dev = nullptr;        // device encoder output
    std::vector<int64_t> dev_row;      // first row of each utterance in it
    Frames pick(const std::vector<int> &idx, size_t i, size_t j) const {
        Frames f;
        f.device = device;
        f.dev = dev;
        for (size_t k = i; k < j; ++k) {
            if (device) f.dev_row.push_back(dev_row[idx[k]]);
            else f.host.push_back(host[idx[k]]);
        }
        return f;
    }
};

// One batched device call; fills per-utterance tokens/steps (+ EOU segments).
int run_batch(detail::SlotPool &pool, int D_enc, int max_symbols, const Frames &fr, const std::vector<int> &n_frames,
              const std::vector<int> &slots, const std::vector<int> &tokens_base,
              std::vector<std::vector<int32_t>> &tokens, std::vector<std::vector<int32_t>> *segments,
              std::vector<int> &steps) {
    const int n = (int)n_frames.size();
    int64_t rows = 0;
    int max_T = 0;
    std::vector<int64_t> row(n);
    for (int u = 0; u < n; ++u) {
        row[u] = rows;
        rows += std::max(0, n_frames[u]);
        max_T = std::max(max_T, n_frames[u]);
    }
    std::vector<float> packed;
    if (fr.device) {
        row = fr.dev_row;
    } else {
        packed.resize((size_t)std::max<int64_t>(rows, 1) * D_enc);
        for (int u = 0; u < n; ++u)
            if (n_frames[u] > 0)
                memcpy(packed.data() + (size_t)row[u] * D_enc, fr.host[u], sizeof(float) * (size_t)n_frames[u] * D_enc);
    }
    const int cap = max_T * std::max(1, max_symbols) + 1;
    std::vector<int32_t> tok((size_t)n * cap), ntok(n), st(n), seg((size_t)n * (cap + 1)), nseg(n);
    std::vector<int32_t> T(n_frames.begin(), n_frames.end()), sl(slots.begin(), slots.end());
    std::vector<int32_t> base(tokens_base.begin(), tokens_base.end());
    pk_batch b{};
    b.n_utts = n;
    b.mem = fr.device ? PK_MEM_DEVICE_FRAMES : PK_MEM_HOST;
    b.d_enc = D_enc;
    b.max_symbols = max_symbols;
    b.enc = fr.device ? fr.dev : packed.data();
    b.enc_row = row.data();
    b.n_frames = T.data();
    b.slot = sl.data();
    b.tokens_base = base.empty() ? nullptr : base.data();
    b.tokens = tok.data();
    b.token_cap = cap;
    b.n_tokens = ntok.data();
    b.steps = st.data();
    b.segments = seg.data();
    b.seg_cap = cap + 1;
    b.n_segments = nseg.data();
    if (int rc = pk_decode(pool.dec, &b)) {
        std::fprintf(stderr, "decode: %s\n", pk_last_error());
        return rc;
    }
    tokens.assign(n, {});
    if (segments) segments->assign(n, {});
    steps.assign(n, 0);
    for (int u = 0; u < n; ++u) {
        tokens[u].assign(tok.begin() + (size_t)u * cap, tok.begin() + (size_t)u * cap + ntok[u]);
        steps[u] = st[u];
        if (segments)
            (*segments)[u].assign(seg.begin() + (size_t)u * (cap + 1), seg.begin() + (size_t)u * (cap + 1) + nseg[u]);
    }
    return 0;
}

// Frames of a device-resident encoder output, checked against its extent.
// Returns 0, 1 (d_model mismatch, the reference's rc) or 3 (bad rows).
int device_frames(const DeviceEncoderOutput &enc, const std::vector<int64_t> &row_offset,
                  const std::vector<int> &n_frames, int D_expected, const char *who, Frames &fr) {
    if (enc.d_model != D_expected) {
        std::fprintf(stderr, "%s: encoder d_model mismatch (%d vs %d)\n", who, enc.d_model, D_expected);
        return 1;
    }
    if (row_offset.size() != n_frames.size()) return 3;
    for (size_t u = 0; u < n_frames.size(); ++u) {
        if (n_frames[u] <= 0) continue;
        if (!enc.data || row_offset[u] < 0 || row_offset[u] + n_frames[u] > enc.n_rows) {
            std::fprintf(stderr, "%s: utterance %zu rows [%lld, %lld) outside the encoder output (%lld rows)\n", who,
                         u, (long long)row_offset[u], (long long)(row_offset[u] + n_frames[u]),
                         (long long)enc.n_rows);
            return 3;
        }
    }
    fr.device = true;
    fr.dev = enc.data;
    fr.dev_row = row_offset;
    return 0;
}

void read_ctrl(detail::SlotPool &pool, int slot, int32_t *ctrl) {
    if (pk_slot_read(pool.dec, slot, nullptr, nullptr, nullptr, ctrl) != 0)
        throw std::runtime_error(std::string("parakeet: slot read failed: ") + pk_last_error());
}

}  // namespace

// ------------------------------------------------------------------ loading

int load_from_gguf(const std::string &gguf_path, ParakeetCtcModel &out, int, int, bool verbose) {
    auto impl = std::make_shared<ParakeetCtcModel::Impl>();
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
    out = ParakeetCtcModel{};
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
    std::string out;
    out.reserve(ids.size() * 3);
    for (int32_t id : ids) {
        if (id < 0 || id >= (int32_t)vocab.pieces.size()) continue;
        if (id == vocab.blank_id || id == vocab.bos_id || id == vocab.eos_id || id == vocab.pad_id) continue;
        const std::string &piece = vocab.pieces[id];
        for (size_t i = 0; i < piece.size();) {
            if ((unsigned char)piece[i] == 0xE2 && i + 2 < piece.size() && (unsigned char)piece[i + 1] == 0x96 &&
                (unsigned char)piece[i + 2] == 0x81) {
                out.push_back(' ');
                i += 3;
            } else {
                out.push_back(piece[i++]);
            }
        }
    }
    size_t start = 0;
    while (start < out.size() && out[start] == ' ') ++start;
    out.erase(0, start);
    return out;
}

// ------------------------------------------------------------------ TDT

int tdt_prepare_runtime(const ParakeetCtcModel &model, TdtRuntimeWeights &W, int n_slots) {
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

void tdt_init_state(TdtRuntimeWeights &W, int, TdtDecodeState &state) {
    if (!state.slot) state.slot = lease(W.pool);
    if (pk_slot_init(W.pool->dec, state.slot->slot) != 0)
        throw std::runtime_error(std::string("tdt_init_state: ") + pk_last_error());
    state.symbols_this_step = 0;
    state.carry_frames = 0;
    state.h_state.clear();
    state.c_state.clear();
    state.pred_out.clear();
    state.initialized = true;
}

namespace {

int tdt_batch(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const Frames &fr, const std::vector<int> &n_frames,
              int D_enc, const TdtDecodeOptions &opts, const std::vector<TdtDecodeState *> &states,
              std::vector<std::vector<int32_t>> &out_tokens, std::vector<int> &out_steps) {
    const int n = (int)n_frames.size();
    std::vector<int> idx, slots, T;
    for (int u = 0; u < n; ++u) {
        if (n_frames[u] <= 0) continue;   // src/parakeet_tdt.cpp:879
        if (!states[u]->initialized) tdt_init_state(W, model.blank_id, *states[u]);
        idx.push_back(u);
        slots.push_back(states[u]->slot->slot);
        T.push_back(n_frames[u]);
    }
    for (size_t i = 0; i < idx.size(); i += PK_MAX_BATCH) {
        const size_t j = std::min(idx.size(), i + PK_MAX_BATCH);
        std::vector<int> tt(T.begin() + i, T.begin() + j), ss(slots.begin() + i, slots.begin() + j);
        std::vector<std::vector<int32_t>> toks;
        std::vector<int> steps;
        if (int rc = run_batch(*W.pool, D_enc, opts.max_symbols_per_step, fr.pick(idx, i, j), tt, ss, {}, toks,
                               nullptr, steps))
            return rc;
        for (size_t k = i; k < j; ++k) {
            const int u = idx[k];
            out_tokens[u] = std::move(toks[k - i]);
            out_steps[u] = steps[k - i];
            int32_t ctrl[PK_CTRL_N];
            read_ctrl(*W.pool, slots[k], ctrl);
            states[u]->symbols_this_step = ctrl[PK_CTRL_SYM];
            states[u]->carry_frames = ctrl[PK_CTRL_CARRY];
        }
    }
    return 0;
}

}  // namespace

int tdt_decode_batch(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const std::vector<const float *> &enc,
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
    return tdt_batch(model, W, fr, n_frames, D_enc, opts, states, out_tokens, out_steps);
}

int tdt_decode_batch_device(const ParakeetCtcModel &model, TdtRuntimeWeights &W, const DeviceEncoderOutput &enc,
                            const std::vector<int64_t> &row_offset, const std::vector<int> &n_frames,
                            const TdtDecodeOptions &opts, const std::vector<TdtDecodeState *> &states,
                            std::vector<std::vector<int32_t>> &out_tokens, std::vector<int> &out_steps) {
    const int n = (int)n_frames.size();
    out_steps.assign(n, 0);
    out_tokens.assign(n, {});
    if ((int)states.size() != n) return 3;
    Frames fr;
    if (int rc = device_frames(enc, row_offset, n_frames, W.D_enc, "tdt_decode_batch_device", fr)) return rc;
    return tdt_batch(model, W, fr, n_frames, W.D_enc, opts, states, out_tokens, out_steps);
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
    result.text = detokenize(model.vocab, result.token_ids);
    result.decode_ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    return 0;
}

// ------------------------------------------------------------------ EOU

int eou_prepare_runtime(const ParakeetCtcModel &model, EouRuntimeWeights &W, int n_slots) {
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

void eou_init_state(const EouRuntimeWeights &W, EouDecodeState &state) {
    if (!state.slot) state.slot = lease(W.pool);
    if (pk_slot_init(W.pool->dec, state.slot->slot) != 0)
        throw std::runtime_error(std::string("eou_init_state: ") + pk_last_error());
    state.h_state.clear();
    state.c_state.clear();
    state.pred_out.clear();
    state.last_token = -1;
    state.symbols_this_step = 0;
    state.segment_start_token = 0;
    state.initialized = true;
}

namespace {

int eou_batch(const EouRuntimeWeights &W, const Frames &fr, const std::vector<int> &n_frames, int D_enc,
              const EouDecodeOptions &opts, const std::vector<EouDecodeState *> &states,
              std::vector<std::vector<int32_t>> &out_tokens, std::vector<std::vector<EouSegmentBoundary>> &out_segments,
              std::vector<int> &out_steps) {
    const int n = (int)n_frames.size();
    std::vector<int> idx(n), slots(n), base(n, 0);
    for (int u = 0; u < n; ++u) {
        if (!states[u]->initialized) eou_init_state(W, *states[u]);
        idx[u] = u;
        slots[u] = states[u]->slot->slot;
    }
    for (int i = 0; i < n; i += PK_MAX_BATCH) {
        const int j = std::min(n, i + PK_MAX_BATCH);
        std::vector<int> tt(n_frames.begin() + i, n_frames.begin() + j), ss(slots.begin() + i, slots.begin() + j);
        std::vector<int> bb(base.begin() + i, base.begin() + j);
        std::vector<std::vector<int32_t>> toks, segs;
        std::vector<int> steps;
        if (int rc = run_batch(*W.pool, D_enc, opts.max_symbols_per_step, fr.pick(idx, i, j), tt, ss, bb, toks, &segs,
                               steps))
            return rc;
        for (int u = i; u < j; ++u) {
            out_tokens[u] = std::move(toks[u - i]);
            out_steps[u] = steps[u - i];
            for (int32_t s : segs[u - i]) out_segments[u].push_back(EouSegmentBoundary{s, true});
            int32_t ctrl[PK_CTRL_N];
            read_ctrl(*W.pool, slots[u], ctrl);
            states[u]->symbols_this_step = ctrl[PK_CTRL_SYM];
            states[u]->last_token = ctrl[PK_CTRL_LAST];
            states[u]->segment_start_token = ctrl[PK_CTRL_SEGSTART];
        }
    }
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
    if ((int)n_frames.size() != n || (int)states.size() != n) return 3;
    Frames fr;
    fr.host = enc;
    return eou_batch(W, fr, n_frames, D_enc, opts, states, out_tokens, out_segments, out_steps);
}

int eou_decode_batch_device(const ParakeetCtcModel &, const EouRuntimeWeights &W, const DeviceEncoderOutput &enc,
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
    return eou_batch(W, fr, n_frames, W.D_enc, opts, states, out_tokens, out_segments, out_steps);
}

int eou_decode_window(const ParakeetCtcModel &model, const EouRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const EouDecodeOptions &opts, EouDecodeState &state,
                      std::vector<int32_t> &out_tokens, std::vector<EouSegmentBoundary> &out_segments,
                      int &out_steps) {
    (void)model;   // kept for the reference signature; the runtime weights carry every size used here
    if (D_enc != W.D_enc) {
        std::fprintf(stderr, "eou_decode_window: encoder d_model mismatch (%d vs %d)\n", D_enc, W.D_enc);
        return 1;
    }
    if (!state.initialized) eou_init_state(W, state);
    // segment indices count from the caller's token vector (src/parakeet_eou.cpp:293-298)
    const int base = (int)out_tokens.size();
    const int n = std::max(0, n_frames);
    std::vector<int32_t> toks;
    std::vector<int> steps;
    std::vector<std::vector<int32_t>> tv, sv;
    Frames fr;
    fr.host = {encoder_out_window};
    if (int rc = run_batch(*W.pool, D_enc, opts.max_symbols_per_step, fr, {n}, {state.slot->slot}, {base}, tv, &sv,
                           steps))
        return rc;
    out_steps = steps[0];
    out_tokens.insert(out_tokens.end(), tv[0].begin(), tv[0].end());
    for (int32_t s : sv[0]) out_segments.push_back(EouSegmentBoundary{s, true});
    int32_t ctrl[PK_CTRL_N];
    read_ctrl(*W.pool, state.slot->slot, ctrl);
    state.symbols_this_step = ctrl[PK_CTRL_SYM];
    state.last_token = ctrl[PK_CTRL_LAST];
    state.segment_start_token = ctrl[PK_CTRL_SEGSTART];
    return 0;
}

namespace {
std::string trim_spaces(const std::string &s) {
    const size_t a = s.find_first_not_of(" \t\r\n");
    if (a == std::string::npos) return std::string();
    const size_t b = s.find_last_not_of(" \t\r\n");
    return s.substr(a, b - a + 1);
}
}  // namespace

int eou_greedy_decode(const ParakeetCtcModel &model, const EouRuntimeWeights &W, const float *encoder_out, int T_enc,
                      int D_enc, const EouDecodeOptions &opts, EouDecodeResult &result) {
    const auto t0 = std::chrono::steady_clock::now();
    EouDecodeState state;
    result.token_ids.clear();
    result.segments.clear();
    if (int rc = eou_decode_window(model, W, encoder_out, T_enc, D_enc, opts, state, result.token_ids,
                                   result.segments, result.steps))
        return rc;
    result.eou_count = (int)result.segments.size();
    // segments joined with '\n' (src/parakeet_eou.cpp:359-382)
    int seg_start = 0;
    std::string text;
    for (size_t i = 0; i <= result.segments.size(); ++i) {
        const int seg_end = i < result.segments.size() ? result.segments[i].token_index : (int)result.token_ids.size();
        if (seg_end <= seg_start) { seg_start = seg_end; continue; }
        std::vector<int32_t> seg(result.token_ids.begin() + seg_start, result.token_ids.begin() + seg_end);
        std::string s = trim_spaces(detokenize(model.vocab, seg));
        if (!s.empty()) {
            if (!text.empty()) text += "\n";
            text += s;
        }
        seg_start = seg_end;
    }
    result.text = std::move(text);
    result.decode_ms =
        std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() / 1000.0;
    return 0;
}

// ------------------------------------------------------------------ Engine

struct Engine::Impl {
    EngineOptions opts;
    ParakeetCtcModel model;
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

const ParakeetCtcModel &Engine::model() const { return pimpl_->model; }

EngineResult Engine::transcribe_features(const float *enc, int T_enc, int D_enc) {
    return transcribe_features_batch({enc}, {T_enc}, D_enc)[0];
}

namespace {

// The Engine's batch decode over either frame source: fresh states, one result per utterance.
std::vector<EngineResult> engine_decode(Engine::Impl &E, const Frames &fr, const std::vector<int> &T_enc, int D_enc) {
    const auto t0 = std::chrono::steady_clock::now();
    const int n = (int)T_enc.size();
    std::vector<EngineResult> out(n);
    const ParakeetCtcModel &m = E.model;
    if (m.model_type == ParakeetModelType::TDT) {
        std::vector<TdtDecodeState> states(n);
        std::vector<TdtDecodeState *> sp(n);
        for (int u = 0; u < n; ++u) sp[u] = &states[u];
        std::vector<std::vector<int32_t>> toks(n);
        std::vector<int> steps(n, 0);
        int rc = D_enc != E.tdt.D_enc ? 1 : 0;
        if (rc == 0) rc = tdt_batch(m, E.tdt, fr, T_enc, D_enc, TdtDecodeOptions{}, sp, toks, steps);
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
        if (rc == 0) rc = eou_batch(E.eou, fr, T_enc, D_enc, o, sp, toks, segs, steps);
        if (rc) throw std::runtime_error("parakeet::Engine: eou decode failed (rc=" + std::to_string(rc) + ")");
        for (int u = 0; u < n; ++u) {
            out[u].token_ids = std::move(toks[u]);
            out[u].steps = steps[u];
            int s0 = 0;
            std::string text;
            for (size_t i = 0; i <= segs[u].size(); ++i) {
                const int e = i < segs[u].size() ? segs[u][i].token_index : (int)out[u].token_ids.size();
                if (e > s0) {
                    std::vector<int32_t> seg(out[u].token_ids.begin() + s0, out[u].token_ids.begin() + e);
                    std::string s = trim_spaces(detokenize(m.vocab, seg));
                    if (!s.empty()) text += (text.empty() ? "" : "\n") + s;
                }
                s0 = e;
            }
            out[u].text = std::move(text);
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
    const ParakeetCtcModel &m = pimpl_->model;
    const int D = m.model_type == ParakeetModelType::TDT ? pimpl_->tdt.D_enc : pimpl_->eou.D_enc;
    Frames fr;
    if (int rc = device_frames(enc, row_offset, T_enc, D, "parakeet::Engine::transcribe_device_batch", fr))
        throw std::runtime_error("parakeet::Engine: device frames rejected (rc=" + std::to_string(rc) + ")");
    return engine_decode(*pimpl_, fr, T_enc, D);
}

// ------------------------------------------------------------------ streaming over features

double encoder_frame_stride_ms(const ParakeetCtcModel &m) {
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
    const ParakeetCtcModel &m = engine->model;
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
    const ParakeetCtcModel &m = E.model;
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

}  // namespace parakeet

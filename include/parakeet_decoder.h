// parakeet_decoder.h -- standalone C++ transducer decoder API of the MI355X
// build, shaped like parakeet.cpp's (src/parakeet_tdt.h, src/parakeet_eou.h,
// include/parakeet/engine.h) and running on the kernels of libparakeet_hip.so
// through the C ABI in parakeet_hip.h.
//
// Everything here lives in namespace parakeet_hip, so it can sit beside the
// reference's own headers.  The model is decoder-only (DecoderModel): the
// loader reads the prediction / joint tensors and the metadata of a GGUF, no
// encoder tensors.  A caller that keeps parakeet.cpp's own model and Engine
// uses the drop-in decoder headers in include/dropin/ instead, which declare
// the reference's decoder functions against its ParakeetCtcModel.
//
// Same names, argument meanings and status codes as the reference otherwise.
// Differences, all on purpose:
//   - decode state lives in a device slot of the runtime; every TdtDecodeState
//     / EouDecodeState holds its own (a copy leases a new slot and copies the
//     state, see parakeet_slot.h).  The host vectors h_state / c_state /
//     pred_out stay empty, as on the reference GPU path;
//   - *_decode_batch entry points decode many utterances in one lockstep launch.
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "parakeet_slot.h"

namespace parakeet_hip {

enum class ParakeetModelType { CTC, TDT, EOU, SORTFORMER };

// src/sentencepiece_bpe.h: pieces plus the ids detokenize skips.
struct BpeVocab {
    std::vector<std::string> pieces;
    int32_t blank_id = -1, unk_id = -1, bos_id = -1, eos_id = -1, pad_id = -1;
};

// The decoder fields of the reference's EncoderConfig (src/parakeet_ctc.h), plus the
// subsampling factor that sets the encoder frame stride.
struct EncoderConfig {
    int d_model = 1024;
    int subsampling_factor = 8;
    int tdt_pred_hidden = 640, tdt_pred_rnn_layers = 2, tdt_joint_hidden = 640, tdt_num_durations = 5;
    int eou_pred_hidden = 640, eou_pred_rnn_layers = 1, eou_joint_hidden = 640;
    int eou_max_symbols_per_step = 5;
};

// The MelConfig fields that set the encoder frame stride (src/parakeet_ctc.cpp:470-473).
struct MelConfig {
    int sample_rate = 16000;
    int hop_length = 160;
};

// The decoder half of a parakeet GGUF: metadata, vocabulary and the tensor
// directory (the file's bytes stay mapped in impl).
struct DecoderModel {
    ParakeetModelType model_type = ParakeetModelType::CTC;
    EncoderConfig encoder_cfg;
    MelConfig mel_cfg;
    BpeVocab vocab;
    int32_t blank_id = 1024;
    int32_t vocab_size = 1025;
    int32_t eou_id = -1;
    int32_t eob_id = -1;
    std::vector<int32_t> tdt_durations;

    struct Impl;
    std::shared_ptr<Impl> impl;   // GGUF bytes + tensor directory
};

// src/parakeet_ctc.cpp:297.  Returns 0, or the reference's codes: 1 open
// failure, 2 wrong architecture / missing decoder tensor.
int load_from_gguf(const std::string &gguf_path, DecoderModel &out_model, int n_threads = 0,
                   int n_gpu_layers = 1, bool verbose = false);

// ---- TDT (src/parakeet_tdt.h) ----

struct TdtRuntimeWeights {
    int H_pred = 640, H_joint = 640, D_enc = 1024, V_plus_1 = 8193, V_out = 8198, L = 2, num_durations = 5;
    const DecoderModel *weights_model = nullptr;
    std::shared_ptr<SlotPool> pool;   // device decoder + state slots
    bool ready() const { return pool != nullptr; }
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
    std::vector<float> h_state;   // left empty: state lives on the device
    std::vector<float> c_state;
    std::vector<float> pred_out;
    int symbols_this_step = 0;    // mirrored from the device after every window
    bool initialized = false;
    int carry_frames = 0;
    SlotHandle slot;               // the device slot holding h, c, pred and the control words
};

// n_slots: concurrent decode states the runtime can hold (default 1024).
int tdt_prepare_runtime(const DecoderModel &model, TdtRuntimeWeights &out, int n_slots = 1024);
void tdt_init_state(TdtRuntimeWeights &W, int blank_id, TdtDecodeState &state);
int tdt_decode_window(const DecoderModel &model, TdtRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const TdtDecodeOptions &opts, TdtDecodeState &state,
                      std::vector<int32_t> &out_tokens, int &out_steps);
int tdt_greedy_decode(const DecoderModel &model, TdtRuntimeWeights &W, const float *encoder_out, int T_enc,
                      int D_enc, const TdtDecodeOptions &opts, TdtDecodeResult &result);
// Batched: utterance u decodes enc[u][0 .. n_frames[u]) with states[u].
int tdt_decode_batch(const DecoderModel &model, TdtRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const TdtDecodeOptions &opts,
                     const std::vector<TdtDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<int> &out_steps);

// ---- EOU (src/parakeet_eou.h) ----

struct EouRuntimeWeights {
    int H_pred = 640, H_joint = 640, D_enc = 512, V_plus_1 = 1027, L = 1;
    int blank_id = 1026, eou_id = 1024, eob_id = 1025;
    std::shared_ptr<SlotPool> pool;
};

struct EouDecodeOptions {
    int max_symbols_per_step = 5;
};

struct EouDecodeState {
    std::vector<float> h_state, c_state, pred_out;   // left empty: state lives on the device
    int32_t last_token = -1;
    int symbols_this_step = 0;
    bool initialized = false;
    int segment_start_token = 0;
    SlotHandle slot;               // the device slot holding h, c, pred and the control words
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

int eou_prepare_runtime(const DecoderModel &model, EouRuntimeWeights &out, int n_slots = 1024);
void eou_init_state(const EouRuntimeWeights &W, EouDecodeState &state);
int eou_decode_window(const DecoderModel &model, const EouRuntimeWeights &W, const float *encoder_out_window,
                      int n_frames, int D_enc, const EouDecodeOptions &opts, EouDecodeState &state,
                      std::vector<int32_t> &out_tokens, std::vector<EouSegmentBoundary> &out_segments,
                      int &out_steps);
int eou_greedy_decode(const DecoderModel &model, const EouRuntimeWeights &W, const float *encoder_out,
                      int T_enc, int D_enc, const EouDecodeOptions &opts, EouDecodeResult &result);
int eou_decode_batch(const DecoderModel &model, const EouRuntimeWeights &W, const std::vector<const float *> &enc,
                     const std::vector<int> &n_frames, int D_enc, const EouDecodeOptions &opts,
                     const std::vector<EouDecodeState *> &states, std::vector<std::vector<int32_t>> &out_tokens,
                     std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps);

// ---- Encoder -> decoder handoff on the device ----
//
// The reference copies the encoder output to the host (EncoderOutputs::encoder_out,
// src/parakeet_ctc.cpp:1660-1667) and decodes from there.  An encoder whose
// output stays in device memory hands it over in place instead: the enc_proj
// kernel reads the rows directly, with no host copy and no upload.  Utterance
// u's window is rows row_offset[u] .. row_offset[u] + n_frames[u] (variable
// lengths, in any order).  The rows must be complete before the call: the
// decoder runs on its own stream, so the caller synchronises the stream that
// produced them.  Return codes as the host-frame calls, plus 3 for windows
// outside the output.
struct DeviceEncoderOutput {
    const float *data = nullptr;   // device address of [n_rows][d_model] f32, 16-byte aligned
    int64_t n_rows = 0;
    int d_model = 0;
};
int tdt_decode_batch_device(const DecoderModel &model, TdtRuntimeWeights &W, const DeviceEncoderOutput &enc,
                            const std::vector<int64_t> &row_offset, const std::vector<int> &n_frames,
                            const TdtDecodeOptions &opts, const std::vector<TdtDecodeState *> &states,
                            std::vector<std::vector<int32_t>> &out_tokens, std::vector<int> &out_steps);
int eou_decode_batch_device(const DecoderModel &model, const EouRuntimeWeights &W, const DeviceEncoderOutput &enc,
                            const std::vector<int64_t> &row_offset, const std::vector<int> &n_frames,
                            const EouDecodeOptions &opts, const std::vector<EouDecodeState *> &states,
                            std::vector<std::vector<int32_t>> &out_tokens,
                            std::vector<std::vector<EouSegmentBoundary>> &out_segments, std::vector<int> &out_steps);

// src/sentencepiece_bpe.cpp:9-38: pieces joined (blank/bos/eos/pad skipped), U+2581 -> ' ',
// leading spaces trimmed.
std::string detokenize(const BpeVocab &vocab, const std::vector<int32_t> &ids);

// ---- Streaming types (include/parakeet/streaming.h) ----

enum class VadState : int { Unknown = 0, Speaking = 1, Silent = 2 };
enum class StreamEventType : int { VadStateChanged = 1, EndOfTurn = 2 };

struct StreamEvent {
    StreamEventType type = StreamEventType::VadStateChanged;
    double timestamp_s = 0.0;     // end of the chunk that produced the event
    int chunk_index = -1;
    VadState vad_state = VadState::Unknown;
    int speaker_id = -1;
    float vad_score = 0.0f;
    float eot_confidence = 0.0f;  // 1.0 when <EOU> fired
};
using StreamEventCallback = std::function<void(const StreamEvent &)>;

struct StreamingSegment {
    std::string text;             // new text of this chunk (cumulative detokenize, minus the previous text)
    std::vector<int32_t> token_ids;
    double start_s = 0.0, end_s = 0.0;
    int chunk_index = 0;
    bool is_final = true;
    bool is_eou_boundary = false; // EOU: the chunk recorded at least one segment boundary
    float eot_confidence = 0.0f;
    double encoder_ms = 0.0;
    double decode_ms = 0.0;
};
using StreamingCallback = std::function<void(const StreamingSegment &)>;

// Streaming over encoder features.  The reference's StreamingOptions (chunk_ms,
// left context, lookahead) also drive mel and encoder windows, which are
// outside this library: a caller hands the frames of each chunk that are to
// be decoded (the reference drops the context frames first,
// src/parakeet_engine.cpp:796-818).
struct FeatureStreamOptions {
    int chunk_ms = 1000;             // StreamingOptions::chunk_ms
    int chunk_frames = 0;            // frames per window of transcribe_features_stream;
                                     // 0: floor(chunk_ms / frame stride), at least 1
    StreamEventCallback on_event = nullptr;
};

class Engine;

// The decode half of StreamSession (src/parakeet_engine.cpp:753-864): each fed
// chunk is decoded with the session's carried state (its own device slot),
// then one StreamingSegment and, for EOU boundaries, EndOfTurn events are
// delivered.  Each chunk is decoded into a fresh token vector, as the
// reference does, so EOU boundary indices count from the chunk's first token
// while segment_start_token carries over (src/parakeet_eou.cpp:293-299).
// Not thread-safe; one Engine may hold many sessions; a session must not
// outlive its Engine.
class FeatureStreamSession {
public:
    struct Impl;
    explicit FeatureStreamSession(std::unique_ptr<Impl> impl);
    ~FeatureStreamSession();
    FeatureStreamSession(const FeatureStreamSession &) = delete;
    FeatureStreamSession &operator=(const FeatureStreamSession &) = delete;

    // One chunk of encoder frames [n_frames][D_enc].  Throws std::runtime_error on
    // a decode failure; does nothing after cancel().
    void feed_frames(const float *encoder_out, int n_frames, int D_enc);
    // Sessions of one Engine fed in one lockstep launch: sessions[i] gets
    // encoder_out[i][0 .. n_frames[i]).  Callbacks run afterwards, in session order.
    static void feed_frames_batch(const std::vector<FeatureStreamSession *> &sessions,
                                  const std::vector<const float *> &encoder_out, const std::vector<int> &n_frames,
                                  int D_enc);
    // No more chunks (the reference flushes its sample remainder here; feature
    // chunks have none).  Later feeds throw.
    void finalize();
    void cancel();
    const FeatureStreamOptions &options() const;
    int chunks_emitted() const;
    const std::vector<int32_t> &token_ids() const;   // every token so far
    const std::string &text() const;                 // detokenize(token_ids())
    int steps() const;                               // decode steps so far

private:
    std::unique_ptr<Impl> pimpl_;
};

// Encoder frame stride in ms: 1000 * hop_length * subsampling / sample_rate
// (src/parakeet_engine.cpp:35-41).
double encoder_frame_stride_ms(const DecoderModel &model);

// ---- Engine-shaped front (include/parakeet/engine.h) over encoder features ----

struct EngineOptions {
    std::string model_gguf_path;
    int n_slots = 1024;
};

struct EngineResult {
    std::string text;
    std::vector<int32_t> token_ids;
    double decode_ms = 0.0;
    int encoder_frames = 0;
    int steps = 0;
};

class Engine {
public:
    explicit Engine(const EngineOptions &opts);   // throws std::runtime_error, as the reference does
    ~Engine();
    // The decode half of Engine::transcribe_samples (src/parakeet_engine.cpp:271-317),
    // dispatched on parakeet.model.type: features are the encoder output [T][D].
    EngineResult transcribe_features(const float *encoder_out, int T_enc, int D_enc);
    std::vector<EngineResult> transcribe_features_batch(const std::vector<const float *> &encoder_out,
                                                        const std::vector<int> &T_enc, int D_enc);
    // The same over an encoder output resident in device memory (see DeviceEncoderOutput).
    std::vector<EngineResult> transcribe_device_batch(const DeviceEncoderOutput &encoder_out,
                                                      const std::vector<int64_t> &row_offset,
                                                      const std::vector<int> &T_enc);
    // The decode half of Engine::transcribe_samples_stream (src/parakeet_engine.cpp:389-489):
    // the encoder output in windows of opts.chunk_frames frames, one segment per window.
    EngineResult transcribe_features_stream(const float *encoder_out, int T_enc, int D_enc,
                                            const FeatureStreamOptions &opts, StreamingCallback on_segment);
    // The decode half of Engine::stream_start (src/parakeet_engine.cpp:1013-1059).
    std::unique_ptr<FeatureStreamSession> stream_start(const FeatureStreamOptions &opts,
                                                       StreamingCallback on_segment);
    const DecoderModel &model() const;
    struct Impl;

private:
    std::unique_ptr<Impl> pimpl_;
};

}  // namespace parakeet_hip

// Drives the drop-in decoder (include/dropin/parakeet_tdt.h, parakeet_eou.h,
// csrc/dropin/parakeet_dropin.cpp) through parakeet.cpp's own model type: the
// ParakeetCtcModel of the reference's src/parakeet_ctc.h, filled here the way
// its loader fills the decoder fields (src/parakeet_ctc.cpp:418-458 metadata,
// :603-665 tensor handles), and prints what the decoder returns as one JSON
// object:
//   - tdt_greedy_decode per utterance, tdt_init_state + tdt_decode_window over
//     fixed windows (src/parakeet_engine.cpp:409-452), tdt_decode_batch;
//   - value semantics of a state: a copy taken mid-utterance decodes the rest
//     of the utterance to the same tokens as the original, whichever runs
//     first, and a state assigned over another replaces it;
//   - a d_model mismatch (rc 1, src/parakeet_tdt.cpp:874-877);
//   - eou_greedy_decode, eou_decode_window over fixed windows, eou_decode_batch;
//   - the wall time of one tdt_greedy_decode call on the first utterance (one
//     launch per call), over `reps` calls.
//
// ggml is not linked: ggml_tensor is defined here as a handle to a tensor of
// the GGUF file read by the library's own reader, and
// parakeet_hip::dropin::tensor_bytes returns its stored bytes, as the ggml
// implementation does with ggml_backend_tensor_get inside parakeet.cpp's build.
//
// Usage: dropin_main TDT.gguf TDT_FRAMES EOU.gguf EOU_FRAMES WINDOW [reps]
// Frame files: int32 n, T, D, then n*T*D float32 (utterance-major).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <deque>
#include <string>
#include <vector>

#include "decoder_core.h"
#include "dropin_tensor.h"
#include "gguf_reader.h"
#include "parakeet_ctc.h"
#include "parakeet_eou.h"
#include "parakeet_tdt.h"

struct ggml_tensor {
    const parakeet_hip::gguf::Tensor *t = nullptr;
};

namespace parakeet_hip {
namespace dropin {

int tensor_bytes(const ggml_tensor *t, pk_tensor *out, std::vector<uint8_t> *storage) {
    *out = pk_tensor{};
    if (!t) return 0;
    if (!t->t || t->t->ne.empty()) return 2;
    storage->assign(t->t->data, t->t->data + t->t->nbytes);
    out->data = storage->data();
    out->type = (int32_t)t->t->type;
    out->ne0 = t->t->ne[0];
    out->ne1 = t->t->ne.size() > 1 ? t->t->ne[1] : 1;
    return 0;
}

}  // namespace dropin
}  // namespace parakeet_hip

namespace {

namespace gguf = parakeet_hip::gguf;
using namespace parakeet;

// A GGUF file and the ggml_tensor handles a model points into.
struct Loaded {
    gguf::File file;
    std::deque<ggml_tensor> handles;
    ParakeetCtcModel model;

    ggml_tensor *handle(const std::string &name) {
        const gguf::Tensor *t = file.tensor(name);
        if (!t) return nullptr;
        handles.push_back(ggml_tensor{t});
        return &handles.back();
    }
};

template <class Weights>
int bind(Loaded &ld, const std::string &p, int L, Weights &w) {
    w.predict_embed = ld.handle(p + "predict.embed.weight");
    w.lstm.resize(L);
    for (int l = 0; l < L; ++l) {
        const std::string q = p + "predict.lstm." + std::to_string(l) + ".";
        w.lstm[l].w_ih = ld.handle(q + "w_ih");
        w.lstm[l].w_hh = ld.handle(q + "w_hh");
        w.lstm[l].b_ih = ld.handle(q + "b_ih");
        w.lstm[l].b_hh = ld.handle(q + "b_hh");
    }
    w.joint_enc_w = ld.handle(p + "joint.enc.weight");
    w.joint_enc_b = ld.handle(p + "joint.enc.bias");
    w.joint_pred_w = ld.handle(p + "joint.pred.weight");
    w.joint_pred_b = ld.handle(p + "joint.pred.bias");
    w.joint_out_w = ld.handle(p + "joint.out.weight");
    w.joint_out_b = ld.handle(p + "joint.out.bias");
    return w.predict_embed && w.joint_out_w ? 0 : 2;
}

// The decoder half of src/parakeet_ctc.cpp:297-682 for one GGUF.
int load(const char *path, Loaded &ld) {
    std::string err;
    if (ld.file.open(path, err)) {
        std::fprintf(stderr, "gguf: %s\n", err.c_str());
        return 1;
    }
    const gguf::File &g = ld.file;
    ParakeetCtcModel &m = ld.model;
    EncoderConfig &c = m.encoder_cfg;
    c.d_model = (int)g.get_u32("parakeet.encoder.d_model", 1024);
    const std::string mt = g.get_str("parakeet.model.type", "ctc");
    if (mt == "tdt") {
        m.model_type = ParakeetModelType::TDT;
        c.tdt_pred_hidden = (int)g.get_u32("parakeet.tdt.pred_hidden", 640);
        c.tdt_pred_rnn_layers = (int)g.get_u32("parakeet.tdt.pred_rnn_layers", 2);
        c.tdt_joint_hidden = (int)g.get_u32("parakeet.tdt.joint_hidden", 640);
        c.tdt_num_durations = (int)g.get_u32("parakeet.tdt.num_durations", 5);
        m.vocab_size = (int32_t)g.get_u32("parakeet.tdt.vocab_size", 8192);
        m.blank_id = (int32_t)g.get_u32("parakeet.tdt.blank_id", (uint32_t)m.vocab_size);
        if (const gguf::Value *v = g.find("parakeet.tdt.durations"))
            m.tdt_durations.assign(v->arr_i.begin(), v->arr_i.end());
        else
            m.tdt_durations = {0, 1, 2, 3, 4};
    } else if (mt == "eou") {
        m.model_type = ParakeetModelType::EOU;
        c.eou_pred_hidden = (int)g.get_u32("parakeet.eou.pred_hidden", 640);
        c.eou_pred_rnn_layers = (int)g.get_u32("parakeet.eou.pred_rnn_layers", 1);
        c.eou_joint_hidden = (int)g.get_u32("parakeet.eou.joint_hidden", 640);
        m.vocab_size = (int32_t)g.get_u32("parakeet.eou.vocab_size", 1026);
        m.blank_id = (int32_t)g.get_u32("parakeet.eou.blank_id", (uint32_t)m.vocab_size);
        m.eou_id = g.find("parakeet.eou.eou_id") ? g.get_i32("parakeet.eou.eou_id", -1) : -1;
        m.eob_id = g.find("parakeet.eou.eob_id") ? g.get_i32("parakeet.eou.eob_id", -1) : -1;
    } else {
        return 2;
    }
    if (const gguf::Value *v = g.find("tokenizer.ggml.tokens")) m.vocab.pieces = v->arr_s;
    m.vocab.blank_id = m.blank_id;
    m.vocab.bos_id = (int32_t)g.get_u32("tokenizer.ggml.bos_token_id", (uint32_t)-1);
    m.vocab.eos_id = (int32_t)g.get_u32("tokenizer.ggml.eos_token_id", (uint32_t)-1);
    m.vocab.pad_id = (int32_t)g.get_u32("tokenizer.ggml.pad_token_id", (uint32_t)-1);
    return m.model_type == ParakeetModelType::TDT ? bind(ld, "tdt.", c.tdt_pred_rnn_layers, m.tdt)
                                                  : bind(ld, "eou.", c.eou_pred_rnn_layers, m.eou);
}

struct Frames {
    int n = 0, T = 0, D = 0;
    std::vector<float> data;
    const float *utt(int u) const { return data.data() + (size_t)u * T * D; }
};

bool read_frames(const char *path, Frames &f) {
    FILE *fp = std::fopen(path, "rb");
    if (!fp) return false;
    int hdr[3];
    bool ok = std::fread(hdr, 4, 3, fp) == 3;
    if (ok) {
        f.n = hdr[0];
        f.T = hdr[1];
        f.D = hdr[2];
        f.data.resize((size_t)f.n * f.T * f.D);
        ok = std::fread(f.data.data(), 4, f.data.size(), fp) == f.data.size();
    }
    std::fclose(fp);
    return ok;
}

void ints(const std::vector<int32_t> &v) {
    std::printf("[");
    for (size_t i = 0; i < v.size(); ++i) std::printf(i ? ",%d" : "%d", v[i]);
    std::printf("]");
}

void lists(const std::vector<std::vector<int32_t>> &v) {
    std::printf("[");
    for (size_t u = 0; u < v.size(); ++u) {
        if (u) std::printf(",");
        ints(v[u]);
    }
    std::printf("]");
}

void str(const std::string &s) {
    std::printf("\"");
    for (char c : s) {
        if (c == '"' || c == '\\') std::printf("\\%c", c);
        else if (c == '\n') std::printf("\\n");
        else std::printf("%c", c);
    }
    std::printf("\"");
}

int fail(const char *what, int rc) {
    std::fprintf(stderr, "%s failed: rc=%d\n", what, rc);
    return 1;
}

}  // namespace

// The reference CLI's pattern (src/main.cpp:745-777): each model type keeps its
// runtime in a function-local static, prepared on first use and destroyed at
// process exit, after main returns.
int run_once(const char *path, const Frames &f, std::vector<int32_t> &ids) {
    Loaded ld;
    if (int rc = load(path, ld)) return rc;
    const ParakeetCtcModel &model = ld.model;
    if (model.model_type == ParakeetModelType::TDT) {
        static TdtRuntimeWeights rt;
        static bool rt_ready = false;
        if (!rt_ready) {
            if (tdt_prepare_runtime(model, rt) != 0) return 20;
            rt_ready = true;
        }
        TdtDecodeOptions dopts;
        TdtDecodeResult dres;
        if (int rc = tdt_greedy_decode(model, rt, f.utt(0), f.T, f.D, dopts, dres)) return rc;
        ids = std::move(dres.token_ids);
    } else {
        static EouRuntimeWeights rt;
        static bool rt_ready = false;
        if (!rt_ready) {
            if (eou_prepare_runtime(model, rt) != 0) return 20;
            rt_ready = true;
        }
        EouDecodeOptions dopts;
        dopts.max_symbols_per_step = model.encoder_cfg.eou_max_symbols_per_step;
        EouDecodeResult dres;
        if (int rc = eou_greedy_decode(model, rt, f.utt(0), f.T, f.D, dopts, dres)) return rc;
        ids = std::move(dres.token_ids);
    }
    return 0;
}

// --static-exit: decode utterance 0 of each model through run_once, print the
// token ids and return from main with both static runtimes alive.
int static_exit(int argc, char **argv) {
    if (argc < 6) return 2;
    Frames ft, fe;
    if (!read_frames(argv[3], ft) || !read_frames(argv[5], fe)) return fail("reading the frames", -1);
    std::vector<std::vector<int32_t>> ids(2);
    if (int rc = run_once(argv[2], ft, ids[0])) return fail("run_once(tdt)", rc);
    if (int rc = run_once(argv[4], fe, ids[1])) return fail("run_once(eou)", rc);
    std::printf("{\"static_exit\":");
    lists(ids);
    std::printf("}\n");
    std::fflush(stdout);
    return 0;
}

// --bench TDT.gguf FRAMES REPS: the reference CLI's decode of one utterance
// (tdt_greedy_decode, src/main.cpp:745-761) timed REPS times after a warm-up:
// wall time per call as the runtime runs it, then, with the handle's timing events on, the
// kernels' share (pk_last_timing).
int bench(int argc, char **argv) {
    if (argc < 5) return 2;
    Frames f;
    if (!read_frames(argv[3], f)) return fail("reading the frames", -1);
    const int reps = std::max(1, std::atoi(argv[4]));
    Loaded ld;
    if (int rc = load(argv[2], ld)) return fail("loading the model", rc);
    const ParakeetCtcModel &model = ld.model;
    TdtRuntimeWeights rt;
    if (int rc = tdt_prepare_runtime(model, rt)) return fail("tdt_prepare_runtime", rc);
    TdtDecodeOptions dopts;
    // pass 0: as the runtime runs (no timing events); pass 1: with them, for the kernels' share
    double wall[2] = {0.0, 0.0}, wmin = 1e30, kern = 0.0;
    int steps = 0;
    for (int pass = 0; pass < 2; ++pass) {
        pk_decoder_set_timing(rt.pool->dec, pass);
        for (int r = 0; r <= reps; ++r) {
            TdtDecodeResult res;
            const auto t0 = std::chrono::steady_clock::now();
            if (int rc = tdt_greedy_decode(model, rt, f.utt(0), f.T, f.D, dopts, res))
                return fail("tdt_greedy_decode", rc);
            const double dt = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
            float ep = 0.f, lp = 0.f;
            int32_t it = 0;
            pk_last_timing(rt.pool->dec, &ep, &lp, &it);
            if (r > 0) {   // the first call of a pass is a warm-up
                wall[pass] += dt;
                if (pass == 0) wmin = std::min(wmin, dt);
                else kern += 1000.0 * (ep + lp);
            }
            steps = res.steps;
        }
    }
    std::printf("{\"call_us\":%.3f,\"call_us_min\":%.3f,\"call_us_timed\":%.3f,\"kernel_us\":%.3f,"
                "\"steps\":%d,\"frames\":%d,\"reps\":%d}\n",
                wall[0] / reps, wmin, wall[1] / reps, kern / reps, steps, f.T, reps);
    return 0;
}

int main(int argc, char **argv) {
    if (argc > 1 && std::strcmp(argv[1], "--static-exit") == 0) return static_exit(argc, argv);
    if (argc > 1 && std::strcmp(argv[1], "--bench") == 0) return bench(argc, argv);
    if (argc < 6) {
        std::fprintf(stderr, "usage: dropin_main TDT.gguf TDT_FRAMES EOU.gguf EOU_FRAMES WINDOW [reps]\n"
                             "       dropin_main --static-exit TDT.gguf TDT_FRAMES EOU.gguf EOU_FRAMES\n"
                             "       dropin_main --bench TDT.gguf TDT_FRAMES REPS\n");
        return 2;
    }
    const int W = std::atoi(argv[5]);
    const int reps = argc > 6 ? std::atoi(argv[6]) : 20;
    Frames ft, fe;
    if (!read_frames(argv[2], ft) || !read_frames(argv[4], fe) || W <= 0) return fail("reading the frames", -1);
    int rc;

    // ---------------- TDT
    Loaded lt;
    if ((rc = load(argv[1], lt)) != 0) return fail("loading the TDT model", rc);
    const ParakeetCtcModel &mt = lt.model;
    TdtRuntimeWeights tw;
    if ((rc = tdt_prepare_runtime(mt, tw)) != 0) return fail("tdt_prepare_runtime", rc);
    if (!tw.ready()) return fail("TdtRuntimeWeights::ready", -1);
    TdtDecodeOptions topt;
    std::vector<std::vector<int32_t>> greedy(ft.n), chunked(ft.n);
    std::vector<std::string> text(ft.n);
    std::vector<int32_t> steps(ft.n);
    for (int u = 0; u < ft.n; ++u) {
        TdtDecodeResult r;
        if ((rc = tdt_greedy_decode(mt, tw, ft.utt(u), ft.T, ft.D, topt, r)) != 0) return fail("tdt_greedy_decode", rc);
        greedy[u] = r.token_ids;
        text[u] = r.text;
        steps[u] = r.steps;
        TdtDecodeState st;
        tdt_init_state(tw, mt.blank_id, st);
        for (int t0 = 0; t0 < ft.T; t0 += W) {
            int s = 0;
            const int n = std::min(W, ft.T - t0);
            if ((rc = tdt_decode_window(mt, tw, ft.utt(u) + (size_t)t0 * ft.D, n, ft.D, topt, st, chunked[u], s)))
                return fail("tdt_decode_window", rc);
        }
    }
    std::vector<TdtDecodeState> bst(ft.n);
    std::vector<TdtDecodeState *> bp;
    std::vector<const float *> enc;
    std::vector<int> nf;
    for (int u = 0; u < ft.n; ++u) {
        tdt_init_state(tw, mt.blank_id, bst[u]);
        bp.push_back(&bst[u]);
        enc.push_back(ft.utt(u));
        nf.push_back(ft.T);
    }
    std::vector<std::vector<int32_t>> batch;
    std::vector<int> bsteps;
    if ((rc = tdt_decode_batch(mt, tw, enc, nf, ft.D, topt, bp, batch, bsteps))) return fail("tdt_decode_batch", rc);

    // value semantics: the first half of utterance 0 through `a`, then b = a
    // (a new slot holding a's state); b finishes first, then a; c is assigned
    // the half-way state over a state of its own and finishes last.
    const int half = (ft.T / 2 / W) * W > 0 ? (ft.T / 2 / W) * W : ft.T / 2;
    std::vector<int32_t> head, tail_a, tail_b, tail_c;
    TdtDecodeState a, c;
    tdt_init_state(tw, mt.blank_id, a);
    tdt_init_state(tw, mt.blank_id, c);
    int s = 0;
    if ((rc = tdt_decode_window(mt, tw, ft.utt(0), half, ft.D, topt, a, head, s))) return fail("head", rc);
    std::vector<int32_t> scratch;
    if ((rc = tdt_decode_window(mt, tw, ft.utt(1), 3, ft.D, topt, c, scratch, s))) return fail("c's own", rc);
    TdtDecodeState b = a;
    c = a;
    const int slots_distinct = a.slot.slot() != b.slot.slot() && a.slot.slot() != c.slot.slot() &&
                               b.slot.slot() != c.slot.slot();
    const float *rest = ft.utt(0) + (size_t)half * ft.D;
    if ((rc = tdt_decode_window(mt, tw, rest, ft.T - half, ft.D, topt, b, tail_b, s))) return fail("tail b", rc);
    if ((rc = tdt_decode_window(mt, tw, rest, ft.T - half, ft.D, topt, a, tail_a, s))) return fail("tail a", rc);
    if ((rc = tdt_decode_window(mt, tw, rest, ft.T - half, ft.D, topt, c, tail_c, s))) return fail("tail c", rc);
    std::vector<int32_t> bad;
    const int bad_dim_rc = tdt_decode_window(mt, tw, ft.utt(0), ft.T, ft.D + 1, topt, a, bad, s);

    // one launch per call: wall time of tdt_greedy_decode on utterance 0
    double us = 0.0;
    int tsteps = 0;
    for (int r = 0; r <= reps; ++r) {
        TdtDecodeResult res;
        const auto t0 = std::chrono::steady_clock::now();
        if ((rc = tdt_greedy_decode(mt, tw, ft.utt(0), ft.T, ft.D, topt, res))) return fail("timed decode", rc);
        const double dt = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        if (r > 0) us += dt;   // the first call is a warm-up
        tsteps = res.steps;
    }

    std::printf("{\"tdt\":{\"greedy\":");
    lists(greedy);
    std::printf(",\"chunked\":");
    lists(chunked);
    std::printf(",\"batch\":");
    lists(batch);
    std::printf(",\"steps\":");
    ints(steps);
    std::printf(",\"text\":[");
    for (int u = 0; u < ft.n; ++u) {
        if (u) std::printf(",");
        str(text[u]);
    }
    std::printf("],\"head\":");
    ints(head);
    std::printf(",\"tail_a\":");
    ints(tail_a);
    std::printf(",\"tail_b\":");
    ints(tail_b);
    std::printf(",\"tail_c\":");
    ints(tail_c);
    std::printf(",\"slots_distinct\":%d,\"bad_dim_rc\":%d,\"call_us\":%.3f,\"call_steps\":%d}", slots_distinct,
                bad_dim_rc, reps > 0 ? us / reps : 0.0, tsteps);

    // ---------------- EOU
    Loaded le;
    if ((rc = load(argv[3], le)) != 0) return fail("loading the EOU model", rc);
    const ParakeetCtcModel &me = le.model;
    EouRuntimeWeights ew;
    if ((rc = eou_prepare_runtime(me, ew)) != 0) return fail("eou_prepare_runtime", rc);
    EouDecodeOptions eopt;
    std::vector<std::vector<int32_t>> eg(fe.n), esg(fe.n), ec(fe.n), ecs(fe.n), eb, ebs(fe.n);
    std::vector<std::string> etext(fe.n);
    for (int u = 0; u < fe.n; ++u) {
        EouDecodeResult r;
        if ((rc = eou_greedy_decode(me, ew, fe.utt(u), fe.T, fe.D, eopt, r))) return fail("eou_greedy_decode", rc);
        eg[u] = r.token_ids;
        for (const auto &b : r.segments) esg[u].push_back(b.token_index);
        etext[u] = r.text;
        // windows into fresh vectors, as the Engine's streaming modes decode them
        EouDecodeState st;
        eou_init_state(ew, st);
        for (int t0 = 0; t0 < fe.T; t0 += W) {
            std::vector<int32_t> toks;
            std::vector<EouSegmentBoundary> segs;
            int es = 0;
            const int n = std::min(W, fe.T - t0);
            if ((rc = eou_decode_window(me, ew, fe.utt(u) + (size_t)t0 * fe.D, n, fe.D, eopt, st, toks, segs, es)))
                return fail("eou_decode_window", rc);
            ec[u].insert(ec[u].end(), toks.begin(), toks.end());
            for (const auto &b : segs) ecs[u].push_back(b.token_index);
        }
    }
    std::vector<EouDecodeState> est(fe.n);
    std::vector<EouDecodeState *> ep;
    std::vector<const float *> eenc;
    std::vector<int> enf;
    for (int u = 0; u < fe.n; ++u) {
        eou_init_state(ew, est[u]);
        ep.push_back(&est[u]);
        eenc.push_back(fe.utt(u));
        enf.push_back(fe.T);
    }
    std::vector<std::vector<EouSegmentBoundary>> eseg;
    std::vector<int> esteps;
    if ((rc = eou_decode_batch(me, ew, eenc, enf, fe.D, eopt, ep, eb, eseg, esteps)))
        return fail("eou_decode_batch", rc);
    for (int u = 0; u < fe.n; ++u)
        for (const auto &b : eseg[u]) ebs[u].push_back(b.token_index);

    std::printf(",\"eou\":{\"greedy\":");
    lists(eg);
    std::printf(",\"segments\":");
    lists(esg);
    std::printf(",\"chunked\":");
    lists(ec);
    std::printf(",\"chunked_segments\":");
    lists(ecs);
    std::printf(",\"batch\":");
    lists(eb);
    std::printf(",\"batch_segments\":");
    lists(ebs);
    std::printf(",\"text\":[");
    for (int u = 0; u < fe.n; ++u) {
        if (u) std::printf(",");
        str(etext[u]);
    }
    std::printf("],\"ids\":[%d,%d,%d]}}\n", ew.blank_id, ew.eou_id, ew.eob_id);
    return 0;
}

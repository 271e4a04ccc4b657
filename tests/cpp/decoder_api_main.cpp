// Drives the reference-shaped C++ decoder API (include/parakeet_decoder.h) the
// way parakeet.cpp's callers do, and prints what it returns as one JSON object:
//   - tdt_greedy_decode per utterance (src/parakeet_engine.cpp:273-297);
//   - tdt_init_state + tdt_decode_window over fixed-size windows (Mode 2,
//     src/parakeet_engine.cpp:409-452);
//   - tdt_decode_batch over all utterances;
//   - the same three for EOU, with segment boundaries;
//   - Engine::transcribe_features on the first TDT utterance;
//   - Engine::transcribe_features_stream (Mode 2) on the first TDT utterance, and
//     EOU FeatureStreamSessions (Mode 3) fed chunk by chunk: all sessions in one
//     launch per chunk, and one session per launch;
//   - the encoder output resident in device memory: tdt/eou_decode_batch_device
//     and Engine::transcribe_device_batch on ragged windows, beside the same
//     windows decoded from host memory, plus their argument checks.
// Usage: decoder_api_main TDT.gguf TDT_FRAMES EOU.gguf EOU_FRAMES WINDOW
//        decoder_api_main --bench-eou-stream EOU.gguf FRAMES CHUNK   (timing; see bench_eou_stream)
// Frame files: int32 n, T, D, then n*T*D float32 (utterance-major).
#include <cstdio>
#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <memory>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "parakeet_decoder.h"

namespace {

struct Frames {
    int n = 0, T = 0, D = 0;
    std::vector<float> data;
    const float *utt(int u) const { return data.data() + (size_t)u * T * D; }
};

bool read_frames(const char *path, Frames &f) {
    FILE *fp = fopen(path, "rb");
    if (!fp) return false;
    int hdr[3];
    bool ok = fread(hdr, 4, 3, fp) == 3;
    if (ok) {
        f.n = hdr[0];
        f.T = hdr[1];
        f.D = hdr[2];
        f.data.resize((size_t)f.n * f.T * f.D);
        ok = fread(f.data.data(), 4, f.data.size(), fp) == f.data.size();
    }
    fclose(fp);
    return ok;
}

void ints(const std::vector<int32_t> &v) {
    printf("[");
    for (size_t i = 0; i < v.size(); ++i) printf(i ? ",%d" : "%d", v[i]);
    printf("]");
}

void str(const std::string &s) {
    printf("\"");
    for (char c : s) {
        if (c == '"' || c == '\\') printf("\\%c", c);
        else printf("%c", c);
    }
    printf("\"");
}

struct SegLog {
    std::vector<parakeet_hip::StreamingSegment> segs;
    std::vector<parakeet_hip::StreamEvent> events;
};

void print_log(const SegLog &l) {
    printf("{\"segments\":[");
    for (size_t i = 0; i < l.segs.size(); ++i) {
        const auto &g = l.segs[i];
        printf(i ? ",{" : "{");
        printf("\"chunk\":%d,\"tokens\":", g.chunk_index);
        ints(g.token_ids);
        printf(",\"text\":");
        str(g.text);
        printf(",\"start\":%.6f,\"end\":%.6f,\"eou\":%d,\"final\":%d}", g.start_s, g.end_s,
               g.is_eou_boundary ? 1 : 0, g.is_final ? 1 : 0);
    }
    printf("],\"events\":[");
    for (size_t i = 0; i < l.events.size(); ++i) {
        const auto &e = l.events[i];
        printf(i ? ",{" : "{");
        printf("\"type\":%d,\"chunk\":%d,\"t\":%.6f,\"conf\":%.3f}", (int)e.type, e.chunk_index, e.timestamp_s,
               e.eot_confidence);
    }
    printf("]}");
}

int fail(const char *what, int rc) {
    fprintf(stderr, "%s failed: rc=%d\n", what, rc);
    return 1;
}

}  // namespace

// Ragged windows over utterance-major frames: utterance u decodes rows
// u*T .. u*T + len(u) (len(u) = T, 7T/8, 3T/4, 5T/8, ...).
int window_len(const Frames &f, int u) { return std::max(1, f.T - (u % 4) * (f.T / 8)); }

// Frames uploaded to device memory, freed with the object.
struct DeviceCopy {
    float *p = nullptr;
    bool ok = false;
    explicit DeviceCopy(const Frames &f) {
        const size_t bytes = f.data.size() * sizeof(float);
        ok = hipMalloc(reinterpret_cast<void **>(&p), bytes) == hipSuccess &&
             hipMemcpy(p, f.data.data(), bytes, hipMemcpyHostToDevice) == hipSuccess &&
             hipDeviceSynchronize() == hipSuccess;
    }
    ~DeviceCopy() { if (p) (void)hipFree(p); }
};

void int_lists(const std::vector<std::vector<int32_t>> &v) {
    printf("[");
    for (size_t u = 0; u < v.size(); ++u) {
        if (u) printf(",");
        ints(v[u]);
    }
    printf("]");
}

int device_section(const char *tdt_path, const char *eou_path, const Frames &ft, const Frames &fe) {
    using namespace parakeet_hip;
    int rc;
    DeviceCopy dt(ft), de(fe);
    if (!dt.ok || !de.ok) return fail("device copy of the frames", -1);
    // TDT: host windows and device rows, fresh states each
    DecoderModel tdt;
    if ((rc = load_from_gguf(tdt_path, tdt)) != 0) return fail("load_from_gguf(tdt)", rc);
    TdtRuntimeWeights tw;
    if ((rc = tdt_prepare_runtime(tdt, tw, 2 * ft.n + 4)) != 0) return fail("tdt_prepare_runtime", rc);
    const DeviceEncoderOutput dout{dt.p, (int64_t)ft.n * ft.T, ft.D};
    std::vector<const float *> hp;
    std::vector<int64_t> rows;
    std::vector<int> nf;
    for (int u = 0; u < ft.n; ++u) {
        hp.push_back(ft.utt(u));
        rows.push_back((int64_t)u * ft.T);
        nf.push_back(window_len(ft, u));
    }
    std::vector<std::vector<int32_t>> th, td;
    std::vector<int> sh, sd;
    {
        std::vector<TdtDecodeState> a(ft.n), b(ft.n);
        std::vector<TdtDecodeState *> pa, pb;
        for (int u = 0; u < ft.n; ++u) {
            pa.push_back(&a[u]);
            pb.push_back(&b[u]);
        }
        if ((rc = tdt_decode_batch(tdt, tw, hp, nf, ft.D, TdtDecodeOptions{}, pa, th, sh)) != 0)
            return fail("tdt_decode_batch", rc);
        if ((rc = tdt_decode_batch_device(tdt, tw, dout, rows, nf, TdtDecodeOptions{}, pb, td, sd)) != 0)
            return fail("tdt_decode_batch_device", rc);
    }
    printf("{\"tdt_host\":");
    int_lists(th);
    printf(",\"tdt_dev\":");
    int_lists(td);
    printf(",\"tdt_steps_host\":");
    ints(std::vector<int32_t>(sh.begin(), sh.end()));
    printf(",\"tdt_steps_dev\":");
    ints(std::vector<int32_t>(sd.begin(), sd.end()));
    {   // argument checks: a window past the end of the output, a d_model mismatch
        TdtDecodeState st;
        std::vector<std::vector<int32_t>> t;
        std::vector<int> s;
        const int rc_range = tdt_decode_batch_device(tdt, tw, dout, {(int64_t)ft.n * ft.T - 1}, {2}, TdtDecodeOptions{},
                                                     {&st}, t, s);
        DeviceEncoderOutput bad = dout;
        bad.d_model = ft.D + 1;
        const int rc_dim = tdt_decode_batch_device(tdt, tw, bad, {0}, {1}, TdtDecodeOptions{}, {&st}, t, s);
        printf(",\"rc_range\":%d,\"rc_dim\":%d", rc_range, rc_dim);
    }
    // EOU: the same with segment boundaries
    DecoderModel eou;
    if ((rc = load_from_gguf(eou_path, eou)) != 0) return fail("load_from_gguf(eou)", rc);
    EouRuntimeWeights ew;
    if ((rc = eou_prepare_runtime(eou, ew, 2 * fe.n + 4)) != 0) return fail("eou_prepare_runtime", rc);
    EouDecodeOptions eopt;
    eopt.max_symbols_per_step = eou.encoder_cfg.eou_max_symbols_per_step;
    const DeviceEncoderOutput eout{de.p, (int64_t)fe.n * fe.T, fe.D};
    std::vector<const float *> ehp;
    std::vector<int64_t> erows;
    std::vector<int> enf;
    for (int u = 0; u < fe.n; ++u) {
        ehp.push_back(fe.utt(u));
        erows.push_back((int64_t)u * fe.T);
        enf.push_back(window_len(fe, u));
    }
    std::vector<std::vector<int32_t>> eh, ed;
    std::vector<std::vector<EouSegmentBoundary>> gh, gd;
    std::vector<int> esh, esd;
    {
        std::vector<EouDecodeState> a(fe.n), b(fe.n);
        std::vector<EouDecodeState *> pa, pb;
        for (int u = 0; u < fe.n; ++u) {
            pa.push_back(&a[u]);
            pb.push_back(&b[u]);
        }
        if ((rc = eou_decode_batch(eou, ew, ehp, enf, fe.D, eopt, pa, eh, gh, esh)) != 0)
            return fail("eou_decode_batch", rc);
        if ((rc = eou_decode_batch_device(eou, ew, eout, erows, enf, eopt, pb, ed, gd, esd)) != 0)
            return fail("eou_decode_batch_device", rc);
    }
    auto seg_ints = [](const std::vector<std::vector<EouSegmentBoundary>> &g) {
        std::vector<std::vector<int32_t>> v(g.size());
        for (size_t u = 0; u < g.size(); ++u)
            for (auto &b : g[u]) v[u].push_back(b.token_index);
        return v;
    };
    printf(",\"eou_host\":");
    int_lists(eh);
    printf(",\"eou_dev\":");
    int_lists(ed);
    printf(",\"eou_seg_host\":");
    int_lists(seg_ints(gh));
    printf(",\"eou_seg_dev\":");
    int_lists(seg_ints(gd));
    // Engine over the TDT model
    try {
        EngineOptions eo;
        eo.model_gguf_path = tdt_path;
        eo.n_slots = 2 * ft.n + 4;
        Engine engine(eo);
        const std::vector<EngineResult> rh = engine.transcribe_features_batch(hp, nf, ft.D);
        const std::vector<EngineResult> rd = engine.transcribe_device_batch(dout, rows, nf);
        std::vector<std::vector<int32_t>> a, b;
        for (auto &r : rh) a.push_back(r.token_ids);
        for (auto &r : rd) b.push_back(r.token_ids);
        printf(",\"engine_host\":");
        int_lists(a);
        printf(",\"engine_dev\":");
        int_lists(b);
        printf(",\"engine_text_equal\":%d", (int)(rh.size() == rd.size() && !rh.empty() && rh[0].text == rd[0].text));
    } catch (const std::exception &e) {
        fprintf(stderr, "Engine (device frames): %s\n", e.what());
        return 1;
    }
    printf("}");
    return 0;
}

// --bench-eou-stream EOU.gguf FRAMES CHUNK: the streaming form of the EOU decode
// over an encoder output resident in device memory.  FRAMES holds n sessions of T
// frames; every session is fed T / CHUNK chunks of CHUNK frames, all sessions of a
// chunk in one eou_decode_batch_device call with their states carried (Mode 3 over
// many sessions at once, src/parakeet_engine.cpp:753-886).  The stream runs twice
// on fresh states (a warm-up, then the timed pass); one JSON line: wall time per
// chunk call (outputs back in the caller's vectors), decode steps.
int bench_eou_stream(int argc, char **argv) {
    if (argc != 5) return 2;
    using namespace parakeet_hip;
    Frames fe;
    if (!read_frames(argv[3], fe)) return fail("read frames", -1);
    const int F = atoi(argv[4]);
    if (F <= 0 || fe.T % F) return fail("chunk frames", -1);
    const int chunks = fe.T / F;
    DecoderModel eou;
    int rc;
    if ((rc = load_from_gguf(argv[2], eou)) != 0) return fail("load_from_gguf(eou)", rc);
    EouRuntimeWeights ew;
    if ((rc = eou_prepare_runtime(eou, ew, 2 * fe.n)) != 0) return fail("eou_prepare_runtime", rc);
    EouDecodeOptions eopt;
    eopt.max_symbols_per_step = eou.encoder_cfg.eou_max_symbols_per_step;
    float *d = nullptr;
    const size_t bytes = fe.data.size() * sizeof(float);
    if (hipMalloc(reinterpret_cast<void **>(&d), bytes) != hipSuccess ||
        hipMemcpy(d, fe.data.data(), bytes, hipMemcpyHostToDevice) != hipSuccess)
        return fail("device frames", -1);
    const DeviceEncoderOutput enc{d, (int64_t)fe.n * fe.T, fe.D};
    std::vector<int> nf(fe.n, F);
    std::vector<int64_t> rows(fe.n);
    double wall = 0.0, wmin = 1e30;
    long steps = 0, tokens = 0;
    for (int pass = 0; pass < 2; ++pass) {
        std::vector<EouDecodeState> st(fe.n);
        std::vector<EouDecodeState *> sp(fe.n);
        for (int u = 0; u < fe.n; ++u) {
            eou_init_state(ew, st[u]);
            sp[u] = &st[u];
        }
        for (int c = 0; c < chunks; ++c) {
            for (int u = 0; u < fe.n; ++u) rows[u] = (int64_t)u * fe.T + (int64_t)c * F;
            std::vector<std::vector<int32_t>> toks;
            std::vector<std::vector<EouSegmentBoundary>> segs;
            std::vector<int> stp;
            const auto t0 = std::chrono::steady_clock::now();
            if ((rc = eou_decode_batch_device(eou, ew, enc, rows, nf, eopt, sp, toks, segs, stp)) != 0)
                return fail("eou_decode_batch_device", rc);
            const double dt = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
            if (pass == 1) {
                wall += dt;
                wmin = std::min(wmin, dt);
                for (int u = 0; u < fe.n; ++u) {
                    steps += stp[u];
                    tokens += (long)toks[u].size();
                }
            }
        }
    }
    (void)hipFree(d);
    printf("{\"call_us\":%.3f,\"call_us_min\":%.3f,\"steps\":%ld,\"tokens\":%ld,\"sessions\":%d,"
           "\"chunks\":%d,\"frames_per_chunk\":%d}\n",
           wall / chunks, wmin, steps, tokens, fe.n, chunks, F);
    return 0;
}

int main(int argc, char **argv) {
    if (argc > 1 && std::string(argv[1]) == "--bench-eou-stream") return bench_eou_stream(argc, argv);
    if (argc != 6) {
        fprintf(stderr, "usage: %s TDT.gguf TDT_FRAMES EOU.gguf EOU_FRAMES WINDOW\n", argv[0]);
        return 2;
    }
    const int W = atoi(argv[5]);
    Frames ft, fe;
    if (!read_frames(argv[2], ft) || !read_frames(argv[4], fe)) return fail("read frames", -1);
    using namespace parakeet_hip;
    int rc;

    // ---- TDT ----
    DecoderModel tdt;
    if ((rc = load_from_gguf(argv[1], tdt)) != 0) return fail("load_from_gguf(tdt)", rc);
    TdtRuntimeWeights tw;
    if ((rc = tdt_prepare_runtime(tdt, tw, 2 * ft.n + 4)) != 0) return fail("tdt_prepare_runtime", rc);
    TdtDecodeOptions topt;
    printf("{\"tdt\":{\"greedy\":[");
    std::vector<int> steps;
    std::vector<std::string> texts;
    for (int u = 0; u < ft.n; ++u) {
        TdtDecodeResult r;
        if ((rc = tdt_greedy_decode(tdt, tw, ft.utt(u), ft.T, ft.D, topt, r)) != 0) return fail("tdt_greedy_decode", rc);
        if (u) printf(",");
        ints(r.token_ids);
        steps.push_back(r.steps);
        texts.push_back(r.text);
    }
    printf("],\"steps\":");
    ints(std::vector<int32_t>(steps.begin(), steps.end()));
    printf(",\"text\":[");
    for (size_t i = 0; i < texts.size(); ++i) {
        if (i) printf(",");
        str(texts[i]);
    }
    printf("],\"chunked\":[");
    for (int u = 0; u < ft.n; ++u) {
        TdtDecodeState st;
        tdt_init_state(tw, tdt.blank_id, st);
        std::vector<int32_t> all;
        for (int t0 = 0; t0 < ft.T; t0 += W) {
            const int n = std::min(W, ft.T - t0);
            std::vector<int32_t> toks;
            int s = 0;
            if ((rc = tdt_decode_window(tdt, tw, ft.utt(u) + (size_t)t0 * ft.D, n, ft.D, topt, st, toks, s)) != 0)
                return fail("tdt_decode_window", rc);
            all.insert(all.end(), toks.begin(), toks.end());
        }
        if (u) printf(",");
        ints(all);
    }
    printf("],\"batch\":[");
    {
        std::vector<TdtDecodeState> sts(ft.n);
        std::vector<TdtDecodeState *> ps;
        std::vector<const float *> enc;
        std::vector<int> nf;
        for (int u = 0; u < ft.n; ++u) {
            tdt_init_state(tw, tdt.blank_id, sts[u]);
            ps.push_back(&sts[u]);
            enc.push_back(ft.utt(u));
            nf.push_back(ft.T);
        }
        std::vector<std::vector<int32_t>> toks;
        std::vector<int> bs;
        if ((rc = tdt_decode_batch(tdt, tw, enc, nf, ft.D, topt, ps, toks, bs)) != 0) return fail("tdt_decode_batch", rc);
        for (int u = 0; u < ft.n; ++u) {
            if (u) printf(",");
            ints(toks[u]);
        }
    }
    printf("],\"bad_dim_rc\":");
    {
        TdtDecodeResult r;
        printf("%d", tdt_greedy_decode(tdt, tw, ft.utt(0), ft.T, ft.D + 1, topt, r));
    }
    printf("},");

    // ---- EOU ----
    DecoderModel eou;
    if ((rc = load_from_gguf(argv[3], eou)) != 0) return fail("load_from_gguf(eou)", rc);
    EouRuntimeWeights ew;
    if ((rc = eou_prepare_runtime(eou, ew, 2 * fe.n + 4)) != 0) return fail("eou_prepare_runtime", rc);
    EouDecodeOptions eopt;
    eopt.max_symbols_per_step = eou.encoder_cfg.eou_max_symbols_per_step;
    printf("\"eou\":{\"greedy\":[");
    std::vector<std::vector<int32_t>> segs;
    for (int u = 0; u < fe.n; ++u) {
        EouDecodeResult r;
        if ((rc = eou_greedy_decode(eou, ew, fe.utt(u), fe.T, fe.D, eopt, r)) != 0) return fail("eou_greedy_decode", rc);
        if (u) printf(",");
        ints(r.token_ids);
        std::vector<int32_t> b;
        for (auto &sb : r.segments) b.push_back(sb.token_index);
        segs.push_back(b);
    }
    printf("],\"segments\":[");
    for (size_t u = 0; u < segs.size(); ++u) {
        if (u) printf(",");
        ints(segs[u]);
    }
    printf("],\"chunked\":[");
    std::vector<std::vector<int32_t>> csegs;
    for (int u = 0; u < fe.n; ++u) {
        EouDecodeState st;
        eou_init_state(ew, st);
        std::vector<int32_t> all, bounds;
        for (int t0 = 0; t0 < fe.T; t0 += W) {
            const int n = std::min(W, fe.T - t0);
            std::vector<int32_t> toks;
            std::vector<EouSegmentBoundary> sb;
            int s = 0;
            if ((rc = eou_decode_window(eou, ew, fe.utt(u) + (size_t)t0 * fe.D, n, fe.D, eopt, st, toks, sb, s)) != 0)
                return fail("eou_decode_window", rc);
            all.insert(all.end(), toks.begin(), toks.end());
            for (auto &x : sb) bounds.push_back(x.token_index);
        }
        if (u) printf(",");
        ints(all);
        csegs.push_back(bounds);
    }
    printf("],\"chunked_segments\":[");
    for (size_t u = 0; u < csegs.size(); ++u) {
        if (u) printf(",");
        ints(csegs[u]);
    }
    printf("]},");

    // ---- Engine ----
    try {
        EngineOptions eo;
        eo.model_gguf_path = argv[1];
        eo.n_slots = 4;
        Engine engine(eo);
        EngineResult er = engine.transcribe_features(ft.utt(0), ft.T, ft.D);
        printf("\"engine\":{\"tokens\":");
        ints(er.token_ids);
        printf(",\"text\":");
        str(er.text);
        printf(",\"steps\":%d}", er.steps);

        // ---- streaming over features ----
        printf(",\"stream\":{\"tdt\":");
        SegLog tl;
        FeatureStreamOptions so;
        so.chunk_frames = W;
        EngineResult sr = engine.transcribe_features_stream(
            ft.utt(0), ft.T, ft.D, so, [&](const StreamingSegment &g) { tl.segs.push_back(g); });
        print_log(tl);
        printf(",\"tdt_tokens\":");
        ints(sr.token_ids);
        printf(",\"tdt_text\":");
        str(sr.text);
        printf(",\"tdt_steps\":%d,\"stride_ms\":%.6f", sr.steps, encoder_frame_stride_ms(engine.model()));

        EngineOptions eeo;
        eeo.model_gguf_path = argv[3];
        eeo.n_slots = 2 * fe.n + 4;
        Engine eng(eeo);
        for (int mode = 0; mode < 2; ++mode) {   // 0: all sessions per launch, 1: one per launch
            std::vector<SegLog> logs(fe.n);
            std::vector<std::unique_ptr<FeatureStreamSession>> ss;
            for (int u = 0; u < fe.n; ++u) {
                FeatureStreamOptions o;
                o.on_event = [&logs, u](const StreamEvent &ev) { logs[u].events.push_back(ev); };
                ss.push_back(eng.stream_start(o, [&logs, u](const StreamingSegment &g) { logs[u].segs.push_back(g); }));
            }
            for (int t0 = 0; t0 < fe.T; t0 += W) {
                const int n = std::min(W, fe.T - t0);
                if (mode == 0) {
                    std::vector<FeatureStreamSession *> ps;
                    std::vector<const float *> en;
                    std::vector<int> nf;
                    for (int u = 0; u < fe.n; ++u) {
                        ps.push_back(ss[u].get());
                        en.push_back(fe.utt(u) + (size_t)t0 * fe.D);
                        nf.push_back(n);
                    }
                    FeatureStreamSession::feed_frames_batch(ps, en, nf, fe.D);
                } else {
                    for (int u = 0; u < fe.n; ++u) ss[u]->feed_frames(fe.utt(u) + (size_t)t0 * fe.D, n, fe.D);
                }
            }
            printf(mode == 0 ? ",\"eou_batch\":[" : ",\"eou_single\":[");
            for (int u = 0; u < fe.n; ++u) {
                ss[u]->finalize();
                if (u) printf(",");
                print_log(logs[u]);
            }
            printf("]");
        }
        printf("}");
    } catch (const std::exception &e) {
        fprintf(stderr, "Engine: %s\n", e.what());
        return 1;
    }
    printf(",\"device\":");
    if ((rc = device_section(argv[1], argv[3], ft, fe)) != 0) return rc;
    printf("}\n");
    return 0;
}

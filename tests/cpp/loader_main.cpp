// Loads a GGUF with the reference-shaped loader (load_from_gguf,
// src/parakeet_ctc.cpp:297) and prints what it read as one JSON object, plus
// detokenize() of the token ids given after the path.  Host only: no device
// call is made.
// Usage: loader_main MODEL.gguf [id ...]
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "parakeet_decoder.h"

namespace {
void str(const std::string &s) {
    printf("\"");
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') printf("\\%c", c);
        else if (c < 0x20) printf("\\u%04x", c);
        else printf("%c", c);
    }
    printf("\"");
}
}  // namespace

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s MODEL.gguf [id ...]\n", argv[0]);
        return 2;
    }
    using namespace parakeet_hip;
    DecoderModel m;
    const int rc = load_from_gguf(argv[1], m);
    printf("{\"rc\":%d", rc);
    if (rc == 0) {
        const char *type[] = {"ctc", "tdt", "eou", "sortformer"};
        const EncoderConfig &c = m.encoder_cfg;
        printf(",\"type\":\"%s\",\"d_model\":%d,\"vocab\":%d,\"blank\":%d,\"eou\":%d,\"eob\":%d", type[(int)m.model_type],
               c.d_model, m.vocab_size, m.blank_id, m.eou_id, m.eob_id);
        printf(",\"tdt\":[%d,%d,%d,%d],\"eou_cfg\":[%d,%d,%d,%d]", c.tdt_pred_hidden, c.tdt_pred_rnn_layers,
               c.tdt_joint_hidden, c.tdt_num_durations, c.eou_pred_hidden, c.eou_pred_rnn_layers, c.eou_joint_hidden,
               c.eou_max_symbols_per_step);
        printf(",\"durations\":[");
        for (size_t i = 0; i < m.tdt_durations.size(); ++i) printf(i ? ",%d" : "%d", m.tdt_durations[i]);
        printf("],\"stride_ms\":%.6f,\"n_pieces\":%zu", encoder_frame_stride_ms(m), m.vocab.pieces.size());
        printf(",\"special\":[%d,%d,%d,%d]", m.vocab.unk_id, m.vocab.bos_id, m.vocab.eos_id, m.vocab.pad_id);
        std::vector<int32_t> ids;
        for (int i = 2; i < argc; ++i) ids.push_back(atoi(argv[i]));
        printf(",\"detok\":");
        str(detokenize(m.vocab, ids));
    }
    printf("}\n");
    return 0;
}

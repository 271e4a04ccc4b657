// Mutation fuzzer of the GGUF reader (gguf::File::parse) and of the decoder
// loader (load_from_gguf) on corrupted copies of a valid decoder GGUF.  Built
// with AddressSanitizer and UndefinedBehaviorSanitizer (host code only): any
// out-of-bounds access, overflow or bad allocation aborts the run.
//
// Each iteration mutates a copy of the seed: a truncation, byte flips, an
// extreme value written over a 4- or 8-byte field of the header (counts,
// lengths, dimensions, types, offsets), or a byte inserted / removed in the
// header.  The reader must either reject the copy or accept it with every
// tensor inside the buffer; every accepted tensor's first and last byte is
// read.  Every 8th copy also goes through load_from_gguf from a file.
//
// Usage: gguf_fuzz_main SEED.gguf ITERATIONS RNG_SEED SCRATCH_FILE
// Prints {"iterations":N,"accepted":A,"rejected":R,"loaded":L,"load_rejected":M}.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <random>
#include <string>
#include <vector>

#include "gguf_reader.h"
#include "parakeet_decoder.h"

namespace gguf = parakeet_hip::gguf;

int main(int argc, char **argv) {
    if (argc < 5) {
        std::fprintf(stderr, "usage: gguf_fuzz_main SEED.gguf ITERATIONS RNG_SEED SCRATCH_FILE\n");
        return 2;
    }
    std::ifstream in(argv[1], std::ios::binary);
    const std::vector<uint8_t> seed((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    const long iters = std::atol(argv[2]);
    std::mt19937_64 rng((uint64_t)std::atoll(argv[3]));
    const std::string scratch = argv[4];

    // the header ends where the first tensor's data starts
    size_t header = seed.size();
    {
        gguf::File f;
        std::string err;
        if (f.parse(seed, err)) {
            std::fprintf(stderr, "seed does not parse: %s\n", err.c_str());
            return 1;
        }
        for (const auto &kv : f.tensors()) header = std::min<size_t>(header, kv.second.offset);
    }
    static const uint64_t extremes[] = {0ull, 1ull, 2ull, 31ull, 32ull, 33ull, 0x7Full, 0xFFull, 0xFFFFull,
                                        0x7FFFFFFFull, 0x80000000ull, 0xFFFFFFFFull, 0x100000000ull,
                                        0x7FFFFFFFFFFFFFFFull, 0x8000000000000000ull, 0xFFFFFFFFFFFFFFFFull};
    long accepted = 0, rejected = 0, loaded = 0, load_rejected = 0;
    volatile uint8_t sink = 0;
    for (long it = 0; it < iters; ++it) {
        std::vector<uint8_t> b = seed;
        auto pick = [&](size_t n) { return n ? (size_t)(rng() % n) : 0; };
        switch (rng() % 5) {
            case 0:   // truncation
                b.resize(pick(b.size()));
                break;
            case 1: {   // byte flips, mostly in the header
                const int n = 1 + (int)(rng() % 8);
                for (int k = 0; k < n; ++k) {
                    const size_t at = (rng() % 4) ? pick(header) : pick(b.size());
                    b[at] ^= (uint8_t)(1u << (rng() % 8));
                }
                break;
            }
            case 2: {   // an extreme 8-byte value at a random header offset
                const size_t at = pick(header > 8 ? header - 8 : 1);
                const uint64_t v = extremes[rng() % (sizeof extremes / sizeof *extremes)];
                for (int k = 0; k < 8 && at + k < b.size(); ++k) b[at + k] = (uint8_t)(v >> (8 * k));
                break;
            }
            case 3: {   // an extreme 4-byte value
                const size_t at = pick(header > 4 ? header - 4 : 1);
                const uint32_t v = (uint32_t)extremes[rng() % (sizeof extremes / sizeof *extremes)];
                for (int k = 0; k < 4 && at + k < b.size(); ++k) b[at + k] = (uint8_t)(v >> (8 * k));
                break;
            }
            default: {   // a byte inserted or removed in the header
                const size_t at = pick(header);
                if (rng() % 2) b.insert(b.begin() + (long)at, (uint8_t)rng());
                else if (at < b.size()) b.erase(b.begin() + (long)at);
                break;
            }
        }
        gguf::File f;
        std::string err;
        if (f.parse(b, err) == 0) {
            ++accepted;
            for (const auto &kv : f.tensors()) {
                const gguf::Tensor &t = kv.second;
                sink ^= t.data[0];
                sink ^= t.data[t.nbytes - 1];
            }
            (void)f.get_u32("parakeet.tdt.vocab_size", 0);
            (void)f.get_str("parakeet.model.type", "");
            if (const gguf::Value *v = f.find("tokenizer.ggml.tokens")) sink ^= (uint8_t)v->arr_s.size();
        } else {
            ++rejected;
        }
        if (it % 8 == 0) {
            {
                std::ofstream out(scratch, std::ios::binary | std::ios::trunc);
                out.write(reinterpret_cast<const char *>(b.data()), (std::streamsize)b.size());
            }
            parakeet_hip::DecoderModel m;
            if (parakeet_hip::load_from_gguf(scratch, m) == 0) {
                ++loaded;
                std::vector<int32_t> ids;
                for (int k = -2; k < (int)m.vocab.pieces.size() + 2; k += 3) ids.push_back(k);
                sink ^= (uint8_t)parakeet_hip::detokenize(m.vocab, ids).size();
            } else {
                ++load_rejected;
            }
        }
    }
    std::printf("{\"iterations\":%ld,\"accepted\":%ld,\"rejected\":%ld,\"loaded\":%ld,\"load_rejected\":%ld}\n", iters,
                accepted, rejected, loaded, load_rejected);
    return 0;
}

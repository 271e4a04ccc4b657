// gguf_reader.h -- minimal GGUF v2/v3 reader for parakeet decoder tensors.
//
// Reads the metadata and tensor directory of a GGUF file and keeps the file
// bytes in memory.  Covers what the reference's loader reads for the
// transducer decoders (src/parakeet_ctc.cpp:297-682): scalar / string / array
// metadata and f32 / f16 / q4_0 / q5_0 / q8_0 tensors (ggml type ids 0, 1, 2, 6, 8).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace parakeet_hip {
namespace gguf {

struct Value {
    uint32_t type = 0;             // GGUF value type
    int64_t i = 0;                 // integer / bool scalars
    double f = 0.0;                // float scalars
    std::string s;                 // string scalar
    uint32_t arr_type = 0;         // array element type
    std::vector<int64_t> arr_i;    // integer arrays
    std::vector<std::string> arr_s;// string arrays
};

struct Tensor {
    std::string name;
    uint32_t type = 0;             // ggml type
    std::vector<int64_t> ne;       // innermost first
    uint64_t offset = 0;           // absolute offset in the file
    uint64_t nbytes = 0;
    const uint8_t *data = nullptr; // into File::bytes
};

class File {
public:
    // Returns 0 on success, non-zero with a message in err otherwise.
    int open(const std::string &path, std::string &err);
    // The same over the bytes of a file already in memory (kept by the File).
    int parse(std::vector<uint8_t> bytes, std::string &err);
    const Value *find(const std::string &key) const;
    const Tensor *tensor(const std::string &name) const;
    uint32_t get_u32(const std::string &key, uint32_t def) const;
    int32_t get_i32(const std::string &key, int32_t def) const;
    bool get_bool(const std::string &key, bool def) const;
    std::string get_str(const std::string &key, const std::string &def) const;
    const std::map<std::string, Tensor> &tensors() const { return tensors_; }

private:
    std::vector<uint8_t> bytes_;
    std::map<std::string, Value> kv_;
    std::map<std::string, Tensor> tensors_;
};

uint64_t tensor_nbytes(uint32_t type, int64_t n_elements);

}  // namespace gguf
}  // namespace parakeet_hip

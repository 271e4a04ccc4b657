// dropin_tensor.h -- the one ggml-dependent step of the drop-in decoder: the
// stored bytes of a GGUF tensor held by parakeet.cpp's model.
//
// ggml_tensor_bytes.cpp implements it with ggml inside parakeet.cpp's build
// (ggml_backend_tensor_get, as src/parakeet_tdt.cpp:78-95 reads the decoder
// tensors); a test links its own implementation for handles it made itself.
#pragma once

#include <cstdint>
#include <vector>

#include "parakeet_hip.h"

struct ggml_tensor;

namespace parakeet_hip {
namespace dropin {

// out <- the tensor's ggml type id, ne[0], ne[1] and a pointer to its stored
// bytes, copied into storage (which must outlive the use of out).  A null
// tensor gives an empty pk_tensor (data == nullptr).  Returns 0 or 2.
int tensor_bytes(const ggml_tensor *t, pk_tensor *out, std::vector<uint8_t> *storage);

}  // namespace dropin
}  // namespace parakeet_hip

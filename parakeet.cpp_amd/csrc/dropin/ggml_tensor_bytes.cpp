// ggml_tensor_bytes.cpp -- dropin::tensor_bytes over ggml, compiled inside
// parakeet.cpp's own build (it needs ggml.h / ggml-backend.h, which that
// build provides).  The bytes are read with ggml_backend_tensor_get whatever
// backend holds the tensor, as src/parakeet_tdt.cpp:78-95 does.
#include "dropin_tensor.h"

#include "ggml-backend.h"
#include "ggml.h"

namespace parakeet_hip {
namespace dropin {

int tensor_bytes(const ggml_tensor *t, pk_tensor *out, std::vector<uint8_t> *storage) {
    *out = pk_tensor{};
    if (!t) return 0;
    storage->resize(ggml_nbytes(t));
    ggml_backend_tensor_get(t, storage->data(), 0, storage->size());
    out->data = storage->data();
    out->type = (int32_t)t->type;   // pk_tensor types are ggml type ids
    out->ne0 = t->ne[0];
    out->ne1 = t->ne[1];
    return 0;
}

}  // namespace dropin
}  // namespace parakeet_hip

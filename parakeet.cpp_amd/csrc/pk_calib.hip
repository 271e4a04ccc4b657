// pk_calib.hip -- a plain device-to-device copy of known size.
//
// Hardware byte counters (FETCH_SIZE / WRITE_SIZE) are read per dispatch in
// units whose exact scale is set by the counter block.  Reading the same
// counters for this copy, whose traffic is exactly `bytes` read plus `bytes`
// written, gives the factor that turns them into HBM bytes for the decode
// kernels profiled in the same run.  Not part of the decoder ABI.
#include <hip/hip_runtime.h>

#include <cstddef>

__global__ void __launch_bounds__(256) calib_copy_kernel(const float4 *__restrict src, float4 *__restrict dst,
                                                         size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// Copies `bytes` (a multiple of 16) from src to dst; both device pointers.
// Returns 0, or the HIP error code.
extern "C" int pk_calib_copy(void *dst, const void *src, size_t bytes) {
    if (bytes % 16 != 0 || !dst || !src) return (int)hipErrorInvalidValue;
    const size_t n = bytes / 16;
    calib_copy_kernel<<<2048, 256>>>(static_cast<const float4 *>(src), static_cast<float4 *>(dst), n);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return (int)e;
}

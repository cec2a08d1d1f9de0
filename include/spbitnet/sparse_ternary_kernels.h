// spbitnet/sparse_ternary_kernels.h -- drop-in C++17 host API for the
// MI355X build, over the C ABI in spbitnet_amd.h.
//
// Same namespace, names, argument order and meaning as the reference's
// include/spbitnet/sparse_ternary_kernels.h:16-48, with hipStream_t in place of
// cudaStream_t (the quantiser and the other per-op wrappers are in
// spbitnet/inference_kernels.h, as in the reference).  Error behaviour matches the reference's CUDA_CHECK
// (include/spbitnet/cuda_utils.h:13-21): a failing call prints the error and
// exits the process; rows == 0 or cols == 0 is a no-op.  Callers that prefer
// status codes use the C ABI directly.
//
// Link with spbitnet_amd/libspbitnet_amd.so.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "spbitnet_amd.h"

namespace spbitnet {

namespace detail {
inline void check(int rc, const char* what, const char* file, int line) {
    if (rc != 0) {
        std::fprintf(stderr, "HIP error at %s:%d (%s): %s\n", file, line, what,
                     spb_last_error_string());
        std::exit(EXIT_FAILURE);
    }
}
inline const uint16_t* bits(const half* p) { return reinterpret_cast<const uint16_t*>(p); }
inline uint16_t* bits(half* p) { return reinterpret_cast<uint16_t*>(p); }
inline const uint16_t* bits(const __hip_bfloat16* p) {
    return reinterpret_cast<const uint16_t*>(p);
}
inline uint16_t* bits(__hip_bfloat16* p) { return reinterpret_cast<uint16_t*>(p); }
}  // namespace detail

#define SPBITNET_AMD_CHECK(call) ::spbitnet::detail::check((call), #call, __FILE__, __LINE__)

// reference include/spbitnet/sparse_ternary_kernels.h:16-19
inline void sparse_ternary_unpack_gpu(const uint32_t* meta, const uint32_t* values, int8_t* out,
                                      int rows, int cols, int meta_row_stride,
                                      int values_row_stride, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_sparse_ternary_unpack(meta, values, out, rows, cols, meta_row_stride,
                                                 values_row_stride, stream));
}

// reference include/spbitnet/sparse_ternary_kernels.h:29-33
inline void sparse_ternary_gemv_gpu(const uint32_t* meta, const uint32_t* values,
                                    const int8_t* x, int32_t* y, int rows, int cols,
                                    int meta_row_stride, int values_row_stride,
                                    hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_sparse_ternary_gemv(meta, values, x, y, rows, cols, meta_row_stride,
                                               values_row_stride, stream));
}

// reference include/spbitnet/sparse_ternary_kernels.h:43-48 (fp16 activations)
inline void fused_sparse_bitlinear_gpu(const uint32_t* meta, const uint32_t* values,
                                       const half* x, half* output, const float* d_absmax,
                                       float gamma, int rows, int cols, int meta_row_stride,
                                       int values_row_stride, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_fused_sparse_bitlinear_f16(meta, values, detail::bits(x),
                                                      detail::bits(output), d_absmax, gamma,
                                                      rows, cols, meta_row_stride,
                                                      values_row_stride, stream));
}

// bf16 activations (same semantics; the bf16 decode configuration)
inline void fused_sparse_bitlinear_gpu(const uint32_t* meta, const uint32_t* values,
                                       const __hip_bfloat16* x, __hip_bfloat16* output,
                                       const float* d_absmax, float gamma, int rows, int cols,
                                       int meta_row_stride, int values_row_stride,
                                       hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_fused_sparse_bitlinear_bf16(meta, values, detail::bits(x),
                                                       detail::bits(output), d_absmax, gamma,
                                                       rows, cols, meta_row_stride,
                                                       values_row_stride, stream));
}

}  // namespace spbitnet

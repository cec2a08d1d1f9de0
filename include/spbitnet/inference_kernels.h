// spbitnet/inference_kernels.h -- drop-in C++17 host API for the MI355X
// build, over the C ABI in spbitnet_amd.h.
//
// Same namespace, names, argument order and meaning as the reference's
// include/spbitnet/inference_kernels.h:14-89, with hipStream_t in place of
// cudaStream_t; every function has a half overload (the reference's type) and
// a __hip_bfloat16 overload.  Error behaviour matches the reference's
// CUDA_CHECK (include/spbitnet/cuda_utils.h:13-21): a failing call prints the
// error and exits.  Callers that prefer status codes use the C ABI.
//
// Link with spbitnet_amd/libspbitnet_amd.so.
#pragma once

#include "spbitnet/sparse_ternary_kernels.h"

namespace spbitnet {

// reference include/spbitnet/inference_kernels.h:19-20
inline void absmax_quantize_gpu(const half* input, int8_t* output, float* d_absmax, int size,
                                hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_absmax_quantize_f16(detail::bits(input), output, d_absmax, size, stream));
}
inline void absmax_quantize_gpu(const __hip_bfloat16* input, int8_t* output, float* d_absmax,
                                int size, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_absmax_quantize_bf16(detail::bits(input), output, d_absmax, size, stream));
}

// reference include/spbitnet/inference_kernels.h:24-25
inline void absmax_reduce_gpu(const half* input, float* d_absmax, int size,
                              hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_absmax_reduce_f16(detail::bits(input), d_absmax, size, stream));
}
inline void absmax_reduce_gpu(const __hip_bfloat16* input, float* d_absmax, int size,
                              hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_absmax_reduce_bf16(detail::bits(input), d_absmax, size, stream));
}

// reference include/spbitnet/inference_kernels.h:29-30
inline void dequantize_gpu(const int32_t* input, half* output, const float* d_absmax,
                           float gamma, int size, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_dequantize_f16(input, detail::bits(output), d_absmax, gamma, size, stream));
}
inline void dequantize_gpu(const int32_t* input, __hip_bfloat16* output, const float* d_absmax,
                           float gamma, int size, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_dequantize_bf16(input, detail::bits(output), d_absmax, gamma, size, stream));
}

// reference include/spbitnet/inference_kernels.h:14-15
inline void rms_norm_gpu(const half* input, const float* weight, half* output, int size,
                         float eps, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_rms_norm_f16(detail::bits(input), weight, detail::bits(output), size,
                                        eps, stream));
}
inline void rms_norm_gpu(const __hip_bfloat16* input, const float* weight, __hip_bfloat16* output,
                         int size, float eps, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_rms_norm_bf16(detail::bits(input), weight, detail::bits(output), size,
                                         eps, stream));
}

// reference include/spbitnet/inference_kernels.h:33-34
inline void rope_gpu(half* vec, int num_heads, int head_dim, int pos, float theta,
                     hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_rope_f16(detail::bits(vec), num_heads, head_dim, pos, theta, stream));
}
inline void rope_gpu(__hip_bfloat16* vec, int num_heads, int head_dim, int pos, float theta,
                     hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_rope_bf16(detail::bits(vec), num_heads, head_dim, pos, theta, stream));
}

// reference include/spbitnet/inference_kernels.h:38-40
inline void scatter_kv_gpu(const half* src, half* cache, int num_kv_heads, int head_dim,
                           int max_seq_len, int pos, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_scatter_kv(detail::bits(src), detail::bits(cache), num_kv_heads,
                                      head_dim, max_seq_len, pos, stream));
}
inline void scatter_kv_gpu(const __hip_bfloat16* src, __hip_bfloat16* cache, int num_kv_heads,
                           int head_dim, int max_seq_len, int pos, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_scatter_kv(detail::bits(src), detail::bits(cache), num_kv_heads,
                                      head_dim, max_seq_len, pos, stream));
}

// reference include/spbitnet/inference_kernels.h:45-48
inline void attention_scores_gpu(const half* Q, const half* K_cache, float* scores, int num_heads,
                                 int num_kv_heads, int head_dim, int max_seq_len, int seq_len,
                                 float scale, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_attention_scores_f16(detail::bits(Q), detail::bits(K_cache), scores,
                                                num_heads, num_kv_heads, head_dim, max_seq_len,
                                                seq_len, scale, stream));
}
inline void attention_scores_gpu(const __hip_bfloat16* Q, const __hip_bfloat16* K_cache,
                                 float* scores, int num_heads, int num_kv_heads, int head_dim,
                                 int max_seq_len, int seq_len, float scale,
                                 hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_attention_scores_bf16(detail::bits(Q), detail::bits(K_cache), scores,
                                                 num_heads, num_kv_heads, head_dim, max_seq_len,
                                                 seq_len, scale, stream));
}

// reference include/spbitnet/inference_kernels.h:52-53
inline void softmax_gpu(float* scores, int num_heads, int max_seq_len, int seq_len,
                        hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_softmax(scores, num_heads, max_seq_len, seq_len, stream));
}

// reference include/spbitnet/inference_kernels.h:58-61
inline void attention_output_gpu(const float* scores, const half* V_cache, half* output,
                                 int num_heads, int num_kv_heads, int head_dim, int max_seq_len,
                                 int seq_len, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_attention_output_f16(scores, detail::bits(V_cache), detail::bits(output),
                                                num_heads, num_kv_heads, head_dim, max_seq_len,
                                                seq_len, stream));
}
inline void attention_output_gpu(const float* scores, const __hip_bfloat16* V_cache,
                                 __hip_bfloat16* output, int num_heads, int num_kv_heads,
                                 int head_dim, int max_seq_len, int seq_len,
                                 hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_attention_output_bf16(scores, detail::bits(V_cache),
                                                 detail::bits(output), num_heads, num_kv_heads,
                                                 head_dim, max_seq_len, seq_len, stream));
}

// reference include/spbitnet/inference_kernels.h:64-65
inline void relu2_mul_gpu(const half* gate, const half* up, half* output, int size,
                          hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_relu2_mul_f16(detail::bits(gate), detail::bits(up), detail::bits(output),
                                         size, stream));
}
inline void relu2_mul_gpu(const __hip_bfloat16* gate, const __hip_bfloat16* up,
                          __hip_bfloat16* output, int size, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_relu2_mul_bf16(detail::bits(gate), detail::bits(up),
                                          detail::bits(output), size, stream));
}

// reference include/spbitnet/inference_kernels.h:70-71
inline void relu2_mul_f32_gpu(const half* gate, const half* up, float* output, int size,
                              hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_relu2_mul_f32_f16(detail::bits(gate), detail::bits(up), output, size, stream));
}
inline void relu2_mul_f32_gpu(const __hip_bfloat16* gate, const __hip_bfloat16* up, float* output,
                              int size, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_relu2_mul_f32_bf16(detail::bits(gate), detail::bits(up), output, size, stream));
}

// reference include/spbitnet/inference_kernels.h:75-76
inline void rms_norm_f32in_gpu(const float* input, const float* weight, half* output, int size,
                               float eps, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_rms_norm_f32in_f16(input, weight, detail::bits(output), size, eps, stream));
}
inline void rms_norm_f32in_gpu(const float* input, const float* weight, __hip_bfloat16* output,
                               int size, float eps, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(
        spb_rms_norm_f32in_bf16(input, weight, detail::bits(output), size, eps, stream));
}

// reference include/spbitnet/inference_kernels.h:79-80 (and its bf16 counterpart)
inline void float_to_half_gpu(const float* input, half* output, int size,
                              hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_float_to_f16(input, detail::bits(output), size, stream));
}
inline void float_to_half_gpu(const float* input, __hip_bfloat16* output, int size,
                              hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_float_to_bf16(input, detail::bits(output), size, stream));
}

// reference include/spbitnet/inference_kernels.h:83-84
inline void residual_add_gpu(const half* a, const half* b, half* output, int size,
                             hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_residual_add_f16(detail::bits(a), detail::bits(b), detail::bits(output),
                                            size, stream));
}
inline void residual_add_gpu(const __hip_bfloat16* a, const __hip_bfloat16* b,
                             __hip_bfloat16* output, int size, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_residual_add_bf16(detail::bits(a), detail::bits(b),
                                             detail::bits(output), size, stream));
}

// reference include/spbitnet/inference_kernels.h:87-89
inline void half_gemv_gpu(const half* W, const half* x, float* y, int rows, int cols,
                          hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_gemv_f16(detail::bits(W), detail::bits(x), y, rows, cols, stream));
}
inline void half_gemv_gpu(const __hip_bfloat16* W, const __hip_bfloat16* x, float* y, int rows,
                          int cols, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_gemv_bf16(detail::bits(W), detail::bits(x), y, rows, cols, stream));
}

// Device argmax for greedy decoding (no reference wrapper: the reference
// copies the logits to the host, src/main.cpp:194-200).
inline void argmax_gpu(const float* x, int n, int* out_index, hipStream_t stream = nullptr) {
    SPBITNET_AMD_CHECK(spb_argmax_f32(x, n, out_index, stream));
}

}  // namespace spbitnet

// quant.hip -- per-token absmax reduction, int8 quantisation and int32
// dequantisation (reference src/kernels/inference_kernels.cu:69-171).
//
// absmax is a max over |x|: exact and order-independent, so the reduction
// tree is free.  One 1024-thread block per vector (16 waves): the vectors on
// this path are a hidden or FFN activation of one token (2560 or 6912
// elements), which one workgroup reads in a few hundred nanoseconds.
#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

template <class T>
__global__ __launch_bounds__(kRedBlock) void absmax_reduce_kernel(const uint16_t* __restrict__ x,
                                                                  float* __restrict__ d_absmax,
                                                                  int n) {
    const float m = block_absmax<T>(x, n);
    if (threadIdx.x == 0) *d_absmax = m;
}

template <class T>
__global__ __launch_bounds__(kRedBlock) void absmax_quantize_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ d_absmax, int n) {
    const float m = block_absmax<T>(x, n);
    if (threadIdx.x == 0) *d_absmax = m;
    const float scale = quant_scale(m);
    for (int i = threadIdx.x; i < n; i += kRedBlock)
        q[i] = static_cast<int8_t>(quant_round_clamp(T::to_float(x[i]) * scale));
}

template <class T>
__global__ __launch_bounds__(256) void dequantize_kernel(const int32_t* __restrict__ in,
                                                         uint16_t* __restrict__ out,
                                                         const float* __restrict__ d_absmax,
                                                         float gamma, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float s = dequant_scale(gamma, *d_absmax);
    out[i] = T::from_float(static_cast<float>(in[i]) * s);
}

template <class T>
int absmax_reduce(const char* fn, const uint16_t* x, float* d_absmax, int n, hipStream_t st) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!x || !d_absmax) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(absmax_reduce_kernel<T>, dim3(1), dim3(kRedBlock), 0, st, x, d_absmax, n);
    return launch_status(fn);
}

template <class T>
int absmax_quantize(const char* fn, const uint16_t* x, int8_t* q, float* d_absmax, int n,
                    hipStream_t st) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!x || !q || !d_absmax) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(absmax_quantize_kernel<T>, dim3(1), dim3(kRedBlock), 0, st, x, q,
                       d_absmax, n);
    return launch_status(fn);
}

template <class T>
int dequantize(const char* fn, const int32_t* in, uint16_t* out, const float* d_absmax,
               float gamma, int n, hipStream_t st) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!in || !out || !d_absmax) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(dequantize_kernel<T>, dim3((n + 255) / 256), dim3(256), 0, st, in, out,
                       d_absmax, gamma, n);
    return launch_status(fn);
}

}  // namespace
}  // namespace spb

using namespace spb;

extern "C" int spb_absmax_reduce_f16(const uint16_t* x, float* d_absmax, int n, spb_stream_t s) {
    return absmax_reduce<F16>("spb_absmax_reduce_f16", x, d_absmax, n, as_stream(s));
}
extern "C" int spb_absmax_reduce_bf16(const uint16_t* x, float* d_absmax, int n, spb_stream_t s) {
    return absmax_reduce<BF16>("spb_absmax_reduce_bf16", x, d_absmax, n, as_stream(s));
}
extern "C" int spb_absmax_quantize_f16(const uint16_t* x, int8_t* q, float* d_absmax, int n,
                                       spb_stream_t s) {
    return absmax_quantize<F16>("spb_absmax_quantize_f16", x, q, d_absmax, n, as_stream(s));
}
extern "C" int spb_absmax_quantize_bf16(const uint16_t* x, int8_t* q, float* d_absmax, int n,
                                        spb_stream_t s) {
    return absmax_quantize<BF16>("spb_absmax_quantize_bf16", x, q, d_absmax, n, as_stream(s));
}
extern "C" int spb_dequantize_f16(const int32_t* in, uint16_t* out, const float* d_absmax,
                                  float gamma, int n, spb_stream_t s) {
    return dequantize<F16>("spb_dequantize_f16", in, out, d_absmax, gamma, n, as_stream(s));
}
extern "C" int spb_dequantize_bf16(const int32_t* in, uint16_t* out, const float* d_absmax,
                                   float gamma, int n, spb_stream_t s) {
    return dequantize<BF16>("spb_dequantize_bf16", in, out, d_absmax, gamma, n, as_stream(s));
}

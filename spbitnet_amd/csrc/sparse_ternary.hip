// sparse_ternary.hip -- 2:4 sparse-ternary unpack, GEMV and fused BitLinear
// for gfx950 (MI355X).
//
// What the reference computes (src/kernels/sparse_ternary.cu:116-234):
//   y[r] = sum_g  (s_lo ? -1 : 1) * x[4g+p0] + (s_hi ? -1 : 1) * x[4g+p1]
// with p0 < p1 the two set bits of group g's 4-bit bitmap.  The sum is exact
// int32 arithmetic, so any evaluation order gives the same bits.
//
// How it is computed here (bit-plane kernel):
//   * A meta word is directly a 32-column keep mask K (bit j <=> column
//     32w+j kept).  The 2-bit sign pairs are expanded in registers into a
//     mask M holding each kept column's sign bit, with nibble-parallel bit
//     tricks and no lookup table: D = K - 0x1111_1111 clears the lower kept
//     bit of every group and keeps the higher one (no borrow crosses a
//     nibble since each holds two set bits), so M = D ? s_hi : s_lo.
//   * The int8 activations are used as 8 bit planes (X_b: bit j = bit b of
//     column j's two's-complement byte).  For the columns of a meta word,
//     with P / N the kept columns holding +1 / -1,
//       sum_{j in P} x_j - sum_{j in N} x_j
//         = sum_b c_b * popc((X_b & P) | (~X_b & N)) + popc(N),
//     c_b = 2^b (b < 7), c_7 = -128, and (X_b & P) | (~X_b & N) = K & (X_b ^ M):
//     one v_bitop3_b32 and one accumulating v_bcnt_u32_b32 per plane per 32
//     columns, additions and bit operations only, no multiplies on the
//     activations.  popc(N) is the number of set sign bits.
//   * Plane layouts.  Global "activation planes" format: word [w * 8 + b]
//     holds plane b of columns 32w .. 32w+31 (the 8 planes of a 128-column
//     chunk are 128 contiguous bytes).  In LDS the planes are plane-major,
//     word (b, w) at b * (cols / 32) + w, so a thread reads its chunk with one
//     16-byte read per plane and neighbouring chunks fall in neighbouring
//     banks (the global layout would put every chunk of a wave in the same
//     banks).  Planes come either from a prologue that transposes the
//     activations 8 columns per thread (SWAR 8x8 bit transpose,
//     lane-parallel, one load per thread), or precomputed in global memory by
//     spb_activation_planes / spb_absmax_quantize_planes_* and rearranged on
//     the copy into LDS.
//   * Work mapping (streaming kernel): a thread owns one 128-column chunk
//     (16 bytes of meta, 8 of signs, 128/64-bit buffer loads) and keeps that
//     chunk's 32 plane words in registers for every row it visits;
//     consecutive threads take consecutive chunks of consecutive rows, so
//     each load instruction of a block reads one contiguous span.  Each block
//     streams a contiguous range of rows with three steps of loads in flight;
//     per-row partial sums meet in LDS (integer atomics: exact in any order).
// Shapes the bit-plane kernel does not take (cols % 128 != 0, cols > 32768,
// unaligned rows or activations) go to a general wave-per-row kernel.
#include "bitplane.hpp"
#include "spbitnet_amd.h"

namespace spb {

namespace {

// ---- activation planes in global memory ------------------------------------------

// The 8 plane words of one 32-column group g: 4 x (8-column load, transpose),
// byte gathers, two 16-byte stores.  Columns at or beyond cols read as 0
// (cols % 8 == 0).
template <class Src>
__device__ __forceinline__ void group_planes(const Src& src, int g, int cols, uint32_t* out) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int c0 = g * 32 + k * 8;
        if (c0 < cols) {
            src.load8(c0, lo[k], hi[k]);
        } else {
            lo[k] = 0;
            hi[k] = 0;
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) transpose8x8(lo[k], hi[k]);
    uint32_t w[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        // perm(a, b, sel): selector bytes 0..3 pick b's bytes, 4..7 a's, 0x0C -> 0.
        const uint32_t s01 = 0x0C0C0000u | ((4u + b) << 8) | b;      // [k0.b, k1.b, 0, 0]
        const uint32_t s23 = ((4u + b) << 24) | (b << 16) | 0x0C0Cu;  // [0, 0, k2.b, k3.b]
        w[b] = __builtin_amdgcn_perm(lo[1], lo[0], s01) | __builtin_amdgcn_perm(lo[3], lo[2], s23);
        w[b + 4] =
            __builtin_amdgcn_perm(hi[1], hi[0], s01) | __builtin_amdgcn_perm(hi[3], hi[2], s23);
    }
    uint4* o = reinterpret_cast<uint4*>(out + g * 8);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

__global__ __launch_bounds__(256) void activation_planes_kernel(Int8Src src, uint32_t* planes,
                                                                int cols) {
    const int ngroups = (cols + 31) >> 5;
    for (int g = blockIdx.x * 256 + threadIdx.x; g < ngroups; g += gridDim.x * 256)
        group_planes(src, g, cols, planes);
}

// absmax + int8 quantisation (reference src/kernels/inference_kernels.cu:69-114)
// emitting the plane layout, and optionally the int8 vector too; one block.
template <class T>
__global__ __launch_bounds__(kRedBlock) void absmax_quantize_planes_kernel(
    const uint16_t* __restrict__ x, uint32_t* __restrict__ planes, int8_t* __restrict__ q,
    float* __restrict__ d_absmax, int n) {
    const float m = block_absmax<T>(x, n);
    if (threadIdx.x == 0) *d_absmax = m;
    const QuantSrc<T> src{x, nullptr, quant_scale(m)};
    const int ngroups = (n + 31) >> 5;
    for (int g = threadIdx.x; g < ngroups; g += kRedBlock) group_planes(src, g, n, planes);
    if (q)
        for (int i = threadIdx.x; i < n; i += kRedBlock) q[i] = static_cast<int8_t>(src.load(i));
}

// ---- unpack -------------------------------------------------------------------

__global__ __launch_bounds__(256) void unpack_kernel(Weights wt, int8_t* out) {
    const long gid = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    const int gpr = wt.cols >> 2;
    if (gid >= static_cast<long>(wt.rows) * gpr) return;
    const long row = gid / gpr;
    const int g = static_cast<int>(gid - row * gpr);
    const uint32_t bm = (wt.meta[row * wt.ms + (g >> 3)] >> ((g & 7) * 4)) & 0xFu;
    const uint32_t sg = (wt.values[row * wt.vs + (g >> 4)] >> ((g & 15) * 2)) & 0x3u;
    const bool ok = __builtin_popcount(bm) == 2;
    const int p0 = ok ? __builtin_ctz(bm) : 0;
    const int p1 = ok ? __builtin_ctz(bm & (bm - 1)) : 0;
    int8_t v[4] = {0, 0, 0, 0};
    v[p0] = (sg & 1u) ? -1 : 1;
    v[p1] = (sg & 2u) ? -1 : 1;  // for (0,0) the second write wins, as in the reference
    int8_t* dst = out + row * wt.cols + 4 * g;
    const uint32_t packed = static_cast<uint8_t>(v[0]) | (static_cast<uint8_t>(v[1]) << 8) |
                            (static_cast<uint8_t>(v[2]) << 16) |
                            (static_cast<uint32_t>(static_cast<uint8_t>(v[3])) << 24);
    if ((reinterpret_cast<uintptr_t>(dst) & 3u) == 0) {
        *reinterpret_cast<uint32_t*>(dst) = packed;
    } else {
        for (int i = 0; i < 4; ++i) dst[i] = v[i];
    }
}

template <class T>
int fused_bitlinear(const char* fn, const uint32_t* meta, const uint32_t* values,
                    const uint16_t* x, uint16_t* output, const float* d_absmax, float gamma,
                    int rows, int cols, int ms, int vs, spb_stream_t stream) {
    clear_error();
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !output || !d_absmax) return invalid("%s: null pointer argument", fn);
    const Weights wt{meta, values, rows, cols, ms, vs};
    const QuantSrc<T> src{x, d_absmax, 0.0f};
    const DequantSink<T> sink{output, d_absmax, gamma, 0.0f};
    if (bitplane_ok(meta, values, cols, ms, vs) && aligned(x, 16))
        launch_stream(wt, BuildPlanes<QuantSrc<T>>{src}, sink, as_stream(stream));
    else
        launch_general(wt, src, sink, as_stream(stream));
    return launch_status(fn);
}

template <class T>
int fused_bitlinear_planes(const char* fn, const uint32_t* meta, const uint32_t* values,
                           const uint32_t* planes, uint16_t* output, const float* d_absmax,
                           float gamma, int rows, int cols, int ms, int vs, spb_stream_t stream) {
    clear_error();
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!planes || !output || !d_absmax) return invalid("%s: null pointer argument", fn);
    if (!aligned(planes, 16)) return invalid("%s: planes must be 16-byte aligned", fn);
    const Weights wt{meta, values, rows, cols, ms, vs};
    const DequantSink<T> sink{output, d_absmax, gamma, 0.0f};
    if (bitplane_ok(meta, values, cols, ms, vs))
        launch_stream(wt, GlobalPlanes{planes}, sink, as_stream(stream));
    else
        launch_general(wt, PlaneSrc{planes}, sink, as_stream(stream));
    return launch_status(fn);
}

template <class T>
int absmax_quantize_planes(const char* fn, const uint16_t* x, uint32_t* planes, int8_t* q,
                           float* d_absmax, int n, spb_stream_t stream) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (n % 8) return invalid("%s: size=%d is not a multiple of 8", fn, n);
    if (!x || !planes || !d_absmax) return invalid("%s: null pointer", fn);
    if (!aligned(x, 16) || !aligned(planes, 16))
        return invalid("%s: input and planes must be 16-byte aligned", fn);
    hipLaunchKernelGGL(absmax_quantize_planes_kernel<T>, dim3(1), dim3(kRedBlock), 0,
                       as_stream(stream), x, planes, q, d_absmax, n);
    return launch_status(fn);
}

}  // namespace
}  // namespace spb

using namespace spb;

extern "C" int spb_sparse_ternary_gemv_kernel_id(const uint32_t* meta, const uint32_t* values,
                                                 int rows, int cols, int ms, int vs) {
    (void)rows;
    return bitplane_ok(meta, values, cols, ms, vs) ? 1 : 0;
}

extern "C" int spb_sparse_ternary_unpack(const uint32_t* meta, const uint32_t* values,
                                         int8_t* out, int rows, int cols, int ms, int vs,
                                         spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_ternary_unpack";
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!out) return invalid("%s: null output", fn);
    const long groups = static_cast<long>(rows) * (cols / 4);
    const long blocks = (groups + 255) / 256;
    hipLaunchKernelGGL(unpack_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                       Weights{meta, values, rows, cols, ms, vs}, out);
    return launch_status(fn);
}

extern "C" int spb_sparse_ternary_gemv(const uint32_t* meta, const uint32_t* values,
                                       const int8_t* x, int32_t* y, int rows, int cols, int ms,
                                       int vs, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_ternary_gemv";
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !y) return invalid("%s: null activation or output pointer", fn);
    const Weights wt{meta, values, rows, cols, ms, vs};
    if (bitplane_ok(meta, values, cols, ms, vs) && aligned(x, 16))
        launch_stream(wt, BuildPlanes<Int8Src>{Int8Src{x}}, Int32Sink{y}, as_stream(stream));
    else
        launch_general(wt, Int8Src{x}, Int32Sink{y}, as_stream(stream));
    return launch_status(fn);
}

extern "C" int spb_sparse_ternary_gemv_resident(const uint32_t* meta, const uint32_t* values,
                                                const int8_t* x, int32_t* y, int rows, int cols,
                                                int ms, int vs, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_ternary_gemv_resident";
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !y) return invalid("%s: null activation or output pointer", fn);
    const Weights wt{meta, values, rows, cols, ms, vs};
    if (bitplane_ok(meta, values, cols, ms, vs) && aligned(x, 16))
        launch_stream<BuildPlanes<Int8Src>, Int32Sink, kResidentLoadPolicy>(
            wt, BuildPlanes<Int8Src>{Int8Src{x}}, Int32Sink{y}, as_stream(stream));
    else
        launch_general(wt, Int8Src{x}, Int32Sink{y}, as_stream(stream));
    return launch_status(fn);
}

extern "C" int spb_sparse_ternary_gemv_planes(const uint32_t* meta, const uint32_t* values,
                                              const uint32_t* planes, int32_t* y, int rows,
                                              int cols, int ms, int vs, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_ternary_gemv_planes";
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!planes || !y) return invalid("%s: null planes or output pointer", fn);
    if (!aligned(planes, 16)) return invalid("%s: planes must be 16-byte aligned", fn);
    const Weights wt{meta, values, rows, cols, ms, vs};
    if (bitplane_ok(meta, values, cols, ms, vs))
        launch_stream(wt, GlobalPlanes{planes}, Int32Sink{y}, as_stream(stream));
    else
        launch_general(wt, PlaneSrc{planes}, Int32Sink{y}, as_stream(stream));
    return launch_status(fn);
}

extern "C" int spb_fused_sparse_bitlinear_f16(const uint32_t* meta, const uint32_t* values,
                                              const uint16_t* x, uint16_t* output,
                                              const float* d_absmax, float gamma, int rows,
                                              int cols, int ms, int vs, spb_stream_t stream) {
    return fused_bitlinear<F16>("spb_fused_sparse_bitlinear_f16", meta, values, x, output,
                                d_absmax, gamma, rows, cols, ms, vs, stream);
}

extern "C" int spb_fused_sparse_bitlinear_bf16(const uint32_t* meta, const uint32_t* values,
                                               const uint16_t* x, uint16_t* output,
                                               const float* d_absmax, float gamma, int rows,
                                               int cols, int ms, int vs, spb_stream_t stream) {
    return fused_bitlinear<BF16>("spb_fused_sparse_bitlinear_bf16", meta, values, x, output,
                                 d_absmax, gamma, rows, cols, ms, vs, stream);
}

extern "C" int spb_fused_sparse_bitlinear_planes_f16(const uint32_t* meta,
                                                     const uint32_t* values,
                                                     const uint32_t* planes, uint16_t* output,
                                                     const float* d_absmax, float gamma,
                                                     int rows, int cols, int ms, int vs,
                                                     spb_stream_t stream) {
    return fused_bitlinear_planes<F16>("spb_fused_sparse_bitlinear_planes_f16", meta, values,
                                       planes, output, d_absmax, gamma, rows, cols, ms, vs,
                                       stream);
}

extern "C" int spb_fused_sparse_bitlinear_planes_bf16(const uint32_t* meta,
                                                      const uint32_t* values,
                                                      const uint32_t* planes, uint16_t* output,
                                                      const float* d_absmax, float gamma,
                                                      int rows, int cols, int ms, int vs,
                                                      spb_stream_t stream) {
    return fused_bitlinear_planes<BF16>("spb_fused_sparse_bitlinear_planes_bf16", meta, values,
                                        planes, output, d_absmax, gamma, rows, cols, ms, vs,
                                        stream);
}

extern "C" int spb_activation_planes(const int8_t* x, uint32_t* planes, int cols,
                                     spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_activation_planes";
    if (cols < 0) return invalid("%s: negative size", fn);
    if (cols == 0) return 0;
    if (cols % 8) return invalid("%s: cols=%d is not a multiple of 8", fn, cols);
    if (!x || !planes) return invalid("%s: null pointer", fn);
    if (!aligned(x, 8) || !aligned(planes, 16))
        return invalid("%s: x must be 8-byte and planes 16-byte aligned", fn);
    const int groups = (cols + 31) / 32;
    const int blocks = (groups + 255) / 256;
    hipLaunchKernelGGL(activation_planes_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                       Int8Src{x}, planes, cols);
    return launch_status(fn);
}

extern "C" int spb_absmax_quantize_planes_f16(const uint16_t* input, uint32_t* planes,
                                              int8_t* output, float* d_absmax, int size,
                                              spb_stream_t stream) {
    return absmax_quantize_planes<F16>("spb_absmax_quantize_planes_f16", input, planes, output,
                                       d_absmax, size, stream);
}

extern "C" int spb_absmax_quantize_planes_bf16(const uint16_t* input, uint32_t* planes,
                                               int8_t* output, float* d_absmax, int size,
                                               spb_stream_t stream) {
    return absmax_quantize_planes<BF16>("spb_absmax_quantize_planes_bf16", input, planes,
                                        output, d_absmax, size, stream);
}

// Batched add/sub GEMM: the bit-plane GEMV kernel with tokens on grid.y (each
// token's activations decoded into planes by its own blocks; weights re-read
// per token from L2).  X token-major [n][cols] int8, Y token-major [n][rows].
extern "C" int spb_sparse_ternary_gemm_addsub(const uint32_t* meta, const uint32_t* values,
                                              const int8_t* X, int32_t* Y, int rows, int cols,
                                              int n, int ms, int vs, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_ternary_gemm_addsub";
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (n < 0) return invalid("%s: negative batch", fn);
    if (rows == 0 || cols == 0 || n == 0) return 0;
    if (!X || !Y) return invalid("%s: null activation or output pointer", fn);
    if (n > 65535) return invalid("%s: batch %d exceeds 65535", fn, n);
    if (!bitplane_ok(meta, values, cols, ms, vs) || !aligned(X, 16) || (cols % 16))
        return invalid("%s: needs cols %% 128 == 0, aligned rows and 16-byte aligned X", fn);
    Int8Src src{X};
    src.token_stride = cols;
    Int32Sink sink{Y};
    sink.token_stride = rows;
    launch_bitplane(Weights{meta, values, rows, cols, ms, vs}, BuildPlanes<Int8Src>{src}, sink,
                    as_stream(stream), n);
    return launch_status(fn);
}

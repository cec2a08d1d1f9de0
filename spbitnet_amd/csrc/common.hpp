// common.hpp -- shared device helpers and C-ABI error plumbing for the
// gfx950 sparse-ternary library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

namespace spb {

constexpr int kWave = 64;  // CDNA wavefront width

// ---- error reporting (per host thread) -------------------------------------

void set_error(const char* fmt, ...);
void clear_error();
const char* last_error();

// Returns hipErrorInvalidValue after recording a message.
int invalid(const char* fmt, ...);

// Checks the launch status and records it.
int launch_status(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of compute units of the current device (cached per device).
int device_cu_count();

// LDS bytes per compute unit of the current device (cached per device).
int device_lds_per_cu();

}  // namespace spb

struct spb_sparse_linear;

namespace spb {

// Up to three stacked projections with equal columns and strides in one
// matrix-core GEMM launch (gemm.hip); 1 = not possible (nothing launched),
// 2 = launch error, 0 = launched.  Y is [n][sum of rows].
int gemm_stacked(const spb_sparse_linear* const* segs, int nseg, const int8_t* X, int32_t* Y,
                 int n, hipStream_t st);

// Raises the LDS limit of the matrix-core GEMM kernels that need more than
// 64 KB on the current device (idempotent; 0 = done).  Engines call it before
// capturing graphs, so no attribute change happens inside a capture.
int gemm_prepare();

// ---- 16-bit float conversions (bit patterns in uint16_t) --------------------

struct F16 {
    static __device__ __forceinline__ float to_float(uint16_t b) {
        return static_cast<float>(__builtin_bit_cast(_Float16, b));
    }
    // IEEE round-to-nearest-even of a float32 value, as __float2half.  The
    // empty asm keeps f an already-rounded float32: without it the backend
    // folds a preceding float multiply into v_fma_mixlo_f16, which rounds the
    // exact product once to fp16 instead of rounding to fp32 and then fp16.
    static __device__ __forceinline__ uint16_t from_float(float f) {
        asm("" : "+v"(f));
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
    }
};

struct BF16 {
    static __device__ __forceinline__ float to_float(uint16_t b) {
        return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
    }
    // Round to nearest even; a NaN keeps its sign and upper payload bits and
    // becomes quiet ((bits >> 16) | 0x40).  One v_cvt_pk_bf16_f32 on gfx950,
    // whose results equal that rule's for all 2^32 float inputs (compared
    // exhaustively on an MI355X); the integer form took ~6 instructions.
    static __device__ __forceinline__ uint16_t from_float(float f) {
        return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
    }
};

// ---- activation quantisation, shared by every kernel that quantises --------
// scale = absmax > 0 ? 127/absmax : 0 (correctly rounded float32 divide), and
// q = clamp(rint_ne(x * scale), -128, 127); NaN products give -128, which is
// what clamping the INT_MIN that __float2int_rn returns for NaN produces
// (reference src/kernels/sparse_ternary.cu:199, 214-217).
__device__ __forceinline__ float quant_scale(float absmax) {
    return absmax > 0.0f ? 127.0f / absmax : 0.0f;
}

__device__ __forceinline__ int quant_round_clamp(float v) {
    float r = __builtin_rintf(v);
    r = __builtin_fmaxf(r, -128.0f);  // maxnum: NaN -> -128
    r = __builtin_fminf(r, 127.0f);
    return static_cast<int>(r);
}

// (gamma * absmax) / 127, each step rounded to float32
// (reference src/kernels/sparse_ternary.cu:231, inference_kernels.cu:169).
__device__ __forceinline__ float dequant_scale(float gamma, float absmax) {
    const float ga = gamma * absmax;
    return ga / 127.0f;
}

// ---- wave64 reductions -------------------------------------------------------

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// max |x| over x[0..n) for a block of kRedBlock threads; every thread gets
// the result.  Exact and order-independent (a max of absolute values).
constexpr int kRedBlock = 1024;

template <class T>
__device__ __forceinline__ float block_absmax(const uint16_t* __restrict__ x, int n) {
    __shared__ float part[kRedBlock / kWave];
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += kRedBlock) m = __builtin_fmaxf(m, __builtin_fabsf(T::to_float(x[i])));
    m = wave_max(m);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) part[wave] = m;
    __syncthreads();
    float r = lane < kRedBlock / kWave ? part[lane] : 0.0f;
    r = wave_max(r);
    return r;  // every thread holds the block result
}

}  // namespace spb

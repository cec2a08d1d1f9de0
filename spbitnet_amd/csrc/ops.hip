// ops.hip -- the reference's per-op inference kernels
// (include/spbitnet/inference_kernels.h:14-87, src/kernels/inference_kernels.cu)
// as C-ABI entry points for fp16 and bf16 storage, for callers that keep the
// reference engine's op-by-op dataflow.  The fused decode engine (engine.hip)
// does not call these; they are the drop-in replacements of the individual
// wrappers.
//
// Semantics follow the reference kernels (formula, operation order, storage
// type of every output); arithmetic is float32.  Differences by design:
// 1/sqrt is correctly rounded where the reference uses rsqrtf, and reductions
// use wave-64 trees.  Shapes are validated on the host; every kernel bounds-
// checks its own indices.
#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

constexpr int kOpBlock = 256;
constexpr int kNormBlock = 1024;

template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wave-64 sum (pairwise tree over adjacent lanes; every lane gets the result).
__device__ __forceinline__ float wsum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wmax(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

template <int kThreads, bool kMax>
__device__ __forceinline__ float block_reduce(float v, float* slot) {
    v = kMax ? wmax(v) : wsum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) slot[threadIdx.x / kWave] = v;
    __syncthreads();
    float s = slot[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) s = kMax ? fmaxf(s, slot[w]) : s + slot[w];
    return s;
}

struct F32 {
    static __device__ __forceinline__ float to_float(float v) { return v; }
};

// rms_norm_kernel / rms_norm_f32in_kernel (inference_kernels.cu:15-56, 418-455):
// y = T((x * inv) * w), inv = 1 / sqrt(mean(x^2) + eps).  One block; input
// and output may alias (each element is read before the thread that reads
// it writes it).
template <class T, class In, class InT>
__global__ __launch_bounds__(kNormBlock) void rms_norm_kernel(const InT* x, const float* w,
                                                              uint16_t* y, int n, float eps) {
    __shared__ float slot[kNormBlock / kWave];
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += kNormBlock) {
        const float v = In::to_float(x[i]);
        ss = fmaf(v, v, ss);
    }
    ss = block_reduce<kNormBlock, false>(ss, slot);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
    __syncthreads();  // every thread has read its inputs before any output aliasing them
    for (int i = threadIdx.x; i < n; i += kNormBlock)
        y[i] = T::from_float((In::to_float(x[i]) * inv) * w[i]);
}

// rope_kernel (inference_kernels.cu:185-206): pair (2i, 2i+1) of each head
// rotated by angle pos * theta^(-2i/hd), in place.
template <class T>
__global__ __launch_bounds__(kOpBlock) void rope_kernel(uint16_t* v, int nheads, int hd, int pos,
                                                        float theta) {
    const int t = blockIdx.x * kOpBlock + threadIdx.x;
    const int half = hd / 2;
    if (t >= nheads * half) return;
    const int head = t / half, pair = t - head * half;
    const float freq =
        1.0f / powf(theta, static_cast<float>(2 * pair) / static_cast<float>(hd));
    const float angle = static_cast<float>(pos) * freq;
    float s, c;
    sincosf(angle, &s, &c);
    const int idx = head * hd + 2 * pair;
    const float x0 = T::to_float(v[idx]), x1 = T::to_float(v[idx + 1]);
    v[idx] = T::from_float(x0 * c - x1 * s);
    v[idx + 1] = T::from_float(x0 * s + x1 * c);
}

// scatter_kv_kernel (inference_kernels.cu:215-227)
__global__ __launch_bounds__(kOpBlock) void scatter_kv_kernel(const uint16_t* src, uint16_t* cache,
                                                              int nkv, int hd, int max_seq,
                                                              int pos) {
    const int t = blockIdx.x * kOpBlock + threadIdx.x;
    if (t >= nkv * hd) return;
    const int h = t / hd, d = t - h * hd;
    cache[(static_cast<long>(h) * max_seq + pos) * hd + d] = src[t];
}

// attention_scores_kernel (inference_kernels.cu:241-275): one wave per
// (position, head); lanes over head_dim; GQA kv = h * nkv / nh.
template <class T>
__global__ __launch_bounds__(kOpBlock) void attention_scores_kernel(
    const uint16_t* Q, const uint16_t* K, float* scores, int nh, int nkv, int hd, int max_seq,
    int seq_len, float scale) {
    const int lane = threadIdx.x & (kWave - 1);
    const int j = blockIdx.x * (kOpBlock / kWave) + threadIdx.x / kWave;
    const int h = blockIdx.y;
    if (j >= seq_len) return;
    const int kvh = h * nkv / nh;
    const uint16_t* q = Q + static_cast<long>(h) * hd;
    const uint16_t* k = K + (static_cast<long>(kvh) * max_seq + j) * hd;
    float acc = 0.0f;
    for (int d = lane; d < hd; d += kWave) acc = fmaf(T::to_float(q[d]), T::to_float(k[d]), acc);
    acc = wsum(acc);
    if (lane == 0) scores[static_cast<long>(h) * max_seq + j] = acc * scale;
}

// softmax_kernel (inference_kernels.cu:283-339): per head, in place over the
// first seq_len entries: max, exp, sum, multiply by 1/sum.
__global__ __launch_bounds__(kNormBlock) void softmax_kernel(float* scores, int max_seq,
                                                             int seq_len) {
    __shared__ float slot[2][kNormBlock / kWave];
    float* hs = scores + static_cast<long>(blockIdx.x) * max_seq;
    float m = -INFINITY;
    for (int j = threadIdx.x; j < seq_len; j += kNormBlock) m = fmaxf(m, hs[j]);
    m = block_reduce<kNormBlock, true>(m, slot[0]);
    float s = 0.0f;
    for (int j = threadIdx.x; j < seq_len; j += kNormBlock) {
        const float e = expf(hs[j] - m);
        hs[j] = e;
        s += e;
    }
    s = block_reduce<kNormBlock, false>(s, slot[1]);
    const float inv = 1.0f / s;
    for (int j = threadIdx.x; j < seq_len; j += kNormBlock) hs[j] *= inv;
}

// attention_output_kernel (inference_kernels.cu:350-371):
// out[h][d] = sum_j score[h][j] * V[kv_h][j][d].  One block per head; wave w
// takes positions w, w + 4, ...; lane d, d + 64, ...; wave partials summed
// in LDS (head_dim <= 256).
template <class T>
__global__ __launch_bounds__(kOpBlock) void attention_output_kernel(
    const float* scores, const uint16_t* V, uint16_t* out, int nh, int nkv, int hd, int max_seq,
    int seq_len) {
    __shared__ float part[kOpBlock / kWave][256];
    const int h = blockIdx.x, lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int kvh = h * nkv / nh;
    const float* p = scores + static_cast<long>(h) * max_seq;
    const uint16_t* v = V + static_cast<long>(kvh) * max_seq * hd;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = wave; j < seq_len; j += kOpBlock / kWave) {
        const float pj = p[j];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = lane + r * kWave;
            if (d < hd) acc[r] = fmaf(pj, T::to_float(v[static_cast<long>(j) * hd + d]), acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int d = lane + r * kWave;
        if (d < hd) part[wave][d] = acc[r];
    }
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += kOpBlock) {
        float s = part[0][d];
#pragma unroll
        for (int w = 1; w < kOpBlock / kWave; ++w) s += part[w][d];
        out[static_cast<long>(h) * hd + d] = T::from_float(s);
    }
}

// relu2_mul_kernel / relu2_mul_f32_kernel (inference_kernels.cu:380-410)
template <class T, bool kF32Out>
__global__ __launch_bounds__(kOpBlock) void relu2_mul_kernel(const uint16_t* g, const uint16_t* u,
                                                             void* out, long n) {
    for (long i = static_cast<long>(blockIdx.x) * kOpBlock + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * kOpBlock) {
        const float r = fmaxf(0.0f, T::to_float(g[i]));
        const float v = (r * r) * T::to_float(u[i]);
        if (kF32Out)
            static_cast<float*>(out)[i] = v;
        else
            static_cast<uint16_t*>(out)[i] = T::from_float(v);
    }
}

// float_to_half_kernel (inference_kernels.cu:460-466)
template <class T>
__global__ __launch_bounds__(kOpBlock) void float_to_16_kernel(const float* x, uint16_t* y, long n) {
    for (long i = static_cast<long>(blockIdx.x) * kOpBlock + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * kOpBlock)
        y[i] = T::from_float(x[i]);
}

// residual_add_kernel (inference_kernels.cu:471-479): T(float(a) + float(b))
template <class T>
__global__ __launch_bounds__(kOpBlock) void residual_add_kernel(const uint16_t* a, const uint16_t* b,
                                                                uint16_t* y, long n) {
    for (long i = static_cast<long>(blockIdx.x) * kOpBlock + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * kOpBlock)
        y[i] = T::from_float(T::to_float(a[i]) + T::to_float(b[i]));
}

// half_gemv_kernel (inference_kernels.cu:488-531): y[r] = sum_c W[r][c] x[c]
// in float32, one wave per row; 16-byte chunks when rows are 16-byte aligned.
template <class T>
__global__ __launch_bounds__(kOpBlock) void gemv16_kernel(const uint16_t* W, const uint16_t* x,
                                                          float* y, int rows, int cols,
                                                          bool vec) {
    const int lane = threadIdx.x & (kWave - 1);
    const long r = static_cast<long>(blockIdx.x) * (kOpBlock / kWave) + threadIdx.x / kWave;
    if (r >= rows) return;
    const uint16_t* w = W + r * cols;
    float acc = 0.0f;
    int tail = 0;
    if (vec) {
        const int nch = cols >> 3;
        for (int c = lane; c < nch; c += kWave) {
            const uint4 a = reinterpret_cast<const uint4*>(w)[c];
            const uint4 b = reinterpret_cast<const uint4*>(x)[c];
            const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                acc = fmaf(T::to_float(static_cast<uint16_t>(aw[k] & 0xFFFFu)),
                           T::to_float(static_cast<uint16_t>(bw[k] & 0xFFFFu)), acc);
                acc = fmaf(T::to_float(static_cast<uint16_t>(aw[k] >> 16)),
                           T::to_float(static_cast<uint16_t>(bw[k] >> 16)), acc);
            }
        }
        tail = nch << 3;
    }
    for (int c = tail + lane; c < cols; c += kWave) acc = fmaf(T::to_float(w[c]), T::to_float(x[c]), acc);
    acc = wsum(acc);
    if (lane == 0) y[r] = acc;
}

// Greedy token pick: index of the maximum (lowest index among equal maxima,
// as std::max_element in src/main.cpp:194-200); NaN entries never win.
__global__ __launch_bounds__(kNormBlock) void argmax_kernel(const float* x, int n, int* out) {
    __shared__ float sv[kNormBlock / kWave];
    __shared__ int si[kNormBlock / kWave];
    float b = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += kNormBlock)
        if (x[i] > b) {  // ascending per thread: strict > keeps the first
            b = x[i];
            bi = i;
        }
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const float ov = __shfl_xor(b, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (ov > b || (ov == b && oi < bi)) {
            b = ov;
            bi = oi;
        }
    }
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) {
        sv[wave] = b;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kNormBlock / kWave; ++w)
            if (sv[w] > b || (sv[w] == b && si[w] < bi)) {
                b = sv[w];
                bi = si[w];
            }
        *out = bi == 0x7FFFFFFF ? 0 : bi;
    }
}

int grid_for(long n) {
    long g = (n + kOpBlock - 1) / kOpBlock;
    return static_cast<int>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <class T, class In, class InT>
int rms_norm(const char* fn, const InT* x, const float* w, uint16_t* y, int n, float eps,
             spb_stream_t s) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!x || !w || !y) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL((rms_norm_kernel<T, In, InT>), dim3(1), dim3(kNormBlock), 0, as_stream(s),
                       x, w, y, n, eps);
    return launch_status(fn);
}

template <class T>
int rope(const char* fn, uint16_t* v, int nh, int hd, int pos, float theta, spb_stream_t s) {
    clear_error();
    if (nh < 0 || hd < 0 || pos < 0) return invalid("%s: negative argument", fn);
    if (hd % 2) return invalid("%s: head_dim must be even", fn);
    if (nh == 0 || hd == 0) return 0;
    if (!v) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(rope_kernel<T>, dim3(grid_for(static_cast<long>(nh) * hd / 2)),
                       dim3(kOpBlock), 0, as_stream(s), v, nh, hd, pos, theta);
    return launch_status(fn);
}

int check_attn(const char* fn, int nh, int nkv, int hd, int max_seq, int seq_len) {
    if (nh <= 0 || nkv <= 0 || hd <= 0 || max_seq <= 0)
        return invalid("%s: non-positive dimension", fn);
    if (seq_len < 0 || seq_len > max_seq) return invalid("%s: seq_len outside [0, max_seq]", fn);
    if (nkv > nh) return invalid("%s: more kv heads than heads", fn);
    return 0;
}

template <class T>
int attention_scores(const char* fn, const uint16_t* Q, const uint16_t* K, float* sc, int nh,
                     int nkv, int hd, int max_seq, int seq_len, float scale, spb_stream_t s) {
    clear_error();
    if (int e = check_attn(fn, nh, nkv, hd, max_seq, seq_len)) return e;
    if (seq_len == 0) return 0;
    if (!Q || !K || !sc) return invalid("%s: null pointer", fn);
    const dim3 grid((seq_len + kOpBlock / kWave - 1) / (kOpBlock / kWave), nh);
    hipLaunchKernelGGL(attention_scores_kernel<T>, grid, dim3(kOpBlock), 0, as_stream(s), Q, K, sc,
                       nh, nkv, hd, max_seq, seq_len, scale);
    return launch_status(fn);
}

template <class T>
int attention_output(const char* fn, const float* sc, const uint16_t* V, uint16_t* out, int nh,
                     int nkv, int hd, int max_seq, int seq_len, spb_stream_t s) {
    clear_error();
    if (int e = check_attn(fn, nh, nkv, hd, max_seq, seq_len)) return e;
    if (hd > 256) return invalid("%s: head_dim %d > 256", fn, hd);
    if (!sc || !V || !out) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(attention_output_kernel<T>, dim3(nh), dim3(kOpBlock), 0, as_stream(s), sc, V,
                       out, nh, nkv, hd, max_seq, seq_len);
    return launch_status(fn);
}

template <class T, bool kF32>
int relu2_mul(const char* fn, const uint16_t* g, const uint16_t* u, void* out, int n,
              spb_stream_t s) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!g || !u || !out) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL((relu2_mul_kernel<T, kF32>), dim3(grid_for(n)), dim3(kOpBlock), 0,
                       as_stream(s), g, u, out, static_cast<long>(n));
    return launch_status(fn);
}

template <class T>
int float_to_16(const char* fn, const float* x, uint16_t* y, int n, spb_stream_t s) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!x || !y) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(float_to_16_kernel<T>, dim3(grid_for(n)), dim3(kOpBlock), 0, as_stream(s), x,
                       y, static_cast<long>(n));
    return launch_status(fn);
}

template <class T>
int residual_add(const char* fn, const uint16_t* a, const uint16_t* b, uint16_t* y, int n,
                 spb_stream_t s) {
    clear_error();
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!a || !b || !y) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(residual_add_kernel<T>, dim3(grid_for(n)), dim3(kOpBlock), 0, as_stream(s),
                       a, b, y, static_cast<long>(n));
    return launch_status(fn);
}

template <class T>
int gemv16(const char* fn, const uint16_t* W, const uint16_t* x, float* y, int rows, int cols,
           spb_stream_t s) {
    clear_error();
    if (rows < 0 || cols < 0) return invalid("%s: negative shape", fn);
    if (rows == 0) return 0;
    if (!W || !x || !y) return invalid("%s: null pointer", fn);
    const bool vec = cols % 8 == 0 && al16(W) && al16(x);
    const long blocks = (static_cast<long>(rows) + kOpBlock / kWave - 1) / (kOpBlock / kWave);
    hipLaunchKernelGGL(gemv16_kernel<T>, dim3(blocks), dim3(kOpBlock), 0, as_stream(s), W, x, y,
                       rows, cols, vec);
    return launch_status(fn);
}

}  // namespace
}  // namespace spb

using namespace spb;

extern "C" {

int spb_rms_norm_f16(const uint16_t* x, const float* w, uint16_t* y, int size, float eps,
                     spb_stream_t s) {
    return rms_norm<F16, F16, uint16_t>("spb_rms_norm_f16", x, w, y, size, eps, s);
}
int spb_rms_norm_bf16(const uint16_t* x, const float* w, uint16_t* y, int size, float eps,
                      spb_stream_t s) {
    return rms_norm<BF16, BF16, uint16_t>("spb_rms_norm_bf16", x, w, y, size, eps, s);
}
int spb_rms_norm_f32in_f16(const float* x, const float* w, uint16_t* y, int size, float eps,
                           spb_stream_t s) {
    return rms_norm<F16, F32, float>("spb_rms_norm_f32in_f16", x, w, y, size, eps, s);
}
int spb_rms_norm_f32in_bf16(const float* x, const float* w, uint16_t* y, int size, float eps,
                            spb_stream_t s) {
    return rms_norm<BF16, F32, float>("spb_rms_norm_f32in_bf16", x, w, y, size, eps, s);
}
int spb_rope_f16(uint16_t* v, int nh, int hd, int pos, float theta, spb_stream_t s) {
    return rope<F16>("spb_rope_f16", v, nh, hd, pos, theta, s);
}
int spb_rope_bf16(uint16_t* v, int nh, int hd, int pos, float theta, spb_stream_t s) {
    return rope<BF16>("spb_rope_bf16", v, nh, hd, pos, theta, s);
}
int spb_scatter_kv(const uint16_t* src, uint16_t* cache, int nkv, int hd, int max_seq, int pos,
                   spb_stream_t s) {
    clear_error();
    const char* fn = "spb_scatter_kv";
    if (nkv < 0 || hd < 0 || max_seq < 0) return invalid("%s: negative argument", fn);
    if (pos < 0 || pos >= max_seq) return invalid("%s: pos %d outside [0, %d)", fn, pos, max_seq);
    if (nkv == 0 || hd == 0) return 0;
    if (!src || !cache) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(scatter_kv_kernel, dim3(grid_for(static_cast<long>(nkv) * hd)),
                       dim3(kOpBlock), 0, as_stream(s), src, cache, nkv, hd, max_seq, pos);
    return launch_status(fn);
}
int spb_attention_scores_f16(const uint16_t* Q, const uint16_t* K, float* sc, int nh, int nkv,
                             int hd, int max_seq, int seq_len, float scale, spb_stream_t s) {
    return attention_scores<F16>("spb_attention_scores_f16", Q, K, sc, nh, nkv, hd, max_seq,
                                 seq_len, scale, s);
}
int spb_attention_scores_bf16(const uint16_t* Q, const uint16_t* K, float* sc, int nh, int nkv,
                              int hd, int max_seq, int seq_len, float scale, spb_stream_t s) {
    return attention_scores<BF16>("spb_attention_scores_bf16", Q, K, sc, nh, nkv, hd, max_seq,
                                  seq_len, scale, s);
}
int spb_softmax(float* sc, int nh, int max_seq, int seq_len, spb_stream_t s) {
    clear_error();
    const char* fn = "spb_softmax";
    if (nh < 0 || max_seq < 0 || seq_len < 0 || seq_len > max_seq)
        return invalid("%s: bad shape", fn);
    if (nh == 0 || seq_len == 0) return 0;
    if (!sc) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(softmax_kernel, dim3(nh), dim3(kNormBlock), 0, as_stream(s), sc, max_seq,
                       seq_len);
    return launch_status(fn);
}
int spb_attention_output_f16(const float* sc, const uint16_t* V, uint16_t* out, int nh, int nkv,
                             int hd, int max_seq, int seq_len, spb_stream_t s) {
    return attention_output<F16>("spb_attention_output_f16", sc, V, out, nh, nkv, hd, max_seq,
                                 seq_len, s);
}
int spb_attention_output_bf16(const float* sc, const uint16_t* V, uint16_t* out, int nh, int nkv,
                              int hd, int max_seq, int seq_len, spb_stream_t s) {
    return attention_output<BF16>("spb_attention_output_bf16", sc, V, out, nh, nkv, hd, max_seq,
                                  seq_len, s);
}
int spb_relu2_mul_f16(const uint16_t* g, const uint16_t* u, uint16_t* out, int n, spb_stream_t s) {
    return relu2_mul<F16, false>("spb_relu2_mul_f16", g, u, out, n, s);
}
int spb_relu2_mul_bf16(const uint16_t* g, const uint16_t* u, uint16_t* out, int n, spb_stream_t s) {
    return relu2_mul<BF16, false>("spb_relu2_mul_bf16", g, u, out, n, s);
}
int spb_relu2_mul_f32_f16(const uint16_t* g, const uint16_t* u, float* out, int n, spb_stream_t s) {
    return relu2_mul<F16, true>("spb_relu2_mul_f32_f16", g, u, out, n, s);
}
int spb_relu2_mul_f32_bf16(const uint16_t* g, const uint16_t* u, float* out, int n,
                           spb_stream_t s) {
    return relu2_mul<BF16, true>("spb_relu2_mul_f32_bf16", g, u, out, n, s);
}
int spb_float_to_f16(const float* x, uint16_t* y, int n, spb_stream_t s) {
    return float_to_16<F16>("spb_float_to_f16", x, y, n, s);
}
int spb_float_to_bf16(const float* x, uint16_t* y, int n, spb_stream_t s) {
    return float_to_16<BF16>("spb_float_to_bf16", x, y, n, s);
}
int spb_residual_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, int n,
                         spb_stream_t s) {
    return residual_add<F16>("spb_residual_add_f16", a, b, y, n, s);
}
int spb_residual_add_bf16(const uint16_t* a, const uint16_t* b, uint16_t* y, int n,
                          spb_stream_t s) {
    return residual_add<BF16>("spb_residual_add_bf16", a, b, y, n, s);
}
int spb_gemv_f16(const uint16_t* W, const uint16_t* x, float* y, int rows, int cols,
                 spb_stream_t s) {
    return gemv16<F16>("spb_gemv_f16", W, x, y, rows, cols, s);
}
int spb_gemv_bf16(const uint16_t* W, const uint16_t* x, float* y, int rows, int cols,
                  spb_stream_t s) {
    return gemv16<BF16>("spb_gemv_bf16", W, x, y, rows, cols, s);
}
int spb_argmax_f32(const float* x, int n, int* out_index, spb_stream_t s) {
    clear_error();
    const char* fn = "spb_argmax_f32";
    if (n <= 0) return invalid("%s: need n > 0", fn);
    if (!x || !out_index) return invalid("%s: null pointer", fn);
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kNormBlock), 0, as_stream(s), x, n, out_index);
    return launch_status(fn);
}

}  // extern "C"

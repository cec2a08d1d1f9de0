// sparse_i8.hip -- 2:4 structured-sparse int8 GEMM on the int8 sparse matrix
// cores of gfx950 (v_smfmac_i32_16x16x128_i8): the drop-in for the
// reference's cuSPARSELt backend, CuSparseLtGemm (include/spbitnet/
// cusparselt_backend.h:28-77, src/cusparselt_backend.cu:38-219), whose
// prepare() prunes a dense int8 weight matrix to 2:4 and compresses it and
// whose execute() computes D = A_pruned * B with int32 accumulation.
//
// Unlike spbitnet's ternary format, the weights here are any int8 values
// (the reference's tests feed {-1, 0, +1} with kept zeros,
// tests/test_cusparselt.cu:68-117), so the compressed operand keeps two int8
// values per group of four.
//
// Pruning rule (cuSPARSELt's STRIP selection is not specified by the
// reference and is not reproduced): in each group of four along k keep the
// two largest |a|, on equal magnitudes the higher index -- the rule of the
// stable argsort in python/convert_model.py:88-119 that the ternary
// converter uses.  A group with at most two non-zeros keeps all of them, so
// a matrix already in 2:4 form is unchanged.
//
// Compressed operand ("tile order"): the matrix is cut into tiles of 16 rows
// x 128 columns (rows padded to a multiple of 16, columns to 128, with
// zeros); tile (strip s, step j) sits at byte (s * steps + j) * 1280 and
// holds, for SMFMAC lane l = 16 a + i (row 16 s + i, columns 128 j + 32 a +
// [0, 32)), the lane's 16 compressed values at byte 16 l (value 2g, 2g + 1
// = the kept entries of group g, lower column first) and its index word at
// byte 1024 + 4 l (nibble g = p0 | p1 << 2, the kept positions inside
// group g).  That is exactly the A operand of v_smfmac_i32_16x16x128_i8, so
// a wave loads a tile's operand with one 16-byte and one 4-byte load per
// lane, both fully coalesced, and decodes nothing.  Empty groups hold zeros
// with positions (0, 1).
//
// B is int8 [k x n] column-major (= token-major [n][k]) and D int32 [m x n]
// column-major (= [n][m]), as the reference declares them
// (src/cusparselt_backend.cu:53-78).
#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));

constexpr int kI8TileBytes = 1280;  // 16 rows x 128 columns: values then index words
constexpr int kI8ValBytes = 1024;
constexpr uint32_t kI8EmptyNibble = 0x4u;  // positions (0, 1)
constexpr int kI8RawBufferFlags = 0x00020000;  // gfx9 raw buffer resource word 3

long i8_steps(int k) { return (k + 127) / 128; }
long i8_strips(int m) { return (m + 15) / 16; }

// Kept positions of a group (v[0..3]): nibble p0 | p1 << 2, p0 < p1.
__device__ __forceinline__ uint32_t i8_top2_nibble(int v0, int v1, int v2, int v3) {
    const int a[4] = {v0 < 0 ? -v0 : v0, v1 < 0 ? -v1 : v1, v2 < 0 ? -v2 : v2, v3 < 0 ? -v3 : v3};
    uint32_t keep = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int beaten = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (j != i && (a[j] > a[i] || (a[j] == a[i] && j > i))) ++beaten;
        if (beaten < 2) keep |= 1u << i;
    }
    const uint32_t p0 = __builtin_ctz(keep), p1 = __builtin_ctz(keep & (keep - 1));
    return p0 | (p1 << 2);
}

// One wave per tile: lane (a, i) prunes row 16 s + i, columns 128 j + 32 a +
// [0, 32) and writes its compressed values, its index word and (optionally)
// the pruned dense row segment.
__global__ __launch_bounds__(256) void sparse_i8_prune_kernel(const int8_t* __restrict__ A,
                                                              int8_t* __restrict__ pruned,
                                                              uint8_t* __restrict__ comp, int m,
                                                              int k, int steps, long ntiles) {
    const long tile = static_cast<long>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (tile >= ntiles) return;
    const int lane = threadIdx.x & (kWave - 1), a = lane >> 4, li = lane & 15;
    const long row = (tile / steps) * 16 + li;
    const int c0 = static_cast<int>(tile % steps) * 128 + 32 * a;
    uint32_t vals[4] = {0u, 0u, 0u, 0u}, idx = 0u;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const int c = c0 + 4 * g;
        const bool in = row < m && c < k;  // k % 4 == 0: a group is wholly inside or outside
        uint32_t w = 0u;
        if (in) w = *reinterpret_cast<const uint32_t*>(A + row * k + c);
        const int v0 = static_cast<int8_t>(w), v1 = static_cast<int8_t>(w >> 8);
        const int v2 = static_cast<int8_t>(w >> 16), v3 = static_cast<int8_t>(w >> 24);
        const uint32_t nib = in ? i8_top2_nibble(v0, v1, v2, v3) : kI8EmptyNibble;
        const uint32_t p0 = nib & 3u, p1 = nib >> 2;
        const uint32_t b0 = (w >> (8 * p0)) & 0xFFu, b1 = (w >> (8 * p1)) & 0xFFu;
        vals[g >> 1] |= (b0 | (b1 << 8)) << (16 * (g & 1));
        idx |= nib << (4 * g);
        if (pruned && in)
            *reinterpret_cast<uint32_t*>(pruned + row * k + c) = (b0 << (8 * p0)) | (b1 << (8 * p1));
    }
    uint8_t* t = comp + tile * kI8TileBytes;
    *reinterpret_cast<v4i*>(t + lane * 16) =
        (v4i){static_cast<int>(vals[0]), static_cast<int>(vals[1]), static_cast<int>(vals[2]),
              static_cast<int>(vals[3])};
    *reinterpret_cast<uint32_t*>(t + kI8ValBytes + lane * 4) = idx;
}

// Groups of A with more than two non-zeros, counted into *bad (set to 0
// first by sparse_i8_zero_kernel on the same stream).
__global__ void sparse_i8_zero_kernel(int* bad) { *bad = 0; }

__global__ __launch_bounds__(256) void sparse_i8_check_kernel(const int8_t* __restrict__ A, int m,
                                                              int k, int* bad) {
    const long groups = static_cast<long>(m) * (k / 4);
    const long g = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    int over = 0;
    if (g < groups) {
        const long row = g / (k / 4);
        const int c = static_cast<int>(g - row * (k / 4)) * 4;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(A + row * k + c);
        const int nz = ((w & 0xFFu) != 0) + ((w & 0xFF00u) != 0) + ((w & 0xFF0000u) != 0) +
                       ((w & 0xFF000000u) != 0);
        over = nz > 2;
    }
    const unsigned long long ball = __ballot(over);
    if ((threadIdx.x & (kWave - 1)) == 0 && ball) atomicAdd(bad, __popcll(ball));
}

// Compressed -> dense [m][k] (the pruned matrix): one thread per group.
__global__ __launch_bounds__(256) void sparse_i8_decompress_kernel(const uint8_t* __restrict__ comp,
                                                                   int8_t* __restrict__ out, int m,
                                                                   int k, int steps) {
    const long groups = static_cast<long>(m) * (k / 4);
    const long g = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
    if (g >= groups) return;
    const long row = g / (k / 4);
    const int c = static_cast<int>(g - row * (k / 4)) * 4;
    const int j = c >> 7, cl = c & 127, a = cl >> 5, gl = (cl & 31) >> 2;
    const int lane = 16 * a + static_cast<int>(row & 15);
    const uint8_t* t = comp + ((row >> 4) * steps + j) * kI8TileBytes;
    const uint32_t nib = (*reinterpret_cast<const uint32_t*>(t + kI8ValBytes + lane * 4) >> (4 * gl)) & 0xFu;
    const uint32_t b0 = t[lane * 16 + 2 * gl], b1 = t[lane * 16 + 2 * gl + 1];
    const uint32_t p0 = nib & 3u, p1 = nib >> 2;
    *reinterpret_cast<uint32_t*>(out + row * k + c) = (b0 << (8 * p0)) | (b1 << (8 * p1));
}

// D[t][r] = sum_c A[r][c] B[t][c] on the matrix cores.  Block: W waves on
// S strips (16 S rows) and T token tiles (16 T tokens, grid.y); wave w takes
// the 128-column steps w, w + W, ... of every (strip, tile) and the W partial
// sums meet in LDS.  A tiles load straight from the compressed operand (one
// 16-byte and one 4-byte load per lane, 1.25 KB contiguous per wave); B
// lane (token i, group q) loads columns 16 q + [0, 16) and 64 + 16 q + [0,
// 16) of the step through a buffer resource covering B's n * k bytes, so
// tokens past n read zeros; columns past k meet zero A values.
template <int S, int T, int W>
__global__ __launch_bounds__(W * kWave) void sparse_i8_gemm_kernel(
    const uint8_t* __restrict__ comp, const int8_t* __restrict__ B, int32_t* __restrict__ D,
    int m, int k, int n, int steps, int strips, int quads) {
    __shared__ v4i red[W * S * T * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int q = lane >> 4, li = lane & 15;
    const int s0 = blockIdx.x * S, t0 = blockIdx.y * (16 * T);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(B), static_cast<short>(0), n * k, kI8RawBufferFlags);
    v4i acc[S][T];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = (v4i){0, 0, 0, 0};
    for (int j = wave; j < steps; j += W) {
        v4i av[S];
        int idx[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            av[s] = (v4i){0, 0, 0, 0};
            idx[s] = 0x44444444;
            if (s0 + s < strips) {
                const uint8_t* tp = comp + (static_cast<long>(s0 + s) * steps + j) * kI8TileBytes;
                av[s] = *reinterpret_cast<const v4i*>(tp + lane * 16);
                idx[s] = *reinterpret_cast<const int*>(tp + kI8ValBytes + lane * 4);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int off = (t0 + 16 * t + li) * k + 128 * j + 16 * q;
            const v4i lo = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
            const v4i hi =
                __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, off + 64, 0, 0));
            const v8i b = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int s = 0; s < S; ++s)
                acc[s][t] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(av[s], b, acc[s][t], idx[s], 0, 0);
        }
    }
    if (W > 1) {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t) red[((wave * S + s) * T + t) * kWave + lane] = acc[s][t];
        __syncthreads();
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                if ((s * T + t) % W == wave) {
                    v4i sum = red[(s * T + t) * kWave + lane];
#pragma unroll
                    for (int w = 1; w < W; ++w) sum += red[((w * S + s) * T + t) * kWave + lane];
                    acc[s][t] = sum;
                }
    }
    // lane (i, q) of (strip, tile) holds rows 16 strip + 4 q .. + 3 of token 16 tile + i
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int row = (s0 + s) * 16 + 4 * q;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int tok = t0 + 16 * t + li;
            if ((W == 1 || (s * T + t) % W == wave) && tok < n && row < m) {
                int32_t* y = D + static_cast<long>(tok) * m + row;
                if (quads) {
                    *reinterpret_cast<v4i*>(y) = acc[s][t];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (row + e < m) y[e] = acc[s][t][e];
                }
            }
        }
    }
}

// Any shape with k % 4 == 0 and any alignment: one wave per row, tokens on
// grid.y, groups decoded from the compressed operand.
__global__ __launch_bounds__(256) void sparse_i8_gemm_general_kernel(
    const uint8_t* __restrict__ comp, const int8_t* __restrict__ B, int32_t* __restrict__ D,
    int m, int k, int n, int steps) {
    const int lane = threadIdx.x & (kWave - 1);
    const long row = static_cast<long>(blockIdx.x) * 4 + threadIdx.x / kWave;
    const int tok = blockIdx.y;
    if (row >= m) return;
    const int8_t* x = B + static_cast<long>(tok) * k;
    int acc = 0;
    for (int g = lane; g < (k >> 2); g += kWave) {
        const int c = 4 * g, j = c >> 7, cl = c & 127, a = cl >> 5, gl = (cl & 31) >> 2;
        const int ln = 16 * a + static_cast<int>(row & 15);
        const uint8_t* t = comp + ((row >> 4) * steps + j) * kI8TileBytes;
        const uint32_t nib =
            (*reinterpret_cast<const uint32_t*>(t + kI8ValBytes + ln * 4) >> (4 * gl)) & 0xFu;
        const int v0 = static_cast<int8_t>(t[ln * 16 + 2 * gl]);
        const int v1 = static_cast<int8_t>(t[ln * 16 + 2 * gl + 1]);
        acc += v0 * static_cast<int>(x[c + (nib & 3u)]) + v1 * static_cast<int>(x[c + (nib >> 2)]);
    }
    acc = wave_sum(acc);
    if (lane == 0) D[static_cast<long>(tok) * m + row] = acc;
}

bool i8_aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

template <int S, int T, int W>
void launch_i8_gemm(const uint8_t* comp, const int8_t* B, int32_t* D, int m, int k, int n,
                    hipStream_t st) {
    const int steps = static_cast<int>(i8_steps(k)), strips = static_cast<int>(i8_strips(m));
    const dim3 grid((strips + S - 1) / S, (n + 16 * T - 1) / (16 * T));
    const int quads = (m % 4 == 0 && i8_aligned(D, 16)) ? 1 : 0;
    hipLaunchKernelGGL((sparse_i8_gemm_kernel<S, T, W>), grid, dim3(W * kWave), 0, st, comp, B, D,
                       m, k, n, steps, strips, quads);
}

const char* i8_shape_error(int m, int k) {
    if (m < 0 || k < 0) return "negative shape";
    if (k % 4) return "k is not a multiple of 4 (2:4 groups along k)";
    if (static_cast<long>(m) * k >= (1L << 31)) return "m * k must stay below 2^31";
    return nullptr;
}

}  // namespace
}  // namespace spb

using namespace spb;

extern "C" long spb_sparse_i8_compressed_size(int m, int k) {
    clear_error();
    if (const char* e = i8_shape_error(m, k)) {
        set_error("spb_sparse_i8_compressed_size: %s", e);
        return -1;
    }
    return i8_strips(m) * i8_steps(k) * kI8TileBytes;
}

extern "C" int spb_sparse_i8_prune_compress(const int8_t* A, int8_t* pruned, void* compressed,
                                            int m, int k, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_i8_prune_compress";
    if (const char* e = i8_shape_error(m, k)) return invalid("%s: %s", fn, e);
    if (m == 0 || k == 0) return 0;
    if (!A || !compressed) return invalid("%s: null pointer", fn);
    if (!i8_aligned(A, 4) || (pruned && !i8_aligned(pruned, 4)) || !i8_aligned(compressed, 16))
        return invalid("%s: A and pruned need 4-byte, compressed 16-byte alignment", fn);
    const long ntiles = i8_strips(m) * i8_steps(k);
    hipLaunchKernelGGL(sparse_i8_prune_kernel, dim3(static_cast<unsigned>((ntiles + 3) / 4)),
                       dim3(256), 0, as_stream(stream), A, pruned,
                       static_cast<uint8_t*>(compressed), m, k, static_cast<int>(i8_steps(k)),
                       ntiles);
    return launch_status(fn);
}

extern "C" int spb_sparse_i8_prune_check(const int8_t* A, int m, int k, int* d_invalid,
                                         spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_i8_prune_check";
    if (const char* e = i8_shape_error(m, k)) return invalid("%s: %s", fn, e);
    if (!d_invalid) return invalid("%s: null result pointer", fn);
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(sparse_i8_zero_kernel, dim3(1), dim3(1), 0, st, d_invalid);
    const long groups = static_cast<long>(m) * (k / 4);
    if (groups > 0) {
        if (!A) return invalid("%s: null pointer", fn);
        if (!i8_aligned(A, 4)) return invalid("%s: A needs 4-byte alignment", fn);
        hipLaunchKernelGGL(sparse_i8_check_kernel, dim3(static_cast<unsigned>((groups + 255) / 256)),
                           dim3(256), 0, st, A, m, k, d_invalid);
    }
    return launch_status(fn);
}

extern "C" int spb_sparse_i8_decompress(const void* compressed, int8_t* out, int m, int k,
                                        spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_i8_decompress";
    if (const char* e = i8_shape_error(m, k)) return invalid("%s: %s", fn, e);
    if (m == 0 || k == 0) return 0;
    if (!compressed || !out) return invalid("%s: null pointer", fn);
    if (!i8_aligned(out, 4) || !i8_aligned(compressed, 16))
        return invalid("%s: out needs 4-byte, compressed 16-byte alignment", fn);
    const long groups = static_cast<long>(m) * (k / 4);
    hipLaunchKernelGGL(sparse_i8_decompress_kernel, dim3(static_cast<unsigned>((groups + 255) / 256)),
                       dim3(256), 0, as_stream(stream), static_cast<const uint8_t*>(compressed),
                       out, m, k, static_cast<int>(i8_steps(k)));
    return launch_status(fn);
}

extern "C" int spb_sparse_i8_gemm_kernel_id(const void* compressed, const int8_t* B, int m,
                                            int k, int n) {
    (void)compressed;
    (void)m;
    if (k <= 0 || k % 16 || !i8_aligned(B, 16)) return 0;
    if ((static_cast<long>(n) + 64) * k >= (1L << 31) || (n + 15) / 16 > 65535) return 0;
    return 1;
}

extern "C" int spb_sparse_i8_gemm(const void* compressed, const int8_t* B, int32_t* D, int m,
                                  int k, int n, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_i8_gemm";
    if (const char* e = i8_shape_error(m, k)) return invalid("%s: %s", fn, e);
    if (n < 0) return invalid("%s: negative n", fn);
    if (m == 0 || k == 0 || n == 0) return 0;  // a no-op, as the reference's wrappers
    if (!compressed || !D || !B) return invalid("%s: null pointer", fn);
    if (!i8_aligned(compressed, 16)) return invalid("%s: compressed needs 16-byte alignment", fn);
    hipStream_t st = as_stream(stream);
    const auto* comp = static_cast<const uint8_t*>(compressed);
    if (spb_sparse_i8_gemm_kernel_id(compressed, B, m, k, n)) {
        if (n <= 16)
            launch_i8_gemm<2, 1, 4>(comp, B, D, m, k, n, st);
        else if (n <= 64)
            launch_i8_gemm<2, 4, 4>(comp, B, D, m, k, n, st);
        else
            launch_i8_gemm<2, 4, 4>(comp, B, D, m, k, n, st);
    } else {
        if (n > 65535) return invalid("%s: n = %d exceeds 65535 on the general kernel", fn, n);
        hipLaunchKernelGGL(sparse_i8_gemm_general_kernel,
                           dim3(static_cast<unsigned>((m + 3) / 4), static_cast<unsigned>(n)),
                           dim3(256), 0, st, comp, B, D, m, k, n, static_cast<int>(i8_steps(k)));
    }
    return launch_status(fn);
}

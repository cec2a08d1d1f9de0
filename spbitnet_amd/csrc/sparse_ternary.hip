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
//     32w+j kept).  The 2-bit sign pairs are expanded in registers into the
//     mask N of columns holding -1 (P = K ^ N holds +1) with nibble-parallel
//     bit tricks: H = K & (K - 0x1111_1111) isolates the higher kept bit of
//     every group (no borrow crosses a nibble since each holds two set bits),
//     L = K ^ H the lower one; no lookup table.
//   * The int8 activations are staged once per block in LDS as 8 bit planes
//     (X_b, one bit per column), built with 64-lane ballots.
//   * For column set S, sum_{j in P} x_j - sum_{j in N} x_j
//       = sum_b c_b * popc((X_b & P) | (~X_b & N)) + popc(N),
//     c_b = 2^b (b < 7), c_7 = -128 (two's complement).  The select is one
//     v_bitop3_b32 and the count one accumulating v_bcnt_u32_b32, so each 32
//     columns cost two VALU ops per bit plane: additions and bit operations
//     only, no multiplies on the activations.
//   * Work mapping: a thread owns one 128-column chunk (16 bytes of meta, 8 of
//     signs, loaded with 128/64-bit vector loads) and keeps that chunk's 32
//     plane words in registers for every row it visits; consecutive threads
//     take consecutive chunks of consecutive rows, so each load instruction
//     of a block reads one contiguous span.  Per-row partial sums meet in LDS
//     (integer atomics: exact in any order).  Blocks stride over row tiles so
//     a large matrix is streamed by a grid sized to the chip.
// Shapes the bit-plane kernel does not take (cols % 128 != 0, cols > 32768,
// unaligned rows) go to a general wave-per-row kernel.
#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {

namespace {

constexpr int kBlock = 512;
constexpr int kChunk = 128;           // columns per thread per row (bit-plane kernel)
constexpr int kMaxPlaneCols = 32768;  // bit-plane kernel column limit (C <= kBlock/2)

struct Weights {
    const uint32_t* meta;
    const uint32_t* values;
    int rows, cols, ms, vs;
};

// ---- activation sources ------------------------------------------------------

struct Int8Src {
    const int8_t* x;
    __device__ void prepare() {}
    __device__ int load(int c) const { return x[c]; }
};

template <class T>
struct QuantSrc {
    const uint16_t* x;
    const float* d_absmax;
    float scale;
    __device__ void prepare() { scale = quant_scale(*d_absmax); }
    __device__ int load(int c) const { return quant_round_clamp(T::to_float(x[c]) * scale); }
};

// ---- output sinks --------------------------------------------------------------

struct Int32Sink {
    int32_t* y;
    __device__ void prepare() {}
    __device__ void store(long r, int acc) const { y[r] = acc; }
};

template <class T>
struct DequantSink {
    uint16_t* out;
    const float* d_absmax;
    float gamma;
    float dq;
    __device__ void prepare() { dq = dequant_scale(gamma, *d_absmax); }
    __device__ void store(long r, int acc) const {
        out[r] = T::from_float(static_cast<float>(acc) * dq);
    }
};

// ---- bit-plane decode of one 128-column chunk ---------------------------------

// v_bitop3_b32 truth tables: bit i of the table is f(a, b, c) with a, b, c
// the bits of 0xF0, 0xCC, 0xAA at position i (a = first operand).
constexpr uint32_t kOrAnd = 0xC8;   // (a | c) & b
constexpr uint32_t kSelect = 0xCA;  // (a & b) | (~a & c)
constexpr uint32_t kXorAnd = 0x28;  // (a ^ b) & c

template <uint32_t kTable>
__device__ __forceinline__ uint32_t bitop3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, kTable);
}

// popcount(v) + acc in one v_bcnt_u32_b32 (the compiler otherwise sums
// separate popcounts with extra adds).
__device__ __forceinline__ int bcnt_acc(uint32_t v, int acc) {
    int r;
    asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(acc));
    return r;
}

// 7 * v on each 16-bit half (one v_pk_mul_lo_u16).  Used on words whose set
// bits sit at nibble bases (or bit 1 of nibbles), where 7*v copies each bit
// to the two bits above it without carries.
__device__ __forceinline__ uint32_t times7_halves(uint32_t v) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 h = __builtin_bit_cast(u16x2, v);
    h = h * (u16x2){7, 7};
    return __builtin_bit_cast(uint32_t, h);
}

// Negative / positive column masks of one meta word (8 groups, 32 columns).
// k: the meta word; vw: the values word holding these groups' sign pairs,
// in its low (upper_half = false) or high 16 bits.
__device__ __forceinline__ void sign_masks(uint32_t k, uint32_t vw, bool upper_half,
                                           uint32_t& neg, uint32_t& pos) {
    // Spread group g's sign pair to nibble g: s_lo -> bit 4g, s_hi -> bit 4g+1.
    // perm gives bytes [b0, 0, b1, 0] (or [b2, 0, b3, 0]); selector 0x0C is 0x00.
    uint32_t t = __builtin_amdgcn_perm(vw, vw, upper_half ? 0x0C030C02u : 0x0C010C00u);
    t = bitop3<kOrAnd>(t << 4, 0x0F0F0F0Fu, t);
    const uint32_t a0 = bitop3<kOrAnd>(t << 2, 0x11111111u, t);  // s_lo at nibble bit 0
    const uint32_t a1 = bitop3<kOrAnd>(t << 2, 0x22222222u, t);  // s_hi at nibble bit 1
    const uint32_t s_lo = times7_halves(a0);                      // over nibble bits 0..2
    const uint32_t s_hi = times7_halves(a1);                      // over nibble bits 1..3
    // Each nibble of k holds exactly two set bits, so subtracting 1 per nibble
    // never borrows across nibbles: hi = higher kept column, k ^ hi = lower.
    const uint32_t hi = k & (k - 0x11111111u);
    neg = (hi & s_hi) | bitop3<kXorAnd>(k, hi, s_lo);
    pos = k ^ neg;
}

__device__ __forceinline__ int chunk_dot(const uint4 K, const uint2 V, const uint32_t (&X)[8][4]) {
    const uint32_t kw[4] = {K.x, K.y, K.z, K.w};
    int cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int cneg = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t neg, pos;
        sign_masks(kw[w], w < 2 ? V.x : V.y, (w & 1) != 0, neg, pos);
#pragma unroll
        for (int b = 0; b < 8; ++b)
            cnt[b] = bcnt_acc(bitop3<kSelect>(X[b][w], pos, neg), cnt[b]);
        cneg = bcnt_acc(neg, cneg);
    }
    int s = cneg - (cnt[7] << 7);
#pragma unroll
    for (int b = 0; b < 7; ++b) s += cnt[b] << b;
    return s;
}

template <class Src, class Sink>
__global__ __launch_bounds__(kBlock) void gemv_bitplane_kernel(Weights wt, Src src, Sink sink,
                                                               int tile_steps) {
    extern __shared__ uint32_t smem[];
    const int nwords = wt.cols >> 5;
    uint32_t* planes = smem;  // planes[b * nwords + w]
    int* acc = reinterpret_cast<int*>(smem + 8 * nwords);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int C = wt.cols / kChunk;
    const int RS = kBlock / C;  // rows per step
    const int tile_rows = RS * tile_steps;

    src.prepare();
    sink.prepare();

    // Bit planes of the int8 activations, 64 columns per ballot.
    for (int s = wave; s < (wt.cols >> 6); s += kBlock / kWave) {
        const int q = src.load(s * kWave + lane);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const unsigned long long m = __ballot((q >> b) & 1);
            if (lane == 0) {
                planes[b * nwords + 2 * s] = static_cast<uint32_t>(m);
                planes[b * nwords + 2 * s + 1] = static_cast<uint32_t>(m >> 32);
            }
        }
    }
    for (int i = tid; i < tile_rows; i += kBlock) acc[i] = 0;
    __syncthreads();

    const int c = tid % C;
    const int ro = tid / C;
    const bool active = ro < RS;
    uint32_t X[8][4];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint4 v = active ? *reinterpret_cast<const uint4*>(planes + b * nwords + 4 * c)
                               : make_uint4(0, 0, 0, 0);
        X[b][0] = v.x;
        X[b][1] = v.y;
        X[b][2] = v.z;
        X[b][3] = v.w;
    }

    for (long tile = blockIdx.x;; tile += gridDim.x) {
        const long row0 = tile * tile_rows;
        if (row0 >= wt.rows) break;  // uniform across the block
        for (int s = 0; s < tile_steps; ++s) {
            const long r = row0 + static_cast<long>(s) * RS + ro;
            if (active && r < wt.rows) {
                const uint4 K = *reinterpret_cast<const uint4*>(wt.meta + r * wt.ms + 4 * c);
                const uint2 V = *reinterpret_cast<const uint2*>(wt.values + r * wt.vs + 2 * c);
                atomicAdd(&acc[s * RS + ro], chunk_dot(K, V, X));
            }
        }
        __syncthreads();
        for (int i = tid; i < tile_rows; i += kBlock) {
            const long r = row0 + i;
            if (r < wt.rows) sink.store(r, acc[i]);
            acc[i] = 0;
        }
        __syncthreads();
    }
}

// ---- general kernel: one wave per row, any cols % 4 == 0, any strides ---------

template <class Src, class Sink>
__global__ __launch_bounds__(256) void gemv_general_kernel(Weights wt, Src src, Sink sink) {
    const int lane = threadIdx.x & (kWave - 1);
    const long row = static_cast<long>(blockIdx.x) * (256 / kWave) + (threadIdx.x / kWave);
    src.prepare();
    sink.prepare();
    if (row >= wt.rows) return;
    const uint32_t* mr = wt.meta + row * wt.ms;
    const uint32_t* vr = wt.values + row * wt.vs;
    int acc = 0;
    for (int g = lane; g < (wt.cols >> 2); g += kWave) {
        const uint32_t bm = (mr[g >> 3] >> ((g & 7) * 4)) & 0xFu;
        const uint32_t sg = (vr[g >> 4] >> ((g & 15) * 2)) & 0x3u;
        // Lower / higher set bit; a bitmap without exactly two bits decodes to
        // positions (0, 0), as the reference's table does (sparse_ternary.cu:34-51).
        const bool ok = __builtin_popcount(bm) == 2;
        const int p0 = ok ? __builtin_ctz(bm) : 0;
        const int p1 = ok ? __builtin_ctz(bm & (bm - 1)) : 0;
        const int x0 = src.load(4 * g + p0);
        const int x1 = src.load(4 * g + p1);
        acc += (sg & 1u) ? -x0 : x0;
        acc += (sg & 2u) ? -x1 : x1;
    }
    acc = wave_sum(acc);
    if (lane == 0) sink.store(row, acc);
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

// ---- host side ------------------------------------------------------------------

int check_weights(const char* fn, const uint32_t* meta, const uint32_t* values, int rows,
                  int cols, int ms, int vs) {
    if (rows < 0 || cols < 0) return invalid("%s: negative shape (%d, %d)", fn, rows, cols);
    if (cols % 4) return invalid("%s: cols=%d is not a multiple of 4", fn, cols);
    const int need_m = (cols / 4 + 7) / 8, need_v = (cols / 4 + 15) / 16;
    if (ms < need_m)
        return invalid("%s: meta_row_stride=%d < ceil(cols/32)=%d", fn, ms, need_m);
    if (vs < need_v)
        return invalid("%s: values_row_stride=%d < ceil(cols/64)=%d", fn, vs, need_v);
    if (rows && cols && (!meta || !values)) return invalid("%s: null weight pointer", fn);
    return 0;
}

bool bitplane_ok(const uint32_t* meta, const uint32_t* values, int cols, int ms, int vs) {
    return cols > 0 && cols % kChunk == 0 && cols <= kMaxPlaneCols && ms % 4 == 0 &&
           vs % 2 == 0 && (reinterpret_cast<uintptr_t>(meta) & 15u) == 0 &&
           (reinterpret_cast<uintptr_t>(values) & 7u) == 0;
}

template <class Src, class Sink>
int launch_gemv(const char* fn, const Weights& wt, Src src, Sink sink, hipStream_t stream) {
    if (bitplane_ok(wt.meta, wt.values, wt.cols, wt.ms, wt.vs)) {
        const int C = wt.cols / kChunk;
        const int RS = kBlock / C;
        const long target = 4L * device_cu_count();
        long steps = (static_cast<long>(wt.rows) + RS * target - 1) / (RS * target);
        steps = steps < 1 ? 1 : (steps > 8 ? 8 : steps);
        const long tile_rows = RS * steps;
        long tiles = (wt.rows + tile_rows - 1) / tile_rows;
        const int grid = static_cast<int>(tiles < target ? tiles : target);
        const size_t lds = static_cast<size_t>(wt.cols) + static_cast<size_t>(tile_rows) * 4;
        hipLaunchKernelGGL((gemv_bitplane_kernel<Src, Sink>), dim3(grid), dim3(kBlock), lds,
                           stream, wt, src, sink, static_cast<int>(steps));
    } else {
        const long blocks = (static_cast<long>(wt.rows) + 3) / 4;
        hipLaunchKernelGGL((gemv_general_kernel<Src, Sink>), dim3(blocks), dim3(256), 0, stream,
                           wt, src, sink);
    }
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
    return launch_gemv(fn, Weights{meta, values, rows, cols, ms, vs}, Int8Src{x}, Int32Sink{y},
                       as_stream(stream));
}

template <class T>
static int fused_bitlinear(const char* fn, const uint32_t* meta, const uint32_t* values,
                           const uint16_t* x, uint16_t* output, const float* d_absmax,
                           float gamma, int rows, int cols, int ms, int vs, spb_stream_t stream) {
    clear_error();
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !output || !d_absmax) return invalid("%s: null pointer argument", fn);
    return launch_gemv(fn, Weights{meta, values, rows, cols, ms, vs},
                       QuantSrc<T>{x, d_absmax, 0.0f}, DequantSink<T>{output, d_absmax, gamma, 0.0f},
                       as_stream(stream));
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

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
//     mask N of columns holding -1 with nibble-parallel bit tricks:
//     H = K & (K - 0x1111_1111) isolates the higher kept bit of every group
//     (no borrow crosses a nibble since each holds two set bits), K ^ H the
//     lower one; no lookup table.
//   * The int8 activations are used as 8 bit planes (X_b: bit j = bit b of
//     column j's two's-complement byte).  For the columns of a meta word,
//       sum_{j in P} x_j - sum_{j in N} x_j
//         = sum_b c_b * popc((X_b & P) | (~X_b & N)) + popc(N),
//     P = K & ~N, c_b = 2^b (b < 7), c_7 = -128.  The select is one
//     v_bitop3_b32 of (X_b, K, N) and the count one accumulating
//     v_bcnt_u32_b32: two VALU ops per plane per 32 columns, additions and
//     bit operations only, no multiplies on the activations.
//   * Plane layout (shared by LDS and the global "activation planes" format):
//     word [w * 8 + b] holds plane b of columns 32w .. 32w+31, so the 8
//     planes of a 128-column chunk are 128 contiguous bytes.  Planes come
//     either from a prologue that transposes the activations 8 columns per
//     thread (SWAR 8x8 bit transpose, lane-parallel, one load per thread),
//     or precomputed in global memory by spb_activation_planes /
//     spb_absmax_quantize_planes_*.
//   * Work mapping: a thread owns one 128-column chunk (16 bytes of meta, 8 of
//     signs, 128/64-bit vector loads) and keeps that chunk's 32 plane words
//     in registers for every row it visits; consecutive threads take
//     consecutive chunks of consecutive rows, so each load instruction of a
//     block reads one contiguous span.  Per-row partial sums meet in LDS
//     (integer atomics: exact in any order).  Blocks stride over row tiles so
//     a large matrix is streamed by a grid sized to the resident capacity.
// Shapes the bit-plane kernel does not take (cols % 128 != 0, cols > 32768,
// unaligned rows or activations) go to a general wave-per-row kernel.
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

// ---- SWAR helpers ----------------------------------------------------------------

// v_bitop3_b32 truth tables: bit i of the table is f(a, b, c) with a, b, c
// the bits of 0xF0, 0xCC, 0xAA at position i (a = first operand).
constexpr uint32_t kOrAnd = 0xC8;       // (a | c) & b
constexpr uint32_t kXorAnd = 0x28;      // (a ^ b) & c
constexpr uint32_t kSelectKeep = 0x4A;  // a ? (b & ~c) : c
constexpr uint32_t kXor3 = 0x96;        // a ^ b ^ c

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

// 8x8 bit transpose of 8 int8 columns (lo = columns 0..3, hi = 4..7, byte i =
// column i): afterwards byte b of lo (b < 4) or of hi (b >= 4) holds plane b,
// bit i = bit b of column i.  Three delta swaps (Hacker's Delight, 7-13).
__device__ __forceinline__ void transpose8x8(uint32_t& lo, uint32_t& hi) {
    uint32_t t;
    t = bitop3<kXorAnd>(lo, lo >> 7, 0x00AA00AAu);
    lo = bitop3<kXor3>(lo, t, t << 7);
    t = bitop3<kXorAnd>(hi, hi >> 7, 0x00AA00AAu);
    hi = bitop3<kXor3>(hi, t, t << 7);
    t = bitop3<kXorAnd>(lo, lo >> 14, 0x0000CCCCu);
    lo = bitop3<kXor3>(lo, t, t << 14);
    t = bitop3<kXorAnd>(hi, hi >> 14, 0x0000CCCCu);
    hi = bitop3<kXor3>(hi, t, t << 14);
    t = bitop3<kXorAnd>(lo, hi << 4, 0xF0F0F0F0u);
    lo ^= t;
    hi ^= t >> 4;
}

// ---- activation sources ----------------------------------------------------------

// int8 activations.
struct Int8Src {
    const int8_t* x;
    long token_stride = 0;  // batched use: token t reads x + t * token_stride
    __device__ void offset(long t) { x += t * token_stride; }
    __device__ void prepare() {}
    __device__ int load(int c) const { return x[c]; }
    // Columns c0..c7 as two little-endian dwords (c0 % 8 == 0, x 8-byte aligned).
    __device__ void load8(int c0, uint32_t& lo, uint32_t& hi) const {
        const uint2 v = *reinterpret_cast<const uint2*>(x + c0);
        lo = v.x;
        hi = v.y;
    }
};

// fp16 / bf16 activations quantised on the fly with the reference's rule.
template <class T>
struct QuantSrc {
    const uint16_t* x;
    const float* d_absmax;
    float scale;
    __device__ void offset(long) {}
    __device__ void prepare() { scale = quant_scale(*d_absmax); }
    __device__ int load(int c) const { return quant_round_clamp(T::to_float(x[c]) * scale); }
    __device__ uint32_t q8(uint32_t h) const {
        return static_cast<uint32_t>(
                   quant_round_clamp(T::to_float(static_cast<uint16_t>(h)) * scale)) &
               0xFFu;
    }
    // Columns c0..c7 (c0 % 8 == 0, x 16-byte aligned), quantised, as two dwords.
    __device__ void load8(int c0, uint32_t& lo, uint32_t& hi) const {
        const uint4 v = *reinterpret_cast<const uint4*>(x + c0);  // 8 x 16-bit
        lo = q8(v.x & 0xFFFF) | (q8(v.x >> 16) << 8) | (q8(v.y & 0xFFFF) << 16) |
             (q8(v.y >> 16) << 24);
        hi = q8(v.z & 0xFFFF) | (q8(v.z >> 16) << 8) | (q8(v.w & 0xFFFF) << 16) |
             (q8(v.w >> 16) << 24);
    }
};

// Activations already in the plane layout (global memory), for the general
// kernel: column c's int8 value reassembled from its 8 plane bits.
struct PlaneSrc {
    const uint32_t* p;
    __device__ void prepare() {}
    __device__ int load(int c) const {
        const uint32_t* g = p + (c >> 5) * 8;
        int v = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) v |= static_cast<int>((g[b] >> (c & 31)) & 1u) << b;
        return static_cast<int>(static_cast<int8_t>(v));
    }
};

// ---- how a bit-plane block obtains its activation planes ----------------------

// Planes built in LDS by the block itself from an activation source.
template <class Src>
struct BuildPlanes {
    Src src;
    __device__ void offset(long t) { src.offset(t); }
    __device__ void prepare() { src.prepare(); }
    // Transposes the activations, 8 columns per thread, into LDS planes
    // (bytes of word [w*8+b]).  The loads of up to two units are issued
    // before either is transposed.
    __device__ void build(uint32_t* planes, int cols, int tid) const {
        const int units = cols >> 3;
        uint8_t* pb = reinterpret_cast<uint8_t*>(planes);
        for (int u0 = tid; u0 < units; u0 += 2 * kBlock) {
            const int u1 = u0 + kBlock;
            uint32_t lo0, hi0, lo1 = 0, hi1 = 0;
            src.load8(u0 * 8, lo0, hi0);
            if (u1 < units) src.load8(u1 * 8, lo1, hi1);
            transpose8x8(lo0, hi0);
            const int w0 = u0 >> 2, q0 = u0 & 3;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                pb[(w0 * 8 + b) * 4 + q0] = static_cast<uint8_t>(lo0 >> (8 * b));
                pb[(w0 * 8 + b + 4) * 4 + q0] = static_cast<uint8_t>(hi0 >> (8 * b));
            }
            if (u1 < units) {
                transpose8x8(lo1, hi1);
                const int w1 = u1 >> 2, q1 = u1 & 3;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    pb[(w1 * 8 + b) * 4 + q1] = static_cast<uint8_t>(lo1 >> (8 * b));
                    pb[(w1 * 8 + b + 4) * 4 + q1] = static_cast<uint8_t>(hi1 >> (8 * b));
                }
            }
        }
    }
};

// Planes precomputed in global memory (spb_activation_planes or
// spb_absmax_quantize_planes_*): the block copies the cols bytes into LDS with
// 16-byte loads (every thread of the block then reads its chunk from LDS; a
// direct global read per thread would request 128 B x 512 threads per block
// from L2 for cols bytes of data).
struct GlobalPlanes {
    const uint32_t* p;
    __device__ void offset(long) {}
    __device__ void prepare() {}
    __device__ void build(uint32_t* planes, int cols, int tid) const {
        const uint4* src = reinterpret_cast<const uint4*>(p);
        uint4* dst = reinterpret_cast<uint4*>(planes);
        for (int i = tid; i < (cols >> 4); i += kBlock) dst[i] = src[i];
    }
};

// ---- output sinks ------------------------------------------------------------------

struct Int32Sink {
    int32_t* y;
    long token_stride = 0;  // batched use: token t writes y + t * token_stride
    __device__ void offset(long t) { y += t * token_stride; }
    __device__ void prepare() {}
    __device__ void store(long r, int acc) const { y[r] = acc; }
};

template <class T>
struct DequantSink {
    uint16_t* out;
    const float* d_absmax;
    float gamma;
    float dq;
    __device__ void offset(long) {}
    __device__ void prepare() { dq = dequant_scale(gamma, *d_absmax); }
    __device__ void store(long r, int acc) const {
        out[r] = T::from_float(static_cast<float>(acc) * dq);
    }
};

// ---- bit-plane decode of one 128-column chunk ----------------------------------

// Mask of the columns holding -1 in one meta word (8 groups, 32 columns).
// k: the meta word; vw: the values word holding these groups' sign pairs,
// in its low (upper_half = false) or high 16 bits.
__device__ __forceinline__ uint32_t neg_mask(uint32_t k, uint32_t vw, bool upper_half) {
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
    return (hi & s_hi) | bitop3<kXorAnd>(k, hi, s_lo);
}

// X[w][b]: plane b of the chunk's meta word w.
__device__ __forceinline__ int chunk_dot(const uint4 K, const uint2 V, const uint32_t (&X)[4][8]) {
    const uint32_t kw[4] = {K.x, K.y, K.z, K.w};
    int cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int cneg = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t neg = neg_mask(kw[w], w < 2 ? V.x : V.y, (w & 1) != 0);
        // (X & P) | (~X & N) with P = k & ~N, as one 3-input op of (X, k, N)
#pragma unroll
        for (int b = 0; b < 8; ++b)
            cnt[b] = bcnt_acc(bitop3<kSelectKeep>(X[w][b], kw[w], neg), cnt[b]);
        cneg = bcnt_acc(neg, cneg);
    }
    int s = cneg - (cnt[7] << 7);
#pragma unroll
    for (int b = 0; b < 7; ++b) s += cnt[b] << b;
    return s;
}

// Work item of one thread: the 128-column chunk c of one row.
struct ChunkLoad {
    uint4 k;
    uint2 v;
    bool ok;
};

__device__ __forceinline__ ChunkLoad load_chunk(const Weights& wt, long r, int c, bool active) {
    ChunkLoad L;
    L.ok = active && r < wt.rows;
    if (L.ok) {
        L.k = *reinterpret_cast<const uint4*>(wt.meta + r * wt.ms + 4 * c);
        L.v = *reinterpret_cast<const uint2*>(wt.values + r * wt.vs + 2 * c);
    } else {
        L.k = make_uint4(0, 0, 0, 0);
        L.v = make_uint2(0, 0);
    }
    return L;
}

// The 32 plane words of one 128-column chunk (128 contiguous bytes).
__device__ __forceinline__ void load_x(const uint32_t* src, uint32_t (&X)[4][8]) {
    const uint4* p = reinterpret_cast<const uint4*>(src);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint4 a = p[2 * w], b = p[2 * w + 1];
        X[w][0] = a.x;
        X[w][1] = a.y;
        X[w][2] = a.z;
        X[w][3] = a.w;
        X[w][4] = b.x;
        X[w][5] = b.y;
        X[w][6] = b.z;
        X[w][7] = b.w;
    }
}

// Rows are processed in tiles of RS * tile_steps rows (RS = rows per step:
// kBlock / C threads per row).  Block b takes tiles b, b + gridDim.x, ...; a
// thread visits its chunk of row tile*tile_rows + s*RS + ro for each step s.
// The first weight load is issued before the activation prologue, the next
// item's weights are loaded before the current one is reduced (prefetch
// distance 1), and per-row sums collect in two LDS buffers used by alternate
// tiles, so one barrier per tile orders accumulation and write-out.
template <class Act, class Sink>
__global__ __launch_bounds__(kBlock) void gemv_bitplane_kernel(Weights wt, Act act, Sink sink,
                                                               int tile_steps, long ntiles) {
    extern __shared__ uint32_t smem[];
    const int nwords = wt.cols >> 5;
    const int C = wt.cols / kChunk;
    const int RS = kBlock / C;
    const int tile_rows = RS * tile_steps;
    uint32_t* planes = smem;  // word [w * 8 + b]
    int* acc0 = reinterpret_cast<int*>(smem + 8 * nwords);
    int* acc1 = acc0 + tile_rows;

    const int tid = threadIdx.x;
    const int c = tid % C;
    const int ro = tid / C;
    const bool active = ro < RS;

    // (tile, step) advance uniformly across the block (scalar registers); each
    // thread's row follows from them without divisions.
    long tile = blockIdx.x;
    int step = 0;
    long row = tile * tile_rows + ro;
    int parity = 0;

    act.offset(blockIdx.y);
    sink.offset(blockIdx.y);
    ChunkLoad cur = load_chunk(wt, row, c, active);
    act.prepare();
    sink.prepare();
    uint32_t X[4][8];
    act.build(planes, wt.cols, tid);
    for (int i = tid; i < 2 * tile_rows; i += kBlock) acc0[i] = 0;
    __syncthreads();
    if (active) load_x(planes + c * 32, X);

    for (;;) {
        int step_n = step + 1;
        long tile_n = tile;
        long row_n = row + RS;
        if (step_n == tile_steps) {
            step_n = 0;
            tile_n = tile + gridDim.x;
            row_n = tile_n * tile_rows + ro;
        }
        const bool more = tile_n < ntiles;
        const ChunkLoad nxt = more ? load_chunk(wt, row_n, c, active) : ChunkLoad{};
        int* acc = parity ? acc1 : acc0;
        if (cur.ok) atomicAdd(&acc[step * RS + ro], chunk_dot(cur.k, cur.v, X));
        if (step == tile_steps - 1) {
            __syncthreads();  // uniform: (tile, step) are the same in every thread
            const long row0 = tile * tile_rows;
            for (int j = tid; j < tile_rows; j += kBlock) {
                if (row0 + j < wt.rows) sink.store(row0 + j, acc[j]);
                acc[j] = 0;
            }
            parity ^= 1;
        }
        if (!more) break;
        cur = nxt;
        step = step_n;
        tile = tile_n;
        row = row_n;
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

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool bitplane_ok(const uint32_t* meta, const uint32_t* values, int cols, int ms, int vs) {
    return cols > 0 && cols % kChunk == 0 && cols <= kMaxPlaneCols && ms % 4 == 0 &&
           vs % 2 == 0 && aligned(meta, 16) && aligned(values, 8);
}

// Resident blocks per CU for one bit-plane instantiation (cached per LDS size).
template <class Act, class Sink>
int bitplane_blocks_per_cu(size_t lds) {
    static size_t cached_lds[4] = {0, 0, 0, 0};
    static int cached_n[4] = {0, 0, 0, 0};
    for (int i = 0; i < 4; ++i)
        if (cached_lds[i] == lds && cached_n[i] > 0) return cached_n[i];
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_bitplane_kernel<Act, Sink>, kBlock,
                                                     lds) != hipSuccess ||
        n <= 0)
        n = 1;
    for (int i = 0; i < 4; ++i)
        if (cached_n[i] == 0) {
            cached_lds[i] = lds;
            cached_n[i] = n;
            break;
        }
    return n;
}

template <class Act, class Sink>
void launch_bitplane(const Weights& wt, Act act, Sink sink, hipStream_t stream, int tokens = 1) {
    const int C = wt.cols / kChunk;
    const long RS = kBlock / C;
    const long steps_max = 8;
    const size_t plane_lds = static_cast<size_t>(wt.cols);
    const size_t lds_max = plane_lds + 2 * RS * steps_max * 4;
    long resident =
        static_cast<long>(bitplane_blocks_per_cu<Act, Sink>(lds_max)) * device_cu_count();
    resident = (resident + tokens - 1) / tokens;  // tokens share the resident capacity
    // Enough tiles for every resident block; longer tiles once the matrix
    // is several times the resident capacity.
    long steps = (static_cast<long>(wt.rows) + RS * resident - 1) / (RS * resident);
    steps = steps < 1 ? 1 : (steps > steps_max ? steps_max : steps);
    const long tile_rows = RS * steps;
    const long tiles = (wt.rows + tile_rows - 1) / tile_rows;
    const int grid = static_cast<int>(tiles < resident ? tiles : resident);
    const size_t lds = plane_lds + 2 * static_cast<size_t>(tile_rows) * 4;
    hipLaunchKernelGGL((gemv_bitplane_kernel<Act, Sink>), dim3(grid, tokens), dim3(kBlock), lds,
                       stream, wt, act, sink, static_cast<int>(steps), tiles);
}

template <class Src, class Sink>
void launch_general(const Weights& wt, Src src, Sink sink, hipStream_t stream) {
    const long blocks = (static_cast<long>(wt.rows) + 3) / 4;
    hipLaunchKernelGGL((gemv_general_kernel<Src, Sink>), dim3(blocks), dim3(256), 0, stream, wt,
                       src, sink);
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
        launch_bitplane(wt, BuildPlanes<QuantSrc<T>>{src}, sink, as_stream(stream));
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
        launch_bitplane(wt, GlobalPlanes{planes}, sink, as_stream(stream));
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
        launch_bitplane(wt, BuildPlanes<Int8Src>{Int8Src{x}}, Int32Sink{y}, as_stream(stream));
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
        launch_bitplane(wt, GlobalPlanes{planes}, Int32Sink{y}, as_stream(stream));
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

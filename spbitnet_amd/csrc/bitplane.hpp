// bitplane.hpp -- the gfx950 bit-plane sparse-ternary GEMV core, shared by
// the plain/fused BitLinear entry points and the fused decode engine.
//
// What it computes (reference src/kernels/sparse_ternary.cu:116-234):
//   y[r] = sum_g  (s_lo ? -1 : 1) * x[4g+p0] + (s_hi ? -1 : 1) * x[4g+p1]
// exact int32 for int8 x; the producer of the int8 activations (Act) and the
// consumer of each row's sum (Sink) are template policies, so a prologue
// (quantise, normalise + quantise, ...) and an epilogue (int32 store,
// dequantise, dequantise + residual add, ...) fuse into one launch.  The
// algorithm itself is described in sparse_ternary.hip.
#pragma once

#include "common.hpp"

namespace spb {
namespace {

constexpr int kBlock = 512;
constexpr int kChunk = 128;           // columns per thread per row (bit-plane kernel)
constexpr int kMaxPlaneCols = 32768;  // bit-plane kernel column limit (C <= kBlock/2)

// Work item of one thread: the 128-column chunk c of one row.
// Weight loads with the non-temporal hint (nt): in a decode step every weight
// byte is read once.  On MI355X, bs=1 decode of the 2.4B model ran 1090 tok/s
// with the projections' and the LM head's weight loads non-temporal, against
// 1026 with ordinary loads (1026 / 1041 with only one of the two).
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 nt_load(const uint4* p) {
    const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 nt_load(const uint2* p) {
    const nt_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x2*>(p));
    return make_uint2(v.x, v.y);
}

struct ChunkLoad {
    uint4 k;
    uint2 v;
    bool ok;
};

__device__ __forceinline__ ChunkLoad chunk_at(const uint32_t* meta, const uint32_t* values,
                                              long r, int ms, int vs, int c, bool ok) {
    ChunkLoad L;
    L.ok = ok;
    if (ok) {
        L.k = *reinterpret_cast<const uint4*>(meta + r * ms + 4 * c);
        L.v = *reinterpret_cast<const uint2*>(values + r * vs + 2 * c);
    } else {
        L.k = make_uint4(0, 0, 0, 0);
        L.v = make_uint2(0, 0);
    }
    return L;
}

// A value passed through an empty asm: selects between such values
// stay selects of registers (the compiler otherwise turns a select between
// two fields of a kernel-argument struct into a dynamically indexed load,
// which moves the struct to scratch memory).
template <class T>
__device__ __forceinline__ T opaque(T v) {
    asm volatile("" : "+v"(v));
    return v;
}

// One packed matrix (reference SparseLinear, include/spbitnet/model.h:46-60).
struct Weights {
    const uint32_t* meta;
    const uint32_t* values;
    int rows, cols, ms, vs;
    __device__ ChunkLoad load(long r, int c, bool active) const {
        return chunk_at(meta, values, r, ms, vs, c, active && r < rows);
    }
    // unconditional (non-temporal) load of a row known to be in range
    __device__ ChunkLoad load_in(long r, int c) const {
        return ChunkLoad{nt_load(reinterpret_cast<const uint4*>(meta + r * ms + 4 * c)),
                         nt_load(reinterpret_cast<const uint2*>(values + r * vs + 2 * c)), true};
    }
};

// Up to three packed matrices with the same cols, stacked by rows: the
// projections of one layer that read the same activation (q/k/v, gate/up)
// run as one launch.  Row r belongs to segment (r >= end0) + (r >= end1).
// Segments 1 and 2 are addressed as element offsets from segment 0's arrays
// (dm1 = meta1 - meta0, dm2 = meta2 - meta1, likewise for values and the
// strides), so every load stays a global load off one kernel-argument base.
struct SegWeights {
    const uint32_t* meta;
    const uint32_t* values;
    long dm1, dm2, dv1, dv2;
    int ms, vs, dms1, dms2, dvs1, dvs2;
    int end0, end1;
    int rows, cols;
    __device__ ChunkLoad load(long r, int c, bool active) const {
        const bool s1 = r >= end0, s2 = r >= end1;
        const long om = (s1 ? dm1 : 0) + (s2 ? dm2 : 0);
        const long ov = (s1 ? dv1 : 0) + (s2 ? dv2 : 0);
        const int sm = ms + (s1 ? dms1 : 0) + (s2 ? dms2 : 0);
        const int sv = vs + (s1 ? dvs1 : 0) + (s2 ? dvs2 : 0);
        const long lr = r - (s1 ? end0 : 0) - (s2 ? end1 - end0 : 0);
        return chunk_at(meta + om, values + ov, lr, sm, sv, c, active && r < rows);
    }
    // unconditional (non-temporal) load of a row known to be in range
    __device__ ChunkLoad load_in(long r, int c) const {
        const bool s1 = r >= end0, s2 = r >= end1;
        const long om = (s1 ? dm1 : 0) + (s2 ? dm2 : 0);
        const long ov = (s1 ? dv1 : 0) + (s2 ? dv2 : 0);
        const int sm = ms + (s1 ? dms1 : 0) + (s2 ? dms2 : 0);
        const int sv = vs + (s1 ? dvs1 : 0) + (s2 ? dvs2 : 0);
        const long lr = r - (s1 ? end0 : 0) - (s2 ? end1 - end0 : 0);
        return ChunkLoad{nt_load(reinterpret_cast<const uint4*>(meta + om + lr * sm + 4 * c)),
                         nt_load(reinterpret_cast<const uint2*>(values + ov + lr * sv + 2 * c)), true};
    }
};

// ---- SWAR helpers ----------------------------------------------------------------

// v_bitop3_b32 truth tables: bit i of the table is f(a, b, c) with a, b, c
// the bits of 0xF0, 0xCC, 0xAA at position i (a = first operand).
constexpr uint32_t kOrAnd = 0xC8;    // (a | c) & b
constexpr uint32_t kXorAnd = 0x28;   // (a ^ b) & c
constexpr uint32_t kKeptXor = 0x48;  // b & (a ^ c)
constexpr uint32_t kSelect = 0xCA;   // a ? b : c
constexpr uint32_t kXor3 = 0x96;     // a ^ b ^ c

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

// ---- one unit of activations from registers into the LDS planes ---------------------
//
// q = clamp(rint_ne(v * scale), -128, 127), the reference's rule
// (src/kernels/sparse_ternary.cu:199, 216-217), as v * scale (rounded) plus
// 1.5 * 2^23: the sum's ulp is 1, so the addition rounds to the nearest
// integer, ties to even, while |v * scale| < 2^22, and one med3 clamps the
// biased value (anything beyond 2^22 clamps to the same end).  The low byte
// of the biased float is q's two's-complement byte.  (NaN inputs are not
// defined here: activations are finite.)
__device__ __forceinline__ uint32_t q8_biased(float v, float scale) {
    constexpr float kBias = 12582912.0f;
    return __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_fmed3f(v * scale + kBias, kBias - 128.0f, kBias + 127.0f));
}

// Unit u (columns 8u .. 8u+7) of the activations, 8 floats in registers,
// quantised and stored into the plane-major LDS planes.  The 4 units of a
// plane word sit in the 4 lanes of a quad (u % 4 == lane % 4 for
// u = tid + k * kBlock); after the 8x8 bit transpose each lane holds one byte
// of every plane, and a byte transpose across the quad (two DPP exchanges,
// lane ^ 1 then lane ^ 2) gives lane q the whole words of planes q and q + 4:
// two dword stores instead of eight byte stores.  All 4 lanes of a quad run
// this together.
__device__ __forceinline__ void store_unit_planes(uint32_t* planes, int nw, int u,
                                                  const float (&v)[8], float scale) {
    uint32_t t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = q8_biased(v[e], scale);
    // byte e of (lo, hi) = column 8u + e
    uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], 0x0C0C0400u) | __builtin_amdgcn_perm(t[3], t[2], 0x04000C0Cu);
    uint32_t hi = __builtin_amdgcn_perm(t[5], t[4], 0x0C0C0400u) | __builtin_amdgcn_perm(t[7], t[6], 0x04000C0Cu);
    transpose8x8(lo, hi);  // byte b of lo / hi: plane b / b + 4 of the unit's 8 columns
    const int q = u & 3;
    // stage 1 (partner lane ^ 1): even lanes [own0, p0, own2, p2], odd [p1, own1, p3, own3];
    // stage 2 (partner lane ^ 2): lanes 0, 1 [own0, own1, p0, p1], lanes 2, 3 [p2, p3, own2, own3]
    const uint32_t sel1 = (q & 1) ? 0x03070105u : 0x06020400u;
    const uint32_t sel2 = (q & 2) ? 0x03020706u : 0x05040100u;
    auto quad_t = [&](uint32_t x) {
        const uint32_t p1 = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xF, 0xF, true));
        x = __builtin_amdgcn_perm(p1, x, sel1);
        const uint32_t p2 = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xF, 0xF, true));
        return __builtin_amdgcn_perm(p2, x, sel2);
    };
    const int w = u >> 2;
    planes[q * nw + w] = quad_t(lo);
    planes[(q + 4) * nw + w] = quad_t(hi);
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
    // Transposes the activations, 8 columns per thread, into the LDS planes
    // (plane-major: word (b, w) at b * nw + w, nw = cols / 32; a unit is one
    // byte of each plane).  The loads of up to two units are issued before
    // either is transposed.
    struct Regs {};
    static size_t extra_lds(int) { return 0; }
    __device__ bool skip() const { return false; }
    __device__ void issue(int, Regs&) {}
    __device__ void build(uint32_t* planes, int cols, int tid, float* s, Regs&) const {
        build(planes, cols, tid, s);
    }
    __device__ void build(uint32_t* planes, int cols, int tid, float*) const {
        const int units = cols >> 3;
        const int nw = cols >> 5;
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
                pb[(b * nw + w0) * 4 + q0] = static_cast<uint8_t>(lo0 >> (8 * b));
                pb[((b + 4) * nw + w0) * 4 + q0] = static_cast<uint8_t>(hi0 >> (8 * b));
            }
            if (u1 < units) {
                transpose8x8(lo1, hi1);
                const int w1 = u1 >> 2, q1 = u1 & 3;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    pb[(b * nw + w1) * 4 + q1] = static_cast<uint8_t>(lo1 >> (8 * b));
                    pb[((b + 4) * nw + w1) * 4 + q1] = static_cast<uint8_t>(hi1 >> (8 * b));
                }
            }
        }
    }
};

// Planes precomputed in global memory (spb_activation_planes or
// spb_absmax_quantize_planes_*, word [w*8+b]): the block copies the cols bytes
// into the plane-major LDS layout with 16-byte loads (every thread of the
// block then reads its chunk from LDS; a direct global read per thread would
// request 128 B x 512 threads per block from L2 for cols bytes of data).
struct GlobalPlanes {
    const uint32_t* p;
    __device__ void offset(long) {}
    __device__ void prepare() {}
    struct Regs {};
    static size_t extra_lds(int) { return 0; }
    __device__ bool skip() const { return false; }
    __device__ void issue(int, Regs&) {}
    __device__ void build(uint32_t* planes, int cols, int tid, float*, Regs&) const {
        const uint4* src = reinterpret_cast<const uint4*>(p);
        const int nw = cols >> 5;
        for (int i = tid; i < (cols >> 4); i += kBlock) {
            const uint4 v = src[i];  // words w*8 + b .. +3 with w = i / 2, b = 4 * (i % 2)
            uint32_t* d = planes + (4 * (i & 1)) * nw + (i >> 1);
            d[0] = v.x;
            d[nw] = v.y;
            d[2 * nw] = v.z;
            d[3 * nw] = v.w;
        }
    }
};

// ---- output sinks ------------------------------------------------------------------

struct Int32Sink {
    int32_t* y;
    long token_stride = 0;  // batched use: token t writes y + t * token_stride
    __device__ void offset(long t) { y += t * token_stride; }
    __device__ void prepare() {}
    __device__ void prefetch(long, int, int) {}
    template <class A>
    __device__ void bind(const A&) {}
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
    __device__ void prefetch(long, int, int) {}
    template <class A>
    __device__ void bind(const A&) {}
    __device__ void store(long r, int acc) const {
        out[r] = T::from_float(static_cast<float>(acc) * dq);
    }
};

// ---- bit-plane decode of one 128-column chunk ----------------------------------

// A mask that holds, at each kept column of one meta word (8 groups, 32
// columns), that column's sign bit; its other bits are unspecified.
// k: the meta word; vw: the values word holding these groups' sign pairs, in
// its low (upper_half = false) or high 16 bits.
//   * The 2-bit sign pairs are spread to nibble g: s_lo of group g to bit 4g,
//     s_hi to bit 4g+1 (perm, then two shift-and-mask steps), and each is
//     copied over three bits by one packed 16-bit multiply by 7 (set bits at
//     nibble bases or nibble bit 1, so no carries): s_lo over bits 0..2 of the
//     nibble (where the lower kept column can be), s_hi over bits 1..3.
//   * d = k - 0x11111111 subtracts 1 from every nibble without borrows (each
//     nibble holds two set bits): it clears the lower kept bit and keeps the
//     higher one, so "d ? s_hi : s_lo" is s_lo at the lower kept column and
//     s_hi at the higher.
__device__ __forceinline__ uint32_t sign_mask(uint32_t k, uint32_t vw, bool upper_half) {
    // perm gives bytes [b0, 0, b1, 0] (or [b2, 0, b3, 0]); selector 0x0C is 0x00.
    uint32_t t = __builtin_amdgcn_perm(vw, vw, upper_half ? 0x0C030C02u : 0x0C010C00u);
    t = bitop3<kOrAnd>(t << 4, 0x0F0F0F0Fu, t);
    const uint32_t a0 = bitop3<kOrAnd>(t << 2, 0x11111111u, t);  // s_lo at nibble bit 0
    const uint32_t a1 = bitop3<kOrAnd>(t << 2, 0x22222222u, t);  // s_hi at nibble bit 1
    return bitop3<kSelect>(k - 0x11111111u, times7_halves(a1), times7_halves(a0));
}

// X[w][b]: plane b of the chunk's meta word w.  Per plane, with P / N the
// kept columns holding +1 / -1 and M = sign_mask (M = N on kept columns):
//   popc((X & P) | (~X & N)) = popc(K & (X ^ M)),
// one v_bitop3 and one accumulating v_bcnt.  The popc(N) term (weight 1, like
// plane 0) is the number of set sign bits: popc of the two values words.
// The weighted sum of the plane counts is evaluated by Horner's rule from
// plane 7 (weight -128) down, one shift-and-add per plane.
__device__ __forceinline__ int chunk_dot(const uint4 K, const uint2 V, const uint32_t (&X)[4][8]) {
    const uint32_t kw[4] = {K.x, K.y, K.z, K.w};
    int cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t m = sign_mask(kw[w], w < 2 ? V.x : V.y, (w & 1) != 0);
#pragma unroll
        for (int b = 0; b < 8; ++b) cnt[b] = bcnt_acc(bitop3<kKeptXor>(X[w][b], kw[w], m), cnt[b]);
    }
    cnt[0] = bcnt_acc(V.x, cnt[0]);
    cnt[0] = bcnt_acc(V.y, cnt[0]);
    int s = cnt[6] - 2 * cnt[7];
#pragma unroll
    for (int b = 5; b >= 0; --b) s = (s << 1) + cnt[b];
    return s;
}

// The 4 x 8 plane words of chunk c (columns 128c .. 128c+127) from the
// plane-major LDS layout: one 16-byte read per plane, at 16c bytes into the
// plane, so the chunks of neighbouring threads sit in neighbouring banks.
__device__ __forceinline__ void load_x(const uint32_t* planes, int c, int nw, uint32_t (&X)[4][8]) {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint4 v = *reinterpret_cast<const uint4*>(planes + b * nw + 4 * c);
        X[0][b] = v.x;
        X[1][b] = v.y;
        X[2][b] = v.z;
        X[3][b] = v.w;
    }
}

// Rows are processed in tiles of RS * tile_steps rows (RS = rows per step:
// kBlock / C threads per row).  Block b takes tiles b, b + gridDim.x, ...; a
// thread visits its chunk of row tile*tile_rows + s*RS + ro for each step s.
// The first weight load is issued before the activation prologue, the next
// item's weights are loaded before the current one is reduced (prefetch
// distance 1), and per-row sums collect in two LDS buffers used by alternate
// tiles, so one barrier per tile orders accumulation and write-out.
//
// Act (activation planes) and Sink (output epilogue) are policies:
//   act.skip() (uniform early exit), act.issue(tid, regs) (loads issued
//   before the first weight loads into Act::Regs, a kernel-local register
//   block), act.prepare(), act.build(planes, cols, tid, scratch, regs)
//   -- scratch: the
//   Act::extra_lds(cols) bytes of LDS after the row sums;
//   sink.prepare() before the prologue, sink.prefetch(row0, n, tid) with the
//   block's first tile (loads the epilogue will need), sink.bind(act) after
//   the prologue (a sink may take a scale the prologue computed), and
//   sink.store(row, acc) per row -- or, for a sink with SinkPairs<S>::value,
//   sink.store_pair(row, acc_row, acc_row_plus_1) per even row (tiles then
//   hold an even number of rows).
template <class S>
struct SinkPairs {
    static constexpr bool value = false;
};

template <class Sink>
__host__ __device__ constexpr int rows_per_step(int C) {
    return SinkPairs<Sink>::value ? (kBlock / C) & ~1 : kBlock / C;
}

template <class W, class Act, class Sink>
__global__ __launch_bounds__(kBlock) void gemv_bitplane_kernel(W wt, Act act, Sink sink,
                                                               int tile_steps, long ntiles) {
    extern __shared__ uint32_t smem[];
    if (act.skip()) return;
    const int nwords = wt.cols >> 5;
    const int C = wt.cols / kChunk;
    const int RS = rows_per_step<Sink>(C);
    const int tile_rows = RS * tile_steps;
    uint32_t* planes = smem;  // plane-major: word (b, w) at b * nwords + w
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
    typename Act::Regs regs;
    act.issue(tid, regs);  // activation loads first: they head the critical path
    ChunkLoad cur = wt.load(row, c, active);
    act.prepare();
    sink.prepare();
    sink.prefetch(tile * tile_rows, tile_rows, tid);
    uint32_t X[4][8];
    // prologue scratch after the row sums, 16-byte aligned
    act.build(planes, wt.cols, tid,
              reinterpret_cast<float*>(smem + ((8 * nwords + 2 * tile_rows + 3) & ~3)), regs);
    for (int i = tid; i < 2 * tile_rows; i += kBlock) acc0[i] = 0;
    __syncthreads();
    sink.bind(act);
    if (active) load_x(planes, c, nwords, X);

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
        const ChunkLoad nxt = more ? wt.load(row_n, c, active) : ChunkLoad{};
        int* acc = parity ? acc1 : acc0;
        if (cur.ok) atomicAdd(&acc[step * RS + ro], chunk_dot(cur.k, cur.v, X));
        if (step == tile_steps - 1) {
            __syncthreads();  // uniform: (tile, step) are the same in every thread
            const long row0 = tile * tile_rows;
            if constexpr (SinkPairs<Sink>::value) {
                for (int j = 2 * tid; j < tile_rows; j += 2 * kBlock) {
                    if (row0 + j < wt.rows) sink.store_pair(row0 + j, acc[j], acc[j + 1]);
                    acc[j] = 0;
                    acc[j + 1] = 0;
                }
            } else {
                for (int j = tid; j < tile_rows; j += kBlock) {
                    if (row0 + j < wt.rows) sink.store(row0 + j, acc[j]);
                    acc[j] = 0;
                }
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

// ---- latency-bound kernel: one row span per block -------------------------------
//
// For matrices of a few steps per CU (the decode engine's projections, where
// one launch reads a few MB and its time is a chain of latencies): block b of
// G owns the rows [b*R/G, (b+1)*R/G) (R counted in row pairs for a pair
// sink), thread (ro, c) the chunk c of rows start + i*RS + ro for i < MS.
// Every chunk load of the thread is issued right after the activation loads
// and before the prologue (rows past the span read the span's last row and
// drop it), so the weight latency overlaps the prologue's instead of
// following it.  Same per-chunk arithmetic and LDS row sums as
// gemv_bitplane_kernel, so the results are identical.
// The row split of a span launch, computed on the host: block b owns
// base + (b < rem) units (rows, or row pairs for a pair sink) from
// b * base + min(b, rem), so the kernel divides nothing (a 64-bit division
// by the grid size is a chain of ~100 dependent scalar instructions ahead of
// the first load).
struct SpanSplit {
    int base, rem;  // units per block, blocks with one more
    int RS;         // rows per step
};

// kPairAdd (C even): the chunk sums of lanes 2i and 2i + 1 (the same row:
// a row's C lanes start at an even lane) are added by one DPP move first,
// so half as many lanes meet at each row's LDS counter (bs=1 decode of the
// 2.4B model: 1,184 -> 1,191 tok/s; quads of lanes: no further change).
template <class W, class Act, class Sink, int MS, bool kPairAdd = false>
__global__ __launch_bounds__(kBlock) void gemv_span_kernel(W wt, Act act, Sink sink, SpanSplit sp) {
    extern __shared__ uint32_t smem[];
    if (act.skip()) return;
    constexpr bool kPairs = SinkPairs<Sink>::value;
    const int nwords = wt.cols >> 5;
    const int C = wt.cols >> 7;  // 128-column chunks
    const int RS = sp.RS;
    uint32_t* planes = smem;  // plane-major: word (b, w) at b * nwords + w
    int* acc = reinterpret_cast<int*>(smem + 8 * nwords);
    const int tid = threadIdx.x;
    const int ro = static_cast<int>(static_cast<unsigned>(tid) / static_cast<unsigned>(C));
    const int c = tid - ro * C;
    const int b = blockIdx.x;
    const int u0 = b * sp.base + (b < sp.rem ? b : sp.rem);
    const int nu = sp.base + (b < sp.rem ? 1 : 0);
    const long start = kPairs ? 2L * u0 : static_cast<long>(u0);
    const long end = start + (kPairs ? 2L * nu : static_cast<long>(nu));
    const int n = static_cast<int>(end - start);

    act.offset(blockIdx.y);
    sink.offset(blockIdx.y);
    typename Act::Regs regs;
    // Loads in three groups, kept in this order (the scheduler barriers stop
    // the compiler from interleaving them): the activations, which head the
    // critical path, then the weights, then the epilogue's.  The wait counter
    // retires loads in issue order, so the prologue's waits then cover the
    // activations alone.
    act.issue(tid, regs);
    __builtin_amdgcn_sched_barrier(0);
    ChunkLoad L[MS];
#pragma unroll
    for (int i = 0; i < MS; ++i) {
        const long r = start + i * RS + ro;
        L[i] = wt.load_in(r < end ? r : end - 1, c);
    }
    __builtin_amdgcn_sched_barrier(0);
    act.prepare();
    sink.prepare();
    sink.prefetch(start, n, tid);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t X[4][8];
    // prologue scratch after the row sums, 16-byte aligned
    act.build(planes, wt.cols, tid,
              reinterpret_cast<float*>(smem + ((8 * nwords + MS * RS + 3) & ~3)), regs);
    for (int i = tid; i < MS * RS; i += kBlock) acc[i] = 0;
    __syncthreads();
    sink.bind(act);
    if (ro < RS) {
        load_x(planes, c, nwords, X);
#pragma unroll
        for (int i = 0; i < MS; ++i) {
            const int j = i * RS + ro;
            if (j < n) {
                int d = chunk_dot(L[i].k, L[i].v, X);
                if constexpr (kPairAdd) {
                    d += __builtin_amdgcn_mov_dpp(d, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
                    if ((c & 1) == 0) atomicAdd(&acc[j], d);
                } else {
                    atomicAdd(&acc[j], d);
                }
            }
        }
    }
    __syncthreads();
    if constexpr (kPairs) {
        for (int j = 2 * tid; j < n; j += 2 * kBlock) sink.store_pair(start + j, acc[j], acc[j + 1]);
    } else {
        for (int j = tid; j < n; j += kBlock) sink.store(start + j, acc[j]);
    }
}

// ---- streaming kernel for one packed matrix -------------------------------------
//
// The same per-chunk arithmetic, laid out for matrices much larger than one
// pass of the grid.  Thread (ro, c) = (tid / C, tid % C) owns the 128-column
// chunk c of row s * RS + ro in step s.  The F = rows / RS full steps are
// split into contiguous ranges [b*F/G, (b+1)*F/G), one per block, so every
// block streams one contiguous span of the matrix and the blocks differ by at
// most one step; the last block also takes the rows % RS tail rows.  A
// block's row sums all live in LDS (integer atomics) and are written once,
// after the loop.  In the loop a load is a buffer load through a resource
// whose base is the step's first row (scalar registers) plus the thread's
// fixed byte offset, with no bounds test (threads beyond RS rows per step and
// the pipeline's loads past the block's last step are out of the buffer's
// range: they return zeros without reading memory, and their sums are
// dropped).  Four register sets rotate, so
// three steps are in flight while one is reduced.  The loop body holds only
// loads, bit arithmetic and LDS atomics (no barrier, no global store, no
// early exit), which keeps the compiler's wait counts exact: each wait
// covers the step being reduced and never the ones in flight.
struct StreamLoad {
    uint4 k;
    uint2 v;
};

// Buffer resource word 3 for gfx9-family raw (unformatted, stride 0) loads.
constexpr int kBufferFlags = 0x00020000;
// Cache policy of the streamed weight loads: nt (non-temporal).  Every weight
// byte is read once; on MI355X the hint took a cold 265 MB launch with three
// blocks per CU from ~49.5 to ~46.8 us (it made no difference with one).
// kResidentLoadPolicy (0, the default policy) is for weights meant to stay in
// the Infinity Cache between launches (spb_sparse_ternary_gemv_resident).
constexpr int kStreamLoadPolicy = 2;
constexpr int kResidentLoadPolicy = 0;
// Buffer extents are capped at kExtentCap bytes, so an offset of kOutOfRange
// puts every dword of a 16-byte load out of range (the load returns zeros and
// reads no memory).
constexpr int kExtentCap = 0x7FFF0000;
constexpr int kOutOfRange = 0x7FFFFFF0;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 as_uint4(u32x4_t v) { return make_uint4(v.x, v.y, v.z, v.w); }
__device__ __forceinline__ uint2 as_uint2(u32x2_t v) { return make_uint2(v.x, v.y); }

constexpr int kStreamMaxRows = 8192;  // LDS row sums per block (32 KB)

constexpr int kStreamDepth = 4;  // register sets: kStreamDepth - 1 steps in flight

// Host-computed launch constants of the streaming kernel (no division in the
// kernel: a 64-bit division is a chain of ~100 dependent scalar instructions).
struct StreamSplit {
    int nfull;         // full steps of RS rows
    int base, rem;     // steps per block: base, plus one for blocks b < rem
    int RS;            // rows per step
    int cap_m, cap_v;  // kExtentCap / (row stride in bytes) of meta and signs
    int row_base;      // first row of this launch in the output
};

template <class Act, class Sink, int D, int Pol>
__global__ __launch_bounds__(kBlock) void gemv_stream_kernel(Weights wt, Act act, Sink sink, StreamSplit sp) {
    extern __shared__ uint32_t smem[];
    const int nwords = wt.cols >> 5;
    const int C = wt.cols >> 7;  // 128-column chunks
    const int RS = sp.RS;
    const int rows = wt.rows;
    const int nfull = sp.nfull, row_base = sp.row_base;
    // step indices stay 32-bit (scalar compares; rows < 2^31)
    const int bi = blockIdx.x;
    const int s_begin = bi * sp.base + (bi < sp.rem ? bi : sp.rem);
    const int s_end = s_begin + sp.base + (bi < sp.rem ? 1 : 0);
    const bool last = blockIdx.x == gridDim.x - 1;
    const int tail = last ? rows - nfull * RS : 0;   // rows after the full steps
    const int span = (s_end - s_begin) * RS + tail;  // rows of this block
    uint32_t* planes = smem;  // plane-major: word (b, w) at b * nwords + w
    int* acc = reinterpret_cast<int*>(smem + 8 * nwords);
    const int acc_slots = (span + RS + 3) & ~3;
    const int n = s_end - s_begin;
    const int s_last = n > 0 ? s_end - 1 : 0;

    const int tid = threadIdx.x;
    const int ro = static_cast<int>(static_cast<unsigned>(tid) / static_cast<unsigned>(C));
    const int c = tid - ro * C;
    const bool active = ro < RS;
    // Per-thread byte offsets from the step's first row.  Inactive threads get
    // an offset past every buffer extent: their loads return zeros and read
    // no memory.
    const int om = active ? (ro * wt.ms + 4 * c) * 4 : kOutOfRange;
    const int ov = active ? (ro * wt.vs + 2 * c) * 4 : kOutOfRange;

    // Buffer extents in bytes from the step's first row to the matrix end,
    // capped at kExtentCap (all scalar 32-bit arithmetic).
    const int ms4 = wt.ms * 4, vs4 = wt.vs * 4;
    const int cap_m = sp.cap_m, cap_v = sp.cap_v;
    // Steps past the block's range (the pipeline's loads beyond its last step)
    // get an empty extent, so they read no memory either.
    auto load = [&](int s) {
        const bool live = s < s_end;
        const int ub = (live ? s : s_last) * RS;
        const int left = live ? rows - ub : 0;
        const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(wt.meta + static_cast<long>(ub) * wt.ms), static_cast<short>(0),
            (left < cap_m ? left : cap_m) * ms4, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(wt.values + static_cast<long>(ub) * wt.vs),
            static_cast<short>(0), (left < cap_v ? left : cap_v) * vs4, kBufferFlags);
        StreamLoad L;
        L.k = as_uint4(__builtin_amdgcn_raw_buffer_load_b128(rm, om, 0, Pol));
        L.v = as_uint2(__builtin_amdgcn_raw_buffer_load_b64(rv, ov, 0, Pol));
        return L;
    };


    // The activation loads go first (they head the prologue's chain), then
    // the first D - 1 steps' weights, which arrive while the prologue runs.
    typename Act::Regs regs;
    act.issue(tid, regs);
    StreamLoad S[D];
#pragma unroll
    for (int i = 0; i < D - 1; ++i) S[i] = load(s_begin + i);
    act.prepare();
    sink.prepare();
    act.build(planes, wt.cols, tid,
              reinterpret_cast<float*>(smem + ((8 * nwords + acc_slots + 3) & ~3)), regs);
    for (int i = tid; i < acc_slots; i += kBlock) acc[i] = 0;
    __syncthreads();
    sink.bind(act);
    uint32_t X[4][8];
    load_x(planes, c, nwords, X);

    auto reduce = [&](int s, const StreamLoad& L) {
        const int d = chunk_dot(L.k, L.v, X);
        if (active) atomicAdd(&acc[(s - s_begin) * RS + ro], d);
    };

    if (n > 0) {
        // A counted loop over groups of D steps with its only exit at the
        // latch (a mid-body exit would join the loop head on a path with fewer
        // loads in flight, and the compiler's merged wait state would then
        // drain every load each iteration).  In a group, step s + i is reduced
        // from set i after the load of step s + i + D - 1 into the set freed
        // last.
        // sched_barrier keeps each load where it is written (the scheduler
        // otherwise sinks loads into the reduction before them).
        __builtin_amdgcn_sched_barrier(0);
        int s = s_begin;
        for (int q = 0; q < n / D; ++q, s += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                S[(i + D - 1) % D] = load(s + i + D - 1);
                __builtin_amdgcn_sched_barrier(0);
                reduce(s + i, S[i]);
            }
        }
        // the n % D remaining steps s, s+1, ... are held in S[0], S[1], ...
#pragma unroll
        for (int i = 0; i < D - 1; ++i)
            if (i < n % D) reduce(s + i, S[i]);
    }
    if (tail > 0 && active && ro < tail) {  // the last block's partial step
        const long r = static_cast<long>(nfull) * RS + ro;
        const uint4 k = *reinterpret_cast<const uint4*>(wt.meta + r * wt.ms + 4 * c);
        const uint2 v = *reinterpret_cast<const uint2*>(wt.values + r * wt.vs + 2 * c);
        atomicAdd(&acc[n * RS + ro], chunk_dot(k, v, X));
    }
    __syncthreads();
    const int row0 = s_begin * RS;
    for (int j = tid; j < span; j += kBlock)
        sink.store(static_cast<long>(row_base) + row0 + j, acc[j]);
}

// Grid: kStreamBlocksPerCU blocks per CU where their LDS fits (fewer
// otherwise), each a contiguous range of steps.  Three 512-thread blocks are
// six waves per SIMD, the register limit at 73 VGPRs.  On MI355X, with the
// clocks settled (after ~2 ms of load) and non-temporal loads, a cold 265 MB
// pass (80 x 6912x2560 alternating with 80 x 2560x6912) ran ~51 / ~49.3 /
// ~46.8 us per launch with one / two / three blocks per CU.  A matrix whose
// per-block span would exceed kStreamMaxRows is split into consecutive row
// ranges, one launch each.
constexpr int kStreamBlocksPerCU = 3;

template <class Act, class Sink, int Pol = kStreamLoadPolicy>
void launch_stream(const Weights& wt, Act act, Sink sink, hipStream_t stream) {
    const int C = wt.cols / kChunk;
    const long RS = kBlock / C;
    const long cus = device_cu_count();
    const long lds_cu = device_lds_per_cu();
    const long fixed = static_cast<long>(wt.cols) + static_cast<long>(Act::extra_lds(wt.cols)) + 48;
    const long max_rows = cus * (kStreamMaxRows / RS - 1) * RS;  // <= kStreamMaxRows sums per block
    for (long r0 = 0; r0 < wt.rows;) {
        const long n = wt.rows - r0 < max_rows ? wt.rows - r0 : max_rows;
        const long nfull = n / RS;
        long grid = 1, steps_per_block = 0;
        size_t lds = 0;
        for (long per_cu = kStreamBlocksPerCU; per_cu >= 1; --per_cu) {
            grid = nfull < per_cu * cus ? nfull : per_cu * cus;
            if (grid < 1) grid = 1;
            steps_per_block = (nfull + grid - 1) / grid;
            lds = static_cast<size_t>(fixed + ((steps_per_block + 2) * RS + 8) * 4);
            if (per_cu == 1 || static_cast<long>(lds) * per_cu <= lds_cu) break;
        }
        Weights part{wt.meta + r0 * wt.ms, wt.values + r0 * wt.vs, static_cast<int>(n), wt.cols,
                     wt.ms, wt.vs};
        const StreamSplit sp{static_cast<int>(nfull), static_cast<int>(nfull / grid),
                             static_cast<int>(nfull % grid), static_cast<int>(RS),
                             kExtentCap / (wt.ms * 4), kExtentCap / (wt.vs * 4), static_cast<int>(r0)};
        hipLaunchKernelGGL((gemv_stream_kernel<Act, Sink, kStreamDepth, Pol>), dim3(static_cast<int>(grid)),
                           dim3(kBlock), lds, stream, part, act, sink, sp);
        r0 += n;
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
template <class W, class Act, class Sink>
int bitplane_blocks_per_cu(size_t lds) {
    static size_t cached_lds[4] = {0, 0, 0, 0};
    static int cached_n[4] = {0, 0, 0, 0};
    for (int i = 0; i < 4; ++i)
        if (cached_lds[i] == lds && cached_n[i] > 0) return cached_n[i];
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_bitplane_kernel<W, Act, Sink>, kBlock,
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

template <class W, class Act, class Sink>
void launch_bitplane(const W& wt, Act act, Sink sink, hipStream_t stream, int tokens = 1) {
    const int C = wt.cols / kChunk;
    const long RS = rows_per_step<Sink>(C);
    const long steps_max = 8;
    const size_t plane_lds = static_cast<size_t>(wt.cols) + Act::extra_lds(wt.cols);
    const size_t lds_max = plane_lds + 2 * RS * steps_max * 4 + 12;
    // One token (the GEMV and the decode engine): at most one block per CU.
    // With more tiles than CUs, the CUs that run two blocks finish last and
    // set the kernel time (measured: 277 blocks on 256 CUs took ~2x the
    // median block), so longer tiles on fewer blocks win.  Batched use:
    // the resident capacity, shared by the tokens.
    long resident = device_cu_count();
    if (tokens > 1) {
        resident *= bitplane_blocks_per_cu<W, Act, Sink>(lds_max);
        resident = (resident + tokens - 1) / tokens;
    }
    // Enough tiles for every block; longer tiles once the matrix is several
    // times that.
    long steps = (static_cast<long>(wt.rows) + RS * resident - 1) / (RS * resident);
    steps = steps < 1 ? 1 : (steps > steps_max ? steps_max : steps);
    const long tile_rows = RS * steps;
    const long tiles = (wt.rows + tile_rows - 1) / tile_rows;
    const int grid = static_cast<int>(tiles < resident ? tiles : resident);
    const size_t lds = plane_lds + 2 * static_cast<size_t>(tile_rows) * 4 + 12;
    hipLaunchKernelGGL((gemv_bitplane_kernel<W, Act, Sink>), dim3(grid, tokens), dim3(kBlock),
                       lds, stream, wt, act, sink, static_cast<int>(steps), tiles);
}

// Span launch over every CU (at most one block per CU) when each block's
// span fits kSpanMaxSteps steps; returns false (nothing launched) otherwise.
constexpr int kSpanMaxSteps = 4;

template <class W, class Act, class Sink>
bool launch_span(const W& wt, Act act, Sink sink, hipStream_t stream) {
    const int C = wt.cols / kChunk;
    const long RS = rows_per_step<Sink>(C);
    const long unit = SinkPairs<Sink>::value ? 2 : 1;
    const long units = wt.rows / unit;
    if (units * unit != wt.rows || units == 0) return false;
    long G = device_cu_count();
    G = G < units ? G : units;
    const long per = (units + G - 1) / G * unit;  // most rows of one block
    const long ms = (per + RS - 1) / RS;
    if (ms > kSpanMaxSteps) return false;
    const size_t lds = static_cast<size_t>(wt.cols) + Act::extra_lds(wt.cols) +
                       static_cast<size_t>(ms * RS) * 4 + 16;
    const SpanSplit sp{static_cast<int>(units / G), static_cast<int>(units % G), static_cast<int>(RS)};
    const dim3 grid(static_cast<unsigned>(G)), block(kBlock);
    if (C % 2 == 0) {
        switch (ms) {
        case 1: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 1, true>), grid, block, lds, stream, wt, act, sink, sp); break;
        case 2: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 2, true>), grid, block, lds, stream, wt, act, sink, sp); break;
        case 3: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 3, true>), grid, block, lds, stream, wt, act, sink, sp); break;
        default: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 4, true>), grid, block, lds, stream, wt, act, sink, sp); break;
        }
        return true;
    }
    switch (ms) {
    case 1: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 1>), grid, block, lds, stream, wt, act, sink, sp); break;
    case 2: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 2>), grid, block, lds, stream, wt, act, sink, sp); break;
    case 3: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 3>), grid, block, lds, stream, wt, act, sink, sp); break;
    default: hipLaunchKernelGGL((gemv_span_kernel<W, Act, Sink, 4>), grid, block, lds, stream, wt, act, sink, sp); break;
    }
    return true;
}

template <class Src, class Sink>
void launch_general(const Weights& wt, Src src, Sink sink, hipStream_t stream) {
    const long blocks = (static_cast<long>(wt.rows) + 3) / 4;
    hipLaunchKernelGGL((gemv_general_kernel<Src, Sink>), dim3(blocks), dim3(256), 0, stream, wt,
                       src, sink);
}


}  // namespace
}  // namespace spb

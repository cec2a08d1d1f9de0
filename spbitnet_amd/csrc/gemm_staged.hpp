// gemm_staged.hpp -- the staged 2:4 sparse-ternary GEMM kernel on the
// int8 structured-sparse matrix cores of gfx950 (v_smfmac_i32_16x16x128_i8)
// with an epilogue policy: the entry point spb_sparse_ternary_gemm stores the
// int32 products (Int32Out, gemm.hip); the engines apply their per-token
// output stages (dequantise, RoPE and KV-cache write, residual add) to the
// products in registers (engine.hip), so no int32 buffer is written or read.
//
// What it computes: Y[t][r] = sum_c W[r][c] * X[t][c] (exact int32), X
// token-major int8 [n][cols]; the reference's cuSPARSELt product D = A * B
// (src/cusparselt_backend.cu:53-62, 83-89, 186-207) computed directly on
// spbitnet's packed format.  The operand layouts are described in gemm.hip.
#pragma once

#include <cstdint>

#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {

// Raises a kernel's dynamic-LDS limit to the CU's LDS, once per device
// (gemm.hip); false if the runtime refuses.
bool gemm_allow_lds(const void* fn);

namespace {

// Up to three matrices stacked along the rows (q | k | v, gate | up), with
// equal columns and strides: rows [0, end0) are the first, [end0, end1) the
// second (words at meta + om1 for global row r, i.e. om1 = offset of the
// second matrix - end0 * ms), [end1, rows) the third.  One matrix: end0 =
// end1 = rows.
struct GemmSegs {
    long om1, om2, ov1, ov2;
    int end0, end1;
};

// Split-K (engines' decode GEMMs whose row tiles leave most CUs idle): the
// chunks of K split over gridDim.z blocks per tile.  Each block writes its
// partial tile to part with write-through stores (cache policy sc1), waits
// for them, and counts itself in the tile's counter; the block that counts
// last reads the partials back with sc1 loads (past the per-XCD L2s, which
// do not see each other's writes), adds them in z order (exact int32) and
// runs the epilogue, then clears the counter for the next launch.  part
// holds [tile][z][WS x S x T][64 lanes] x 4 int32; count one zeroed word per
// tile (blockIdx.y * gridDim.x + blockIdx.x).
struct GemmSplit {
    int32_t* part;
    unsigned* count;
    long part_words;   // int32 capacity of part
    int count_words;   // capacity of count
};
constexpr int kCachePolicySc1 = 16;  // buffer-op cache policy: agent-coherent (sc1)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));


template <uint32_t kTable>
__device__ __forceinline__ uint32_t gemm_bitop3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, kTable);
}

// Index word of one meta word (8 groups): nibble g = p0 | p1 << 2.
__device__ __forceinline__ int smfmac_index(uint32_t k) {
    const uint32_t a = k >> 1, c = k << 1;
    const uint32_t t0 = gemm_bitop3<0x20>(a, k, 0x11111111u);  // (a & ~b) & m : ~b0 & b1
    const uint32_t t1 = gemm_bitop3<0x02>(c, k, 0x22222222u);  // ~(a | b) & m : ~(b0 | b1)
    const uint32_t t2 = gemm_bitop3<0xA2>(a, k, 0x44444444u);  // (a | ~b) & m : b3 | ~b2
    const uint32_t t3 = gemm_bitop3<0xA8>(c, k, 0x88888888u);  // (a | b) & m  : b3 | b2
    return static_cast<int>(gemm_bitop3<0xFE>(t0, t1, t2) | t3);
}

// Four compressed-value dwords (16 int8 +-1) from 16 sign bits: bit j -> byte j.
__device__ __forceinline__ v4i smfmac_values(uint32_t s16) {
    v4i a;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t nib = (s16 >> (4 * d)) & 0xFu;
        const uint32_t nb = (nib * 0x00204081u) & 0x01010101u;  // bit i -> byte i (0/1)
        // per 16-bit half: 0/1 bytes * 0xFE + 0x0101 -> 0x01 / 0xFF bytes, no carries
        u16x2 h = __builtin_bit_cast(u16x2, nb);
        h = h * (u16x2){0xFE, 0xFE} + (u16x2){0x0101, 0x0101};
        a[d] = __builtin_bit_cast(int, h);
    }
    return a;
}

// ---------------------------------------------------------------------------
// Staged kernel (the path for column counts that are a multiple of 256 and
// 16-byte aligned rows).  The direct kernel above reads each lane's A words
// and B bytes straight from memory: 4- and 16-byte pieces of 16 different
// rows per instruction, with each K step's loads consumed at once, so its
// time is the memory pipeline's per-request cost and latency (~20 us at
// n=256 on 6912x2560, nearly independent of the grid size).  This kernel
// moves whole tiles with 16-byte buffer loads of consecutive addresses into
// LDS, double-buffered over chunks of KCP column pairs, and the waves read
// their operands from LDS.
//
// Column pairs.  SMFMAC lane group q covers logical K [32q, 32q + 32) of a
// 128-K step.  Two steps are taken over 256 columns ("a pair") such that lane
// group q of step i reads meta word 8p + 2q + i of the pair p: the lane's two
// steps are adjacent words, and its sign bits for both are one values word
// (4p + q, half i).  The B operand follows: lane (token, q) of step i holds
// columns 64(q >> 1) + 32i + 16(q & 1) + [0, 16) and the same + 128 (the
// k-th byte of its two 16-byte halves pairs with the k-th compressed value
// of A lane group q >> 1 and 2 + (q >> 1)).  Staging stores each lane
// group's 32 bytes of step i adjacent in LDS.
//
// LDS layout per buffer (bank-conflict free for the operand reads and the
// staging writes, as measured with SQ_LDS_BANK_CONFLICT on gfx950 for these
// access patterns):
//   meta   [8 KCP words][RBM rows]   (transposed; RBM = 8 or 24 mod 32)
//   values [4 KCP words][RBV rows]   (transposed; RBV = 16 or 48 mod 64)
//   B      [4 lane groups q][KCP pairs][TB tokens][4 units]: units 2i, 2i+1
//          of (q, pair, token t) are lane group q's step-i bytes, unit c
//          stored at c ^ ((t >> 2) & 3); the q-parts are 4 mod 8 units apart
// Block: WS x KW waves.  Wave (ws, kw) owns strips ws*S .. ws*S + S - 1 and
// all T token tiles, and takes the chunk's steps kw, kw + KW, ...; the KW
// partial sums of a tile meet in LDS after the last chunk, and the epilogue
// policy Epi takes each lane's four rows of one token (store4).
constexpr int low_pow2(int x) { return x & -x; }
constexpr int cmin(int a, int b) { return a < b ? a : b; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int pitch_mod(int rb, int m, int r1, int r2) {  // smallest p >= rb with p % m in {r1, r2}
    return (rb % m <= r1) ? rb - rb % m + r1 : (rb % m <= r2 ? rb - rb % m + r2 : rb - rb % m + m + r1);
}
constexpr int kRawBufferFlags = 0x00020000;  // gfx9 raw buffer resource word 3
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

template <int S, int T, int WS, int KW, int KCP>
struct StagedTile {
    static constexpr int NT = WS * KW * kWave;
    static constexpr int RB = WS * S * 16, TB = T * 16;
    static constexpr int RBM = pitch_mod(RB, 32, 8, 24), RBV = pitch_mod(RB, 64, 16, 48);
    // B: lane group q of a step reads 32 bytes of its token (units c = 2i, 2i+1
    // of its q-part); the chunk is stored as 4 q-parts of [pair][token][4 units]
    // (unit c of token t at c ^ ((t >> 2) & 3)), the q-parts QS units apart
    static constexpr int QS = KCP * TB * 4 + 4;
    // staging maps: a thread owns unit column j < G of rows tr, tr + NT/G, ...
    static constexpr int GM = cmin(low_pow2(2 * KCP), 16);
    static constexpr int RMK = NT / GM, KRM = (RB + RMK - 1) / RMK, KJM = 2 * KCP / GM;
    static constexpr int GV = cmin(low_pow2(KCP), 16);
    static constexpr int RVK = NT / GV, KRV = (RB + RVK - 1) / RVK, KJV = KCP / GV;
    // B staging: 16 threads move one token's 256-byte pair; G16 such groups
    // take items (token t, pair p) = g + G16 r, t fastest
    static constexpr int G16 = NT / 16, KIB = (TB * KCP + G16 - 1) / G16;
    static_assert((TB & (TB - 1)) == 0 && (G16 & (G16 - 1)) == 0, "power-of-two staging maps");
    static constexpr int kABytes = (8 * KCP * RBM + 4 * KCP * RBV) * 4;
    static constexpr int kBufBytes = kABytes + 4 * QS * 16;
    static constexpr int NSW = 2 * KCP / KW;  // steps per wave and chunk
    static_assert((2 * KCP) % KW == 0, "KW must divide a chunk's steps");
    static constexpr int kRedBytes = KW * WS * S * T * kWave * 16;
    static __host__ __device__ int lds_bytes(int nch) {
        const int b = (nch > 1 ? 2 : 1) * kBufBytes;
        return b > kRedBytes ? b : kRedBytes;
    }
};

template <int S, int T, int WS, int KW, int KCP, class Epi, bool kSplit = false>
__global__ __launch_bounds__(WS * KW * kWave) void gemm_smfmac_kernel(
    const uint32_t* __restrict__ meta, const uint32_t* __restrict__ values,
    const int8_t* __restrict__ X, Epi epi, int rows, int cols, int n, int ms, int vs,
    GemmSegs segs, GemmSplit sk) {
    using P = StagedTile<S, T, WS, KW, KCP>;
    extern __shared__ __align__(16) uint8_t gemm_smem[];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int ws = wave % WS, kw = wave / WS;
    const int q = lane >> 4, li = lane & 15;
    const int r0 = blockIdx.x * P::RB;
    const int t0 = blockIdx.y * P::TB;
    if (r0 >= segs.end0) {
        const bool last = r0 >= segs.end1;
        meta += last ? segs.om2 : segs.om1;
        values += last ? segs.ov2 : segs.ov1;
    }
    const int npairs = cols >> 8;
    const int nch = (npairs + KCP - 1) / KCP;
    // this block's chunks: all of them, or split-K part blockIdx.z
    int c_begin = 0, c_end = nch;
    if constexpr (kSplit) {
        const int cpb = (nch + gridDim.z - 1) / gridDim.z;
        c_begin = blockIdx.z * cpb;
        c_end = min(nch, c_begin + cpb);
    }
    // Block-relative buffer resources: rows and tokens past the matrix read
    // zeros (their results are not stored); columns past the end in the last
    // chunk read other in-range bytes or zeros and feed only masked steps.
    // Every byte offset, the chunk's included, goes in the VGPR offset, which
    // the hardware checks against the resource's extent (the scalar offset
    // is not checked), so no load reads past a buffer's end.
    const int brows = min(rows - r0, P::RB), btoks = min(n - t0, P::TB);
    const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(meta + static_cast<long>(r0) * ms), static_cast<short>(0),
        brows * ms * 4, kRawBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(values + static_cast<long>(r0) * vs), static_cast<short>(0),
        brows * vs * 4, kRawBufferFlags);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(X + static_cast<long>(t0) * cols), static_cast<short>(0),
        btoks * cols, kRawBufferFlags);
    const int jm = tid % P::GM, trm = tid / P::GM;
    const int jv = tid % P::GV, trv = tid / P::GV;
    const int gm0 = (trm * ms + 4 * jm) * 4, gv0 = (trv * vs + 4 * jv) * 4;
    // B: thread k of a 16-group loads unit src(k) of the 256-byte pair (the
    // group's 16 loads cover it) and stores it as (q, c) = (k >> 2, k & 3):
    // each 8-thread half then writes 8 distinct bank groups (q-parts 4 mod 8
    // units apart), and the reads of a 16-lane group hit 16.
    const int gk = tid >> 4, kq = (tid & 15) >> 2, kc = tid & 3;
    const int src16 = 16 * ((kq >> 1) * 4 + 2 * (kc >> 1) + (kq & 1) + 8 * (kc & 1));
    const int lm0 = (4 * jm * P::RBM + trm) * 4;
    const int lv0 = (8 * KCP * P::RBM + 4 * jv * P::RBV + trv) * 4;

    u32x4v sm[P::KRM][P::KJM], sv[P::KRV][P::KJV], sb[P::KIB];
    auto load_chunk = [&](int c) {
        const int cm = c * 32 * KCP, cv = c * 16 * KCP, cb = c * 256 * KCP;
#pragma unroll
        for (int kr = 0; kr < P::KRM; ++kr)
#pragma unroll
            for (int kj = 0; kj < P::KJM; ++kj)
                if (P::RMK * (kr + 1) <= P::RB || trm + kr * P::RMK < P::RB)
                    sm[kr][kj] = __builtin_amdgcn_raw_buffer_load_b128(
                        rm, gm0 + kr * P::RMK * ms * 4 + kj * P::GM * 16 + cm, 0, 0);
#pragma unroll
        for (int kr = 0; kr < P::KRV; ++kr)
#pragma unroll
            for (int kj = 0; kj < P::KJV; ++kj)
                if (P::RVK * (kr + 1) <= P::RB || trv + kr * P::RVK < P::RB)
                    sv[kr][kj] = __builtin_amdgcn_raw_buffer_load_b128(
                        rv, gv0 + kr * P::RVK * vs * 4 + kj * P::GV * 16 + cv, 0, 0);
#pragma unroll
        for (int r = 0; r < P::KIB; ++r) {
            const int item = gk + r * P::G16, t = item & (P::TB - 1), pr = item / P::TB;
            if ((P::TB * KCP) % P::G16 == 0 || item < P::TB * KCP)
                sb[r] = __builtin_amdgcn_raw_buffer_load_b128(rx, t * cols + pr * 256 + src16 + cb,
                                                              0, 0);
        }
    };
    auto store_chunk = [&](int buf) {
        uint8_t* base = gemm_smem + buf * P::kBufBytes;
#pragma unroll
        for (int kr = 0; kr < P::KRM; ++kr)
#pragma unroll
            for (int kj = 0; kj < P::KJM; ++kj)
                if (P::RMK * (kr + 1) <= P::RB || trm + kr * P::RMK < P::RB) {
                    uint32_t* d = reinterpret_cast<uint32_t*>(
                        base + lm0 + kr * P::RMK * 4 + kj * P::GM * 16 * P::RBM);
#pragma unroll
                    for (int e = 0; e < 4; ++e) d[e * P::RBM] = sm[kr][kj][e];
                }
#pragma unroll
        for (int kr = 0; kr < P::KRV; ++kr)
#pragma unroll
            for (int kj = 0; kj < P::KJV; ++kj)
                if (P::RVK * (kr + 1) <= P::RB || trv + kr * P::RVK < P::RB) {
                    uint32_t* d = reinterpret_cast<uint32_t*>(
                        base + lv0 + kr * P::RVK * 4 + kj * P::GV * 16 * P::RBV);
#pragma unroll
                    for (int e = 0; e < 4; ++e) d[e * P::RBV] = sv[kr][kj][e];
                }
#pragma unroll
        for (int r = 0; r < P::KIB; ++r) {
            const int item = gk + r * P::G16, t = item & (P::TB - 1), pr = item / P::TB;
            if ((P::TB * KCP) % P::G16 == 0 || item < P::TB * KCP)
                *reinterpret_cast<u32x4v*>(
                    base + P::kABytes +
                    (kq * P::QS + (pr * P::TB + t) * 4 + (kc ^ ((t >> 2) & 3))) * 16) = sb[r];
        }
    };

    v4i acc[S][T];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[s][t] = (v4i){0, 0, 0, 0};

    // The epilogue's own loads (Epi::preload: the sink's per-token inputs),
    // issued ahead of the first chunk in the small tiles (the batched decode's
    // few-chunk launches, whose end would otherwise wait a memory round trip
    // for them), at the end in the tiles of more than four 16x16 products
    // per wave (the 64x64 and 128x64 tiles: held through the loop, their
    // registers cost the 64x64 tile its second block per CU); rows and
    // tokens past the matrix load row 0 /
    // the last token (nothing is stored for them).
    constexpr bool kEarly = S * T <= 4;
    typename Epi::Pre pre[S][T];
    auto preload = [&](int s, int t) {
        const int row = r0 + (ws * S + s) * 16 + 4 * q, tok = t0 + t * 16 + li;
        pre[s][t] = epi.preload(tok < n ? tok : n - 1, row < rows ? row : 0);
    };
    if constexpr (kEarly) {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                if (KW == 1 || (s * T + t) % KW == kw) preload(s, t);
    }

    load_chunk(c_begin);
    store_chunk(0);
    __syncthreads();
    for (int c = c_begin; c < c_end; ++c) {
        if (c + 1 < c_end) load_chunk(c + 1);  // in flight during this chunk's steps
        const uint8_t* base = gemm_smem + ((c - c_begin) & 1) * P::kBufBytes;
        const uint32_t* am = reinterpret_cast<const uint32_t*>(base);
        const uint32_t* av = am + 8 * KCP * P::RBM;
        const u32x4v* bb = reinterpret_cast<const u32x4v*>(base + P::kABytes);
        const int nst = 2 * min(KCP, npairs - c * KCP);  // steps in this chunk
        uint32_t mw[P::NSW][S], vw[P::NSW][S];
        u32x4v blo[P::NSW][T], bhi[P::NSW][T];
        // every operand of the wave's steps is read first, then decoded and used
#pragma unroll
        for (int j = 0; j < P::NSW; ++j) {
            const int stp = kw + j * KW;
            const int pp = stp >> 1, i = stp & 1;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int r = (ws * S + s) * 16 + li;
                mw[j][s] = am[(8 * pp + 2 * q + i) * P::RBM + r];
                vw[j][s] = av[(4 * pp + q) * P::RBV + r];
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int tr = t * 16 + li, sw = (tr >> 2) & 3;
                const u32x4v* row = bb + q * P::QS + (pp * P::TB + tr) * 4;
                blo[j][t] = row[(2 * i) ^ sw];
                bhi[j][t] = row[(2 * i + 1) ^ sw];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < P::NSW; ++j) {
            const int stp = kw + j * KW;
            const bool ok = stp < nst;  // the last chunk's missing steps add zero
            const int i = stp & 1;
            v4i a[S];
            int idx[S];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                idx[s] = smfmac_index(mw[j][s]);
                a[s] = smfmac_values(vw[j][s] >> (16 * i));
                if (!ok) a[s] = (v4i){0, 0, 0, 0};
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const v8i b = (v8i){(int)blo[j][t][0], (int)blo[j][t][1], (int)blo[j][t][2],
                                    (int)blo[j][t][3], (int)bhi[j][t][0], (int)bhi[j][t][1],
                                    (int)bhi[j][t][2], (int)bhi[j][t][3]};
#pragma unroll
                for (int s = 0; s < S; ++s)
                    acc[s][t] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a[s], b, acc[s][t],
                                                                           idx[s], 0, 0);
            }
        }
        if (c + 1 < c_end) store_chunk((c + 1 - c_begin) & 1);  // that buffer was last read a chunk ago
        __syncthreads();
    }
    // split-K sum: every wave parks its partials; wave kw adds up and stores
    // the (strip, tile) pairs e with e % KW == kw (exact integer adds)
    if (KW > 1) {
        v4i* red = reinterpret_cast<v4i*>(gemm_smem);
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                red[((kw * WS + ws) * S * T + s * T + t) * kWave + lane] = acc[s][t];
        __syncthreads();
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                if ((s * T + t) % KW == kw) {
                    v4i sum = red[(ws * S * T + s * T + t) * kWave + lane];
#pragma unroll
                    for (int k = 1; k < KW; ++k)
                        sum += red[((k * WS + ws) * S * T + s * T + t) * kWave + lane];
                    acc[s][t] = sum;
                }
    }
    if constexpr (kSplit) {
        // the flag goes in the (no longer read) LDS of the K-way sums: a static
        // LDS variable would lower the dynamic limit below the CU's LDS
        int& last_part = *reinterpret_cast<int*>(gemm_smem);
        const int tile = blockIdx.y * gridDim.x + blockIdx.x, ks = gridDim.z;
        // v4i slot of (tile, z, ws, s, t, lane); the extent ends the buffer
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
            sk.part, static_cast<short>(0), static_cast<int>(sk.part_words * 4), kRawBufferFlags);
        auto slot = [&](int z, int s, int t) {
            return (((static_cast<int>(tile) * ks + z) * WS + ws) * S * T + s * T + t) * kWave + lane;
        };
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                if (KW == 1 || (s * T + t) % KW == kw)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4v, acc[s][t]), rp, slot(blockIdx.z, s, t) * 16, 0,
                        kCachePolicySc1);
        __builtin_amdgcn_s_waitcnt(0);  // the partial stores are complete
        __syncthreads();
        if (tid == 0)
            last_part = __hip_atomic_fetch_add(sk.count + tile, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT) == static_cast<unsigned>(ks - 1);
        __syncthreads();
        if (!last_part) return;  // uniform
        if (tid == 0) __hip_atomic_store(sk.count + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int t = 0; t < T; ++t)
                if (KW == 1 || (s * T + t) % KW == kw) {
                    v4i sum = (v4i){0, 0, 0, 0};
                    for (int z = 0; z < ks; ++z)
                        sum += __builtin_bit_cast(
                            v4i, __builtin_amdgcn_raw_buffer_load_b128(rp, slot(z, s, t) * 16, 0,
                                                                       kCachePolicySc1));
                    acc[s][t] = sum;
                }
    }
    // lane (li, q) of tile (s, t) holds rows 16(ws S + s) + 4q .. +3 of token 16t + li
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int row = r0 + (ws * S + s) * 16 + 4 * q;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int tok = t0 + t * 16 + li;
            if ((KW == 1 || (s * T + t) % KW == kw) && tok < n && row < rows) {
                if constexpr (!kEarly) preload(s, t);
                epi.store4(tok, row, acc[s][t], pre[s][t]);
            }
        }
    }
}

bool gemm_aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// The staged kernel needs whole column pairs, 16-byte aligned rows and
// 16-byte aligned base pointers.
bool staged_ok(const void* meta, const void* values, const void* X, int cols, int ms, int vs) {
    return cols >= 256 && cols % 256 == 0 && ms % 4 == 0 && vs % 4 == 0 &&
           gemm_aligned(meta, 16) && gemm_aligned(values, 16) && gemm_aligned(X, 16);
}

// Staged tile per batch size (sweep on MI355X over 6912x2560, 2560x6912,
// 2560x2560 and 640x2560 at n = 16, 32, 64, 256 against the direct kernel):
//   n <= 16: 32 rows x 16 tokens, 8 waves splitting K 4 ways, chunks of 2560
//            columns (a 2560-column row in one memory round trip; longer rows
//            double-buffer 123 KB of LDS)
//   n <= 64: 64 rows x 32 tokens, 8 waves (2 row groups x 4 K ways)
//   n > 64 : 64 rows x 64 tokens, 8 waves (2 row groups x 4 K ways), 78 KB;
//            128 rows x 64 tokens (4 row groups x 2 K ways, one column pair
//            per chunk, 64 KB) when that grid has at least 4/5 as many
//            blocks as there are CUs
// Kernels above 64 KB of LDS need their limit raised (gemm_prepare).
enum StagedShape {
    kStagedN16, kStagedN16R16, kStagedN16Long, kStagedN16R64, kStagedN64, kStagedWide, kStagedWide128
};
// Batches of up to 16 tokens take the 32x16 tile; so do batches of up to 32
// whose 64x32 grid would fill at most half the CUs (the token tiles side by
// side, one chunk per 2560-column row: more blocks, one memory round trip
// each).  On the 2.4B model's batch-32 decode step the 32x16 tile took q|k|v
// from 9.25 to 6.44 us (240 blocks instead of 60) and o / down from 7.2 /
// 10.1 to ~6.4 us, but gate|up (216 tiles of 64x32 already) from 7.77 to
// 11.8 us (864 blocks); at 64 tokens it lost (6912x2560: 10.5 against 5.6 us).
// Up to 16 tokens: the smallest row block (16, 32 or 64 rows) whose grid
// stays within one block per CU -- these launches are a few chunks long, and
// a second block on some CUs sets the time.  8 tokens, back to back (us per
// launch, 32-row tile against the chosen one): 13824 x 2560 5.79 -> 4.63
// (64 rows, 216 blocks), 3840 x 2560 3.58 -> 3.39 and 2560 x 2560 3.53 ->
// 3.36 (16 rows, 240 / 160 blocks).  16-row blocks of rows longer than one
// 2560-column chunk take 3584-column chunks (two chunk round trips instead of
// three at 6912 columns; 140 KB of LDS): 2560 x 6912 5.89 -> 5.52.
constexpr int kStagedN16Max = 32;
StagedShape staged_shape(int n, int rows, int cols) {
    if (n <= 16) {
        const long cus = device_cu_count();
        if ((rows + 15) / 16 <= cus) return cols > 10 * 256 ? kStagedN16Long : kStagedN16R16;
        if ((rows + 31) / 32 <= cus) return kStagedN16;
        if ((rows + 63) / 64 <= cus) return kStagedN16R64;
        return kStagedN16;
    }
    if (n <= kStagedN16Max &&
        2L * ((rows + 63) / 64) * ((n + 31) / 32) <= static_cast<long>(device_cu_count()))
        return kStagedN16;
    if (n <= 64) return kStagedN64;
    // The 128x64 tile reads 5.4 operand bytes per product and chunk where the
    // 64x64 tile reads 9.3, the launch's L2-to-CU traffic (82 MB at n = 256 on
    // 6912 x 2560: the token block re-read by every row block) with it; it
    // pays once its grid nearly fills the chip.  Sweep on MI355X, us per
    // launch, 64x64 -> 128x64: 6912 x 2560 n = 256 / 512 / 1024 11.37 ->
    // 11.18, 19.57 -> 17.13, 33.29 -> 30.34; 13824 x 2560 n = 128 / 256 /
    // 1024 11.74 -> 11.20, 19.71 -> 16.79, 65.93 -> 54.95; 3840 x 2560
    // n = 1024 20.36 -> 17.47; 2560 x 6912 n = 1024 35.48 -> 33.48, while at
    // 160 blocks (2560 x 6912, n = 512) it lost (21.68 -> 26.08).
    const long wide128 = static_cast<long>((rows + 127) / 128) * ((n + 63) / 64);
    return 5 * wide128 >= 4 * device_cu_count() ? kStagedWide128 : kStagedWide;
}
int staged_row_block(int n, int rows, int cols) {
    switch (staged_shape(n, rows, cols)) {
        case kStagedN16R16:
        case kStagedN16Long: return 16;
        case kStagedN16: return 32;
        case kStagedWide128: return 128;
        default: return 64;
    }
}

template <int S, int T, int WS, int KW, int KCP, class Epi, bool kSplit = false>
const void* staged_fn() {
    return reinterpret_cast<const void*>(&gemm_smfmac_kernel<S, T, WS, KW, KCP, Epi, kSplit>);
}

// Split-K parts for a launch of `tiles` row x token tiles over nch chunks:
// only for long rows (at least kSplitMinChunks chunks) whose tiles fill at
// most half the CUs; enough parts to reach about one block per CU, at least
// two chunks each (1: no split).  Measured on the 2.4B model's batch-32
// decode step on the 64x32 tile: the down projection (14 chunks, 40 tiles)
// went from 15.2 to 10.3 us in 7 parts, while the 5-chunk q|k|v and o
// launches got slower (9.5 -> 10.8 and 7.2 -> 7.7 us): the partials' round
// trip through memory and the last block's sum cost more than their shorter
// chunk loops saved.  (Batch 32 now takes the 32x16 tile, whose rows are at
// most 3 chunks long; the split serves batches of 33-64 tokens.)
constexpr int kSplitMinChunks = 6;
int staged_split_parts(long tiles, int nch) {
    const long cus = device_cu_count();
    if (nch < kSplitMinChunks || 2 * tiles > cus) return 1;
    int ks = static_cast<int>((cus + tiles - 1) / tiles);
    if (ks > nch / 2) ks = nch / 2;
    const int cpb = (nch + ks - 1) / ks;
    return (nch + cpb - 1) / cpb;
}

template <int S, int T, int WS, int KW, int KCP, class Epi>
int launch_staged(const uint32_t* meta, const uint32_t* values, const int8_t* X, const Epi& epi,
                  int rows, int cols, int n, int ms, int vs, hipStream_t st, const GemmSegs& segs,
                  const GemmSplit* split = nullptr) {
    using P = StagedTile<S, T, WS, KW, KCP>;
    const int nch = (cols / 256 + KCP - 1) / KCP;
    const int lds = P::lds_bytes(nch);
    const dim3 grid((rows + P::RB - 1) / P::RB, (n + P::TB - 1) / P::TB);
    const long tiles = static_cast<long>(grid.x) * grid.y;
    int ks = split ? staged_split_parts(tiles, nch) : 1;
    // a workspace too small for this launch runs it unsplit
    if (ks > 1 && (tiles > split->count_words ||
                   tiles * ks * P::RB * P::TB > split->part_words))
        ks = 1;
    const void* fn = ks > 1 ? staged_fn<S, T, WS, KW, KCP, Epi, true>()
                            : staged_fn<S, T, WS, KW, KCP, Epi, false>();
    if (lds > 65536 && (lds > device_lds_per_cu() || !gemm_allow_lds(fn)))
        return invalid("spb_sparse_ternary_gemm: %d bytes of LDS unavailable", lds);
    if (ks > 1) {
        hipLaunchKernelGGL((gemm_smfmac_kernel<S, T, WS, KW, KCP, Epi, true>),
                           dim3(grid.x, grid.y, ks), dim3(P::NT), lds, st, meta, values, X, epi,
                           rows, cols, n, ms, vs, segs, *split);
    } else {
        hipLaunchKernelGGL((gemm_smfmac_kernel<S, T, WS, KW, KCP, Epi, false>), grid, dim3(P::NT),
                           lds, st, meta, values, X, epi, rows, cols, n, ms, vs, segs,
                           GemmSplit{nullptr, nullptr, 0, 0});
    }
    return 0;
}

// The staged launch for n tokens (the tile of staged_shape); the caller has
// checked staged_ok.  split: the caller's split-K workspace, or null.
template <class Epi>
int launch_staged_for(const uint32_t* meta, const uint32_t* values, const int8_t* X,
                      const Epi& epi, int rows, int cols, int n, int ms, int vs, hipStream_t st,
                      const GemmSegs& g, const GemmSplit* split = nullptr) {
    switch (staged_shape(n, rows, cols)) {
        case kStagedN16:
            return launch_staged<1, 1, 2, 4, 10>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                 split);
        case kStagedN16R16:
            return launch_staged<1, 1, 1, 4, 10>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                 split);
        case kStagedN16Long:
            return launch_staged<1, 1, 1, 4, 14>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                 split);
        case kStagedN16R64:
            return launch_staged<2, 1, 2, 4, 10>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                 split);
        case kStagedN64:
            return launch_staged<2, 2, 2, 4, 2>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                split);
        case kStagedWide128:
            return launch_staged<2, 4, 4, 2, 1>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                split);
        default:
            return launch_staged<2, 4, 2, 4, 2>(meta, values, X, epi, rows, cols, n, ms, vs, st, g,
                                                split);
    }
}

// Split-K workspace (int32 words of part) that launches of up to n tokens
// on these row counts and columns need at most.
long staged_split_words(const int* rows, int nrows, int cols, int n) {
    long words = 0;
    for (int i = 0; i < nrows; ++i) {
        const StagedShape sh = staged_shape(n, rows[i], cols);
        const bool t16 = n <= 16 || sh == kStagedN16;  // 16-token tiles
        const int rb = staged_row_block(n, rows[i], cols);
        const int tb = t16 ? 16 : (n <= 64 ? 32 : 64);
        const int kcp = sh == kStagedN16Long ? 14 : (t16 ? 10 : (sh == kStagedWide128 ? 1 : 2));
        const int nch = (cols / 256 + kcp - 1) / kcp;
        const long tiles = static_cast<long>((rows[i] + rb - 1) / rb) * ((n + tb - 1) / tb);
        const long w = tiles * staged_split_parts(tiles, nch) * rb * tb;
        if (w > words) words = w;
    }
    return words;
}

// Raises the LDS limit of the staged tiles with epilogue Epi, unsplit
// and split (0 = done).
template <class Epi>
int staged_prepare() {
    return gemm_allow_lds(staged_fn<1, 1, 2, 4, 10, Epi>()) &&
                   gemm_allow_lds(staged_fn<1, 1, 1, 4, 10, Epi>()) &&
                   gemm_allow_lds(staged_fn<1, 1, 1, 4, 10, Epi, true>()) &&
                   gemm_allow_lds(staged_fn<1, 1, 1, 4, 14, Epi>()) &&
                   gemm_allow_lds(staged_fn<1, 1, 1, 4, 14, Epi, true>()) &&
                   gemm_allow_lds(staged_fn<2, 1, 2, 4, 10, Epi>()) &&
                   gemm_allow_lds(staged_fn<2, 1, 2, 4, 10, Epi, true>()) &&
                   gemm_allow_lds(staged_fn<2, 2, 2, 4, 2, Epi>()) &&
                   gemm_allow_lds(staged_fn<2, 4, 2, 4, 2, Epi>()) &&
                   gemm_allow_lds(staged_fn<1, 1, 2, 4, 10, Epi, true>()) &&
                   gemm_allow_lds(staged_fn<2, 2, 2, 4, 2, Epi, true>()) &&
                   gemm_allow_lds(staged_fn<2, 4, 2, 4, 2, Epi, true>()) &&
                   gemm_allow_lds(staged_fn<2, 4, 4, 2, 1, Epi>()) &&
                   gemm_allow_lds(staged_fn<2, 4, 4, 2, 1, Epi, true>())
               ? 0
               : 1;
}

// The int32 products, token-major Y [n][rows] (the entry point's output).
// A lane's four rows row .. row + 3 (row a multiple of 4, row < rows) are one
// 16-byte store when every token's run of Y starts 16-byte aligned (rows a
// multiple of 4 and Y aligned, `quads`); otherwise each row is stored on its
// own and rows past the last are dropped, so no token's rows spill into the
// next token's and nothing is written past Y's end.
struct Int32Out {
    int32_t* Y;
    int rows;
    bool quads;
    struct Pre {};
    __device__ Pre preload(int, int) const { return {}; }
    __device__ void store4(int tok, int row, v4i acc, const Pre&) const {
        int32_t* y = Y + static_cast<long>(tok) * rows + row;
        if (quads) {
            *reinterpret_cast<v4i*>(y) = acc;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (row + k < rows) y[k] = acc[k];
        }
    }
};

// Up to three stacked projections (equal columns and strides) in one
// launch with epilogue Epi, rows of the stack in order.  Returns 1 (nothing
// launched) when the shapes do not allow it: columns or strides differ, the
// staged kernel's conditions fail, or a segment boundary falls inside a
// block's row tile; 2 on a launch error, 0 when launched.
template <class Epi>
int gemm_stacked_epi(const spb_sparse_linear* const* segs, int nseg, const int8_t* X,
                     const Epi& epi, int n, hipStream_t st, const GemmSplit* split = nullptr) {
    if (nseg < 1 || nseg > 3 || n <= 0 || (n + 15) / 16 > 65535) return 1;
    const spb_sparse_linear& a = *segs[0];
    int rows = 0, ends[3] = {0, 0, 0};
    for (int i = 0; i < nseg; ++i) {
        const spb_sparse_linear& l = *segs[i];
        if (l.cols != a.cols || l.meta_stride != a.meta_stride ||
            l.values_stride != a.values_stride || !l.meta || !l.values)
            return 1;
        rows += l.rows;
        ends[i] = rows;
    }
    if (!staged_ok(a.meta, a.values, X, a.cols, a.meta_stride, a.values_stride)) return 1;
    const int rb = staged_row_block(n, rows, a.cols);
    GemmSegs g{0, 0, 0, 0, ends[0], nseg > 1 ? ends[1] : ends[0]};
    if (nseg == 1) g.end0 = g.end1 = rows;
    for (int i = 1; i < nseg; ++i) {
        // every segment's rows must start a block, on a 16-byte boundary
        if (ends[i - 1] % rb || !gemm_aligned(segs[i]->meta, 16) ||
            !gemm_aligned(segs[i]->values, 16))
            return 1;
        const long om = (segs[i]->meta - a.meta) - static_cast<long>(ends[i - 1]) * a.meta_stride;
        const long ov = (segs[i]->values - a.values) -
                        static_cast<long>(ends[i - 1]) * a.values_stride;
        if (i == 1) {
            g.om1 = om;
            g.ov1 = ov;
            g.om2 = om;  // two segments: rows past end1 do not exist
            g.ov2 = ov;
        } else {
            g.om2 = om;
            g.ov2 = ov;
        }
    }
    if (nseg == 2) g.end1 = rows;
    if (launch_staged_for(a.meta, a.values, X, epi, rows, a.cols, n, a.meta_stride,
                          a.values_stride, st, g, split))
        return 2;
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace
}  // namespace spb

// gemm.hip -- batched 2:4 sparse-ternary GEMM on the int8 structured-sparse
// matrix cores of gfx950 (v_smfmac_i32_16x16x128_i8).
//
// What it computes: Y[t][r] = sum_c W[r][c] * X[t][c] (exact int32), X
// token-major int8 [n][cols], Y token-major int32 [n][rows]; this is the
// reference's cuSPARSELt product D = A * B with B [K x N] and D [M x N]
// column-major (src/cusparselt_backend.cu:53-62, 83-89, 186-207), computed
// directly on spbitnet's packed format instead of a library-pruned copy.
//
// Why the format maps onto SMFMAC with no repacking:
//   * The sparse A operand of v_smfmac_i32_16x16x128_i8 is 16 rows x 128 K in
//     compressed form: lane l holds row l%16, logical K [32*(l/16), +32) as 8
//     groups of 4, two int8 values per group (16 bytes), plus a 32-bit index
//     word with the 2-bit position of compressed byte j at bits [2j, 2j+1].
//     One spbitnet meta word is exactly one lane's 32 columns.
//   * The compressed values are the kept weights in column order, lower first;
//     spbitnet's sign bits are in the same order (bit 2g = lower, 2g+1 =
//     higher), so byte j = (sign bit j ? -1 : +1).
//   * The index nibble of group g is p0 | p1 << 2 (p0 < p1 the set bits of
//     bitmap b), computed for 8 groups at once:
//       p0 bit0 = ~b0 & b1,  p0 bit1 = ~(b0 | b1),
//       p1 bit0 =  b3 | ~b2, p1 bit1 =  b3 | b2
//     (four v_bitop3_b32 on the meta word and its 1-bit shifts).
//   * B (activations, 128 K x 16 tokens): lane l holds token l%16; bytes
//     0..15 are K 16*(l/16) + i and bytes 16..31 are K 64 + 16*(l/16) + i.
//     C (16 rows x 16 tokens, int32): lane l holds token l%16, rows
//     4*(l/16) + v in VGPR v.
// These operand layouts were established on the hardware with register-only
// probes and are pinned by the GPU parity tests against the CPU oracle.
//
// Work mapping: a block of 8 waves owns kStrips 16-row strips and one pass
// of kTiles*16 tokens (grid.y); the waves split K in 128-column steps.  Per
// step a wave decodes each strip's A operand once (one meta word and 16 sign
// bits per lane: ~24 VALU ops) and reuses each B tile for kStrips SMFMACs.
// Partial sums are reduced across the waves in LDS.
#include <mutex>
#include <set>
#include <utility>

#include "common.hpp"
#include "spbitnet_amd.h"

namespace spb {
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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));


template <uint32_t kTable>
__device__ __forceinline__ uint32_t bitop3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, kTable);
}

// Index word of one meta word (8 groups): nibble g = p0 | p1 << 2.
__device__ __forceinline__ int smfmac_index(uint32_t k) {
    const uint32_t a = k >> 1, c = k << 1;
    const uint32_t t0 = bitop3<0x20>(a, k, 0x11111111u);  // (a & ~b) & m : ~b0 & b1
    const uint32_t t1 = bitop3<0x02>(c, k, 0x22222222u);  // ~(a | b) & m : ~(b0 | b1)
    const uint32_t t2 = bitop3<0xA2>(a, k, 0x44444444u);  // (a | ~b) & m : b3 | ~b2
    const uint32_t t3 = bitop3<0xA8>(c, k, 0x88888888u);  // (a | b) & m  : b3 | b2
    return static_cast<int>(bitop3<0xFE>(t0, t1, t2) | t3);
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

// Block: kWaves waves on the same kStrips*16 rows and the same pass of
// kTiles*16 tokens (pass = blockIdx.y), splitting K: wave w takes the
// 128-column steps s = w, w + kWaves, ...  Each wave decodes its A operands
// once per step and reuses every B tile for kStrips SMFMACs.  The waves'
// int32 partial sums meet in LDS (integer atomics, exact in any order).
template <int kStrips, int kTiles, int kWaves>
__global__ __launch_bounds__(kWaves * kWave) void gemm_smfmac_direct_kernel(
    const uint32_t* __restrict__ meta, const uint32_t* __restrict__ values,
    const int8_t* __restrict__ X, int32_t* __restrict__ Y, int rows, int cols, int n, int ms,
    int vs, GemmSegs segs) {
    constexpr int kBlock = kWaves * kWave;
    constexpr int kAcc = kStrips * kTiles * 4;  // int32 accumulators per lane
    __shared__ int red[kAcc * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const long r0 = static_cast<long>(blockIdx.x) * (kStrips * 16);
    // stacked matrices: the block's rows lie in one segment, whose words sit
    // at a fixed offset from the row's index in the first (uniform selects)
    if (r0 >= segs.end0) {
        const bool last = r0 >= segs.end1;
        meta += last ? segs.om2 : segs.om1;
        values += last ? segs.ov2 : segs.ov1;
    }
    const int tok0 = blockIdx.y * (kTiles * 16);
    const int q = lane >> 4;   // lane group
    const int li = lane & 15;  // A row / B,C token within a tile

    for (int i = threadIdx.x; i < kAcc * kWave; i += kBlock) red[i] = 0;

    v4i acc[kStrips][kTiles];
#pragma unroll
    for (int st = 0; st < kStrips; ++st)
#pragma unroll
        for (int t = 0; t < kTiles; ++t) acc[st][t] = (v4i){0, 0, 0, 0};

    const int nsteps = cols >> 7;
    for (int s = wave; s < nsteps; s += kWaves) {
        const int w = 4 * s + q;  // this lane's meta word
        v4i a[kStrips];
        int idx[kStrips];
#pragma unroll
        for (int st = 0; st < kStrips; ++st) {
            const long ra = r0 + st * 16 + li;
            a[st] = (v4i){0, 0, 0, 0};
            idx[st] = 0;
            if (ra < rows) {
                const uint32_t k = meta[ra * ms + w];
                const uint32_t vw = values[ra * vs + (w >> 1)];
                idx[st] = smfmac_index(k);
                a[st] = smfmac_values((w & 1) ? (vw >> 16) : (vw & 0xFFFFu));
            }
        }
        const int kb = s * 128 + 16 * q;  // B bytes 0..15 -> K kb.., 16..31 -> K kb+64..
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const int tok = tok0 + t * 16 + li;
            v8i b = (v8i){0, 0, 0, 0, 0, 0, 0, 0};
            if (tok < n) {
                const int8_t* xr = X + static_cast<long>(tok) * cols + kb;
                const uint4 lo = *reinterpret_cast<const uint4*>(xr);
                const uint4 hi = *reinterpret_cast<const uint4*>(xr + 64);
                b = (v8i){static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z),
                          static_cast<int>(lo.w), static_cast<int>(hi.x), static_cast<int>(hi.y),
                          static_cast<int>(hi.z), static_cast<int>(hi.w)};
            }
#pragma unroll
            for (int st = 0; st < kStrips; ++st)
                acc[st][t] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a[st], b, acc[st][t],
                                                                       idx[st], 0, 0);
        }
    }
    __syncthreads();  // red[] zeroed
#pragma unroll
    for (int st = 0; st < kStrips; ++st)
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                atomicAdd(&red[((st * kTiles + t) * 4 + v) * kWave + lane], acc[st][t][v]);
    __syncthreads();
    // Write-out, row-fastest so each token's kStrips*16 outputs are one
    // contiguous run of Y.  Entry (st, t, v) of lane l holds token
    // tok0 + 16t + l%16 and row r0 + 16st + 4(l/16) + v.
    constexpr int kRows = kStrips * 16;
    for (int e = threadIdx.x; e < kAcc * kWave; e += kBlock) {
        const int rl = e % kRows, tl = e / kRows;  // local row, local token
        const int st = rl >> 4, q = (rl >> 2) & 3, v = rl & 3;
        const int t = tl >> 4, l = q * 16 + (tl & 15);
        const int tok = tok0 + tl;
        const long row = r0 + rl;
        if (tok < n && row < rows)
            Y[static_cast<long>(tok) * rows + row] = red[((st * kTiles + t) * 4 + v) * kWave + l];
    }
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
// partial sums of a tile meet in LDS after the last chunk.
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

template <int S, int T, int WS, int KW, int KCP>
__global__ __launch_bounds__(WS * KW * kWave) void gemm_smfmac_kernel(
    const uint32_t* __restrict__ meta, const uint32_t* __restrict__ values,
    const int8_t* __restrict__ X, int32_t* __restrict__ Y, int rows, int cols, int n, int ms,
    int vs, GemmSegs segs) {
    using P = StagedTile<S, T, WS, KW, KCP>;
    extern __shared__ __align__(16) uint8_t smem[];
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
    // Block-relative buffer resources: rows and tokens past the matrix read
    // zeros (their results are not stored); columns past the end in the last
    // chunk read other in-range bytes or zeros and feed only masked steps.
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
                        rm, gm0 + kr * P::RMK * ms * 4 + kj * P::GM * 16, cm, 0);
#pragma unroll
        for (int kr = 0; kr < P::KRV; ++kr)
#pragma unroll
            for (int kj = 0; kj < P::KJV; ++kj)
                if (P::RVK * (kr + 1) <= P::RB || trv + kr * P::RVK < P::RB)
                    sv[kr][kj] = __builtin_amdgcn_raw_buffer_load_b128(
                        rv, gv0 + kr * P::RVK * vs * 4 + kj * P::GV * 16, cv, 0);
#pragma unroll
        for (int r = 0; r < P::KIB; ++r) {
            const int item = gk + r * P::G16, t = item & (P::TB - 1), pr = item / P::TB;
            if ((P::TB * KCP) % P::G16 == 0 || item < P::TB * KCP)
                sb[r] = __builtin_amdgcn_raw_buffer_load_b128(rx, t * cols + pr * 256 + src16, cb, 0);
        }
    };
    auto store_chunk = [&](int buf) {
        uint8_t* base = smem + buf * P::kBufBytes;
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

    load_chunk(0);
    store_chunk(0);
    __syncthreads();
    for (int c = 0; c < nch; ++c) {
        if (c + 1 < nch) load_chunk(c + 1);  // in flight during this chunk's steps
        const uint8_t* base = smem + (c & 1) * P::kBufBytes;
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
        if (c + 1 < nch) store_chunk((c + 1) & 1);  // that buffer was last read a chunk ago
        __syncthreads();
    }
    // split-K sum: every wave parks its partials; wave kw adds up and stores
    // the (strip, tile) pairs e with e % KW == kw (exact integer adds)
    if (KW > 1) {
        v4i* red = reinterpret_cast<v4i*>(smem);
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
    // lane (li, q) of tile (s, t) holds rows 16(ws S + s) + 4q .. +3 of token 16t + li
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int row = r0 + (ws * S + s) * 16 + 4 * q;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int tok = t0 + t * 16 + li;
            if ((KW == 1 || (s * T + t) % KW == kw) && tok < n && row < rows)
                *reinterpret_cast<v4i*>(Y + static_cast<long>(tok) * rows + row) = acc[s][t];
        }
    }
}

// General batched kernel: one wave per row, tokens looped inside; any shape.
__global__ __launch_bounds__(256) void gemm_general_kernel(const uint32_t* __restrict__ meta,
                                                           const uint32_t* __restrict__ values,
                                                           const int8_t* __restrict__ X,
                                                           int32_t* __restrict__ Y, int rows,
                                                           int cols, int n, int ms, int vs) {
    const int lane = threadIdx.x & (kWave - 1);
    const long row = static_cast<long>(blockIdx.x) * 4 + threadIdx.x / kWave;
    const int tok = blockIdx.y;
    if (row >= rows) return;
    const uint32_t* mr = meta + row * ms;
    const uint32_t* vr = values + row * vs;
    const int8_t* x = X + static_cast<long>(tok) * cols;
    int acc = 0;
    for (int g = lane; g < (cols >> 2); g += kWave) {
        const uint32_t bm = (mr[g >> 3] >> ((g & 7) * 4)) & 0xFu;
        const uint32_t sg = (vr[g >> 4] >> ((g & 15) * 2)) & 0x3u;
        const bool ok = __builtin_popcount(bm) == 2;
        const int p0 = ok ? __builtin_ctz(bm) : 0;
        const int p1 = ok ? __builtin_ctz(bm & (bm - 1)) : 0;
        const int x0 = x[4 * g + p0], x1 = x[4 * g + p1];
        acc += (sg & 1u) ? -x0 : x0;
        acc += (sg & 2u) ? -x1 : x1;
    }
    acc = wave_sum(acc);
    if (lane == 0) Y[static_cast<long>(tok) * rows + row] = acc;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

template <int kStrips, int kTiles, int kWaves>
void launch_smfmac(const uint32_t* meta, const uint32_t* values, const int8_t* X, int32_t* Y,
                   int rows, int cols, int n, int ms, int vs, hipStream_t st,
                   const GemmSegs* segs = nullptr) {
    const dim3 grid((rows + kStrips * 16 - 1) / (kStrips * 16), (n + kTiles * 16 - 1) / (kTiles * 16));
    const GemmSegs one{0, 0, 0, 0, rows, rows};
    hipLaunchKernelGGL((gemm_smfmac_direct_kernel<kStrips, kTiles, kWaves>), grid, dim3(kWaves * kWave),
                       0, st, meta, values, X, Y, rows, cols, n, ms, vs, segs ? *segs : one);
}

// The tile shape the direct kernel takes for n tokens over `rows` rows:
// strips (16-row strips per block), tiles (16-token tiles per pass).
void smfmac_tiles(int rows, int n, int* strips, int* tiles) {
    if (n <= 16) {
        *strips = 2, *tiles = 1;
    } else if (n <= 64) {
        *strips = 2, *tiles = 4;
    } else {
        const long cus = device_cu_count();
        const long tl = (n + 63) / 64;
        auto blocks = [&](int st) { return (rows + 16L * st - 1) / (16L * st) * tl; };
        *tiles = 4;
        *strips = blocks(8) * 5 >= cus * 3 ? 8 : (blocks(4) * 5 >= cus * 3 ? 4 : 2);
    }
}

// Raises a kernel's dynamic-LDS limit to the CU's LDS, once per device.
bool allow_lds(const void* fn) {
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({fn, dev})) return true;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, device_lds_per_cu()) !=
        hipSuccess)
        return false;
    done.insert({fn, dev});
    return true;
}

// The staged kernel needs whole column pairs, 16-byte aligned rows and
// 16-byte aligned base pointers.
bool staged_ok(const void* meta, const void* values, const void* X, int cols, int ms, int vs) {
    return cols >= 256 && cols % 256 == 0 && ms % 4 == 0 && vs % 4 == 0 && aligned(meta, 16) &&
           aligned(values, 16) && aligned(X, 16);
}

// Staged tile per batch size (sweep on MI355X over 6912x2560, 2560x6912,
// 2560x2560 and 640x2560 at n = 16, 32, 64, 256 against the direct kernel):
//   n <= 16: 32 rows x 16 tokens, 8 waves splitting K 4 ways, chunks of 2560
//            columns (a 2560-column row in one memory round trip; longer rows
//            double-buffer 123 KB of LDS)
//   n <= 64: 64 rows x 32 tokens, 8 waves (2 row groups x 4 K ways)
//   n > 64 : 64 rows x 64 tokens, 8 waves (2 row groups x 4 K ways), 78 KB
// Kernels above 64 KB of LDS need their limit raised (gemm_prepare).
enum StagedShape { kStagedN16, kStagedN64, kStagedWide };
StagedShape staged_shape(int n) { return n <= 16 ? kStagedN16 : (n <= 64 ? kStagedN64 : kStagedWide); }
int staged_row_block(int n) { return n <= 16 ? 32 : 64; }

template <int S, int T, int WS, int KW, int KCP>
const void* staged_fn() {
    return reinterpret_cast<const void*>(&gemm_smfmac_kernel<S, T, WS, KW, KCP>);
}

template <int S, int T, int WS, int KW, int KCP>
int launch_staged(const uint32_t* meta, const uint32_t* values, const int8_t* X, int32_t* Y,
                  int rows, int cols, int n, int ms, int vs, hipStream_t st, const GemmSegs& segs) {
    using P = StagedTile<S, T, WS, KW, KCP>;
    const int nch = (cols / 256 + KCP - 1) / KCP;
    const int lds = P::lds_bytes(nch);
    if (lds > 65536 && (lds > device_lds_per_cu() || !allow_lds(staged_fn<S, T, WS, KW, KCP>())))
        return invalid("spb_sparse_ternary_gemm: %d bytes of LDS unavailable", lds);
    const dim3 grid((rows + P::RB - 1) / P::RB, (n + P::TB - 1) / P::TB);
    hipLaunchKernelGGL((gemm_smfmac_kernel<S, T, WS, KW, KCP>), grid, dim3(P::NT), lds, st, meta,
                       values, X, Y, rows, cols, n, ms, vs, segs);
    return 0;
}

int launch_smfmac_for(const uint32_t* meta, const uint32_t* values, const int8_t* X, int32_t* Y,
                      int rows, int cols, int n, int ms, int vs, hipStream_t st,
                      const GemmSegs* segs) {
    if (staged_ok(meta, values, X, cols, ms, vs)) {
        const GemmSegs one{0, 0, 0, 0, rows, rows};
        const GemmSegs& g = segs ? *segs : one;
        switch (staged_shape(n)) {
            case kStagedN16:
                return launch_staged<1, 1, 2, 4, 10>(meta, values, X, Y, rows, cols, n, ms, vs, st, g);
            case kStagedN64:
                return launch_staged<2, 2, 2, 4, 2>(meta, values, X, Y, rows, cols, n, ms, vs, st, g);
            default:
                return launch_staged<2, 4, 2, 4, 2>(meta, values, X, Y, rows, cols, n, ms, vs, st, g);
        }
    }
    int strips = 0, tiles = 0;
    smfmac_tiles(rows, n, &strips, &tiles);
    if (strips == 2 && tiles == 1)
        launch_smfmac<2, 1, 4>(meta, values, X, Y, rows, cols, n, ms, vs, st, segs);
    else if (strips == 2)
        launch_smfmac<2, 4, 8>(meta, values, X, Y, rows, cols, n, ms, vs, st, segs);
    else if (strips == 4)
        launch_smfmac<4, 4, 8>(meta, values, X, Y, rows, cols, n, ms, vs, st, segs);
    else
        launch_smfmac<8, 4, 8>(meta, values, X, Y, rows, cols, n, ms, vs, st, segs);
    return 0;
}

// Rows per block of the matrix-core launch launch_smfmac_for makes.
int smfmac_row_block(const void* meta, const void* values, const void* X, int rows, int cols,
                     int n, int ms, int vs) {
    if (staged_ok(meta, values, X, cols, ms, vs)) return staged_row_block(n);
    int strips = 0, tiles = 0;
    smfmac_tiles(rows, n, &strips, &tiles);
    return 16 * strips;
}

}  // namespace
}  // namespace spb

using namespace spb;

extern "C" int spb_sparse_ternary_gemm_kernel_id(const uint32_t* meta, const uint32_t* values,
                                                 const int8_t* X, int rows, int cols, int n,
                                                 int ms, int vs) {
    (void)rows;
    (void)n;
    if (cols <= 0 || cols % 128 != 0 || !aligned(X, 16)) return 0;
    return staged_ok(meta, values, X, cols, ms, vs) ? 2 : 1;
}

extern "C" int spb_sparse_ternary_gemm(const uint32_t* meta, const uint32_t* values,
                                       const int8_t* X, int32_t* Y, int rows, int cols, int n,
                                       int ms, int vs, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_sparse_ternary_gemm";
    if (rows < 0 || cols < 0 || n < 0) return invalid("%s: negative shape", fn);
    if (cols % 4) return invalid("%s: cols=%d is not a multiple of 4", fn, cols);
    if (ms < (cols / 4 + 7) / 8 || vs < (cols / 4 + 15) / 16)
        return invalid("%s: row strides are smaller than the format requires", fn);
    if (rows == 0 || cols == 0 || n == 0) return 0;
    if (!meta || !values || !X || !Y) return invalid("%s: null pointer", fn);
    hipStream_t st = as_stream(stream);
    if (spb_sparse_ternary_gemm_kernel_id(meta, values, X, rows, cols, n, ms, vs)) {
        // The staged kernel when the strides and pointers allow it, else the
        // direct one (launch_smfmac_for picks the tile for the batch).
        if ((n + 15) / 16 > 65535) return invalid("%s: batch %d too large", fn, n);
        const int rc = launch_smfmac_for(meta, values, X, Y, rows, cols, n, ms, vs, st, nullptr);
        if (rc) return rc;
    } else {
        if (n > 65535) return invalid("%s: batch %d exceeds 65535", fn, n);
        hipLaunchKernelGGL(gemm_general_kernel, dim3((rows + 3) / 4, n), dim3(256), 0, st, meta,
                           values, X, Y, rows, cols, n, ms, vs);
    }
    return launch_status(fn);
}

namespace spb {

// Raises the LDS limit of the staged kernels above 64 KB on the current
// device (once per device); 0 on success.  Engines call it at create, so no
// attribute call happens during graph capture.
int gemm_prepare() {
    return allow_lds(staged_fn<1, 1, 2, 4, 10>()) && allow_lds(staged_fn<2, 2, 2, 4, 2>()) &&
                   allow_lds(staged_fn<2, 4, 2, 4, 2>())
               ? 0
               : 1;
}

// Y [n][sum of rows] = (A | B | C) X for up to three stacked projections
// (the engines' q | k | v and gate | up) in one matrix-core launch.
// Returns 1 (nothing launched) when the shapes do not allow it: columns or
// strides differ, the matrix-core conditions fail, or a segment boundary
// falls inside a block's row tile; the caller then launches them apart.
int gemm_stacked(const spb_sparse_linear* const* segs, int nseg, const int8_t* X, int32_t* Y,
                 int n, hipStream_t st) {
    if (nseg < 1 || nseg > 3 || n <= 0) return 1;
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
    if (!spb_sparse_ternary_gemm_kernel_id(a.meta, a.values, X, rows, a.cols, n, a.meta_stride,
                                           a.values_stride) ||
        (n + 15) / 16 > 65535)
        return 1;
    const int rb = smfmac_row_block(a.meta, a.values, X, rows, a.cols, n, a.meta_stride,
                                    a.values_stride);
    GemmSegs g{0, 0, 0, 0, ends[0], nseg > 1 ? ends[1] : ends[0]};
    if (nseg == 1) g.end0 = g.end1 = rows;
    for (int i = 1; i < nseg; ++i) {
        // every segment's rows must start a block, on a 16-byte boundary
        if (ends[i - 1] % rb || !aligned(segs[i]->meta, 16) || !aligned(segs[i]->values, 16))
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
    if (launch_smfmac_for(a.meta, a.values, X, Y, rows, a.cols, n, a.meta_stride,
                          a.values_stride, st, &g))
        return 2;
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace spb

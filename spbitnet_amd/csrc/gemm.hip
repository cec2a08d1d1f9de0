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
#include "gemm_staged.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

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

int launch_smfmac_for(const uint32_t* meta, const uint32_t* values, const int8_t* X, int32_t* Y,
                      int rows, int cols, int n, int ms, int vs, hipStream_t st,
                      const GemmSegs* segs) {
    if (staged_ok(meta, values, X, cols, ms, vs)) {
        const GemmSegs one{0, 0, 0, 0, rows, rows};
        const Int32Out out{Y, rows, rows % 4 == 0 && gemm_aligned(Y, 16)};
        return launch_staged_for(meta, values, X, out, rows, cols, n, ms, vs, st,
                                 segs ? *segs : one);
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
    if (staged_ok(meta, values, X, cols, ms, vs)) return staged_row_block(n, rows, cols);
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
    if (cols <= 0 || cols % 128 != 0 || !gemm_aligned(X, 16)) return 0;
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

bool gemm_allow_lds(const void* fn) {
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

// Raises the LDS limit of the staged kernels above 64 KB on the current
// device (once per device); 0 on success.  Engines call it at create, so no
// attribute call happens during graph capture.
int gemm_prepare() { return staged_prepare<Int32Out>(); }

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
    if (launch_smfmac_for(a.meta, a.values, X, Y, rows, a.cols, n, a.meta_stride,
                          a.values_stride, st, &g))
        return 2;
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace spb

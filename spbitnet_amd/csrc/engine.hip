// engine.hip -- bs=1 greedy decode of a BitNet b1.58 (2:4 sparse-ternary)
// transformer on gfx950, as one HIP graph per token.
//
// Dataflow and semantics follow the reference engine, InferenceEngine::forward
// (src/inference.cu:126-283), with bf16 activations / KV cache and the layer
// order:
//   x = embed[tok]
//   per layer: r = x; h = RMSNorm(r; input_ln); q,k,v = BitLinear(h);
//              RoPE(q, k); cache k, v; a = softmax(q k^T / sqrt(hd)) v;
//              o = BitLinear(a); o = RMSNorm(o; attn_sub_norm); x = o + r;
//              r = x; h = RMSNorm(x; post_ln); g,u = BitLinear(h);
//              m = relu(g)^2 * u (fp32); m = RMSNorm_f32in(m; ffn_sub_norm);
//              d = BitLinear(m); x = d + r
//   logits = lm_head . RMSNorm(x; final_norm);  next = argmax(logits)
//
// Kernels per layer (the reference launches ~25; here 5):
//   qkv     bit-plane GEMV over the stacked q/k/v matrices; its prologue
//           does the embedding lookup (layer 0), input RMSNorm, absmax and
//           int8 quantisation straight into LDS bit planes; its epilogue
//           dequantises each projection with its own gamma.
//   attn    RoPE of q and k, KV-cache write, and split-KV GQA attention
//           (one block per (kv head, 256-position split)).
//   o       GEMV; prologue combines the attention splits, absmax, quantise.
//   gate_up GEMV over stacked gate/up; prologue = attn sub-norm, residual add
//           (block 0 stores the new residual), post-attention RMSNorm,
//           absmax, quantise.
//   down    GEMV; prologue = relu^2 * up in fp32, ffn sub-norm, absmax,
//           quantise; epilogue = dequantise + residual add.
// and one LM-head kernel: final RMSNorm, bf16 GEMV to fp32 logits, argmax
// (last-block reduction), and the token/position update in device memory, so
// a whole greedy generation is graph replays with no host round trip.
//
// Every floating-point reduction has a fixed order (listed at each helper), so
// the CPU oracle in oracle/ reproduces the logits bit for bit.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <new>
#include <type_traits>
#include <vector>

#include "bitplane.hpp"
#include "gemm_staged.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

constexpr int kAttnSplit = 64;    // positions per attention split (one per lane)
constexpr int kAttnThreads = 256;
constexpr int kAttnBucketSplits = 4;  // splits per position bucket of the decode graphs
constexpr int kPrefillChunk = 1024;      // prompt tokens per batched-prefill pass (at most)
constexpr int kGemmSplitCounters = 1024;  // split-K tile counters of a batch engine (split launches have at most CUs / 2 tiles)
// Sequence groups of a batched decode step: two parallel branches of the
// step graph for 24-32 sequences (same-box bench at config 4: batch 32
// 11,943-11,952 -> 12,358-12,380 tok/s with two groups, 11,840-11,878 with
// three, 9,196-11,277 with four; batch 16 7,818-7,819 with one, 7,760-7,761 with two; batch 8
// 4,509-4,512 with one, 4,354-4,384 with two).  Larger batches keep one
// branch, so the GEMMs' split over K (33-64 tokens) sees the whole batch.
int batch_groups(int batch) { return batch >= 24 && batch <= 32 ? 2 : 1; }
constexpr long kPrefillPartialBytes = 1L << 30;  // split partials of one pass (at most)
constexpr int kPrefillMinDefault = 16;   // prompt tokens before the last that switch to it
constexpr int kAttnMaxGroup = 8;  // q heads per kv head
constexpr int kLmBlock = 256;
constexpr int kLmMaxH = 8192;
constexpr int kLmMaxRows = 2048;  // LM-head rows per block (grid >= vocab / 2048)

struct EngineState {
    int pos;         // position of the token the next step processes
    int prompt_len;  // tokens[0 .. prompt_len) are given, later ones generated
    int limit;       // positions available (KV capacity and token buffer)
    int done;        // set by EOS (when stop_eos) or when the limit is reached
    int stop_eos;
    int eos;
    unsigned ticket;  // LM-head blocks finished in the current step
    int generated;
};
static_assert(offsetof(EngineState, pos) == 0 && offsetof(EngineState, done) == 12,
              "state_pos and state_done read these offsets");

// A field of the decode state through a one-dword vector (buffer) load.  A
// plain load of a uniform field compiles to a scalar load, whose wait counter
// is shared with LDS: the first LDS wait of a prologue would then also wait
// for it.  A vector load completes in order with the kernel's other vector
// loads and is waited for only where it is used.  One dword per field: a
// wider load with dead fields lets the register allocator reuse their
// registers, and writing such a register waits for the whole load.
__device__ __forceinline__ int state_load(const EngineState* st, int offset) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<EngineState*>(st), static_cast<short>(0), 16, kBufferFlags);
    return static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(r, offset, 0, 0));
}
__device__ __forceinline__ int state_pos(const EngineState* st) { return state_load(st, 0); }
__device__ __forceinline__ int state_done(const EngineState* st) { return state_load(st, 12); }

// ---- fixed-order arithmetic shared with the oracle ------------------------------

__device__ __forceinline__ float bf16r(float f) { return BF16::to_float(BF16::from_float(f)); }

// Sum over the 64 lanes as the balanced pairwise tree over adjacent lanes
// (lanes 2i and 2i+1 first, then pairs of pairs, ...): DPP steps inside each
// 16-lane row (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror: each adds the partner group's partial sum), then the four row
// sums as (r0 + r1) + (r2 + r3).  Every lane gets the same value.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}

__device__ __forceinline__ float wave_sum_tree(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Maximum over the 64 lanes (exact in any order), same pattern.
__device__ __forceinline__ float wave_max_tree(float v) {
    v = __builtin_fmaxf(v, dpp_f<0xB1>(v));
    v = __builtin_fmaxf(v, dpp_f<0x4E>(v));
    v = __builtin_fmaxf(v, dpp_f<0x141>(v));
    v = __builtin_fmaxf(v, dpp_f<0x140>(v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return __builtin_fmaxf(__builtin_fmaxf(r0, r1), __builtin_fmaxf(r2, r3));
}

// Sum over a block of kThreads threads: the wave tree, then the wave
// totals added in wave order (w0 + w1) + w2 ...  slot: kThreads/64 floats of
// LDS that no other reduction of the same kernel phase uses (so one barrier
// suffices).  Every thread returns the same value.
template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float* slot) {
    v = wave_sum_tree(v);
    if ((threadIdx.x & (kWave - 1)) == 0) slot[threadIdx.x / kWave] = v;
    __syncthreads();
    float s = slot[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) s += slot[w];
    return s;
}

template <int kThreads>
__device__ __forceinline__ float block_max(float v, float* slot) {
    v = wave_max_tree(v);
    if ((threadIdx.x & (kWave - 1)) == 0) slot[threadIdx.x / kWave] = v;
    __syncthreads();
    float s = slot[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) s = __builtin_fmaxf(s, slot[w]);
    return s;
}

// exp(x) for x <= 0 (softmax weights): Cody-Waite reduction x = n ln2 + r,
// |r| <= ln2/2, degree-7 Taylor polynomial in Horner form with fused
// multiply-adds, scaled by 2^n.  Results below ~2^-124 are returned as 0.
// Error < 2 ulp against exp.
__device__ __forceinline__ float exp_neg(float x) {
    if (!(x >= -86.0f)) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860682030941723e-6f, r);
    float p = 1.98412698412698413e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, static_cast<int>(n));
}

// 1 / sqrt(ss / n + eps) with correctly rounded divide and square root
// (the reference uses rsqrtf, inference_kernels.cu:50).
__device__ __forceinline__ float inv_rms(float ss, int n, float eps) {
    return 1.0f / __builtin_sqrtf(ss / static_cast<float>(n) + eps);
}

// ---- GEMV prologues: engine activations -> int8 bit planes ---------------------
//
// Vectors are handled in 16-byte units of 8 elements; thread t of a block of T
// threads owns units t, t + T, t + 2T, ...  A pass issues the loads of up to
// kUnits units before using any of them.  Sums of squares accumulate per
// thread in unit order (element order inside a unit) with fma, then
// block_sum: this "unit order" is what the oracle restates.
// A vector of at most KU * T units, KU = 1 or 2 chosen at compile time (every
// vector of the 2B model), is one pass: issue() loads it whole ahead of the
// GEMV's weight loads, KU units per thread (no duplicate loads of a unit
// beyond the vector's end for the threads a second unit would not reach),
// and the one-pass code then issues no global load at all.  A load issued
// after the weights would make the prologue wait for them too: the memory
// wait counter retires loads in issue order.

constexpr int kUnits = 2;  // units per thread per pass

__device__ __forceinline__ void unpack_bf16x8(const uint4 r, float (&f)[8]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[2 * k] = BF16::to_float(static_cast<uint16_t>(w[k] & 0xFFFFu));
        f[2 * k + 1] = BF16::to_float(static_cast<uint16_t>(w[k] >> 16));
    }
}

__device__ __forceinline__ void load_f8(const float* p, float (&f)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w, f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
}

__device__ __forceinline__ void store_f8(float* p, const float (&f)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
}

// vec[i] = bf16((vec[i] * inv) * w[i]) over units (rms_norm_kernel's output
// expression, inference_kernels.cu:53-55); returns max |result| of the
// thread's elements.
template <int T>
__device__ __forceinline__ float scale_by_weight(float* vec, const float* w, float inv, int units,
                                                 int tid) {
    float m = 0.0f;
    for (int base = 0; base < units; base += kUnits * T) {
        float wf[kUnits][8];
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const int u = base + tid + k * T;
            if (u < units) load_f8(w + 8 * u, wf[k]);
        }
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const int u = base + tid + k * T;
            if (u < units) {
                float f[8];
                load_f8(vec + 8 * u, f);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    f[e] = bf16r((f[e] * inv) * wf[k][e]);
                    m = __builtin_fmaxf(m, __builtin_fabsf(f[e]));
                }
                store_f8(vec + 8 * u, f);
            }
        }
    }
    return m;
}

// Norm weights of the thread's units, loaded together with the activations
// when the vector fits one pass (units <= kUnits * T), else read at use.
template <int T>
struct HeldWeights {
    float f[kUnits][8];
    // unconditional loads, units past the vector clamped to its last (their
    // values are never used), so the wait counts of the prologue stay exact
    template <int KU = kUnits>
    __device__ void load(const float* w, int units, int tid) {
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int u = tid + k * T;
            load_f8(w + 8 * (u < units ? u : units - 1), f[k]);
        }
    }
    // the same on a vector held in registers (unit tid + k * T in v[k])
    template <int KU>
    __device__ float scale_regs(float (&v)[kUnits][8], float inv, int units, int tid) const {
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            if (tid + k * T < units) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[k][e] = bf16r((v[k][e] * inv) * f[k][e]);
                    m = __builtin_fmaxf(m, __builtin_fabsf(v[k][e]));
                }
            }
        }
        return m;
    }
    template <bool kOne>
    __device__ float apply(float* vec, const float* w, float inv, int units, int tid) const {
        if constexpr (!kOne) {
            if (units > kUnits * T) return scale_by_weight<T>(vec, w, inv, units, tid);
        }
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const int u = tid + k * T;
            if (u < units) {
                float v[8];
                load_f8(vec + 8 * u, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[e] = bf16r((v[e] * inv) * f[k][e]);
                    m = __builtin_fmaxf(m, __builtin_fabsf(v[e]));
                }
                store_f8(vec + 8 * u, v);
            }
        }
        return m;
    }
};

// The first pass of a bf16 vector's units, loaded into registers.
template <int T>
struct HeldUnits {
    uint4 r[kUnits];
    template <int KU = kUnits>
    __device__ void load(const uint16_t* src, int units, int tid) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src);
#pragma unroll
        for (int k = 0; k < KU; ++k) {  // unconditional, as HeldWeights::load
            const int u = tid + k * T;
            r[k] = s4[u < units ? u : units - 1];
        }
    }
};

// bf16 vector src -> vec (as float), returning this thread's sum of squares;
// copy (nullable) receives the raw bf16 units.  first: the first pass,
// already loaded.
template <int T, bool kOne>
__device__ __forceinline__ float load_bf16_sumsq(const uint16_t* src, float* vec, int units,
                                                 int tid, uint16_t* copy,
                                                 const HeldUnits<T>& first) {
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    float ss = 0.0f;
    for (int base = 0; base < (kOne ? 1 : units); base += kUnits * T) {
        uint4 r[kUnits];
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const int u = base + tid + k * T;
            if (base == 0)
                r[k] = first.r[k];
            else if (!kOne && u < units)
                r[k] = s4[u];
        }
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const int u = base + tid + k * T;
            if (u < units) {
                float f[8];
                unpack_bf16x8(r[k], f);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
                store_f8(vec + 8 * u, f);
                if (copy) reinterpret_cast<uint4*>(copy)[u] = r[k];
            }
        }
    }
    return ss;
}

// Quantising source over a float vector in LDS (values already bf16-rounded).
struct LdsQuantSrc {
    const float* v;
    float scale;
    __device__ uint32_t q8(float f) const {
        return static_cast<uint32_t>(quant_round_clamp(f * scale)) & 0xFFu;
    }
    __device__ void load8(int c0, uint32_t& lo, uint32_t& hi) const {
        const float4 a = *reinterpret_cast<const float4*>(v + c0);
        const float4 b = *reinterpret_cast<const float4*>(v + c0 + 4);
        lo = q8(a.x) | (q8(a.y) << 8) | (q8(a.z) << 16) | (q8(a.w) << 24);
        hi = q8(b.x) | (q8(b.y) << 8) | (q8(b.z) << 16) | (q8(b.w) << 24);
    }
};

constexpr int kRedSlot = 16;  // floats per reduction slot (>= kBlock / 64)

// P::issue(tid, st) issues the first pass of loads into registers (before the
// GEMV's weight loads); P::fill(vec, aux, n, tid, red, st) writes the GEMV input (bf16-rounded, as
// float) to vec[0..n) (aux: P::kAux further floats of LDS per element; red:
// reduction slots 0 and 1) and returns max |value| over the thread's
// elements; then absmax (reference absmax_reduce, inference_kernels.cu:120-148)
// and the quantised bit planes.  Every block of the launch computes the same
// values.  The GEMVs run even after the decode state is done (their reads
// stay in bounds and their outputs are scratch), so no kernel waits on the
// state before its first loads.
template <class P, int KU>
struct ProducerPlanes {
    P p;
    const EngineState* st;
    float amax;
    static size_t extra_lds(int cols) {
        return static_cast<size_t>(cols) * 4 * (1 + P::kAux) + 4 * 3 * kRedSlot;
    }
    using Regs = typename P::Regs;
    __device__ bool skip() const { return false; }
    __device__ void issue(int tid, Regs& r) const { p.template issue<KU ? KU : kUnits>(tid, st, r); }
    __device__ void offset(long) {}
    __device__ void prepare() {}
    __device__ void build(uint32_t* planes, int cols, int tid, float* scratch, Regs& r) {
        float* vec = scratch;
        float* aux = scratch + cols;
        float* red = scratch + cols * (1 + P::kAux);
        if constexpr (KU > 0) {
            // one pass: the vector stays in registers (unit tid + k * kBlock in
            // v[k], k < KU) and each thread stores its own units' planes
            float v[kUnits][8];
            const float m = p.template fill_one<KU>(v, tid, red, st, r);
            amax = block_max<kBlock>(m, red + 2 * kRedSlot);
            const float scale = quant_scale(amax);
            const int units = cols >> 3, nw = cols >> 5;
#pragma unroll
            for (int k = 0; k < KU; ++k) {
                const int u = tid + k * kBlock;
                if (u < units) store_unit_planes(planes, nw, u, v[k], scale);  // whole quads
            }
        } else {
            const float m = p.template fill<false>(vec, aux, cols, tid, red, st, r);
            amax = block_max<kBlock>(m, red + 2 * kRedSlot);  // its barrier also orders vec
            BuildPlanes<LdsQuantSrc>{LdsQuantSrc{vec, quant_scale(amax)}}.build(planes, cols, tid,
                                                                                nullptr);
        }
    }
    __device__ float absmax() const { return amax; }
};

// Layer input: x (or, in layer 0, the embedding row of tokens[pos], which
// block 0 also stores to x_out as the residual stream), then RMSNorm.
// Reference: inference.cu:134-138, 147-153; rms_norm_kernel
// (inference_kernels.cu:15-56): y = bf16((x * inv) * w).
struct InputNorm {
    static constexpr int kAux = 0;
    const uint16_t* x;
    const uint16_t* embed;  // non-null in layer 0
    const int* tokens;
    uint16_t* x_out;
    const float* w;
    float eps;
    int n;
    int writer = 0;  // the block that stores the residual stream (layer 0)
    long tok_stride = 0;  // batched decode: token buffer of sequence t at tokens + t * tok_stride
    // prefill / batched decode: token t of a batch (x and x_out rows of
    // `stride` elements)
    __device__ void at(int t, long stride) {
        x += t * stride;
        x_out += t * stride;
        tokens += t * tok_stride;
        writer = t;
    }
    struct Regs {
        const uint16_t* src;
        HeldUnits<kBlock> hx;
        HeldWeights<kBlock> hw;
    };
    template <int KU>
    __device__ void issue(int tid, const EngineState* st, Regs& r) const {
        r.src = embed ? embed + static_cast<long>(tokens[st->pos]) * n : x;
        r.hx.template load<KU>(r.src, n >> 3, tid);
        r.hw.template load<KU>(w, n >> 3, tid);
    }
    template <bool kOne>
    __device__ float fill_pass(float* vec, int tid, float* red, Regs& r) const {
        const float ss = load_bf16_sumsq<kBlock, kOne>(
            r.src, vec, n >> 3, tid,
            embed && blockIdx.x == static_cast<unsigned>(writer) ? x_out : nullptr, r.hx);
        const float inv = inv_rms(block_sum<kBlock>(ss, red), n, eps);
        return r.hw.template apply<kOne>(vec, w, inv, n >> 3, tid);
    }
    // one pass, in registers (the order of fill_pass); KU units per thread
    template <int KU>
    __device__ float fill_one(float (&v)[kUnits][8], int tid, float* red, const EngineState*,
                              Regs& r) const {
        const int units = n >> 3;
        uint16_t* copy = embed && blockIdx.x == static_cast<unsigned>(writer) ? x_out : nullptr;
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int u = tid + k * kBlock;
            if (u < units) {
                unpack_bf16x8(r.hx.r[k], v[k]);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[k][e], v[k][e], ss);
                if (copy) reinterpret_cast<uint4*>(copy)[u] = r.hx.r[k];
            }
        }
        const float inv = inv_rms(block_sum<kBlock>(ss, red), n, eps);
        return r.hw.template scale_regs<KU>(v, inv, units, tid);
    }
    // units per thread of the one-pass form (1 or 2), 0 for the general form
    int units_per_thread() const {
        const int u = n >> 3;
        return u <= kBlock ? 1 : (u <= kUnits * kBlock ? 2 : 0);
    }
    template <bool kOne>
    __device__ float fill(float* vec, float*, int, int tid, float* red, const EngineState*,
                          Regs& r) const {
        return fill_pass<kOne>(vec, tid, red, r);
    }
};

// Attention output: combine the splits of every head,
//   M = max_s m_s, w_s = exp(m_s - M), out = (sum_s w_s acc_s) / (sum_s w_s l_s)
// (s ascending, fused multiply-adds), rounded to bf16.  A unit (8 dims)
// never straddles heads (head_dim % 8 == 0).  Loads are issued in batches of
// kBatch splits.
struct AttnCombine {
    static constexpr int kAux = 0;
    static constexpr int kBatch = 4;
    const float* pm;    // [nh][S]
    const float* pl;    // [nh][S]
    const float* pacc;  // [nh][S][hd]
    int hd, S;
    int n;        // nh * hd
    int hd_log2;  // head_dim is 64 or 128
    // prefill: token t of a batch (the partials of token t follow those of
    // t - 1: [t][nh][S] and [t][nh][S][hd])
    __device__ void at(int t, long) {
        const long hs = static_cast<long>(n >> hd_log2) * S;
        pm += t * hs;
        pl += t * hs;
        pacc += t * hs * hd;
    }
    int units_per_thread() const { return (n >> 3) <= kBlock ? 1 : 0; }  // a thread per unit
    struct Batch {
        float pv[kBatch][8], lv[kBatch], mv[kBatch];
    };
    static constexpr int kLongBatch = 8;  // splits per load group past the first batch
    static constexpr int kMaxGroup = 32;  // split maxima per load group
    struct LongBatch {
        float pv[kLongBatch][8], lv[kLongBatch], mv[kLongBatch];
    };
    // batch 0 of the thread's first unit is loaded before pos is known (ahead
    // of the GEMV's weights)
    struct Regs {
        int pos;
        Batch b0;
    };
    // splits s0 .. s0 + N - 1 of unit (h, d0) (N = kBatch or kLongBatch);
    // unconditional, splits clamped to S - 1 (those past pos's are dropped)
    template <class B>
    __device__ void load_batch(int h, int d0, int s0, B& b) const {
        constexpr int kN = sizeof(b.lv) / sizeof(float);
#pragma unroll
        for (int k = 0; k < kN; ++k) {
            const int s = s0 + k < S ? s0 + k : S - 1;
            load_f8(pacc + (static_cast<long>(h) * S + s) * hd + d0, b.pv[k]);
            b.lv[k] = pl[h * S + s];
            b.mv[k] = pm[h * S + s];
        }
    }
    template <int KU>
    __device__ void issue(int tid, const EngineState* st, Regs& r) const {
        r.pos = state_pos(st);
        const int u = tid < (n >> 3) ? tid : (n >> 3) - 1;
        const int h = (8 * u) >> hd_log2;
        load_batch(h, 8 * u - (h << hd_log2), 0, r.b0);
    }
    // unit u over splits 0 .. ns-1 (batch 0 from held when non-null) into a;
    // returns max |a|
    __device__ float combine(float (&a)[8], int u, int ns, const Batch* held) const {
        const int h = (8 * u) >> hd_log2, d0 = 8 * u - (h << hd_log2);
        Batch b0;
        if (held)
            b0 = *held;
        else
            load_batch(h, d0, 0, b0);
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) M = __builtin_fmaxf(M, k < ns ? b0.mv[k] : -INFINITY);
        float l = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = 0.0f;
        auto accumulate = [&](const auto& b, int s0) {
            constexpr int kN = sizeof(b.lv) / sizeof(float);
#pragma unroll
            for (int k = 0; k < kN; ++k) {
                if (s0 + k < ns) {
                    const float w = exp_neg(b.mv[k] - M);
                    l = __builtin_fmaf(w, b.lv[k], l);
#pragma unroll
                    for (int e = 0; e < 8; ++e) a[e] = __builtin_fmaf(w, b.pv[k][e], a[e]);
                }
            }
        };
        if (ns <= kBatch) {
            accumulate(b0, 0);
        } else {
            // Splits past the first batch (long contexts): every load of a
            // group is issued before any of it is used -- kMaxGroup maxima at
            // a time, then kLongBatch splits' partials at a time, the first
            // group of those together with the maxima -- so 33 splits cost 5
            // dependent round trips instead of 16.  Same order of arithmetic.
            LongBatch b;
            load_batch(h, d0, kBatch, b);
            for (int s0 = kBatch; s0 < ns; s0 += kMaxGroup) {
                float t[kMaxGroup];
#pragma unroll
                for (int k = 0; k < kMaxGroup; ++k) t[k] = pm[h * S + (s0 + k < ns ? s0 + k : ns - 1)];
#pragma unroll
                for (int k = 0; k < kMaxGroup; ++k) M = __builtin_fmaxf(M, t[k]);
            }
            accumulate(b0, 0);
            accumulate(b, kBatch);
            for (int s0 = kBatch + kLongBatch; s0 < ns; s0 += kLongBatch) {
                load_batch(h, d0, s0, b);
                accumulate(b, s0);
            }
        }
        float mx = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            a[e] = bf16r(a[e] / l);
            mx = __builtin_fmaxf(mx, __builtin_fabsf(a[e]));
        }
        return mx;
    }
    __device__ float combine_to(float* vec, int u, int ns, const Batch* held) const {
        float a[8];
        const float mx = combine(a, u, ns, held);
        store_f8(vec + 8 * u, a);
        return mx;
    }
    // one pass (a unit per thread), in registers
    template <int KU>
    __device__ float fill_one(float (&v)[kUnits][8], int tid, float*, const EngineState*,
                              Regs& r) const {
        int ns = (opaque(r.pos) >> 6) + 1;  // opaque: as in fill
        ns = ns < S ? ns : S;
        return tid < (n >> 3) ? combine(v[0], tid, ns, &r.b0) : 0.0f;
    }
    template <bool kOne>
    __device__ float fill(float* vec, float*, int, int tid, float*, const EngineState*,
                          Regs& r) const {
        // opaque: pos stays a vector register until here (a scalar copy of a
        // uniform load is otherwise placed right after the load, and waits
        // for it ahead of the GEMV's weight loads)
        int ns = (opaque(r.pos) >> 6) + 1;  // splits holding positions 0..pos
        ns = ns < S ? ns : S;
        if constexpr (kOne) return tid < (n >> 3) ? combine_to(vec, tid, ns, &r.b0) : 0.0f;
        // more units than threads (decode), or any count (prefill)
        float mx = tid < (n >> 3) ? combine_to(vec, tid, ns, &r.b0) : 0.0f;
        for (int u = tid + kBlock; u < (n >> 3); u += kBlock)
            mx = __builtin_fmaxf(mx, combine_to(vec, u, ns, nullptr));
        return mx;
    }
};

// The o projection's input when attn_combine_kernel has already folded the
// splits (long contexts): the nh * hd floats it wrote, which are exactly the
// values AttnCombine computes (same operations in the same order), so the
// quantised input and the outputs are unchanged.
struct CombinedAttn {
    static constexpr int kAux = 0;
    const float* v;  // [nh * hd], bf16-rounded
    int n;
    // batched decode: sequence t's vector at v + t * stride
    __device__ void at(int t, long stride) { v += t * stride; }
    struct Regs {
        float4 a[kUnits], b[kUnits];
    };
    template <int KU>
    __device__ void issue(int tid, const EngineState*, Regs& r) const {
        const int units = n >> 3;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int u = tid + k * kBlock < units ? tid + k * kBlock : units - 1;
            r.a[k] = reinterpret_cast<const float4*>(v)[2 * u];
            r.b[k] = reinterpret_cast<const float4*>(v)[2 * u + 1];
        }
    }
    int units_per_thread() const {
        const int u = n >> 3;
        return u <= kBlock ? 1 : (u <= kUnits * kBlock ? 2 : 0);
    }
    template <int KU>
    __device__ float fill_one(float (&vv)[kUnits][8], int tid, float*, const EngineState*,
                              Regs& r) const {
        const int units = n >> 3;
        float mx = 0.0f;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            if (tid + k * kBlock < units) {
                const float f[8] = {r.a[k].x, r.a[k].y, r.a[k].z, r.a[k].w,
                                    r.b[k].x, r.b[k].y, r.b[k].z, r.b[k].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    vv[k][e] = f[e];
                    mx = __builtin_fmaxf(mx, __builtin_fabsf(f[e]));
                }
            }
        }
        return mx;
    }
    template <bool kOne>
    __device__ float fill(float* vec, float*, int, int tid, float*, const EngineState*,
                          Regs& r) const {
        const int units = n >> 3;
        float mx = 0.0f;
        for (int u = tid, k = 0; u < units; u += kBlock, ++k) {
            float f[8];
            if (k < kUnits) {
                const float4 a = r.a[k < kUnits ? k : 0], b = r.b[k < kUnits ? k : 0];
                f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w;
                f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
            } else {
                load_f8(v + 8 * u, f);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = __builtin_fmaxf(mx, __builtin_fabsf(f[e]));
            store_f8(vec + 8 * u, f);
        }
        return mx;
    }
};

// gate/up input: o = RMSNorm(o; attn_sub_norm) (skipped when absent),
// x = bf16(o + r) (block 0 stores it as the new residual), then
// RMSNorm(x; post_attention_layernorm).  Reference inference.cu:205-230.
struct SubNormResidualNorm {
    static constexpr int kAux = 1;
    const uint16_t* o;
    const uint16_t* res;
    uint16_t* x_out;
    const float* w_sub;
    const float* w_post;
    float eps;
    int n;
    int writer = 0;  // the block that stores the new residual stream
    // prefill: token t of a batch (rows of `stride` elements)
    __device__ void at(int t, long stride) {
        o += t * stride;
        res += t * stride;
        x_out += t * stride;
        writer = t;
    }
    struct Regs {
        HeldUnits<kBlock> ho, hr;
        HeldWeights<kBlock> hs, hp;
    };
    template <int KU>
    __device__ void issue(int tid, const EngineState*, Regs& r) const {
        const int units = n >> 3;
        r.ho.template load<KU>(o, units, tid);
        r.hr.template load<KU>(res, units, tid);
        r.hs.template load<KU>(w_sub ? w_sub : w_post, units, tid);  // unconditional (dropped when absent)
        r.hp.template load<KU>(w_post, units, tid);
    }
    // one pass, in registers (the order of fill_pass); KU units per thread
    template <int KU>
    __device__ float fill_one(float (&v)[kUnits][8], int tid, float* red, const EngineState*,
                              Regs& r) const {
        const int units = n >> 3;
        float g[kUnits][8];
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            if (tid + k * kBlock < units) {
                unpack_bf16x8(r.ho.r[k], v[k]);
                unpack_bf16x8(r.hr.r[k], g[k]);
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[k][e], v[k][e], ss);
            }
        }
        const float inv = w_sub ? inv_rms(block_sum<kBlock>(ss, red), n, eps) : 1.0f;
        float ss2 = 0.0f;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            const int u = tid + k * kBlock;
            if (u < units) {
                uint32_t packed[4];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float f = v[k][e];
                    if (w_sub) f = bf16r((f * inv) * r.hs.f[k][e]);
                    f = bf16r(f + g[k][e]);
                    ss2 = __builtin_fmaf(f, f, ss2);
                    v[k][e] = f;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    packed[q] = static_cast<uint32_t>(BF16::from_float(v[k][2 * q])) |
                                (static_cast<uint32_t>(BF16::from_float(v[k][2 * q + 1])) << 16);
                if (blockIdx.x == static_cast<unsigned>(writer))
                    reinterpret_cast<uint4*>(x_out)[u] =
                        make_uint4(packed[0], packed[1], packed[2], packed[3]);
            }
        }
        const float inv2 = inv_rms(block_sum<kBlock>(ss2, red + kRedSlot), n, eps);
        return r.hp.template scale_regs<KU>(v, inv2, units, tid);
    }
    // units per thread of the one-pass form (1 or 2), 0 for the general form
    int units_per_thread() const {
        const int u = n >> 3;
        return u <= kBlock ? 1 : (u <= kUnits * kBlock ? 2 : 0);
    }
    template <bool kOne>
    __device__ float fill(float* vec, float* aux, int, int tid, float* red, const EngineState*,
                          Regs& r) const {
        return fill_pass<kOne>(vec, aux, tid, red, r);
    }
    template <bool kOne>
    __device__ float fill_pass(float* vec, float* aux, int tid, float* red, Regs& r) const {
        const int units = n >> 3;
        // o -> vec (sum of squares), residual -> aux
        float ss = 0.0f;
        for (int base = 0; base < (kOne ? 1 : units); base += kUnits * kBlock) {
            uint4 ro[kUnits], rr[kUnits];
#pragma unroll
            for (int k = 0; k < kUnits; ++k) {
                const int u = base + tid + k * kBlock;
                if (base == 0) {
                    ro[k] = r.ho.r[k];
                    rr[k] = r.hr.r[k];
                } else if (!kOne && u < units) {
                    ro[k] = reinterpret_cast<const uint4*>(o)[u];
                    rr[k] = reinterpret_cast<const uint4*>(res)[u];
                }
            }
#pragma unroll
            for (int k = 0; k < kUnits; ++k) {
                const int u = base + tid + k * kBlock;
                if (u < units) {
                    float f[8], g[8];
                    unpack_bf16x8(ro[k], f);
                    unpack_bf16x8(rr[k], g);
#pragma unroll
                    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
                    store_f8(vec + 8 * u, f);
                    store_f8(aux + 8 * u, g);
                }
            }
        }
        const float inv = w_sub ? inv_rms(block_sum<kBlock>(ss, red), n, eps) : 1.0f;
        // o = bf16((o * inv) * w_sub) (when present); x = bf16(o + r)
        float ss2 = 0.0f;
        for (int base = 0; base < (kOne ? 1 : units); base += kUnits * kBlock) {
#pragma unroll
            for (int k = 0; k < kUnits; ++k) {
                const int u = base + tid + k * kBlock;
                if (u >= units) continue;
                float f[8], g[8], ws[8];
                load_f8(vec + 8 * u, f);
                load_f8(aux + 8 * u, g);
                if (w_sub) {
                    if (kOne) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) ws[e] = r.hs.f[k][e];
                    } else {
                        load_f8(w_sub + 8 * u, ws);
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) f[e] = bf16r((f[e] * inv) * ws[e]);
                }
                uint32_t packed[4];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    f[e] = bf16r(f[e] + g[e]);
                    ss2 = __builtin_fmaf(f[e], f[e], ss2);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    packed[q] = static_cast<uint32_t>(BF16::from_float(f[2 * q])) |
                                (static_cast<uint32_t>(BF16::from_float(f[2 * q + 1])) << 16);
                store_f8(vec + 8 * u, f);
                if (blockIdx.x == static_cast<unsigned>(writer))
                    reinterpret_cast<uint4*>(x_out)[u] =
                        make_uint4(packed[0], packed[1], packed[2], packed[3]);
            }
        }
        const float inv2 = inv_rms(block_sum<kBlock>(ss2, red + kRedSlot), n, eps);
        return r.hp.template apply<kOne>(vec, w_post, inv2, units, tid);
    }
};

// down input: m = (relu(g) * relu(g)) * u in fp32 (relu2_mul_f32_kernel,
// inference_kernels.cu:399-410), then RMSNorm_f32in(m; ffn_sub_norm)
// (:418-455) or a plain bf16 rounding when the norm is absent (:460-466).
struct Relu2Norm {
    static constexpr int kAux = 0;
    const uint16_t* g;
    const uint16_t* u;
    const float* w;
    const float* w_load;  // w, or any buffer of at least n floats when w is absent
    float eps;
    int n;
    // prefill: token t of a batch (g and u rows of `stride` elements)
    __device__ void at(int t, long stride) {
        g += t * stride;
        u += t * stride;
    }
    struct Regs {
        HeldUnits<kBlock> hg, hu;
        HeldWeights<kBlock> hw;
    };
    template <int KU>
    __device__ void issue(int tid, const EngineState*, Regs& r) const {
        const int units = n >> 3;
        r.hg.template load<KU>(g, units, tid);
        r.hu.template load<KU>(u, units, tid);
        r.hw.template load<KU>(w_load, units, tid);  // unconditional (dropped when w is absent)
    }
    // one pass, in registers (the order of fill_pass); KU units per thread
    template <int KU>
    __device__ float fill_one(float (&v)[kUnits][8], int tid, float* red, const EngineState*,
                              Regs& r) const {
        const int units = n >> 3;
        float ss = 0.0f, mx = 0.0f;
#pragma unroll
        for (int k = 0; k < KU; ++k) {
            if (tid + k * kBlock < units) {
                float fg[8], fu[8];
                unpack_bf16x8(r.hg.r[k], fg);
                unpack_bf16x8(r.hu.r[k], fu);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float rl = __builtin_fmaxf(0.0f, fg[e]);
                    float m = (rl * rl) * fu[e];
                    ss = __builtin_fmaf(m, m, ss);
                    if (!w) {  // no sub-norm: plain rounding
                        m = bf16r(m);
                        mx = __builtin_fmaxf(mx, __builtin_fabsf(m));
                    }
                    v[k][e] = m;
                }
            }
        }
        if (!w) return mx;
        const float inv = inv_rms(block_sum<kBlock>(ss, red), n, eps);
        return r.hw.template scale_regs<KU>(v, inv, units, tid);
    }
    // units per thread of the one-pass form (1 or 2), 0 for the general form
    int units_per_thread() const {
        const int u = n >> 3;
        return u <= kBlock ? 1 : (u <= kUnits * kBlock ? 2 : 0);
    }
    template <bool kOne>
    __device__ float fill(float* vec, float*, int, int tid, float* red, const EngineState*,
                          Regs& r) const {
        return fill_pass<kOne>(vec, tid, red, r);
    }
    template <bool kOne>
    __device__ float fill_pass(float* vec, int tid, float* red, Regs& r) const {
        const int units = n >> 3;
        float ss = 0.0f, mx = 0.0f;
        for (int base = 0; base < (kOne ? 1 : units); base += kUnits * kBlock) {
            uint4 rg[kUnits], ru[kUnits];
#pragma unroll
            for (int k = 0; k < kUnits; ++k) {
                const int q = base + tid + k * kBlock;
                if (base == 0) {
                    rg[k] = r.hg.r[k];
                    ru[k] = r.hu.r[k];
                } else if (!kOne && q < units) {
                    rg[k] = reinterpret_cast<const uint4*>(g)[q];
                    ru[k] = reinterpret_cast<const uint4*>(u)[q];
                }
            }
#pragma unroll
            for (int k = 0; k < kUnits; ++k) {
                const int q = base + tid + k * kBlock;
                if (q < units) {
                    float fg[8], fu[8];
                    unpack_bf16x8(rg[k], fg);
                    unpack_bf16x8(ru[k], fu);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float r = __builtin_fmaxf(0.0f, fg[e]);
                        fg[e] = (r * r) * fu[e];
                        ss = __builtin_fmaf(fg[e], fg[e], ss);
                        if (!w) {  // no sub-norm: plain rounding
                            fg[e] = bf16r(fg[e]);
                            mx = __builtin_fmaxf(mx, __builtin_fabsf(fg[e]));
                        }
                    }
                    store_f8(vec + 8 * q, fg);
                }
            }
        }
        if (!w) return mx;
        const float inv = inv_rms(block_sum<kBlock>(ss, red), n, eps);
        return r.hw.template apply<kOne>(vec, w, inv, units, tid);
    }
};

// ---- GEMV epilogues ----------------------------------------------------------------

// bf16 outputs of up to three stacked projections, each dequantised with its
// own gamma: out[r] = bf16(float(acc) * ((gamma_s * absmax) / 127)).
struct SegBf16Sink {
    uint16_t* out;
    float g0, g1, g2;
    int end0, end1;
    float dq0, dq1, dq2;
    __device__ void at(int t, long stride) { out += t * stride; }
    __device__ void offset(long) {}
    __device__ void prepare() {}
    __device__ void prefetch(long, int, int) {}
    template <class A>
    __device__ void bind(const A& a) {
        const float m = a.absmax();
        dq0 = dequant_scale(g0, m);
        dq1 = dequant_scale(g1, m);
        dq2 = dequant_scale(g2, m);
    }
    __device__ void store(long r, int acc) const {
        const float dq = r < end0 ? opaque(dq0) : (r < end1 ? opaque(dq1) : opaque(dq2));
        out[r] = BF16::from_float(static_cast<float>(acc) * dq);
    }
    // rows r .. r + 3 (r % 4 == 0, out 8-byte aligned there) in one store
    __device__ void store4(long r, const int (&acc)[4]) const {
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const long rk = r + k;
            const float dq = rk < end0 ? opaque(dq0) : (rk < end1 ? opaque(dq1) : opaque(dq2));
            h[k] = BF16::from_float(static_cast<float>(acc[k]) * dq);
        }
        *reinterpret_cast<uint2*>(out + r) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
};

// down projection: x_out[r] = bf16(bf16(acc * dq) + res[r])
// (inference.cu:256-262; residual_add_kernel, inference_kernels.cu:471-479).
// The residual row a thread stores in the block's first tile is loaded at
// kernel start (prefetch), off the epilogue's critical path.
struct ResidualSink {
    uint16_t* x_out;
    const uint16_t* res;
    float gamma;
    float dq;
    long pre_row;
    uint16_t pre_res;
    __device__ void at(int t, long stride) {
        x_out += t * stride;
        res += t * stride;
    }
    __device__ void offset(long) {}
    __device__ void prepare() {}
    __device__ void prefetch(long row0, int n, int tid) {
        pre_row = tid < n ? row0 + tid : -1;
        pre_res = res[row0 + (tid < n ? tid : 0)];  // unconditional
    }
    template <class A>
    __device__ void bind(const A& a) {
        dq = dequant_scale(gamma, a.absmax());
    }
    __device__ void store(long r, int acc) const {
        const float d = bf16r(static_cast<float>(acc) * dq);
        const uint16_t rv = r == pre_row ? static_cast<uint16_t>(opaque(static_cast<uint32_t>(pre_res)))
                                         : res[r];
        x_out[r] = BF16::from_float(d + BF16::to_float(rv));
    }
    // rows r .. r + 3 (r % 4 == 0, 8-byte aligned there): one load, one store
    __device__ void store4(long r, const int (&acc)[4]) const {
        store4_with(r, acc, *reinterpret_cast<const uint2*>(res + r));
    }
    // the same with the four residual values already loaded (rv = res[r .. r+3])
    __device__ void store4_with(long r, const int (&acc)[4], uint2 rv) const {
        const uint32_t rw[2] = {rv.x, rv.y};
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float d = bf16r(static_cast<float>(acc[k]) * dq);
            const uint16_t e = static_cast<uint16_t>(k & 1 ? rw[k >> 1] >> 16 : rw[k >> 1] & 0xFFFFu);
            h[k] = BF16::from_float(d + BF16::to_float(e));
        }
        *reinterpret_cast<uint2*>(x_out + r) =
            make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    }
};

// q/k/v outputs of the stacked projection (q rows [0, end0), k rows
// [end0, end1), v rows [end1, ...)): each row dequantised with its own
// projection's gamma and rounded to bf16, out = bf16(acc * ((gamma*absmax)/127));
// then every (2i, 2i+1) pair of a q or k head rotated by RoPE at the decode
// position (rope_kernel, inference_kernels.cu:185-206),
//   (x0, x1) -> (bf16(x0*cos - x1*sin), bf16(x0*sin + x1*cos)),
// and k and v written to this layer's KV cache at pos (scatter_kv,
// inference_kernels.cu:215-227; the cache is [kv head][max_seq][head_dim])
// unless the decode state is done.  The RoPE row of the decode position is
// cur_rope (written by the previous step's LM head, or by the host when the
// state is set), so no load waits for pos until the cache writes.
struct QkvRopeSink {
    uint16_t* out;
    uint16_t* kc;
    uint16_t* vc;
    const float2* cur_rope;  // [hd/2] (cos, sin) at the decode position
    const EngineState* st;
    float g0, g1, g2;
    int end0, end1;
    int hd, max_seq;
    int hd_log2;  // hd is 64 or 128
    float dq0, dq1, dq2;
    int pos, live;
    long pre_row;
    float2 pre_cs;
    const float2* rope_tab;  // prefill: the [max_seq][hd/2] table and the batch's first position
    int rope_pos0;
    long kv_stride;  // batched decode: cache elements per sequence (0 in the prefill)
    // token t of a batch (its own state record; out rows of `stride`
    // elements).  Prefill (rope_tab set): one sequence, token t at position
    // rope_pos0 + t.  Batched decode (rope_tab null): sequence t, with its
    // own RoPE row (cur_rope + t * hd/2) and its own KV cache (kv_stride).
    __device__ void at(int t, long stride) {
        out += t * stride;
        st += t;
        kc += t * kv_stride;
        vc += t * kv_stride;
        cur_rope = rope_tab ? rope_tab + static_cast<long>(rope_pos0 + t) * (hd >> 1)
                            : cur_rope + static_cast<long>(t) * (hd >> 1);
    }
    __device__ void offset(long) {}
    __device__ void prepare() {}
    __device__ int rope_pair(long r) const {  // pair index of q/k row r within its head
        const int rr = static_cast<int>(r < end0 ? r : r - end0);
        return (rr & (hd - 1)) >> 1;
    }
    // element offset of row r of a k or v segment (r relative to the segment)
    // in the cache [kv head][max_seq][hd] at pos
    __device__ long cache_at(int r) const {
        return ((static_cast<long>(r >> hd_log2) * max_seq + pos) << hd_log2) + (r & (hd - 1));
    }
    __device__ void prefetch(long row0, int n, int tid) {
        pos = state_pos(st);  // pos and done are needed only by the cache writes
        live = !state_done(st);
        pre_row = 2 * tid < n ? row0 + 2 * tid : -1;
        // unconditional (row 0's pair when the thread has no q/k row)
        pre_cs = cur_rope[rope_pair(pre_row >= 0 && pre_row < end1 ? pre_row : 0)];
    }
    template <class A>
    __device__ void bind(const A& a) {
        const float m = a.absmax();
        dq0 = dequant_scale(g0, m);
        dq1 = dequant_scale(g1, m);
        dq2 = dequant_scale(g2, m);
    }
    __device__ void store_pair(long r, int a0, int a1) const {
        const bool is_q = r < end0, is_v = r >= end1;
        const float dq = is_q ? opaque(dq0) : (is_v ? opaque(dq2) : opaque(dq1));
        const float x0 = bf16r(static_cast<float>(a0) * dq);
        const float x1 = bf16r(static_cast<float>(a1) * dq);
        // a pair is one 32-bit store (r is even; the buffers are 4-byte aligned)
        if (is_v) {
            const uint32_t y = static_cast<uint32_t>(BF16::from_float(x0)) |
                               (static_cast<uint32_t>(BF16::from_float(x1)) << 16);
            *reinterpret_cast<uint32_t*>(out + r) = y;
            if (live)
                *reinterpret_cast<uint32_t*>(vc + cache_at(static_cast<int>(r - end1))) = y;
            return;
        }
        // opaque: a select between a member and a load would otherwise become a
        // load from a selected address, which moves the sink to scratch memory
        float2 cs;
        if (r == pre_row)
            cs = make_float2(opaque(pre_cs.x), opaque(pre_cs.y));
        else
            cs = cur_rope[rope_pair(r)];
        const uint32_t y = static_cast<uint32_t>(BF16::from_float(x0 * cs.x - x1 * cs.y)) |
                           (static_cast<uint32_t>(BF16::from_float(x0 * cs.y + x1 * cs.x)) << 16);
        *reinterpret_cast<uint32_t*>(out + r) = y;
        if (!is_q && live)
            *reinterpret_cast<uint32_t*>(kc + cache_at(static_cast<int>(r - end0))) = y;
    }
};

template <>
struct SinkPairs<QkvRopeSink> {
    static constexpr bool value = true;
};

// Sinks with a four-row store (store4): the GEMM epilogue's lane holds four
// consecutive rows of one token.
template <class Sink>
struct SinkQuads {
    static constexpr bool value = false;
};
template <>
struct SinkQuads<SegBf16Sink> {
    static constexpr bool value = true;
};
template <>
struct SinkQuads<ResidualSink> {
    static constexpr bool value = true;
};

// ---- attention -----------------------------------------------------------------------

// One block per (64-position split s, kv head): scores of the group's q
// heads against the split's cached keys, the split's softmax numerator and
// unnormalised weighted sum of V.  q arrives rotated and the cache already
// holds k and v at pos (both written by the qkv projection's epilogue), so
// every load is issued at kernel start; rows past pos are loaded too (the
// cache is allocated to max_seq) and masked.
//   * scores: thread t takes quarter qq = t % 4 of K row t / 4 (one global
//     read of each K element per block, unpacked once) and the quarter of
//     every q head of the group from LDS; the 4 quarter sums of a (head,
//     position) meet in the 4 lanes of a quad (two DPP adds).
//   * V rows of the split stay bf16 in LDS; a PV thread owns dims (d, d+1)
//     of one head, reads both with one 32-bit load, and reads 4 positions'
//     weights with one 16-byte load.
//   score_j = ((a0 + a1) + (a2 + a3)) * scale, a_k = fma over the d of
//     quarter k (ascending) of q[d] * k_j[d]
//   per head: m = max_j score_j, e_j = exp(score_j - m),
//   l = tree sum of e over the 64 lanes (lane = position in the split),
//   acc[d] = sum_j e_j v_j[d] (j ascending, fma).
// Reference: attention_scores, softmax, attention_output
// (inference_kernels.cu:241-371), GQA kv = h * nkv / nh.

// The split's softmax over its jn live positions, per head (wave g % 4 takes
// head g, lane = position): m = the wave maximum, e = exp(score - m) stored
// to sc, l = the wave tree sum of e.  score(g, lane) reads the head's score
// of the lane's position; after a barrier that orders the scores.
template <int G, class Score>
__device__ __forceinline__ void split_softmax(float (&sc)[G][kAttnSplit], float (&hmax)[G],
                                              float (&hsum)[G], int jn, Score score) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    for (int g = wave; g < G; g += kAttnThreads / kWave) {
        const float v = lane < jn ? score(g, lane) : -INFINITY;
        const float m = wave_max_tree(v);
        const float e = lane < jn ? exp_neg(v - m) : 0.0f;
        const float l = wave_sum_tree(e);
        sc[g][lane] = e;
        if (lane == 0) {
            hmax[g] = m;
            hsum[g] = l;
        }
    }
}

// The split's weighted V sums and partials: thread o owns elements (2dp,
// 2dp+1) of head o / (HD/2) (one 32-bit V read per position, one 16-byte
// weight read per 4 positions), j ascending with fma.  After a barrier that
// orders the softmax.
template <int HD, int G>
__device__ __forceinline__ void split_weighted_v(const uint32_t (&vs)[kAttnSplit][HD / 2 + 1],
                                                 const float (&sc)[G][kAttnSplit],
                                                 const float (&hmax)[G], const float (&hsum)[G],
                                                 int jn, int s, int kvh, int S,
                                                 float* __restrict__ pm, float* __restrict__ pl,
                                                 float* __restrict__ pacc) {
    for (int o = threadIdx.x; o < G * (HD / 2); o += kAttnThreads) {
        const int g = o / (HD / 2), dp = o - g * (HD / 2);
        float a0 = 0.0f, a1 = 0.0f;
        auto step = [&](int jj, float e) {
            const uint32_t w = vs[jj][dp];
            a0 = __builtin_fmaf(e, BF16::to_float(static_cast<uint16_t>(w & 0xFFFFu)), a0);
            a1 = __builtin_fmaf(e, BF16::to_float(static_cast<uint16_t>(w >> 16)), a1);
        };
        const int n4 = jn >> 2;
        for (int q = 0; q < n4; ++q) {
            const float4 e = *reinterpret_cast<const float4*>(&sc[g][4 * q]);
            step(4 * q, e.x);
            step(4 * q + 1, e.y);
            step(4 * q + 2, e.z);
            step(4 * q + 3, e.w);
        }
        for (int jj = 4 * n4; jj < jn; ++jj) step(jj, sc[g][jj]);
        const int h = kvh * G + g;
        float* out = pacc + (static_cast<long>(h) * S + s) * HD + 2 * dp;
        *reinterpret_cast<float2*>(out) = make_float2(a0, a1);
        if (dp == 0) {
            pm[h * S + s] = hmax[g];
            pl[h * S + s] = hsum[g];
        }
    }
}

// The per-split work of one query (the bs=1 and batched decode kernels share
// it; the prefill kernel runs the same operations on register-held K and V):
// once its q (qs, float) and the split's V rows (vs, bf16) are in
// LDS behind a barrier and the thread holds its quarter of K row p = tid / 4
// (kq; quarter tid % 4), the scores, the split's softmax and the weighted V
// sum, stored as the split's partials of heads kvh * G .. kvh * G + G - 1.
// Scores: the thread unpacks its K quarter once and runs the quarter's fma
// chain for every head of the group; the four quarters of a position are the
// four lanes of a quad and combine through DPP.  V sums: a thread owns a
// pair of elements of one head (one 32-bit V read per position, one 16-byte
// weight read per 4 positions: the V phase's LDS reads are what its time is
// made of).  jn: positions of the split holding positions 0..pos.  A caller
// that writes qs again barriers first.
template <int HD, int G>
__device__ __forceinline__ void attention_split(const uint4 (&kq)[HD / 32], float (&qs)[G][HD],
                                                uint32_t (&vs)[kAttnSplit][HD / 2 + 1],
                                                float (&sc)[G][kAttnSplit], float (&hmax)[G],
                                                float (&hsum)[G], int jn, float scale, int s,
                                                int kvh, int S, float* __restrict__ pm,
                                                float* __restrict__ pl, float* __restrict__ pacc) {
    constexpr int kQU = HD / 32;  // 16-byte units per quarter row
    constexpr int kQD = HD / 4;   // elements per quarter row
    static_assert(kAttnThreads == 4 * kAttnSplit, "4 quarters x 64 positions");
    const int tid = threadIdx.x;
    const int qq = tid & 3, p = tid >> 2;
    // scores (every lane active: the quads combine through DPP)
    {
        float kf[kQD];
#pragma unroll
        for (int u = 0; u < kQU; ++u) {
            float f[8];
            unpack_bf16x8(kq[u], f);
#pragma unroll
            for (int e = 0; e < 8; ++e) kf[8 * u + e] = f[e];
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < kQD / 4; ++u) {
                const float4 q4 = *reinterpret_cast<const float4*>(&qs[g][qq * kQD + 4 * u]);
                a = __builtin_fmaf(q4.x, kf[4 * u], a);
                a = __builtin_fmaf(q4.y, kf[4 * u + 1], a);
                a = __builtin_fmaf(q4.z, kf[4 * u + 2], a);
                a = __builtin_fmaf(q4.w, kf[4 * u + 3], a);
            }
            a += dpp_f<0xB1>(a);  // quad_perm [1,0,3,2]: a0 + a1, a2 + a3
            a += dpp_f<0x4E>(a);  // quad_perm [2,3,0,1]: (a0 + a1) + (a2 + a3)
            if (qq == 0 && p < jn) sc[g][p] = a * scale;
        }
    }
    __syncthreads();
    split_softmax<G>(sc, hmax, hsum, jn, [&](int g, int p) { return sc[g][p]; });
    __syncthreads();
    split_weighted_v<HD, G>(vs, sc, hmax, hsum, jn, s, kvh, S, pm, pl, pacc);
}

// Split combine of one decode step, once per head (long contexts): block h,
// one wave, folds head h's splits 0 .. ns - 1 (those holding positions
// 0 .. pos) with AttnCombine::combine's operations in its order: M = max of
// the split maxima (a DPP wave tree, no LDS exchange), w_s = exp(m_s - M)
// (computed once per split here, by one lane, and shared through LDS), then
// l and each element's sum accumulated split by split; lane t writes
// bf16r(sum_d / l) for its HD / 64 adjacent elements d.  The element's partials of the
// first NB splits and the split maxima and sums are loaded together, right
// after the position (loads of splits past it, whose partials are old and
// cold, would hold up the live ones).  NB: the token-step graph's splits
// rounded up to a multiple of 4, at most kCombineBatch (a batch of loads per
// thread no larger than the splits the graph can reach).
constexpr int kCombineBatch = 64;
// Token-step graphs whose attention reaches at most this many splits keep the
// combine in the o projection's prologue; longer ones launch attn_combine_kernel.
constexpr int kFusedCombineSplits = 8;
template <int HD, int NB>
__global__ __launch_bounds__(kWave) void attn_combine_kernel(const float* __restrict__ pm,
                                                             const float* __restrict__ pl,
                                                             const float* __restrict__ pacc,
                                                             float* __restrict__ out,
                                                             const EngineState* __restrict__ st,
                                                             int S) {
    constexpr int E = HD / kWave;  // adjacent elements per lane (one wave per head)
    extern __shared__ float wl[];  // [2][S]: w_s, l_s
    const int h = blockIdx.x, t = threadIdx.x;
    {  // sequence blockIdx.y of a batch (its state, partials and output)
        const long b = blockIdx.y, hs = static_cast<long>(gridDim.x) * S;
        st += b;
        pm += b * hs;
        pl += b * hs;
        pacc += b * hs * HD;
        out += b * gridDim.x * HD;
    }
    const int pos = state_pos(st);
    int ns = (pos >> 6) + 1;
    ns = ns < S ? ns : S;
    const float* mh = pm + static_cast<long>(h) * S;
    const float* lh = pl + static_cast<long>(h) * S;
    const float* ph = pacc + static_cast<long>(h) * S * HD + E * t;
    auto load = [&](int s, float (&v)[E]) {
        if constexpr (E == 2) {
            const float2 x = *reinterpret_cast<const float2*>(ph + static_cast<long>(s) * HD);
            v[0] = x.x;
            v[1] = x.y;
        } else {
            v[0] = ph[static_cast<long>(s) * HD];
        }
    };
    float pv[NB][E];
#pragma unroll
    for (int k = 0; k < NB; ++k) load(k < ns ? k : ns - 1, pv[k]);
    const float m0 = t < ns ? mh[t] : -INFINITY;
    const float l0 = t < ns ? lh[t] : 0.0f;
    float M = m0;
    for (int s = t + kWave; s < ns; s += kWave) M = __builtin_fmaxf(M, mh[s]);
    M = wave_max_tree(M);  // DPP rows and readlanes (a maximum: exact in any order)
    if (t < ns) {
        wl[t] = exp_neg(m0 - M);
        wl[S + t] = l0;
    }
    for (int s = t + kWave; s < ns; s += kWave) {
        wl[s] = exp_neg(mh[s] - M);
        wl[S + s] = lh[s];
    }
    __syncthreads();  // one wave: orders its LDS writes and reads
    float l = 0.0f, a[E];
#pragma unroll
    for (int e = 0; e < E; ++e) a[e] = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += NB) {
        if (s0) {
#pragma unroll
            for (int k = 0; k < NB; ++k) load(s0 + k < ns ? s0 + k : ns - 1, pv[k]);
        }
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (s0 + k < ns) {
                const float w = wl[s0 + k];
                l = __builtin_fmaf(w, wl[S + s0 + k], l);
#pragma unroll
                for (int e = 0; e < E; ++e) a[e] = __builtin_fmaf(w, pv[k][e], a[e]);
            }
        }
    }
    if constexpr (E == 2)
        *reinterpret_cast<float2*>(out + h * HD + 2 * t) = make_float2(bf16r(a[0] / l), bf16r(a[1] / l));
    else
        out[h * HD + t] = bf16r(a[0] / l);
}

template <int HD, int G, int HB = G>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, float* __restrict__ pm, float* __restrict__ pl,
    float* __restrict__ pacc, const EngineState* __restrict__ st, int max_seq, int S,
    float scale) {
    constexpr int kU = HD / 8;       // 16-byte units per row
    constexpr int kQU = kU / 4;      // units per quarter row
    constexpr int kVRow = HD / 2 + 1;  // 32-bit words per bf16 V row in LDS (+1: no bank conflicts)
    // HB of the group's G q heads per block, heads z * HB .. z * HB + HB - 1
    // (z = blockIdx.z): the decode step's few blocks (one per split and kv
    // head) split over G / HB blocks each, every block loading the split's
    // K and V
    static_assert(G % HB == 0, "HB divides G");
    __shared__ __align__(16) float qs[HB][HD];
    __shared__ uint32_t vs[kAttnSplit][kVRow];
    __shared__ __align__(16) float sc[HB][kAttnSplit];
    __shared__ float hmax[HB], hsum[HB];
    const int s = blockIdx.x, kvh = blockIdx.y, z = blockIdx.z;
    const int j0 = s * kAttnSplit;
    const int tid = threadIdx.x;
    const long cache0 = static_cast<long>(kvh) * max_seq * HD;
    const int jmax = max_seq - 1;
    // the thread's quarter of K row j0 + tid / 4 (clamped to the cache)
    uint4 kq[kQU];
    {
        const int j = j0 + (tid >> 2) <= jmax ? j0 + (tid >> 2) : jmax;
        const uint4* kr = reinterpret_cast<const uint4*>(kc + cache0 + static_cast<long>(j) * HD) +
                          (tid & 3) * kQU;
#pragma unroll
        for (int u = 0; u < kQU; ++u) kq[u] = kr[u];
    }
    // V rows of the split: kVPer 16-byte units per thread, all loads issued
    // before the first LDS store
    constexpr int kVPer = kAttnSplit * kU / kAttnThreads;
    static_assert(kVPer * kAttnThreads == kAttnSplit * kU, "V units per thread");
    uint4 vraw[kVPer];
#pragma unroll
    for (int t = 0; t < kVPer; ++t) {
        const int idx = tid + t * kAttnThreads;
        const int jj = idx / kU, c = idx - jj * kU;
        const int j = j0 + jj <= jmax ? j0 + jj : jmax;
        vraw[t] = reinterpret_cast<const uint4*>(vc + cache0 + static_cast<long>(j) * HD)[c];
    }
    uint4 qraw = make_uint4(0, 0, 0, 0);
    const bool has_q = tid < HB * kU;
    if (has_q) qraw = reinterpret_cast<const uint4*>(qkv + (kvh * G + z * HB) * HD)[tid];
    const int done = state_done(st), pos = state_pos(st);
#pragma unroll
    for (int t = 0; t < kVPer; ++t) {
        const int idx = tid + t * kAttnThreads;
        const int jj = idx / kU, c = idx - jj * kU;
        uint32_t* row = &vs[jj][4 * c];
        row[0] = vraw[t].x;
        row[1] = vraw[t].y;
        row[2] = vraw[t].z;
        row[3] = vraw[t].w;
    }
    if (has_q) {
        float f[8];
        unpack_bf16x8(qraw, f);
        store_f8(&qs[tid / kU][8 * (tid % kU)], f);
    }
    if (done || j0 > pos) return;  // uniform
    const int jn = (pos + 1 - j0) < kAttnSplit ? (pos + 1 - j0) : kAttnSplit;
    __syncthreads();

    // heads kvh * G + z * HB + g = (kvh * G / HB + z) * HB + g
    attention_split<HD, HB>(kq, qs, vs, sc, hmax, hsum, jn, scale, s, kvh * (G / HB) + z, S, pm,
                            pl, pacc);
}

// Prefill form: the queries of the tokens of a batch (token t at position
// pos0 + t, its q at qkv + t * qkv_stride, its partials after those of
// t - 1).  A block (split s, kv head, kQ consecutive tokens) loads the
// split's K and V once and keeps both in registers for all of its tokens:
//   * wave w holds quarter w of the head dims of K row j0 + lane, unpacked
//     (kf), and reads each token's q quarters with scalar loads (the
//     address is the same for the whole wave), so a score costs no LDS
//     reads; the four quarter sums meet in LDS (red).
//   * a V thread holds the element pair dp = tid % (HD/2) of all 64 rows of
//     the split (vcol, bf16 pairs) and reads only the softmax weights from
//     LDS.
// The arithmetic is attention_split's, operation for operation, so a
// prefilled token's partials equal those of its decode step:
//   score = ((a0 + a1) + (a2 + a3)) * scale, a_w = fma chain over quarter w,
//   the softmax of split_softmax, and acc = fma over j ascending of e_j v_j.
template <int HD, int G, int kQ>
__global__ __launch_bounds__(kAttnThreads) void attention_prefill_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, float* __restrict__ pm, float* __restrict__ pl,
    float* __restrict__ pacc, int max_seq, int S, float scale, int pos0, int nt,
    int qkv_stride) {
    constexpr int kU = HD / 8;
    constexpr int kQU = kU / 4;       // 16-byte units per quarter row
    constexpr int kQD = HD / 4;       // elements per quarter row
    constexpr int kVP = HD / 2;       // element pairs per row
    constexpr int kVRow = kVP + 1;
    static_assert(kAttnThreads == 4 * kWave && kAttnSplit == kWave, "4 waves, lane = position");
    static_assert(kAttnThreads % kVP == 0, "a thread's V pair is the same for all its heads");
    __shared__ uint32_t vs[kAttnSplit][kVRow];
    __shared__ float red[4][G][kAttnSplit];
    __shared__ __align__(16) float sc[G][kAttnSplit];
    __shared__ float hmax[G], hsum[G];
    const int s = blockIdx.x, kvh = blockIdx.y;
    const int j0 = s * kAttnSplit;
    const int t0 = blockIdx.z * kQ;
    const int t1 = t0 + kQ < nt ? t0 + kQ : nt;
    if (j0 > pos0 + t1 - 1) return;  // no token of the block reaches the split
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wq = __builtin_amdgcn_readfirstlane(tid / kWave);
    const long cache0 = static_cast<long>(kvh) * max_seq * HD;
    const int jmax = max_seq - 1;
    // quarter wq of K row j0 + lane (clamped to the cache) and the split's V
    // rows (kVPer 16-byte units per thread), all loads issued together
    uint4 kq[kQU];
    {
        const int j = j0 + lane <= jmax ? j0 + lane : jmax;
        const uint4* kr = reinterpret_cast<const uint4*>(kc + cache0 + static_cast<long>(j) * HD) +
                          wq * kQU;
#pragma unroll
        for (int u = 0; u < kQU; ++u) kq[u] = kr[u];
    }
    constexpr int kVPer = kAttnSplit * kU / kAttnThreads;
    uint4 vraw[kVPer];
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
        const int idx = tid + i * kAttnThreads;
        const int jj = idx / kU, c = idx - jj * kU;
        const int j = j0 + jj <= jmax ? j0 + jj : jmax;
        vraw[i] = reinterpret_cast<const uint4*>(vc + cache0 + static_cast<long>(j) * HD)[c];
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
        const int idx = tid + i * kAttnThreads;
        const int jj = idx / kU, c = idx - jj * kU;
        uint32_t* row = &vs[jj][4 * c];
        row[0] = vraw[i].x;
        row[1] = vraw[i].y;
        row[2] = vraw[i].z;
        row[3] = vraw[i].w;
    }
    float kf[kQD];
#pragma unroll
    for (int u = 0; u < kQU; ++u) {
        float f[8];
        unpack_bf16x8(kq[u], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[8 * u + e] = f[e];
    }
    __syncthreads();
    const int dp = tid % kVP;
    uint32_t vcol[kAttnSplit];
#pragma unroll
    for (int jj = 0; jj < kAttnSplit; ++jj) vcol[jj] = vs[jj][dp];

    // q element pairs of quarter wq of token t's heads (the address is the
    // same for the whole wave: scalar loads); the next token's are loaded
    // during the current token's softmax and V sums when they fit in SGPRs
    constexpr int kQP = kQD / 2;
    constexpr bool kPrefetchQ = G * kQP <= 64;
    const uint32_t* q32 = reinterpret_cast<const uint32_t*>(qkv);
    auto load_q = [&](int tt, uint32_t (&q)[G * kQP]) {
        const uint32_t* qw =
            q32 + (static_cast<long>(tt) * qkv_stride + (kvh * G) * HD + wq * kQD) / 2;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < kQP; ++i) q[g * kQP + i] = qw[g * kVP + i];
    };
    const long hs = static_cast<long>(gridDim.y) * G * S;
    // the first token of the block that reaches the split
    int t = t0;
    if (j0 > pos0 + t) t = j0 - pos0;
    uint32_t qn[G * kQP];
    if (kPrefetchQ) load_q(t, qn);
    for (; t < t1; ++t) {
        const int pos = pos0 + t;
        const int jn = (pos + 1 - j0) < kAttnSplit ? (pos + 1 - j0) : kAttnSplit;
        // V stays packed (64 registers, not 128 unpacked ones): the block
        // keeps 4 waves per SIMD
#pragma unroll
        for (int jj = 0; jj < kAttnSplit; ++jj) asm volatile("" : "+v"(vcol[jj]));
        uint32_t qc[G * kQP];
        if (kPrefetchQ) {
#pragma unroll
            for (int i = 0; i < G * kQP; ++i) qc[i] = qn[i];
        } else {
            load_q(t, qc);
        }
        // scores: quarter wq of every q head of the group against K row j0 + lane
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < kQP; ++i) {
                const uint32_t w = qc[g * kQP + i];
                a = __builtin_fmaf(__uint_as_float(w << 16), kf[2 * i], a);
                a = __builtin_fmaf(__uint_as_float(w & 0xFFFF0000u), kf[2 * i + 1], a);
            }
            red[wq][g][lane] = a;
        }
        __syncthreads();  // red complete; the previous token's reads of sc are done
        if (kPrefetchQ && t + 1 < t1) load_q(t + 1, qn);
        split_softmax<G>(sc, hmax, hsum, jn, [&](int g, int p) {
            return ((red[0][g][p] + red[1][g][p]) + (red[2][g][p] + red[3][g][p])) * scale;
        });
        __syncthreads();
        // weighted V sums of the heads o / kVP, element pair dp (all 64
        // positions without a bound per step in the common full split)
        for (int o = tid; o < G * kVP; o += kAttnThreads) {
            const int g = o / kVP;
            float a0 = 0.0f, a1 = 0.0f;
            auto step = [&](float e, uint32_t w) {
                a0 = __builtin_fmaf(e, __uint_as_float(w << 16), a0);
                a1 = __builtin_fmaf(e, __uint_as_float(w & 0xFFFF0000u), a1);
            };
            if (jn == kAttnSplit) {
#pragma unroll
                for (int q = 0; q < kAttnSplit / 4; ++q) {
                    const float4 e = *reinterpret_cast<const float4*>(&sc[g][4 * q]);
                    step(e.x, vcol[4 * q]);
                    step(e.y, vcol[4 * q + 1]);
                    step(e.z, vcol[4 * q + 2]);
                    step(e.w, vcol[4 * q + 3]);
                }
            } else {
#pragma unroll
                for (int jj = 0; jj < kAttnSplit; ++jj)
                    if (jj < jn) step(sc[g][jj], vcol[jj]);
            }
            const int h = kvh * G + g;
            float* out = pacc + t * hs * HD + (static_cast<long>(h) * S + s) * HD + 2 * dp;
            *reinterpret_cast<float2*>(out) = make_float2(a0, a1);
            if (dp == 0) {
                pm[t * hs + h * S + s] = hmax[g];
                pl[t * hs + h * S + s] = hsum[g];
            }
        }
    }
}

// Batched decode form: one block per (64-position split, kv head, sequence
// b = blockIdx.z), each sequence with its own decode state (st + b), query
// (qkv + b * qkv_stride), KV cache (kc / vc + b * kv_stride) and partials
// (after those of sequence b - 1).  Unlike the bs=1 kernel it reads the
// sequence's position before loading K and V: the grid reaches the end of
// the step graph's position bucket, which is set by the longest sequence,
// so the blocks of shorter sequences past their own positions skip their
// loads.  The per-split arithmetic is attention_split, as in the bs=1
// kernel.
template <int HD, int G>
__global__ __launch_bounds__(kAttnThreads) void attention_batch_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, float* __restrict__ pm, float* __restrict__ pl,
    float* __restrict__ pacc, const EngineState* __restrict__ st, int max_seq, int S,
    float scale, int qkv_stride, long kv_stride) {
    constexpr int kU = HD / 8;
    constexpr int kQU = kU / 4;
    constexpr int kVRow = HD / 2 + 1;
    __shared__ __align__(16) float qs[G][HD];
    __shared__ uint32_t vs[kAttnSplit][kVRow];
    __shared__ __align__(16) float sc[G][kAttnSplit];
    __shared__ float hmax[G], hsum[G];
    const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int j0 = s * kAttnSplit;
    const int tid = threadIdx.x;
    st += b;
    const int done = state_done(st), pos = state_pos(st);
    if (done || j0 > pos) return;  // uniform
    kc += b * kv_stride;
    vc += b * kv_stride;
    qkv += static_cast<long>(b) * qkv_stride;
    const long hs = static_cast<long>(gridDim.y) * G * S;
    pm += b * hs;
    pl += b * hs;
    pacc += b * hs * HD;
    const long cache0 = static_cast<long>(kvh) * max_seq * HD;
    const int jmax = max_seq - 1;
    // the thread's quarter of K row j0 + tid / 4 (clamped to the cache)
    uint4 kq[kQU];
    {
        const int j = j0 + (tid >> 2) <= jmax ? j0 + (tid >> 2) : jmax;
        const uint4* kr = reinterpret_cast<const uint4*>(kc + cache0 + static_cast<long>(j) * HD) +
                          (tid & 3) * kQU;
#pragma unroll
        for (int u = 0; u < kQU; ++u) kq[u] = kr[u];
    }
    constexpr int kVPer = kAttnSplit * kU / kAttnThreads;
    uint4 vraw[kVPer];
#pragma unroll
    for (int t = 0; t < kVPer; ++t) {
        const int idx = tid + t * kAttnThreads;
        const int jj = idx / kU, c = idx - jj * kU;
        const int j = j0 + jj <= jmax ? j0 + jj : jmax;
        vraw[t] = reinterpret_cast<const uint4*>(vc + cache0 + static_cast<long>(j) * HD)[c];
    }
    uint4 qraw = make_uint4(0, 0, 0, 0);
    const bool has_q = tid < G * kU;
    if (has_q) qraw = reinterpret_cast<const uint4*>(qkv + (kvh * G) * HD)[tid];
#pragma unroll
    for (int t = 0; t < kVPer; ++t) {
        const int idx = tid + t * kAttnThreads;
        const int jj = idx / kU, c = idx - jj * kU;
        uint32_t* row = &vs[jj][4 * c];
        row[0] = vraw[t].x;
        row[1] = vraw[t].y;
        row[2] = vraw[t].z;
        row[3] = vraw[t].w;
    }
    if (has_q) {
        float f[8];
        unpack_bf16x8(qraw, f);
        store_f8(&qs[tid / kU][8 * (tid % kU)], f);
    }
    const int jn = (pos + 1 - j0) < kAttnSplit ? (pos + 1 - j0) : kAttnSplit;
    __syncthreads();
    attention_split<HD, G>(kq, qs, vs, sc, hmax, hsum, jn, scale, s, kvh, S, pm, pl, pacc);
}

// ---- batched prefill ---------------------------------------------------------------------
//
// The prompt's tokens (all but the last) go through a layer together: the
// decode GEMV's producers run per token (one kBlock block per token, their
// general form) and write int8 activations and their absmax instead of bit
// planes; the matrix-core GEMM multiplies all tokens' activations at once
// (exact int32, as the GEMV); the decode GEMV's sinks run per token on the
// GEMM's rows.  Each token has its own decode-state record (pos = its
// position), so every per-token value is computed by the same device code,
// in the same order, as a decode step at that position: the KV cache and the
// residual stream equal those of one decode step per token, bit for bit.

struct AmaxOf {
    float m;
    __device__ float absmax() const { return m; }
};

// What a sink's four-row epilogue reads from memory besides the GEMM's
// products, loaded by the staged GEMM before its main loop (SinkOut::preload)
// so that no load waits at the kernel's end: the residual rows of a
// ResidualSink; the decode state and the two RoPE pairs of a QkvRopeSink.
template <class Sink>
struct SinkPreload {
    struct Data {};
    __device__ static Data load(const Sink&, int, int) { return {}; }
};
template <>
struct SinkPreload<ResidualSink> {
    struct Data {
        uint2 res;
    };
    __device__ static Data load(const ResidualSink& sk, int row, int rows) {
        // unconditional (row 0 when the lane's four rows are not all there)
        return {*reinterpret_cast<const uint2*>(sk.res + (row + 3 < rows ? row : 0))};
    }
};
template <>
struct SinkPreload<QkvRopeSink> {
    struct Data {
        int pos, live;
        float2 cs0, cs1;
    };
    __device__ static Data load(const QkvRopeSink& sk, int row, int) {
        Data d;
        d.pos = state_pos(sk.st);
        d.live = !state_done(sk.st);
        d.cs0 = sk.cur_rope[sk.rope_pair(row < sk.end1 ? row : 0)];
        d.cs1 = sk.cur_rope[sk.rope_pair(row + 2 < sk.end1 ? row + 2 : 0)];
        return d;
    }
};

// Epilogue of the staged GEMM (gemm_staged.hpp) that passes the products
// through a per-token sink in registers: the lane holding rows row .. row+3
// of token tok runs the sink for them with the calls and arithmetic of
// prefill_sink_kernel, so the outputs are those of a GEMM followed by that
// kernel, and no int32 product is stored.  The token's absmax and the
// sink's own inputs (SinkPreload) come from preload, which the GEMM calls
// before its main loop.
template <class Sink>
struct SinkOut {
    Sink sink;
    long stride;        // per-token output stride
    const float* amax;  // per-token absmax of the GEMM's int8 input
    int rows;           // rows of the (stacked) product
    struct Pre {
        float am;
        typename SinkPreload<Sink>::Data d;
    };
    __device__ Pre preload(int tok, int row) const {
        Sink sk = sink;
        sk.at(tok, stride);
        return Pre{amax[tok], SinkPreload<Sink>::load(sk, row, rows)};
    }
    __device__ void store4(int tok, int row, v4i acc, const Pre& pre) const {
        Sink sk = sink;
        sk.at(tok, stride);
        sk.prepare();
        if constexpr (SinkQuads<Sink>::value) {
            sk.bind(AmaxOf{pre.am});
            if (row + 3 < rows) {
                const int a[4] = {acc[0], acc[1], acc[2], acc[3]};
                if constexpr (std::is_same<Sink, ResidualSink>::value)
                    sk.store4_with(row, a, pre.d.res);
                else
                    sk.store4(row, a);
            } else {
                sk.prefetch(row, 4, 0);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (row + k < rows) sk.store(row + k, acc[k]);
            }
            return;
        }
        if constexpr (std::is_same<Sink, QkvRopeSink>::value) {
            sk.pos = pre.d.pos;
            sk.live = pre.d.live;
            sk.bind(AmaxOf{pre.am});
            sk.pre_row = row;
            sk.pre_cs = pre.d.cs0;
            sk.store_pair(row, acc[0], acc[1]);  // rows are even, row < rows
            if (row + 2 < rows) {
                sk.pre_row = row + 2;
                sk.pre_cs = pre.d.cs1;
                sk.store_pair(row + 2, acc[2], acc[3]);
            }
            return;
        }
        sk.prefetch(row, 4, 0);
        sk.bind(AmaxOf{pre.am});
        if constexpr (SinkPairs<Sink>::value) {
            sk.store_pair(row, acc[0], acc[1]);  // rows are even, row < rows
            if (row + 2 < rows) sk.store_pair(row + 2, acc[2], acc[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (row + k < rows) sk.store(row + k, acc[k]);
        }
    }
};

template <class P>
__global__ __launch_bounds__(kBlock) void prefill_producer_kernel(P p, long stride,
                                                                  const EngineState* st, int cols,
                                                                  int8_t* __restrict__ xq,
                                                                  float* __restrict__ amax) {
    extern __shared__ float sh[];
    const int t = blockIdx.x, tid = threadIdx.x;
    p.at(t, stride);
    st += t;
    typename P::Regs regs;
    p.template issue<kUnits>(tid, st, regs);
    float* vec = sh;
    float* aux = sh + cols;
    float* red = sh + static_cast<long>(cols) * (1 + P::kAux);
    const float m = p.template fill<false>(vec, aux, cols, tid, red, st, regs);
    const float am = block_max<kBlock>(m, red + 2 * kRedSlot);  // its barrier also orders vec
    const LdsQuantSrc q{vec, quant_scale(am)};
    uint32_t* out = reinterpret_cast<uint32_t*>(xq + static_cast<long>(t) * cols);
    for (int c = tid; c < (cols >> 2); c += kBlock) {
        const float4 v = *reinterpret_cast<const float4*>(vec + 4 * c);
        out[c] = q.q8(v.x) | (q.q8(v.y) << 8) | (q.q8(v.z) << 16) | (q.q8(v.w) << 24);
    }
    if (tid == 0) amax[t] = am;
}

// The same for vectors of at most KU units per thread (P::units_per_thread,
// every vector of the 2B model): the producer's one-pass form (fill_one, the
// order of fill), the values in registers through the norms, and each thread
// quantising and storing its own units (no trip of the vector through LDS).
template <class P, int KU>
__global__ __launch_bounds__(kBlock) void prefill_producer_one_kernel(P p, long stride,
                                                                      const EngineState* st,
                                                                      int cols,
                                                                      int8_t* __restrict__ xq,
                                                                      float* __restrict__ amax) {
    __shared__ float red[3 * kRedSlot];
    const int t = blockIdx.x, tid = threadIdx.x;
    p.at(t, stride);
    st += t;
    typename P::Regs regs;
    p.template issue<KU>(tid, st, regs);
    float v[kUnits][8];
    const float m = p.template fill_one<KU>(v, tid, red, st, regs);
    const float am = block_max<kBlock>(m, red + 2 * kRedSlot);
    const float scale = quant_scale(am);
    uint2* out = reinterpret_cast<uint2*>(xq + static_cast<long>(t) * cols);
    const int units = cols >> 3;
#pragma unroll
    for (int k = 0; k < KU; ++k) {
        const int u = tid + k * kBlock;
        if (u < units) {
            uint32_t w[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                w[h] = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[h] |= (static_cast<uint32_t>(quant_round_clamp(v[k][4 * h + e] * scale)) &
                             0xFFu)
                            << (8 * e);
            }
            out[u] = make_uint2(w[0], w[1]);
        }
    }
    if (tid == 0) amax[t] = am;
}

// Rows [blockIdx.x * R, +R) of token blockIdx.y (R = kBlock, or 2 * kBlock
// for a pair sink), from up to three GEMM outputs: row r < end0 of y0, r <
// end1 of y1 (row r - end0), else y2 (row r - end1); y_k is token-major with
// rows of ld_k.
template <class Sink>
__global__ __launch_bounds__(kBlock) void prefill_sink_kernel(
    Sink sink, long stride, const float* __restrict__ amax, const int32_t* __restrict__ y0,
    const int32_t* __restrict__ y1, const int32_t* __restrict__ y2, int end0, int end1, int rows,
    int ld0, int ld1, int ld2) {
    constexpr bool kPairs = SinkPairs<Sink>::value;
    constexpr int R = kPairs ? 2 * kBlock : kBlock;
    const int t = blockIdx.y, tid = threadIdx.x;
    const long row0 = static_cast<long>(blockIdx.x) * R;
    const int n = rows - row0 < R ? static_cast<int>(rows - row0) : R;
    sink.at(t, stride);
    sink.prepare();
    sink.prefetch(row0, n, tid);
    sink.bind(AmaxOf{amax[t]});
    auto acc = [&](long r) {
        return r < end0 ? y0[static_cast<long>(t) * ld0 + r]
                        : (r < end1 ? y1[static_cast<long>(t) * ld1 + r - end0]
                                    : y2[static_cast<long>(t) * ld2 + r - end1]);
    };
    if constexpr (kPairs) {
        if (2 * tid < n) sink.store_pair(row0 + 2 * tid, acc(row0 + 2 * tid), acc(row0 + 2 * tid + 1));
    } else {
        if (tid < n) sink.store(row0 + tid, acc(row0 + tid));
    }
}

// ---- LM head + greedy argmax ------------------------------------------------------------

// Final RMSNorm (unit order over kLmBlock threads), then
// logits[r] = sum_c W[r][c] * xn[c] in fp32: lane l of the row's wave takes
// the 8-element chunks l, l+64, ... (fma in element order), then the
// wave tree.  Block b streams the contiguous rows [b*V/G, (b+1)*V/G); its
// wave w takes rows b0 + w, b0 + w + 4, ...  A lane keeps its NC chunks of
// the normalised x in registers as bf16 pairs (the values are bf16-rounded,
// so the packing is exact), and NB row buffers rotate: NB - 1 rows are in
// flight while one is reduced (the first rows load before the norm).  The
// loop has no global store (logits are staged in LDS) and no predicated
// load (kFull: H % 512 == 0), so its wait counts cover one row only.
// Argmax = lowest index among the maxima (std::max_element,
// src/main.cpp:194-200).  The last block to finish reduces the per-block
// maxima and advances the decode state.  Reference half_gemv_kernel
// (inference_kernels.cu:488-531) with fp16 -> bf16 weights.
template <int NC, int NB, bool kFull>
__global__ __launch_bounds__(kLmBlock) void lm_head_kernel(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
    const float* __restrict__ wn, float eps, float* __restrict__ logits,
    float* __restrict__ part_v, int* __restrict__ part_i, EngineState* __restrict__ st,
    int* __restrict__ tokens, int V, int H, const float2* __restrict__ rope,
    float2* __restrict__ cur_rope, int half_hd, int max_seq, int rbase, int rrem) {
    static_assert(NB == 2 || NB == 3, "two or three row buffers");
    constexpr int kWaves = kLmBlock / kWave;
    __shared__ __align__(16) float xs[kLmMaxH];
    __shared__ float lg[kLmMaxRows];  // the block's logits, stored after the loop
    __shared__ float red[kWaves];
    __shared__ float wv[kWaves];
    __shared__ int wi[kWaves];
    __shared__ int last;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nch = H >> 3;
    // rows [b0, b1): rbase each, one more for blocks below rrem (host-computed
    // V / grid and V % grid: no division here)
    const int blk = blockIdx.x;
    const long b0 = static_cast<long>(blk) * rbase + (blk < rrem ? blk : rrem);
    const long b1 = b0 + rbase + (blk < rrem ? 1 : 0);
    const long n = (b1 - b0 - wave + kWaves - 1) / kWaves;  // rows of this wave (may be <= 0)
    const long i_last = n > 0 ? n - 1 : 0;
    auto row_of = [&](long i) { return b0 + wave + (i <= i_last ? i : i_last) * kWaves; };
    auto load_row = [&](long i, uint4 (&w)[NC]) {
        const long r = row_of(i);
        const uint4* wr = reinterpret_cast<const uint4*>(W + (r < V ? r : V - 1) * H);
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            const int c = lane + k * kWave;
            if (kFull)  // every chunk exists: unconditional loads (non-temporal)
                w[k] = nt_load(wr + c);
            else
                w[k] = c < nch ? nt_load(wr + c) : make_uint4(0, 0, 0, 0);
        }
    };
    // x and the norm weights first (the prologue waits for them alone), then
    // the first rows; H <= NC * 64 elements are one pass of kLmBlock threads
    constexpr bool kOne = NC * kWave <= kUnits * kLmBlock;
    HeldWeights<kLmBlock> hw;
    HeldUnits<kLmBlock> hx;
    hx.load(x, H >> 3, tid);
    hw.load(wn, H >> 3, tid);
    uint4 wa[NC], wb[NC], wc[NC];
    load_row(0, wa);
    if (NB == 3) load_row(1, wb);
    if (st->done) return;  // after the first row loads (they are in bounds either way)

    const float ss = load_bf16_sumsq<kLmBlock, kOne>(x, xs, H >> 3, tid, nullptr, hx);
    const float inv = inv_rms(block_sum<kLmBlock>(ss, red), H, eps);
    hw.template apply<kOne>(xs, wn, inv, H >> 3, tid);
    __syncthreads();
    uint4 xp[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const int c = lane + k * kWave;
        if (c < nch) {
            float f[8];
            load_f8(xs + 8 * c, f);
            uint32_t u[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                u[q] = (__builtin_bit_cast(uint32_t, f[2 * q]) >> 16) |
                       (__builtin_bit_cast(uint32_t, f[2 * q + 1]) & 0xFFFF0000u);
            xp[k] = make_uint4(u[0], u[1], u[2], u[3]);
        } else {
            xp[k] = make_uint4(0, 0, 0, 0);
        }
    }

    float best = -INFINITY;
    int best_i = 0x7FFFFFFF;
    auto reduce_row = [&](long i, const uint4 (&w)[NC]) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            const int c = lane + k * kWave;
            if (kFull || c < nch) {
                float f[8], xv[8];
                unpack_bf16x8(w[k], f);
                unpack_bf16x8(xp[k], xv);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(f[e], xv[e], acc);
            }
        }
        acc = wave_sum_tree(acc);
        const long r = row_of(i);
        // LDS, not global: a global store in the loop would make the
        // compiler drain the loads in flight
        if (lane == 0) lg[r - b0] = acc;
        if (acc > best) {  // rows ascend within a wave: strict > keeps the first maximum
            best = acc;
            best_i = static_cast<int>(r);
        }
    };
    // Counted loops with their only exit at the latch (exact wait counts, as
    // in the streaming GEMV); loads past the wave's last row re-read it.
    long i = 0;
    if (NB == 3) {
        for (long p = 0; p < n / 3; ++p, i += 3) {
            load_row(i + 2, wc);
            __builtin_amdgcn_sched_barrier(0);
            reduce_row(i, wa);
            load_row(i + 3, wa);
            __builtin_amdgcn_sched_barrier(0);
            reduce_row(i + 1, wb);
            load_row(i + 4, wb);
            __builtin_amdgcn_sched_barrier(0);
            reduce_row(i + 2, wc);
        }
        if (n > 0 && n % 3 > 0) reduce_row(i, wa);
        if (n > 0 && n % 3 > 1) reduce_row(i + 1, wb);
    } else {
        for (long p = 0; p < n / 2; ++p, i += 2) {
            load_row(i + 1, wb);
            __builtin_amdgcn_sched_barrier(0);
            reduce_row(i, wa);
            load_row(i + 2, wa);
            __builtin_amdgcn_sched_barrier(0);
            reduce_row(i + 1, wb);
        }
        if (n > 0 && (n & 1)) reduce_row(i, wa);
    }
    __syncthreads();
    for (long j = tid; j < b1 - b0; j += kLmBlock) logits[b0 + j] = lg[j];
    if (lane == 0) {
        wv[wave] = best;
        wi[wave] = best_i;
    }
    __syncthreads();
    if (tid == 0) {
        float b = wv[0];
        int bi = wi[0];
        for (int w = 1; w < kLmBlock / kWave; ++w)
            if (wv[w] > b || (wv[w] == b && wi[w] < bi)) {
                b = wv[w];
                bi = wi[w];
            }
        // The partials go through to memory (agent-coherent stores, sc1) and
        // are complete before the ticket counts this block, so the last
        // block's agent-coherent loads see every block's; no fence (an L2
        // write-back and invalidate per block) is needed.
        __hip_atomic_store(&part_v[blockIdx.x], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&part_i[blockIdx.x], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        const unsigned t =
            __hip_atomic_fetch_add(&st->ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = t == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    const int pos_old = st->pos;  // read before thread 0 advances it (barrier below)
    float b = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int k = tid; k < static_cast<int>(gridDim.x); k += kLmBlock) {
        const float v = __hip_atomic_load(&part_v[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int i = __hip_atomic_load(&part_i[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (v > b || (v == b && i < bi)) {
            b = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(b, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (ov > b || (ov == b && oi < bi)) {
            b = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        wv[wave] = b;
        wi[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kLmBlock / kWave; ++w)
            if (wv[w] > b || (wv[w] == b && wi[w] < bi)) {
                b = wv[w];
                bi = wi[w];
            }
        const int tok = bi == 0x7FFFFFFF ? 0 : bi;  // all-NaN logits: token 0
        const int nxt = st->pos + 1;
        if (nxt >= st->prompt_len && nxt < st->limit) {
            tokens[nxt] = tok;
            st->generated += 1;
            if (st->stop_eos && tok == st->eos) st->done = 1;
        }
        st->pos = nxt;
        if (nxt >= st->limit) st->done = 1;
        st->ticket = 0u;
    }
    // RoPE row of the next position for the next step's q/k projection
    {
        const int p = pos_old + 1 < max_seq ? pos_old + 1 : max_seq - 1;
        for (int i = tid; i < half_hd; i += kLmBlock) cur_rope[i] = rope[static_cast<long>(p) * half_hd + i];
    }
}

typedef void (*LmKernel)(const uint16_t*, const uint16_t*, const float*, float, float*, float*,
                         int*, EngineState*, int*, int, int, const float2*, float2*, int, int,
                         int, int);

// Instantiation for H: NC = ceil(H / 512) chunks per lane (H <= 8192), two
// row buffers; kFull when H % 512 == 0.
template <bool kFull>
LmKernel lm_head_for_nc(int nc) {
    switch (nc) {
        case 1: return lm_head_kernel<1, 2, kFull>;
        case 2: return lm_head_kernel<2, 2, kFull>;
        case 3: return lm_head_kernel<3, 2, kFull>;
        case 4: return lm_head_kernel<4, 2, kFull>;
        case 5: return lm_head_kernel<5, 2, kFull>;
        case 6: return lm_head_kernel<6, 2, kFull>;
        case 7: return lm_head_kernel<7, 2, kFull>;
        case 8: return lm_head_kernel<8, 2, kFull>;
        case 9: return lm_head_kernel<9, 2, kFull>;
        case 10: return lm_head_kernel<10, 2, kFull>;
        case 11: return lm_head_kernel<11, 2, kFull>;
        case 12: return lm_head_kernel<12, 2, kFull>;
        case 13: return lm_head_kernel<13, 2, kFull>;
        case 14: return lm_head_kernel<14, 2, kFull>;
        case 15: return lm_head_kernel<15, 2, kFull>;
        default: return lm_head_kernel<16, 2, kFull>;
    }
}

LmKernel lm_head_for(int H) {
    const int nc = (H / 8 + kWave - 1) / kWave;
    return (H % 512 == 0) ? lm_head_for_nc<true>(nc) : lm_head_for_nc<false>(nc);
}

// Batched decode: the final norm writes each sequence's normalised vector
// for the batched LM head (lm_head_mfma_kernel / lm_select_kernel below).
// The batched final norm holds a normalised vector in LDS, so the batched
// engine takes hidden sizes up to kLmBatchMaxH.
constexpr int kLmBatchMaxH = 4096;

// float index of chunk c's first element in a padded normalised vector
__device__ __forceinline__ int lm_xpad(int c) { return 8 * c + 4 * (c >> 3); }

// A non-negative double rounded up to float.
__device__ __forceinline__ float lm_round_up(double d) {
    float f = static_cast<float>(d);
    if (static_cast<double>(f) < d) f = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, f) + 1u);
    return f;
}

// Batched decode: the final RMSNorm of sequence blockIdx.x with
// lm_head_kernel's prologue (same threads, same order), written padded for
// the LM head: xn[b][lm_xpad(c) ..] = chunk c of the normalised vector
// (bf16-rounded floats), zeros for chunks c >= H / 8 up to nc64; xnorm[b] =
// its Euclidean norm (summed in double, rounded up to float).
template <bool kOne>
__global__ __launch_bounds__(kLmBlock) void final_norm_batch_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ wn, float eps,
    float* __restrict__ xn, float* __restrict__ xnorm, int H, int nc64, int xstride) {
    __shared__ __align__(16) float xs[kLmBatchMaxH];
    __shared__ float red[kLmBlock / kWave];
    __shared__ double dred[kLmBlock / kWave];
    const int tid = threadIdx.x, nch = H >> 3;
    const uint16_t* xg = x + static_cast<long>(blockIdx.x) * H;
    HeldWeights<kLmBlock> hw;
    HeldUnits<kLmBlock> hx;
    hx.load(xg, nch, tid);
    hw.load(wn, nch, tid);
    const float ss = load_bf16_sumsq<kLmBlock, kOne>(xg, xs, nch, tid, nullptr, hx);
    const float inv = inv_rms(block_sum<kLmBlock>(ss, red), H, eps);
    hw.template apply<kOne>(xs, wn, inv, nch, tid);
    __syncthreads();
    {
        double q = 0.0;
        for (int i = tid; i < H; i += kLmBlock) {
            const double v = xs[i];
            q += v * v;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off, kWave);
        if ((tid & (kWave - 1)) == 0) dred[tid / kWave] = q;
    }
    __syncthreads();
    if (tid == 0) {
        double q = 0.0;
        for (int w = 0; w < kLmBlock / kWave; ++w) q += dred[w];
        xnorm[blockIdx.x] = lm_round_up(__builtin_sqrt(q));
    }
    float* dst = xn + static_cast<long>(blockIdx.x) * xstride;
    for (int c = tid; c < nc64; c += kLmBlock) {
        float f[8];
        if (c < nch) {
            load_f8(xs + 8 * c, f);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = 0.0f;
        }
        store_f8(dst + lm_xpad(c), f);
    }
}

// floats per padded normalised vector: lm_xpad(nc * 64), nc = ceil(H / 512)
int lm_head_batch_xstride(int H) {
    const int nc = (H / 8 + kWave - 1) / kWave;
    return 8 * (nc * kWave) + 4 * ((nc * kWave) >> 3);
}


// ---- batched decode: the LM head on the bf16 matrix cores ------------------------
//
// logits[t][r] = W[r] . xn[t] for the B sequences of a step (W the bf16
// [V][H] table, xn[t] the final-normed vector, bf16 values), in two launches:
//   lm_head_mfma_kernel: v_mfma_f32_16x16x32_bf16 over blocks of 512 rows and
//     32 tokens: approximate logits a[t][r] (every product exact, the sums in
//     the matrix cores' float32 accumulation), stored, and per block and
//     token the largest lower bound a - d and upper bound a + d, with
//     d[t][r] = c |W[r]| |xn[t]| (Euclidean norms rounded up);
//   lm_select_kernel (one block per sequence): M = the largest lower bound;
//     every row whose upper bound reaches M (in the blocks whose largest
//     upper bound does) is recomputed with exactly the operations of the bs=1
//     kernel (lm_head_kernel: 64 fma chains over 8-element chunks, then the
//     pairwise tree), its exact logit stored, and the argmax (lowest index
//     among maxima) taken over those rows.
// Why the token equals the bs=1 kernel's: with e the bs=1 value and S the
// real dot product, |e - S| <= (H/64 + 6) 2^-24 sum |w x| (H/64 fma per
// chain, a 6-level tree), |a - S| <= H 2^-23 sum |w x| (at most one float32
// rounding, truncation allowed, per accumulated product), and sum |w x| <=
// |w| |x|; c = 1.25 (H + H/64 + 8) 2^-23 covers both with a margin for the
// rounding of the bounds themselves.  A row outside the candidates has
// e <= a + d < M <= max_j (a_j - d_j) <= max_j e_j, so it is not the argmax,
// which is therefore among the recomputed rows, whose values are the bs=1
// kernel's.  The other rows keep the approximate logits (|a - e| <= 2 d).
// NaN upper bounds count as candidates; more than kLmCandMax candidates in a
// sequence (e.g. NaN logits everywhere) fall back to recomputing every row.
constexpr int kLmMfmaBlock = 512;                     // 8 waves
constexpr int kLmMfmaStrips = 4;                      // 16-row strips per wave
constexpr int kLmMfmaRows = 8 * kLmMfmaStrips * 16;   // rows per block
constexpr int kLmMfmaSeg = 1024;                      // hidden elements per staged x segment
constexpr int kLmMfmaTok = 32;                        // tokens per block (two 16-token tiles)
constexpr int kLmCandMax = 1024;                      // candidate rows per sequence
constexpr int kLmSelMaxBlocks = 2048;                 // row blocks (vocabulary <= 1M rows)
constexpr int kLmSelectBlock = 256;

typedef __bf16 lm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lm_f32x4 __attribute__((ext_vector_type(4)));

float lm_bound_c(int H) {
    return static_cast<float>(1.25 * (H + H / 64 + 8) * 0x1p-23);
}

// |W[r]| (rounded up), one wave per row, once per engine.
__global__ __launch_bounds__(256) void lm_row_norm_kernel(const uint16_t* __restrict__ W,
                                                          float* __restrict__ out, int V, int H) {
    const long r = static_cast<long>(blockIdx.x) * 4 + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (r >= V) return;
    double s = 0.0;
    for (int c = lane; c < H; c += kWave) {
        const double w = BF16::to_float(W[r * H + c]);
        s += w * w;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
    if (lane == 0) out[r] = lm_round_up(__builtin_sqrt(s));
}

// Block (row block x, token group y): 8 waves, wave w owning the strips
// 4w .. 4w + 3 (16 rows each) of the block's 512 rows and both 16-token
// tiles.  x is staged in LDS segment by segment (1024 hidden elements, 32
// tokens, bf16, the 16-byte chunk c of token t at c ^ (t & 15): the 16 lanes
// of a tile read 16 distinct bank groups).  A 64-element step of a strip is
// two MFMAs: lane (i, q) holds row i's elements 16 q + [0, 8) and 16 q +
// [8, 16) of the step (one 32-byte weight load) and the same elements of
// token i (the dot product's K order inside an MFMA is the matrix cores'
// own, as in any fp32 sum order).
template <int NT>
__global__ __launch_bounds__(kLmMfmaBlock) void lm_head_mfma_kernel(
    const uint16_t* __restrict__ W, const float* __restrict__ xn, int xstride,
    const float* __restrict__ wnorm, const float* __restrict__ xnorm, float cbound,
    float* __restrict__ logits, float* __restrict__ part_lo, float* __restrict__ part_hi, int V,
    int H, int B, int nblk) {
    __shared__ __align__(16) uint16_t xs[kLmMfmaTok * kLmMfmaSeg];
    __shared__ float red_lo[8][kLmMfmaTok], red_hi[8][kLmMfmaTok];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int li = lane & 15, q = lane >> 4;
    const int blk = blockIdx.x, t0 = blockIdx.y * kLmMfmaTok;
    const int ntok = B - t0 < kLmMfmaTok ? B - t0 : kLmMfmaTok;
    const long r0 = static_cast<long>(blk) * kLmMfmaRows + wave * (kLmMfmaStrips * 16);
    const uint16_t* wrow[kLmMfmaStrips];
#pragma unroll
    for (int s = 0; s < kLmMfmaStrips; ++s) {
        const long r = r0 + 16 * s + li;
        wrow[s] = W + (r < V ? r : V - 1) * static_cast<long>(H);
    }
    lm_f32x4 acc[kLmMfmaStrips][NT];
#pragma unroll
    for (int s = 0; s < kLmMfmaStrips; ++s)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[s][t] = (lm_f32x4){0.f, 0.f, 0.f, 0.f};
    // weights of step e0 (global element index) of every strip; elements past
    // H read as zeros (H % 8 == 0: each 16-byte half is wholly in or out).
    // Ordinary loads, not the non-temporal hint of the streaming kernels: a
    // load instruction here takes half of each of 16 rows' 128-byte lines
    // and the next one the other halves, which then hit in the L2 (with the
    // hint, batch 8 / 32 decoded 3,864 / 10,087 tok/s, without 3,911 /
    // 10,158; the same-line halves as contiguous 64-byte pieces: no change).
    auto load_w = [&](int e0, uint4 (&w)[kLmMfmaStrips][2]) {
        const int e = e0 + 16 * q;
#pragma unroll
        for (int s = 0; s < kLmMfmaStrips; ++s) {
            const uint4* p = reinterpret_cast<const uint4*>(wrow[s] + e);
            w[s][0] = e < H ? p[0] : make_uint4(0, 0, 0, 0);
            w[s][1] = e + 8 < H ? p[1] : make_uint4(0, 0, 0, 0);
        }
    };
    for (int seg0 = 0; seg0 < H; seg0 += kLmMfmaSeg) {
        const int sl = H - seg0 < kLmMfmaSeg ? H - seg0 : kLmMfmaSeg;
        const int nstep = (sl + 63) / 64;
        __syncthreads();  // the previous segment's operand reads are done
        for (int i = tid; i < kLmMfmaTok * (kLmMfmaSeg / 8); i += kLmMfmaBlock) {
            const int t = i / (kLmMfmaSeg / 8), c = i % (kLmMfmaSeg / 8);
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t < ntok && 8 * c < sl) {
                float f[8];
                load_f8(xn + static_cast<long>(t0 + t) * xstride + lm_xpad((seg0 >> 3) + c), f);
                uint32_t u[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)  // bf16-rounded floats: the high halves are exact
                    u[k] = (__builtin_bit_cast(uint32_t, f[2 * k]) >> 16) |
                           (__builtin_bit_cast(uint32_t, f[2 * k + 1]) & 0xFFFF0000u);
                v = make_uint4(u[0], u[1], u[2], u[3]);
            }
            *reinterpret_cast<uint4*>(xs + t * kLmMfmaSeg + 8 * (c ^ (t & 15))) = v;
        }
        __syncthreads();
        // step stp (64 elements) of every strip from the weights in w
        auto compute = [&](const uint4 (&w)[kLmMfmaStrips][2], int stp) {
            const int c1 = 8 * stp + 2 * q;  // local 16-byte chunk of the lane's first 8 elements
            lm_bf16x8 xb[NT][2];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint16_t* xr = xs + (16 * t + li) * kLmMfmaSeg;
                xb[t][0] = __builtin_bit_cast(lm_bf16x8,
                                              *reinterpret_cast<const uint4*>(xr + 8 * (c1 ^ li)));
                xb[t][1] = __builtin_bit_cast(
                    lm_bf16x8, *reinterpret_cast<const uint4*>(xr + 8 * ((c1 + 1) ^ li)));
            }
#pragma unroll
            for (int s = 0; s < kLmMfmaStrips; ++s) {
                const lm_bf16x8 w0 = __builtin_bit_cast(lm_bf16x8, w[s][0]);
                const lm_bf16x8 w1 = __builtin_bit_cast(lm_bf16x8, w[s][1]);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0, xb[t][0], acc[s][t], 0, 0, 0);
                    acc[s][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1, xb[t][1], acc[s][t], 0, 0, 0);
                }
            }
        };
        // two weight buffers: each is refilled right after its step is used
        uint4 wa[kLmMfmaStrips][2], wb[kLmMfmaStrips][2];
        load_w(seg0, wa);
        for (int d = 0; d < nstep; d += 2) {
            if (d + 1 < nstep) load_w(seg0 + 64 * (d + 1), wb);
            __builtin_amdgcn_sched_barrier(0);
            compute(wa, d);
            if (d + 2 < nstep) load_w(seg0 + 64 * (d + 2), wa);
            __builtin_amdgcn_sched_barrier(0);
            if (d + 1 < nstep) compute(wb, d + 1);
        }
    }
    // lane (i, q) of strip s, tile t holds rows r0 + 16 s + 4 q + v of token
    // t0 + 16 t + i
    float mlo[NT], mhi[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        mlo[t] = -INFINITY;
        mhi[t] = -INFINITY;
        const int tok = t0 + 16 * t + li;
        if (tok >= B) continue;
        const float xnt = xnorm[tok];
#pragma unroll
        for (int s = 0; s < kLmMfmaStrips; ++s) {
            const long row = r0 + 16 * s + 4 * q;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (row + v >= V) continue;
                const float a = acc[s][t][v];
                const float dd = (cbound * wnorm[row + v]) * xnt;
                logits[static_cast<long>(tok) * V + row + v] = a;
                mlo[t] = __builtin_fmaxf(mlo[t], a - dd);
                const float hi = a + dd;
                mhi[t] = hi != hi ? INFINITY : __builtin_fmaxf(mhi[t], hi);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int off = 16; off < kWave; off <<= 1) {
            mlo[t] = __builtin_fmaxf(mlo[t], __shfl_xor(mlo[t], off, kWave));
            mhi[t] = __builtin_fmaxf(mhi[t], __shfl_xor(mhi[t], off, kWave));
        }
        if (q == 0) {
            red_lo[wave][16 * t + li] = mlo[t];
            red_hi[wave][16 * t + li] = mhi[t];
        }
    }
    __syncthreads();
    if (tid < kLmMfmaTok && tid < ntok) {
        float lo = red_lo[0][tid], hi = red_hi[0][tid];
        for (int w = 1; w < 8; ++w) {
            lo = __builtin_fmaxf(lo, red_lo[w][tid]);
            hi = __builtin_fmaxf(hi, red_hi[w][tid]);
        }
        part_lo[static_cast<long>(t0 + tid) * nblk + blk] = lo;
        part_hi[static_cast<long>(t0 + tid) * nblk + blk] = hi;
    }
}

// Sequence blockIdx.x: the candidate rows' exact logits (the bs=1 chain),
// the argmax over them and the decode-state update of lm_head_batch_kernel.
__global__ __launch_bounds__(kLmSelectBlock) void lm_select_kernel(
    const uint16_t* __restrict__ W, const float* __restrict__ xn, int xstride,
    const float* __restrict__ wnorm, const float* __restrict__ xnorm, float cbound,
    float* __restrict__ logits, const float* __restrict__ part_lo,
    const float* __restrict__ part_hi, EngineState* __restrict__ st, int* __restrict__ tokens,
    long tok_stride, int V, int H, const float2* __restrict__ rope, float2* __restrict__ cur_rope,
    int half_hd, int max_seq, int nblk) {
    constexpr int kWaves = kLmSelectBlock / kWave;
    __shared__ int cand[kLmCandMax];
    __shared__ int selb[kLmSelMaxBlocks];
    __shared__ int ncand, nsel;
    __shared__ float red[kWaves];
    __shared__ float wv[kWaves];
    __shared__ int wi[kWaves];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int b = blockIdx.x;
    const float* lo = part_lo + static_cast<long>(b) * nblk;
    const float* hi = part_hi + static_cast<long>(b) * nblk;
    float* lg = logits + static_cast<long>(b) * V;
    const float* x = xn + static_cast<long>(b) * xstride;
    float m = -INFINITY;
    for (int k = tid; k < nblk; k += kLmSelectBlock) m = __builtin_fmaxf(m, lo[k]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off, kWave));
    if (lane == 0) red[wave] = m;
    if (tid == 0) {
        ncand = 0;
        nsel = 0;
    }
    __syncthreads();
    m = red[0];
    for (int w = 1; w < kWaves; ++w) m = __builtin_fmaxf(m, red[w]);
    // the blocks whose largest upper bound reaches m (NaN bounds are +inf)
    for (int k = tid; k < nblk; k += kLmSelectBlock)
        if (!(hi[k] < m)) selb[atomicAdd(&nsel, 1)] = k;
    __syncthreads();
    const float xnt = xnorm[b];
    const int ns = nsel;
    for (int j = 0; j < ns; ++j) {
        const int k = selb[j];
        const long e = static_cast<long>(k + 1) * kLmMfmaRows < V ? static_cast<long>(k + 1) * kLmMfmaRows : V;
        for (long r = static_cast<long>(k) * kLmMfmaRows + tid; r < e; r += kLmSelectBlock) {
            const float a = lg[r];
            const float dd = (cbound * wnorm[r]) * xnt;
            if (!(a + dd < m)) {
                const int slot = atomicAdd(&ncand, 1);
                if (slot < kLmCandMax) cand[slot] = static_cast<int>(r);
            }
        }
    }
    __syncthreads();
    const int nc = ncand;
    const bool all = nc > kLmCandMax;  // recompute every row
    const int nrows = all ? V : nc;
    const int nch = H >> 3;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int k = wave; k < nrows; k += kWaves) {
        const int r = all ? k : cand[k];
        const uint4* wr = reinterpret_cast<const uint4*>(W + static_cast<long>(r) * H);
        float a = 0.0f;
        for (int c = lane; c < nch; c += kWave) {  // lm_head_kernel's chain of virtual lane `lane`
            float wf[8], xv[8];
            unpack_bf16x8(wr[c], wf);
            load_f8(x + lm_xpad(c), xv);
#pragma unroll
            for (int e = 0; e < 8; ++e) a = __builtin_fmaf(wf[e], xv[e], a);
        }
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) a += __shfl_xor(a, off, kWave);  // pairwise tree
        if (lane == 0) lg[r] = a;
        if (a > bv || (a == bv && r < bi)) {
            bv = a;
            bi = r;
        }
    }
    if (lane == 0) {
        wv[wave] = bv;
        wi[wave] = bi;
    }
    __syncthreads();
    EngineState* sg = st + b;
    const int done = sg->done, pos_old = sg->pos;
    __syncthreads();  // every thread has read the state before thread 0 changes it
    if (done) return;  // uniform
    if (tid == 0) {
        for (int w = 1; w < kWaves; ++w)
            if (wv[w] > bv || (wv[w] == bv && wi[w] < bi)) {
                bv = wv[w];
                bi = wi[w];
            }
        const int tok = bi == 0x7FFFFFFF ? 0 : bi;  // all-NaN logits: token 0
        const int nxt = pos_old + 1;
        int* tk = tokens + static_cast<long>(b) * tok_stride;
        if (nxt >= sg->prompt_len && nxt < sg->limit) {
            tk[nxt] = tok;
            sg->generated += 1;
            if (sg->stop_eos && tok == sg->eos) sg->done = 1;
        }
        sg->pos = nxt;
        if (nxt >= sg->limit) sg->done = 1;
    }
    const int p = pos_old + 1 < max_seq ? pos_old + 1 : max_seq - 1;
    float2* cr = cur_rope + static_cast<long>(b) * half_hd;
    for (int k = tid; k < half_hd; k += kLmSelectBlock) cr[k] = rope[static_cast<long>(p) * half_hd + k];
}

// ---- random-init weights (model generation on the device) ------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// N(0,1) float from the counter (seed, i): Box-Muller on two 24-bit
// uniforms, u1 = (k + 1) / 2^24 in (0, 1] and u2 = j / 2^24 in [0, 1),
// normal = sqrt(-2 ln u1) * cos(2 pi u2).  The logarithm, square root and
// cosine are fixed sequences of IEEE double adds and multiplies (no library
// call, no division, no fused multiply-add: the library is built with
// -ffp-contract=off), so every bit of the result follows from the counter
// alone and a host program evaluating the same sequence reproduces the
// weights exactly.
//   ln: u1 = m 2^(e - 24), m in (1/sqrt2, sqrt2]; ln(1 + t) = t sum_{i<=40}
//       (-1)^i t^i / (i + 1) with t = m - 1 (exact), |t| <= 0.4143, so the
//       truncation is below 1e-17;
//   sqrt: y * rsqrt(y), rsqrt from a bit-pattern guess and four Newton steps
//       r <- r (1.5 - (0.5 y r) r);
//   cos: the octant reduction on the 24-bit integer j (exact), then the
//       Taylor series of cos or sin to degree 20 / 21 on [0, pi/4].
__device__ __constant__ double kGenLogC[41] = {
    0x1.0000000000000p+0, -0x1.0000000000000p-1, 0x1.5555555555555p-2, -0x1.0000000000000p-2,
    0x1.999999999999ap-3, -0x1.5555555555555p-3, 0x1.2492492492492p-3, -0x1.0000000000000p-3,
    0x1.c71c71c71c71cp-4, -0x1.999999999999ap-4, 0x1.745d1745d1746p-4, -0x1.5555555555555p-4,
    0x1.3b13b13b13b14p-4, -0x1.2492492492492p-4, 0x1.1111111111111p-4, -0x1.0000000000000p-4,
    0x1.e1e1e1e1e1e1ep-5, -0x1.c71c71c71c71cp-5, 0x1.af286bca1af28p-5, -0x1.999999999999ap-5,
    0x1.8618618618618p-5, -0x1.745d1745d1746p-5, 0x1.642c8590b2164p-5, -0x1.5555555555555p-5,
    0x1.47ae147ae147bp-5, -0x1.3b13b13b13b14p-5, 0x1.2f684bda12f68p-5, -0x1.2492492492492p-5,
    0x1.1a7b9611a7b96p-5, -0x1.1111111111111p-5, 0x1.0842108421084p-5, -0x1.0000000000000p-5,
    0x1.f07c1f07c1f08p-6, -0x1.e1e1e1e1e1e1ep-6, 0x1.d41d41d41d41dp-6, -0x1.c71c71c71c71cp-6,
    0x1.bacf914c1bad0p-6, -0x1.af286bca1af28p-6, 0x1.a41a41a41a41ap-6, -0x1.999999999999ap-6,
    0x1.8f9c18f9c18fap-6};
__device__ __constant__ double kGenCosC[11] = {
    0x1.0000000000000p+0,  -0x1.0000000000000p-1,  0x1.5555555555555p-5,  -0x1.6c16c16c16c17p-10,
    0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
    0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62};
__device__ __constant__ double kGenSinC[11] = {
    0x1.0000000000000p+0,  -0x1.5555555555555p-3,  0x1.1111111111111p-7,  -0x1.a01a01a01a01ap-13,
    0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41,
    0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57, 0x1.71b8ef6dcf572p-66};

// ln(k / 2^24) for k in [1, 2^24]
__device__ __forceinline__ double gen_ln_u24(uint32_t k) {
    int e = 31 - __builtin_clz(k);  // floor(log2 k)
    double m = static_cast<double>(k) *
               __builtin_bit_cast(double, static_cast<uint64_t>(1023 - e) << 52);  // [1, 2)
    if (m > 0x1.6a09e667f3bcdp+0) {  // sqrt(2)
        m = m * 0.5;
        e = e + 1;
    }
    const double t = m - 1.0;
    double p = kGenLogC[40];
#pragma unroll
    for (int i = 39; i >= 0; --i) p = p * t + kGenLogC[i];
    return static_cast<double>(e - 24) * 0x1.62e42fefa39efp-1 + t * p;
}

__device__ __forceinline__ double gen_sqrt(double y) {
    if (!(y > 0.0)) return 0.0;
    const uint64_t b = 0x5FE6EB50C7B537A9ull - (__builtin_bit_cast(uint64_t, y) >> 1);
    double r = __builtin_bit_cast(double, b);
    const double h = 0.5 * y;
#pragma unroll
    for (int i = 0; i < 4; ++i) r = r * (1.5 - (h * r) * r);
    return y * r;
}

// cos(2 pi j / 2^24) for j in [0, 2^24)
__device__ __forceinline__ double gen_cos_u24(uint32_t j) {
    bool neg = false;
    if (j >= (1u << 23)) j = (1u << 24) - j;  // cos(2 pi - x) = cos x
    if (j > (1u << 22)) {                      // cos(pi - x) = -cos x
        j = (1u << 23) - j;
        neg = true;
    }
    const bool use_sin = j > (1u << 21);  // cos(pi/2 - x) = sin x
    const double x = static_cast<double>(use_sin ? (1u << 22) - j : j) * 0x1.921fb54442d18p-22;
    const double x2 = x * x;
    double p;
    if (use_sin) {
        p = kGenSinC[10];
#pragma unroll
        for (int i = 9; i >= 0; --i) p = p * x2 + kGenSinC[i];
        p = x * p;
    } else {
        p = kGenCosC[10];
#pragma unroll
        for (int i = 9; i >= 0; --i) p = p * x2 + kGenCosC[i];
    }
    return neg ? -p : p;
}

__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    const uint64_t z = splitmix64(seed ^ splitmix64(i));
    const uint32_t k = static_cast<uint32_t>(z >> 40) + 1u;
    const uint32_t j = static_cast<uint32_t>((z >> 16) & 0xFFFFFFull);
    const double r = gen_sqrt(-2.0 * gen_ln_u24(k));
    return static_cast<float>(r * gen_cos_u24(j));
}

constexpr int kGenBlocks = 1024;
__device__ double g_gen_partial[kGenBlocks];

// One thread per 64 columns of a row: latent W ~ N(0,1), 2:4 top-2 |W| mask
// (higher index wins ties), kept value sign(W) (W >= 0 -> +1), packed
// (python/convert_model.py:88-207, 257-316).  Per-block sums of |W| in double
// feed gamma = mean|W|.
__global__ __launch_bounds__(256) void gen_sparse_ternary_kernel(uint64_t seed, int rows,
                                                                 int cols, uint32_t* meta,
                                                                 uint32_t* values, int ms,
                                                                 int vs, float* latent) {
    __shared__ double part[256 / kWave];
    const long units = static_cast<long>(rows) * (cols / 64);
    double sum = 0.0;
    for (long u = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; u < units;
         u += static_cast<long>(gridDim.x) * 256) {
        const long r = u / (cols / 64);
        const int c0 = static_cast<int>(u - r * (cols / 64)) * 64;
        uint32_t mw[2] = {0u, 0u}, sw = 0u;
        for (int g = 0; g < 16; ++g) {
            float w[4];
            for (int i = 0; i < 4; ++i) {
                const long idx = r * cols + c0 + 4 * g + i;
                w[i] = normal_at(seed, static_cast<uint64_t>(idx));
                sum += fabs(static_cast<double>(w[i]));
                if (latent) latent[idx] = w[i];
            }
            uint32_t bm = 0u, sg = 0u;
            int kept = 0;
            for (int i = 0; i < 4; ++i) {
                int beaten = 0;
                for (int j = 0; j < 4; ++j) {
                    if (j == i) continue;
                    const float ai = fabsf(w[i]), aj = fabsf(w[j]);
                    if (aj > ai || (aj == ai && j > i)) ++beaten;
                }
                if (beaten < 2) {
                    bm |= 1u << i;
                    if (w[i] < 0.0f) sg |= 1u << kept;  // bit 0: lower kept, bit 1: higher
                    ++kept;
                }
            }
            mw[g >> 3] |= bm << (4 * (g & 7));
            sw |= sg << (2 * g);
        }
        const int w0 = c0 / 32;
        meta[r * ms + w0] = mw[0];
        meta[r * ms + w0 + 1] = mw[1];
        values[r * vs + c0 / 64] = sw;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = sum;
    __syncthreads();
    if (threadIdx.x == 0) g_gen_partial[blockIdx.x] = ((part[0] + part[1]) + part[2]) + part[3];
}

__global__ void gen_gamma_kernel(int nblocks, double count, float* gamma) {
    double s = 0.0;
    for (int b = 0; b < nblocks; ++b) s += g_gen_partial[b];
    *gamma = static_cast<float>(s / count);
}

__global__ __launch_bounds__(256) void gen_normal_bf16_kernel(uint64_t seed, long n, float std_,
                                                              uint16_t* out) {
    for (long i = static_cast<long>(blockIdx.x) * 256 + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * 256)
        out[i] = BF16::from_float(normal_at(seed, static_cast<uint64_t>(i)) * std_);
}

// ---- host side ------------------------------------------------------------------------

bool aligned_to(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

template <class T>
T* dev_alloc(size_t n, std::vector<void*>& owned) {
    void* p = nullptr;
    if (hipMalloc(&p, n * sizeof(T) < 16 ? 16 : n * sizeof(T)) != hipSuccess) return nullptr;
    owned.push_back(p);
    return static_cast<T*>(p);
}

// Buffers of the batched prefill (chunk tokens per pass).
struct PrefillBufs {
    int8_t* x = nullptr;     // [chunk][max cols] int8 activations
    float* amax = nullptr;   // [chunk]
    int32_t* y[3] = {nullptr, nullptr, nullptr};  // [chunk][max rows] GEMM outputs
    uint16_t *qkv = nullptr, *o = nullptr, *r = nullptr, *r2 = nullptr, *gu = nullptr;
    float *pm = nullptr, *pl = nullptr, *pacc = nullptr;
    float* comb = nullptr;      // [chunk][nh * hd] combined attention outputs
    EngineState* st = nullptr;  // [chunk] one decode-state record per token
    int chunk = 0;  // tokens per prefill pass
    // per-token capacities of x, y[0] and y[1..2] (a group's rows of x and y
    // start at its first token * these when a batch's tokens are split into
    // groups)
    long xrow = 0, yrow0 = 0, yrow = 0;
};

// The batched prefill's buffers: up to kPrefillChunk tokens per pass, fewer
// when the split partials of a pass would exceed kPrefillPartialBytes; or,
// with tokens > 0, exactly that many (the batched decode step's buffers).
bool alloc_prefill(PrefillBufs& pf, const spb_model_config& cfg, int S, std::vector<void*>& own,
                   int tokens = 0) {
    const int H = cfg.hidden_size, nh = cfg.num_attention_heads, hd = cfg.head_dim;
    const int I = cfg.intermediate_size, kvdim = cfg.num_key_value_heads * hd;
    const long part = static_cast<long>(nh) * S * (hd + 2) * 4;  // bytes per token
    long c = kPrefillPartialBytes / part;
    c = c < kPrefillChunk ? c : kPrefillChunk;
    if (tokens > 0) c = tokens;
    pf.chunk = static_cast<int>(c > 0 ? c : 1);
    const size_t C = static_cast<size_t>(pf.chunk);
    const size_t xmax = static_cast<size_t>(std::max(std::max(H, I), nh * hd));
    // y[0] also holds the stacked q|k|v and gate|up products
    const size_t ymax = static_cast<size_t>(std::max(std::max(nh * hd, kvdim), std::max(H, I)));
    const size_t ystack = std::max(ymax, static_cast<size_t>(std::max(nh * hd + 2 * kvdim, 2 * I)));
    pf.xrow = static_cast<long>(xmax);
    pf.yrow0 = static_cast<long>(ystack);
    pf.yrow = static_cast<long>(ymax);
    return (pf.x = dev_alloc<int8_t>(C * xmax, own)) && (pf.amax = dev_alloc<float>(C, own)) &&
           (pf.y[0] = dev_alloc<int32_t>(C * ystack, own)) &&
           (pf.y[1] = dev_alloc<int32_t>(C * ymax, own)) &&
           (pf.y[2] = dev_alloc<int32_t>(C * ymax, own)) &&
           (pf.qkv = dev_alloc<uint16_t>(C * (nh * hd + 2 * kvdim), own)) &&
           (pf.o = dev_alloc<uint16_t>(C * H, own)) && (pf.r = dev_alloc<uint16_t>(C * H, own)) &&
           (pf.r2 = dev_alloc<uint16_t>(C * H, own)) &&
           (pf.gu = dev_alloc<uint16_t>(C * 2 * I, own)) &&
           (pf.pm = dev_alloc<float>(C * nh * S, own)) &&
           (pf.pl = dev_alloc<float>(C * nh * S, own)) &&
           (pf.pacc = dev_alloc<float>(C * nh * S * hd, own)) &&
           (pf.comb = dev_alloc<float>(C * nh * hd, own)) &&
           (pf.st = dev_alloc<EngineState>(C, own));
}

SegWeights seg_weights(const spb_sparse_linear* a, const spb_sparse_linear* b,
                       const spb_sparse_linear* c) {
    const spb_sparse_linear* L2 = c ? c : b;
    SegWeights w{};
    w.meta = a->meta;
    w.values = a->values;
    w.dm1 = b->meta - a->meta;
    w.dm2 = L2->meta - b->meta;
    w.dv1 = b->values - a->values;
    w.dv2 = L2->values - b->values;
    w.ms = a->meta_stride;
    w.vs = a->values_stride;
    w.dms1 = b->meta_stride - a->meta_stride;
    w.dms2 = L2->meta_stride - b->meta_stride;
    w.dvs1 = b->values_stride - a->values_stride;
    w.dvs2 = L2->values_stride - b->values_stride;
    w.end0 = a->rows;
    w.rows = a->rows + b->rows + (c ? c->rows : 0);
    w.end1 = c ? a->rows + b->rows : w.rows;
    w.cols = a->cols;
    return w;
}

Weights single_weights(const spb_sparse_linear& l) {
    return Weights{l.meta, l.values, l.rows, l.cols, l.meta_stride, l.values_stride};
}

}  // namespace
}  // namespace spb

using namespace spb;

// attention_kernel<HD, G> for head_dim 64 / 128 and GQA groups 1, 2, 4, 8
// (checked at engine creation).
template <int HD>
void launch_attention_hd(int G, dim3 grid, hipStream_t s, const uint16_t* qkv,
                         const uint16_t* kc, const uint16_t* vc, float* pm, float* pl,
                         float* pacc, const EngineState* st, int max_seq, int S, float scale) {
    const dim3 block(kAttnThreads);
    // Short contexts (at most kFusedCombineSplits splits: a few blocks per kv
    // head) spread each group's q heads over several blocks, which all load
    // the split's K and V: at config 3 (G = 4) one head per block
    // 1,198.0-1,198.2 -> 1,209.1-1,209.3 tok/s, two per block 1,193.5-1,194.4
    // -> 1,202.2-1,202.5; with every split count, config 4 at bs=1 (36
    // splits) lost 2 % with two per block (1,040.4-1,040.7 against 1,062.4-
    // 1,063.2: the duplicated K and V loads).  G = 8 takes four per block.
    const bool split_heads = grid.x <= kFusedCombineSplits;
    switch (G) {
    case 1: hipLaunchKernelGGL((attention_kernel<HD, 1>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S, scale); break;
    case 2: hipLaunchKernelGGL((attention_kernel<HD, 2>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S, scale); break;
    case 4:
        if (split_heads) hipLaunchKernelGGL((attention_kernel<HD, 4, 1>), dim3(grid.x, grid.y, 4), block, 0, s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S, scale);
        else hipLaunchKernelGGL((attention_kernel<HD, 4>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S, scale);
        break;
    default:
        if (split_heads) hipLaunchKernelGGL((attention_kernel<HD, 8, 4>), dim3(grid.x, grid.y, 2), block, 0, s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S, scale);
        else hipLaunchKernelGGL((attention_kernel<HD, 8>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S, scale);
        break;
    }
}
// The prefill form: c tokens at positions pos0 .. pos0 + c - 1 (grid.z).
constexpr int kPrefillQueries = 16;  // tokens per block of the prefill attention

template <int HD>
void launch_attention_prefill_hd(int G, int sp, int nkv, int c, hipStream_t s,
                                 const uint16_t* qkv, const uint16_t* kc, const uint16_t* vc,
                                 float* pm, float* pl, float* pacc, int max_seq, int S,
                                 float scale, int pos0, int qkv_stride) {
    constexpr int Q = kPrefillQueries;
    const dim3 grid(sp, nkv, (c + Q - 1) / Q), block(kAttnThreads);
    switch (G) {
    case 1: hipLaunchKernelGGL((attention_prefill_kernel<HD, 1, Q>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, max_seq, S, scale, pos0, c, qkv_stride); break;
    case 2: hipLaunchKernelGGL((attention_prefill_kernel<HD, 2, Q>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, max_seq, S, scale, pos0, c, qkv_stride); break;
    case 4: hipLaunchKernelGGL((attention_prefill_kernel<HD, 4, Q>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, max_seq, S, scale, pos0, c, qkv_stride); break;
    default: hipLaunchKernelGGL((attention_prefill_kernel<HD, 8, Q>), grid, block, 0, s, qkv, kc, vc, pm, pl, pacc, max_seq, S, scale, pos0, c, qkv_stride); break;
    }
}

template <class P>
void launch_prefill_producer(const P& p, long stride, const EngineState* st, int cols, int c,
                             int8_t* xq, float* amax, hipStream_t s) {
    switch (p.units_per_thread()) {
    case 1:
        hipLaunchKernelGGL((prefill_producer_one_kernel<P, 1>), dim3(c), dim3(kBlock), 0, s, p,
                           stride, st, cols, xq, amax);
        return;
    case 2:
        hipLaunchKernelGGL((prefill_producer_one_kernel<P, 2>), dim3(c), dim3(kBlock), 0, s, p,
                           stride, st, cols, xq, amax);
        return;
    default: {
        const size_t lds = static_cast<size_t>(cols) * 4 * (1 + P::kAux) + 4 * 3 * kRedSlot;
        hipLaunchKernelGGL((prefill_producer_kernel<P>), dim3(c), dim3(kBlock), lds, s, p, stride,
                           st, cols, xq, amax);
    }
    }
}

template <class Sink>
void launch_prefill_sink(const Sink& sink, long stride, const float* amax, const int32_t* y0,
                         const int32_t* y1, const int32_t* y2, int end0, int end1, int rows,
                         int ld0, int ld1, int ld2, int c, hipStream_t s) {
    constexpr int R = SinkPairs<Sink>::value ? 2 * kBlock : kBlock;
    hipLaunchKernelGGL((prefill_sink_kernel<Sink>), dim3((rows + R - 1) / R, c), dim3(kBlock), 0, s,
                       sink, stride, amax, y0, y1, y2, end0, end1, rows, ld0, ld1, ld2);
}

// attn_combine_kernel for a token-step graph whose attention reaches
// `splits` splits: a load batch of the splits rounded up to a multiple of 4
// (at least 12), at most kCombineBatch.
template <int HD, int NB>
void launch_attn_combine_nb(int nh, hipStream_t s, const float* pm, const float* pl,
                            const float* pacc, float* comb, const EngineState* st, int S,
                            int B) {
    const size_t lds = 2 * static_cast<size_t>(S) * sizeof(float);
    hipLaunchKernelGGL((attn_combine_kernel<HD, NB>), dim3(nh, B), dim3(kWave), lds, s, pm, pl,
                       pacc, comb, st, S);
}
template <int HD>
void launch_attn_combine_hd(int nh, int splits, hipStream_t s, const float* pm, const float* pl,
                            const float* pacc, float* comb, const EngineState* st, int S, int B) {
#define SPB_COMBINE_NB(nb) launch_attn_combine_nb<HD, nb>(nh, s, pm, pl, pacc, comb, st, S, B); break
    switch ((splits + 3) / 4) {
    case 0: case 1: case 2: case 3: SPB_COMBINE_NB(12);
    case 4: SPB_COMBINE_NB(16);
    case 5: SPB_COMBINE_NB(20);
    case 6: SPB_COMBINE_NB(24);
    case 7: SPB_COMBINE_NB(28);
    case 8: SPB_COMBINE_NB(32);
    case 9: SPB_COMBINE_NB(36);
    case 10: SPB_COMBINE_NB(40);
    case 11: SPB_COMBINE_NB(44);
    case 12: SPB_COMBINE_NB(48);
    case 13: SPB_COMBINE_NB(52);
    case 14: SPB_COMBINE_NB(56);
    case 15: SPB_COMBINE_NB(60);
    default: SPB_COMBINE_NB(kCombineBatch);
    }
#undef SPB_COMBINE_NB
}
// B sequences: grid (nh, B), sequence b's state st + b, partials after
// those of b - 1, output comb + b * nh * hd.
void launch_attn_combine(int hd, int nh, int splits, hipStream_t s, const float* pm,
                         const float* pl, const float* pacc, float* comb, const EngineState* st,
                         int S, int B = 1) {
    if (hd == 64)
        launch_attn_combine_hd<64>(nh, splits, s, pm, pl, pacc, comb, st, S, B);
    else
        launch_attn_combine_hd<128>(nh, splits, s, pm, pl, pacc, comb, st, S, B);
}

// The first `splits` splits of S (the partials' stride stays S).
void launch_attention(int hd, int G, int S, int splits, int nkv, hipStream_t s,
                      const uint16_t* qkv, const uint16_t* kc, const uint16_t* vc, float* pm,
                      float* pl, float* pacc, const EngineState* st, int max_seq, float scale) {
    if (hd == 64)
        launch_attention_hd<64>(G, dim3(splits, nkv), s, qkv, kc, vc, pm, pl, pacc, st, max_seq, S,
                                scale);
    else
        launch_attention_hd<128>(G, dim3(splits, nkv), s, qkv, kc, vc, pm, pl, pacc, st, max_seq,
                                 S, scale);
}

// A projection of the decode step: the span kernel (every weight load issued
// before the prologue) when each CU's share fits its few steps, else the
// tiled kernel.
template <class W, class Act, class Sink>
void launch_gemv(const W& wt, Act act, Sink sink, hipStream_t s) {
    if (!launch_span(wt, act, sink, s)) launch_bitplane(wt, act, sink, s);
}
// The prologue in its one-pass form (one or two units per thread) when the
// vector fits one pass.
template <class W, class P, class Sink>
void launch_projection(const W& wt, const P& p, const EngineState* st, Sink sink, hipStream_t s) {
    switch (p.units_per_thread()) {
    case 1: launch_gemv(wt, ProducerPlanes<P, 1>{p, st, 0.f}, sink, s); break;
    case 2: launch_gemv(wt, ProducerPlanes<P, 2>{p, st, 0.f}, sink, s); break;
    default: launch_gemv(wt, ProducerPlanes<P, 0>{p, st, 0.f}, sink, s); break;
    }
}


// What a prefill pass reads of the model and the sequence it fills: every
// layer's KV cache at kcache[l] + kv_off, the sequence's token buffer.
struct PrefillTarget {
    const spb_model_config* cfg;
    const std::vector<spb_transformer_layer>* layers;
    const uint16_t* embed;
    const float2* rope;
    int max_seq, S;
    const std::vector<uint16_t*>* kcache;
    const std::vector<uint16_t*>* vcache;
    long kv_off;
    const int* tokens;
};

// The int32 products of up to three projections of the same int8 input X
// ([n][cols]): one stacked matrix-core launch when gemm_stacked takes them
// (equal columns and strides), else one launch each into y[0..nw).  out[i]
// and ld[i]: where projection i's rows are and their row stride.
hipError_t gemm_group(const spb_sparse_linear* const* w, int nw, const int8_t* X,
                      int32_t* const* y, int n, hipStream_t s, const int32_t** out, int* ld) {
    if (gemm_stacked(w, nw, X, y[0], n, s) == 0) {
        int rows = 0;
        for (int i = 0; i < nw; ++i) rows += w[i]->rows;
        int off = 0;
        for (int i = 0; i < 3; ++i) {
            const int k = i < nw ? i : nw - 1;
            out[i] = y[0] + (i < nw ? off : off - w[k]->rows);
            ld[i] = rows;
            if (i < nw) off += w[i]->rows;
        }
        return hipSuccess;
    }
    for (int i = 0; i < 3; ++i) {
        const int k = i < nw ? i : nw - 1;
        if (i < nw && spb_sparse_ternary_gemm(w[i]->meta, w[i]->values, X, y[i], w[i]->rows,
                                              w[i]->cols, n, w[i]->meta_stride,
                                              w[i]->values_stride, s))
            return hipErrorLaunchFailure;
        out[i] = y[k];
        ld[i] = w[k]->rows;
    }
    return hipSuccess;
}

// Sinks fused into the GEMM at every batch size; the q/k/v sink only up to
// kFuseTokens tokens: in a 1024-token prefill pass its epilogue (decode
// state and RoPE row loads per lane, pair stores to the KV cache) made the
// GEMM longer than GEMM + sink kernel (33.8 against 20.7 + 10.1 us), while
// the bf16 and residual sinks gained (gate|up 69.4 against 61.1 + 28.0 us,
// down 40.1 against 36.3 + 7.6 us).
template <class Sink>
struct SinkFusesWide {
    static constexpr bool value = true;
};
template <>
struct SinkFusesWide<QkvRopeSink> {
    static constexpr bool value = false;
};
constexpr int kFuseTokens = 64;

// The products of up to three stacked projections of the int8 tokens X
// ([n][cols], absmax amax[t]) through a per-token sink (output stride
// `stride`): one staged GEMM launch with the sink as its epilogue when
// gemm_stacked_epi takes the shapes (and the sink fuses at n tokens), else
// the int32 products into y (one launch per projection when they cannot be
// stacked) and prefill_sink_kernel.
template <class Sink>
hipError_t gemm_sink(const spb_sparse_linear* const* w, int nw, const int8_t* X,
                     const float* amax, const Sink& sink, long stride, int32_t* const* y, int n,
                     hipStream_t s, const GemmSplit* split = nullptr) {
    int rows = 0;
    for (int i = 0; i < nw; ++i) rows += w[i]->rows;
    if (n <= kFuseTokens || SinkFusesWide<Sink>::value) {
        const int rc =
            gemm_stacked_epi(w, nw, X, SinkOut<Sink>{sink, stride, amax, rows}, n, s, split);
        if (rc == 0) return hipSuccess;
        if (rc == 2) return hipErrorLaunchFailure;
    }
    const int32_t* yy[3];
    int ld[3];
    if (gemm_group(w, nw, X, y, n, s, yy, ld) != hipSuccess) return hipErrorLaunchFailure;
    const int end0 = w[0]->rows, end1 = nw > 1 ? end0 + w[1]->rows : end0;
    launch_prefill_sink(sink, stride, amax, yy[0], yy[1], yy[2], end0, end1, rows, ld[0], ld[1],
                        ld[2], n, s);
    return hipSuccess;
}

// Raises the LDS limit of the sink-epilogue GEMM kernels (0 = done); at
// engine create, before any graph capture.
int gemm_sink_prepare() {
    return staged_prepare<SinkOut<QkvRopeSink>>() == 0 &&
                   staged_prepare<SinkOut<SegBf16Sink>>() == 0 &&
                   staged_prepare<SinkOut<ResidualSink>>() == 0
               ? 0
               : 1;
}

// Positions pos0 .. pos0 + c - 1 of one sequence (t.tokens holds their ids)
// through every layer, c <= pf.chunk: the KV cache of those positions as c
// decode steps would write it.  Returns a HIP error or hipSuccess.
hipError_t enqueue_prefill_pass(const PrefillTarget& t, const PrefillBufs& pf, int pos0, int c,
                            hipStream_t s) {
const spb_model_config& cfg = *t.cfg;
const std::vector<spb_transformer_layer>& layers = *t.layers;
const uint16_t* embed = t.embed;
const int* tokens = t.tokens;
const int max_seq = t.max_seq, S = t.S;
const float2* rope = t.rope;
auto kcache = [&](size_t l) { return (*t.kcache)[l] + t.kv_off; };
auto vcache = [&](size_t l) { return (*t.vcache)[l] + t.kv_off; };
    const int hd = cfg.head_dim, nh = cfg.num_attention_heads;
    const int nkv = cfg.num_key_value_heads, H = cfg.hidden_size;
    const int I = cfg.intermediate_size, kvdim = nkv * hd, qrows = nh * hd;
    const float eps = cfg.rms_norm_eps;
    const float scale = 1.0f / sqrtf(static_cast<float>(hd));
    std::vector<EngineState> hs(c);
    for (int t = 0; t < c; ++t) {
        hs[t] = EngineState{};
        hs[t].pos = pos0 + t;
        hs[t].prompt_len = max_seq;
        hs[t].limit = max_seq;
    }
    hipError_t err = hipMemcpyAsync(pf.st, hs.data(), sizeof(EngineState) * c,
                                    hipMemcpyHostToDevice, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);  // hs is on this frame
    if (err != hipSuccess) return err;
    for (size_t l = 0; l < layers.size(); ++l) {
        const spb_transformer_layer& L = layers[l];
        {
            InputNorm p{pf.r, l == 0 ? embed : nullptr, tokens, pf.r, L.input_layernorm, eps,
                        H};
            launch_prefill_producer(p, H, pf.st, H, c, pf.x, pf.amax, s);
        }
        const spb_sparse_linear* qkv3[3] = {&L.q_proj, &L.k_proj, &L.v_proj};
        {
            QkvRopeSink sink{};
            sink.out = pf.qkv;
            sink.kc = kcache(l);
            sink.vc = vcache(l);
            sink.st = pf.st;
            sink.g0 = L.q_proj.gamma;
            sink.g1 = L.k_proj.gamma;
            sink.g2 = L.v_proj.gamma;
            sink.end0 = qrows;
            sink.end1 = qrows + kvdim;
            sink.hd = hd;
            sink.hd_log2 = hd == 64 ? 6 : 7;
            sink.max_seq = max_seq;
            sink.rope_tab = rope;
            sink.rope_pos0 = pos0;
            if (gemm_sink(qkv3, 3, pf.x, pf.amax, sink, qrows + 2 * kvdim, pf.y, c, s) !=
                hipSuccess)
                return hipErrorLaunchFailure;
        }
        // splits that some token of the pass reaches
        const int sp = (pos0 + c - 1) / kAttnSplit + 1 < S ? (pos0 + c - 1) / kAttnSplit + 1 : S;
        if (hd == 64)
            launch_attention_prefill_hd<64>(nh / nkv, sp, nkv, c, s, pf.qkv, kcache(l),
                                            vcache(l), pf.pm, pf.pl, pf.pacc, max_seq, S,
                                            scale, pos0, qrows + 2 * kvdim);
        else
            launch_attention_prefill_hd<128>(nh / nkv, sp, nkv, c, s, pf.qkv, kcache(l),
                                             vcache(l), pf.pm, pf.pl, pf.pacc, max_seq, S,
                                             scale, pos0, qrows + 2 * kvdim);
        {  // the split combine over (head, token), then the o input per token
            launch_attn_combine(hd, nh, sp, s, pf.pm, pf.pl, pf.pacc, pf.comb, pf.st, S, c);
            CombinedAttn p{pf.comb, qrows};
            launch_prefill_producer(p, qrows, pf.st, qrows, c, pf.x, pf.amax, s);
        }
        {
            const spb_sparse_linear* o1[1] = {&L.o_proj};
            SegBf16Sink sink{pf.o, L.o_proj.gamma, L.o_proj.gamma, L.o_proj.gamma, H, H,
                             0.f, 0.f, 0.f};
            if (gemm_sink(o1, 1, pf.x, pf.amax, sink, H, pf.y, c, s) != hipSuccess)
                return hipErrorLaunchFailure;
        }
        {
            SubNormResidualNorm p{pf.o, pf.r, pf.r2, L.attn_sub_norm,
                                  L.post_attention_layernorm, eps, H};
            launch_prefill_producer(p, H, pf.st, H, c, pf.x, pf.amax, s);
        }
        {
            const spb_sparse_linear* gu2[2] = {&L.gate_proj, &L.up_proj};
            SegBf16Sink sink{pf.gu, L.gate_proj.gamma, L.up_proj.gamma, L.up_proj.gamma,
                             I, 2 * I, 0.f, 0.f, 0.f};
            if (gemm_sink(gu2, 2, pf.x, pf.amax, sink, 2 * I, pf.y, c, s) != hipSuccess)
                return hipErrorLaunchFailure;
        }
        {
            Relu2Norm p{pf.gu, pf.gu + I, L.ffn_sub_norm,
                        L.ffn_sub_norm ? L.ffn_sub_norm : reinterpret_cast<const float*>(pf.gu),
                        eps, I};
            launch_prefill_producer(p, 2 * I, pf.st, I, c, pf.x, pf.amax, s);
        }
        {
            const spb_sparse_linear* d1[1] = {&L.down_proj};
            ResidualSink sink{pf.r, pf.r2, L.down_proj.gamma, 0.f};
            if (gemm_sink(d1, 1, pf.x, pf.amax, sink, H, pf.y, c, s) != hipSuccess)
                return hipErrorLaunchFailure;
        }
    }
    return hipGetLastError();
}

struct spb_engine {
    spb_model_config cfg{};
    std::vector<spb_transformer_layer> layers;
    const uint16_t* embed = nullptr;
    const uint16_t* lm_head = nullptr;
    const float* final_norm = nullptr;
    int max_seq = 0;
    int S = 0;  // attention splits
    int lm_grid = 0;
    LmKernel lm_kernel = nullptr;
    std::vector<void*> owned;
    std::vector<uint16_t*> kcache, vcache;
    uint16_t *xa = nullptr, *xb = nullptr, *qkv = nullptr, *obuf = nullptr, *gu = nullptr;
    float *pm = nullptr, *pl = nullptr, *pacc = nullptr, *logits = nullptr, *part_v = nullptr;
    float* comb = nullptr;  // combined attention output (steps past kFusedCombineSplits splits)
    int* part_i = nullptr;
    int* tokens = nullptr;
    float2* rope = nullptr;
    float2* cur_rope = nullptr;  // RoPE row of the decode position
    EngineState* st = nullptr;
    hipStream_t stream = nullptr;      // where graphs are launched (null = legacy stream)
    hipStream_t cap_stream = nullptr;  // capture stream
    // One token-step graph per bucket of positions: graph k launches the
    // attention kernel on the splits of positions below (k + 1) * bucket_pos
    // only (the blocks of splits past the position would load their K and V
    // for nothing).  The host replays the graph of pos_hint, an upper bound
    // of the device position (the device advances at most one position per
    // step; a done state stops it), so the grid always covers the position.
    std::vector<hipGraph_t> graphs;
    std::vector<hipGraphExec_t> execs;
    int bucket_pos = 0;  // positions per bucket (a multiple of the split)
    int pos_hint = 0;
    int seq_len = 0;
    // The device state is in generate mode (prompt_len, stop_eos, done as
    // spb_engine_generate left them) or advanced by spb_engine_decode_steps
    // without the host knowing its position: spb_engine_forward first reads
    // the position back and re-arms forward mode.
    bool device_mode = false;
    bool pos_stale = false;
    // batched prefill: prompts with at least prefill_min tokens before the
    // last go through the layers pf.chunk tokens at a time (0: never)
    int prefill_min = kPrefillMinDefault;
    PrefillBufs pf;

    ~spb_engine() {
        for (hipGraphExec_t x : execs) (void)hipGraphExecDestroy(x);
        for (hipGraph_t g : graphs) (void)hipGraphDestroy(g);
        if (cap_stream) (void)hipStreamDestroy(cap_stream);
        for (void* p : owned) (void)hipFree(p);
    }

    // Replays the token-step graph for the position bound pos_hint, then
    // advances the bound.
    hipError_t launch_step() {
        int k = pos_hint / bucket_pos;
        k = k < static_cast<int>(execs.size()) ? k : static_cast<int>(execs.size()) - 1;
        const hipError_t err = hipGraphLaunch(execs[k], stream);
        pos_hint = pos_hint < max_seq ? pos_hint + 1 : max_seq;
        return err;
    }

    // The kernels of one token step, in order, on stream s; the attention
    // kernel runs on the first `splits` splits (positions below 64 * splits).
    void enqueue_step(hipStream_t s, int splits) const {
        const int hd = cfg.head_dim, nh = cfg.num_attention_heads;
        const int nkv = cfg.num_key_value_heads;
        const float eps = cfg.rms_norm_eps;
        const float scale = 1.0f / sqrtf(static_cast<float>(hd));  // inference.cu:182
        for (size_t l = 0; l < layers.size(); ++l) {
            const spb_transformer_layer& L = layers[l];
            {
                InputNorm p{xa, l == 0 ? embed : nullptr, tokens, xa, L.input_layernorm, eps,
                            cfg.hidden_size};
                QkvRopeSink sink{};
                sink.out = qkv;
                sink.kc = kcache[l];
                sink.vc = vcache[l];
                sink.cur_rope = cur_rope;
                sink.st = st;
                sink.g0 = L.q_proj.gamma;
                sink.g1 = L.k_proj.gamma;
                sink.g2 = L.v_proj.gamma;
                sink.end0 = L.q_proj.rows;
                sink.end1 = L.q_proj.rows + L.k_proj.rows;
                sink.hd = hd;
                sink.hd_log2 = hd == 64 ? 6 : 7;
                sink.max_seq = max_seq;
                launch_projection(seg_weights(&L.q_proj, &L.k_proj, &L.v_proj),
                                p, st, sink, s);
            }
            launch_attention(hd, nh / nkv, S, splits, nkv, s, qkv, kcache[l], vcache[l], pm, pl,
                             pacc, st, max_seq, scale);
            {
                static_assert(kAttnSplit == 64, "the combine's split index is pos >> 6");
                SegBf16Sink sink{obuf, L.o_proj.gamma, L.o_proj.gamma, L.o_proj.gamma,
                                 L.o_proj.rows, L.o_proj.rows, 0.f, 0.f, 0.f};
                if (splits <= kFusedCombineSplits) {
                    // every block of the o projection folds the splits itself
                    AttnCombine p{pm, pl, pacc, hd, S, nh * hd, hd == 64 ? 6 : 7};
                    launch_projection(single_weights(L.o_proj), p, st, sink, s);
                } else {
                    // long contexts: fold once per head, then read the result
                    launch_attn_combine(hd, nh, splits, s, pm, pl, pacc, comb, st, S);
                    CombinedAttn p{comb, nh * hd};
                    launch_projection(single_weights(L.o_proj), p, st, sink, s);
                }
            }
            {
                SubNormResidualNorm p{obuf, xa, xb, L.attn_sub_norm, L.post_attention_layernorm,
                                      eps, cfg.hidden_size};
                SegBf16Sink sink{gu, L.gate_proj.gamma, L.up_proj.gamma, L.up_proj.gamma,
                                 L.gate_proj.rows, L.gate_proj.rows + L.up_proj.rows, 0.f, 0.f,
                                 0.f};
                launch_projection(seg_weights(&L.gate_proj, &L.up_proj, nullptr),
                                p, st, sink, s);
            }
            {
                const int I = cfg.intermediate_size;
                // without the sub-norm, the held-weight loads read gu (2I bf16 = I floats)
                Relu2Norm p{gu, gu + I, L.ffn_sub_norm,
                            L.ffn_sub_norm ? L.ffn_sub_norm : reinterpret_cast<const float*>(gu),
                            eps, I};
                ResidualSink sink{xa, xb, L.down_proj.gamma, 0.f};
                launch_projection(single_weights(L.down_proj), p, st, sink, s);
            }
        }
        hipLaunchKernelGGL(lm_kernel, dim3(lm_grid), dim3(kLmBlock), 0, s, lm_head, xa,
                           final_norm, eps, logits, part_v, part_i, st, tokens,
                           cfg.vocab_size, cfg.hidden_size, rope, cur_rope, hd / 2, max_seq,
                           cfg.vocab_size / lm_grid, cfg.vocab_size % lm_grid);
    }

    // Positions pos0 .. pos0 + c - 1 (tokens[] holds their ids) through every
    // layer, c <= pf.chunk: the KV cache of those positions as c decode
    // steps would write it.  Returns a HIP error or hipSuccess.
    hipError_t enqueue_prefill(int pos0, int c, hipStream_t s) {
        const PrefillTarget t{&cfg, &layers, embed, rope, max_seq, S, &kcache, &vcache, 0, tokens};
        return enqueue_prefill_pass(t, pf, pos0, c, s);
    }
};

namespace {

int check_linear(const char* fn, const char* name, const spb_sparse_linear& l, int rows,
                 int cols) {
    if (l.rows != rows || l.cols != cols)
        return invalid("%s: %s is %dx%d, expected %dx%d", fn, name, l.rows, l.cols, rows, cols);
    if (!l.meta || !l.values) return invalid("%s: %s has null weights", fn, name);
    // strides must cover a row (the projection kernels read whole rows)
    char where[128];
    snprintf(where, sizeof(where), "%s: %s", fn, name);
    if (int rc = check_weights(where, l.meta, l.values, l.rows, l.cols, l.meta_stride,
                               l.values_stride))
        return rc;
    if (!bitplane_ok(l.meta, l.values, l.cols, l.meta_stride, l.values_stride))
        return invalid("%s: %s must have cols %% 128 == 0, cols <= %d, meta_stride %% 4 == 0, "
                       "values_stride %% 2 == 0 and 16/8-byte aligned meta/values",
                       fn, name, kMaxPlaneCols);
    return 0;
}

// The model shapes both engines take (every projection on the bit-plane
// kernel, head_dim 64 or 128, GQA groups 1/2/4/8, H <= kLmMaxH).
int check_model(const char* fn, const spb_model_config* cfg, const spb_transformer_layer* layers,
                const uint16_t* embed_tokens, const uint16_t* lm_head, int max_seq) {
    const int H = cfg->hidden_size, nh = cfg->num_attention_heads, nkv = cfg->num_key_value_heads;
    const int hd = cfg->head_dim, I = cfg->intermediate_size, V = cfg->vocab_size;
    if (cfg->num_hidden_layers <= 0 || H <= 0 || nh <= 0 || nkv <= 0 || hd <= 0 || I <= 0 ||
        V <= 0)
        return invalid("%s: non-positive model dimension", fn);
    if (nh * hd != H) return invalid("%s: num_attention_heads * head_dim != hidden_size", fn);
    if (nh % nkv || (nh / nkv) & (nh / nkv - 1) || nh / nkv > kAttnMaxGroup)
        return invalid("%s: heads per kv head must divide evenly and be 1, 2, 4 or %d", fn,
                       kAttnMaxGroup);
    if (hd != 64 && hd != 128) return invalid("%s: head_dim must be 64 or 128", fn);
    if (H > kLmMaxH || H % 8) return invalid("%s: hidden_size must be a multiple of 8, <= %d", fn,
                                             kLmMaxH);
    if (max_seq <= 0 || max_seq > cfg->max_position_embeddings)
        return invalid("%s: max_seq must be in [1, max_position_embeddings]", fn);
    if (!aligned_to(embed_tokens, 16) || (lm_head && !aligned_to(lm_head, 16)))
        return invalid("%s: embedding / lm_head must be 16-byte aligned", fn);
    const int kvdim = nkv * hd;
    for (int l = 0; l < cfg->num_hidden_layers; ++l) {
        const spb_transformer_layer& L = layers[l];
        int rc = 0;
        if ((rc = check_linear(fn, "q_proj", L.q_proj, H, H)) ||
            (rc = check_linear(fn, "k_proj", L.k_proj, kvdim, H)) ||
            (rc = check_linear(fn, "v_proj", L.v_proj, kvdim, H)) ||
            (rc = check_linear(fn, "o_proj", L.o_proj, H, H)) ||
            (rc = check_linear(fn, "gate_proj", L.gate_proj, I, H)) ||
            (rc = check_linear(fn, "up_proj", L.up_proj, I, H)) ||
            (rc = check_linear(fn, "down_proj", L.down_proj, H, I)))
            return rc;
        if (!L.input_layernorm || !L.post_attention_layernorm)
            return invalid("%s: layer %d lacks its RMSNorm weights", fn, l);
    }
    return 0;
}

// RoPE table (inference_kernels.cu:195-198): freq_i = 1 / theta^(2i/hd) in
// float32, angle = float(pos) * freq_i, cos/sin evaluated in double.
std::vector<float2> rope_table(const spb_model_config& cfg, int max_seq) {
    const int hd = cfg.head_dim;
    std::vector<float2> rope(static_cast<size_t>(max_seq) * (hd / 2));
    for (int p = 0; p < max_seq; ++p)
        for (int i = 0; i < hd / 2; ++i) {
            const float freq = 1.0f / powf(cfg.rope_theta,
                                           static_cast<float>(2 * i) / static_cast<float>(hd));
            const float angle = static_cast<float>(p) * freq;
            rope[static_cast<size_t>(p) * (hd / 2) + i] =
                make_float2(static_cast<float>(cos(static_cast<double>(angle))),
                            static_cast<float>(sin(static_cast<double>(angle))));
        }
    return rope;
}

int set_state(spb_engine* e, int pos, int prompt_len, int stop_eos) {
    EngineState h{};
    h.pos = pos;
    h.prompt_len = prompt_len;
    h.limit = e->max_seq;
    h.done = 0;
    h.stop_eos = stop_eos;
    h.eos = e->cfg.eos_token_id;
    h.ticket = 0u;
    h.generated = 0;
    // Synchronous with respect to the host: h lives on this stack frame.
    const int half = e->cfg.head_dim / 2;
    const int rp = pos < e->max_seq ? pos : e->max_seq - 1;
    e->pos_hint = pos;
    if (hipMemcpyAsync(e->st, &h, sizeof(h), hipMemcpyHostToDevice, e->stream) != hipSuccess ||
        hipMemcpyAsync(e->cur_rope, e->rope + static_cast<long>(rp) * half,
                       sizeof(float2) * half, hipMemcpyDeviceToDevice, e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return launch_status("spb_engine: state upload");
    return 0;
}

// Reads the device position back after spb_engine_decode_steps (host sync).
int sync_seq_len(spb_engine* e, const char* fn) {
    if (!e->pos_stale) return 0;
    EngineState h{};
    if (hipMemcpyAsync(&h, e->st, sizeof(h), hipMemcpyDeviceToHost, e->stream) != hipSuccess ||
        hipStreamSynchronize(e->stream) != hipSuccess)
        return launch_status(fn);
    e->seq_len = h.pos < e->max_seq ? h.pos : e->max_seq;
    e->pos_stale = false;
    return 0;
}

}  // namespace

extern "C" int spb_engine_create(const spb_model_config* cfg, const spb_transformer_layer* layers,
                                 const uint16_t* embed_tokens, const uint16_t* lm_head,
                                 const float* final_norm, int max_seq, spb_engine** out) {
    clear_error();
    const char* fn = "spb_engine_create";
    if (!cfg || !layers || !embed_tokens || !final_norm || !out)
        return invalid("%s: null argument", fn);
    *out = nullptr;
    if (int rc = check_model(fn, cfg, layers, embed_tokens, lm_head, max_seq)) return rc;
    if (gemm_prepare() != 0 || gemm_sink_prepare() != 0)  // before any graph capture
        return launch_status(fn);
    const int H = cfg->hidden_size, nh = cfg->num_attention_heads, nkv = cfg->num_key_value_heads;
    const int hd = cfg->head_dim, I = cfg->intermediate_size, V = cfg->vocab_size;
    const int kvdim = nkv * hd;
    spb_engine* e = new (std::nothrow) spb_engine();
    if (!e) return invalid("%s: out of host memory", fn);
    e->cfg = *cfg;
    e->layers.assign(layers, layers + cfg->num_hidden_layers);
    e->embed = embed_tokens;
    e->lm_head = lm_head ? lm_head : embed_tokens;  // tied weights (model.h:131-133)
    e->final_norm = final_norm;
    e->max_seq = max_seq;
    e->S = (max_seq + kAttnSplit - 1) / kAttnSplit;
    e->lm_kernel = lm_head_for(H);
    // One block per CU: every block streams a contiguous range of rows.  On
    // MI355X, with non-temporal weight loads in the projections and here,
    // decode ran 1090 / 1075 / 1061 tok/s with one / two / three 4-wave LM-head
    // blocks per CU.  At least V / 2048 blocks (the logits of a block are
    // staged in LDS).
    const long lm_need = (static_cast<long>(V) + kLmBlock / kWave - 1) / (kLmBlock / kWave);
    const long lm_min = (static_cast<long>(V) + kLmMaxRows - 1) / kLmMaxRows;
    long lm_grid = device_cu_count();
    if (lm_grid > lm_need) lm_grid = lm_need;
    e->lm_grid = static_cast<int>(lm_grid > lm_min ? lm_grid : lm_min);

    auto& own = e->owned;
    const size_t kv = static_cast<size_t>(nkv) * max_seq * hd;
    bool ok = true;
    for (int l = 0; l < cfg->num_hidden_layers && ok; ++l) {
        e->kcache.push_back(dev_alloc<uint16_t>(kv, own));
        e->vcache.push_back(dev_alloc<uint16_t>(kv, own));
        ok = e->kcache.back() && e->vcache.back();
    }
    ok = ok && (e->xa = dev_alloc<uint16_t>(H, own)) && (e->xb = dev_alloc<uint16_t>(H, own)) &&
         (e->qkv = dev_alloc<uint16_t>(H + 2 * kvdim, own)) &&
         (e->obuf = dev_alloc<uint16_t>(H, own)) && (e->gu = dev_alloc<uint16_t>(2 * I, own)) &&
         (e->pm = dev_alloc<float>(static_cast<size_t>(nh) * e->S, own)) &&
         (e->pl = dev_alloc<float>(static_cast<size_t>(nh) * e->S, own)) &&
         (e->pacc = dev_alloc<float>(static_cast<size_t>(nh) * e->S * hd, own)) &&
         (e->comb = dev_alloc<float>(static_cast<size_t>(nh) * hd, own)) &&
         (e->logits = dev_alloc<float>(V, own)) &&
         (e->part_v = dev_alloc<float>(e->lm_grid, own)) &&
         (e->part_i = dev_alloc<int>(e->lm_grid, own)) &&
         (e->tokens = dev_alloc<int>(max_seq + 1, own)) &&
         (e->rope = dev_alloc<float2>(static_cast<size_t>(max_seq) * (hd / 2), own)) &&
         (e->cur_rope = dev_alloc<float2>(hd / 2, own)) &&
         (e->st = dev_alloc<EngineState>(1, own));
    ok = ok && alloc_prefill(e->pf, *cfg, e->S, own);
    if (!ok) {
        delete e;
        return invalid("%s: device allocation failed", fn);
    }
    const std::vector<float2> rope = rope_table(*cfg, max_seq);
    hipError_t err = hipMemcpy(e->rope, rope.data(), rope.size() * sizeof(float2),
                               hipMemcpyHostToDevice);
    for (size_t l = 0; l < e->kcache.size() && err == hipSuccess; ++l) {
        err = hipMemset(e->kcache[l], 0, kv * 2);
        if (err == hipSuccess) err = hipMemset(e->vcache[l], 0, kv * 2);
    }
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&e->cap_stream, hipStreamNonBlocking);
    if (err != hipSuccess) {
        delete e;
        return launch_status(fn);
    }
    // Capture the token step once per position bucket: buckets of 4 splits
    // (256 positions; at most 16 graphs), or of S/8 splits past 64 splits
    // (at most 8 graphs).
    {
        const int per = e->S <= 64 ? kAttnBucketSplits : (e->S + 7) / 8;
        e->bucket_pos = per * kAttnSplit;
        for (int s0 = 0; s0 < e->S && err == hipSuccess; s0 += per) {
            const int splits = s0 + per < e->S ? s0 + per : e->S;
            hipGraph_t g = nullptr;
            hipGraphExec_t x = nullptr;
            err = hipStreamBeginCapture(e->cap_stream, hipStreamCaptureModeThreadLocal);
            if (err == hipSuccess) {
                e->enqueue_step(e->cap_stream, splits);
                err = hipStreamEndCapture(e->cap_stream, &g);
            }
            if (err == hipSuccess) {
                e->graphs.push_back(g);
                err = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
            }
            if (err == hipSuccess) e->execs.push_back(x);
        }
    }
    if (err != hipSuccess) {
        set_error("%s: graph capture failed: %s", fn, hipGetErrorString(err));
        delete e;
        return static_cast<int>(err);
    }
    if (int rc = set_state(e, 0, 0x7FFFFFFF, 0)) {
        delete e;
        return rc;
    }
    *out = e;
    return 0;
}

extern "C" int spb_engine_destroy(spb_engine* e) {
    clear_error();
    if (e) {
        (void)hipStreamSynchronize(e->stream);
        delete e;
    }
    return 0;
}

extern "C" int spb_engine_set_stream(spb_engine* e, spb_stream_t stream) {
    clear_error();
    if (!e) return invalid("spb_engine_set_stream: null engine");
    e->stream = as_stream(stream);
    return 0;
}

extern "C" int spb_engine_reset(spb_engine* e) {
    clear_error();
    if (!e) return invalid("spb_engine_reset: null engine");
    e->seq_len = 0;
    const size_t kv = static_cast<size_t>(e->cfg.num_key_value_heads) * e->max_seq *
                      e->cfg.head_dim * 2;
    for (size_t l = 0; l < e->kcache.size(); ++l) {
        if (hipMemsetAsync(e->kcache[l], 0, kv, e->stream) != hipSuccess ||
            hipMemsetAsync(e->vcache[l], 0, kv, e->stream) != hipSuccess)
            return launch_status("spb_engine_reset");
    }
    e->device_mode = false;
    e->pos_stale = false;
    return set_state(e, 0, 0x7FFFFFFF, 0);
}

extern "C" int spb_engine_seq_len(const spb_engine* e) {
    if (!e) return -1;
    if (e->pos_stale && sync_seq_len(const_cast<spb_engine*>(e), "spb_engine_seq_len")) return -1;
    return e->seq_len;
}

extern "C" int spb_engine_forward(spb_engine* e, int token_id, const float** d_logits) {
    clear_error();
    const char* fn = "spb_engine_forward";
    if (!e) return invalid("%s: null engine", fn);
    if (token_id < 0 || token_id >= e->cfg.vocab_size)
        return invalid("%s: token %d outside [0, %d)", fn, token_id, e->cfg.vocab_size);
    if (e->device_mode || e->pos_stale) {
        // after generate / decode_steps: continue at the device position in
        // forward mode (no EOS stop, no token writes, done cleared)
        if (int rc = sync_seq_len(e, fn)) return rc;
        if (int rc = set_state(e, e->seq_len, 0x7FFFFFFF, 0)) return rc;
        e->device_mode = false;
    }
    if (e->seq_len >= e->max_seq) return invalid("%s: sequence is full (%d)", fn, e->max_seq);
    const int pos = e->seq_len;
    if (hipMemcpyAsync(e->tokens + pos, &token_id, sizeof(int), hipMemcpyHostToDevice,
                       e->stream) != hipSuccess)
        return launch_status(fn);
    // The host copy above is pageable: wait until it has been consumed.
    if (hipStreamSynchronize(e->stream) != hipSuccess) return launch_status(fn);
    e->pos_hint = pos;
    if (e->launch_step() != hipSuccess) return launch_status(fn);
    e->seq_len = pos + 1;
    if (d_logits) *d_logits = e->logits;
    return 0;
}

extern "C" int spb_engine_generate(spb_engine* e, const int* prompt, int n_prompt, int n_new,
                                   int stop_at_eos, int* out_tokens, int* n_generated) {
    clear_error();
    const char* fn = "spb_engine_generate";
    if (!e || !prompt || (!out_tokens && n_new > 0)) return invalid("%s: null argument", fn);
    if (n_prompt <= 0 || n_new < 0) return invalid("%s: need n_prompt >= 1, n_new >= 0", fn);
    if (static_cast<long>(n_prompt) + n_new > e->max_seq)
        return invalid("%s: prompt + new tokens (%d) exceed max_seq %d", fn, n_prompt + n_new,
                       e->max_seq);
    for (int i = 0; i < n_prompt; ++i)
        if (prompt[i] < 0 || prompt[i] >= e->cfg.vocab_size)
            return invalid("%s: prompt token %d outside [0, %d)", fn, prompt[i],
                           e->cfg.vocab_size);
    if (int rc = spb_engine_reset(e)) return rc;
    if (hipMemcpyAsync(e->tokens, prompt, sizeof(int) * n_prompt, hipMemcpyHostToDevice,
                       e->stream) != hipSuccess)
        return launch_status(fn);
    if (int rc = set_state(e, 0, n_prompt, stop_at_eos ? 1 : 0)) return rc;
    // Positions 0 .. n_prompt-2 prefill (in batches through the layers when
    // there are at least prefill_min of them, else one decode step each);
    // step n_prompt-1+t produces token t.
    int start = 0;
    const int pre = n_prompt - 1;
    if (e->prefill_min > 0 && pre >= e->prefill_min) {
        for (int p0 = 0; p0 < pre; p0 += e->pf.chunk) {
            const int c = pre - p0 < e->pf.chunk ? pre - p0 : e->pf.chunk;
            if (e->enqueue_prefill(p0, c, e->stream) != hipSuccess) return launch_status(fn);
        }
        if (int rc = set_state(e, pre, n_prompt, stop_at_eos ? 1 : 0)) return rc;
        start = pre;
    }
    const int steps = n_prompt - 1 - start + n_new;
    for (int i = 0; i < steps; ++i)
        if (e->launch_step() != hipSuccess) return launch_status(fn);
    EngineState h{};
    if (hipMemcpyAsync(&h, e->st, sizeof(h), hipMemcpyDeviceToHost, e->stream) != hipSuccess)
        return launch_status(fn);
    if (hipStreamSynchronize(e->stream) != hipSuccess) return launch_status(fn);
    const int got = h.generated < n_new ? h.generated : n_new;
    if (got > 0 && hipMemcpy(out_tokens, e->tokens + n_prompt, sizeof(int) * got,
                             hipMemcpyDeviceToHost) != hipSuccess)
        return launch_status(fn);
    if (n_generated) *n_generated = got;
    e->seq_len = h.pos < e->max_seq ? h.pos : e->max_seq;
    e->device_mode = true;
    e->pos_stale = false;
    return 0;
}

extern "C" int spb_engine_set_prefill_batch(spb_engine* e, int min_tokens) {
    clear_error();
    if (!e) return invalid("spb_engine_set_prefill_batch: null engine");
    if (min_tokens < 0) return invalid("spb_engine_set_prefill_batch: min_tokens < 0");
    e->prefill_min = min_tokens;
    return 0;
}

extern "C" int spb_engine_decode_steps(spb_engine* e, int steps) {
    clear_error();
    if (!e) return invalid("spb_engine_decode_steps: null engine");
    if (steps < 0) return invalid("spb_engine_decode_steps: steps < 0");
    for (int i = 0; i < steps; ++i)
        if (e->launch_step() != hipSuccess) return launch_status("spb_engine_decode_steps");
    // the device advanced pos (unless the state is done): seq_len and forward
    // read it back when next asked
    if (steps > 0) e->pos_stale = true;
    return 0;
}

extern "C" int spb_engine_buffers(const spb_engine* e, const float** logits, const int** tokens) {
    clear_error();
    if (!e) return invalid("spb_engine_buffers: null engine");
    if (logits) *logits = e->logits;
    if (tokens) *tokens = e->tokens;
    return 0;
}

extern "C" int spb_generate_sparse_ternary(uint64_t seed, int rows, int cols, uint32_t* meta,
                                           uint32_t* values, int meta_stride, int values_stride,
                                           float* d_gamma, float* latent, spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_generate_sparse_ternary";
    if (rows <= 0 || cols <= 0 || cols % 64) return invalid("%s: need rows > 0, cols %% 64 == 0", fn);
    if (meta_stride < cols / 32 || values_stride < cols / 64)
        return invalid("%s: strides smaller than the format requires", fn);
    if (!meta || !values || !d_gamma) return invalid("%s: null pointer", fn);
    const long units = static_cast<long>(rows) * (cols / 64);
    long blocks = (units + 255) / 256;
    if (blocks > kGenBlocks) blocks = kGenBlocks;
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(gen_sparse_ternary_kernel, dim3(blocks), dim3(256), 0, s, seed, rows, cols,
                       meta, values, meta_stride, values_stride, latent);
    hipLaunchKernelGGL(gen_gamma_kernel, dim3(1), dim3(1), 0, s, static_cast<int>(blocks),
                       static_cast<double>(rows) * cols, d_gamma);
    return launch_status(fn);
}

extern "C" int spb_generate_normal_bf16(uint64_t seed, long n, float std_, uint16_t* out,
                                        spb_stream_t stream) {
    clear_error();
    const char* fn = "spb_generate_normal_bf16";
    if (n < 0) return invalid("%s: negative size", fn);
    if (n == 0) return 0;
    if (!out) return invalid("%s: null pointer", fn);
    long blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(gen_normal_bf16_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                       seed, n, std_, out);
    return launch_status(fn);
}

// ---- batched decode engine ------------------------------------------------------------
//
// B independent sequences per step (BASELINE config 4 at batch 8 / 32).  The
// reference engine decodes one sequence (InferenceEngine::forward,
// src/inference.cu:123-283); this engine computes, for each sequence, every
// value of that step with the same device code in the same order as the bs=1
// engine: the decode producers per token around the matrix-core GEMM over
// the B tokens (the batched prefill's building blocks, with the token of
// sequence t at that sequence's own position), the per-split attention body
// over each sequence's own KV cache, and an LM head whose rows are computed
// exactly as the bs=1 kernel computes them.  So every sequence's tokens equal
// those of a bs=1 generation of that sequence alone.

namespace {

// Launches the splits below `splits` (of S, the partials' stride).
void launch_attention_batch(int hd, int G, int S, int splits, int nkv, int B, hipStream_t s,
                            const uint16_t* qkv, const uint16_t* kc, const uint16_t* vc, float* pm,
                            float* pl, float* pacc, const EngineState* st, int max_seq,
                            float scale, int qkv_stride, long kv_stride) {
    const dim3 grid(splits, nkv, B), block(kAttnThreads);
#define SPB_ATTN_BATCH(HD, GG)                                                                     \
    hipLaunchKernelGGL((attention_batch_kernel<HD, GG>), grid, block, 0, s, qkv, kc, vc, pm, pl,  \
                       pacc, st, max_seq, S, scale, qkv_stride, kv_stride)
    if (hd == 64) {
        switch (G) {
        case 1: SPB_ATTN_BATCH(64, 1); break;
        case 2: SPB_ATTN_BATCH(64, 2); break;
        case 4: SPB_ATTN_BATCH(64, 4); break;
        default: SPB_ATTN_BATCH(64, 8); break;
        }
    } else {
        switch (G) {
        case 1: SPB_ATTN_BATCH(128, 1); break;
        case 2: SPB_ATTN_BATCH(128, 2); break;
        case 4: SPB_ATTN_BATCH(128, 4); break;
        default: SPB_ATTN_BATCH(128, 8); break;
        }
    }
#undef SPB_ATTN_BATCH
}

}  // namespace

struct spb_batch_engine {
    spb_model_config cfg{};
    std::vector<spb_transformer_layer> layers;
    const uint16_t* embed = nullptr;
    const uint16_t* lm_head = nullptr;
    const float* final_norm = nullptr;
    int max_seq = 0, S = 0, batch = 0, lm_grid = 0;
    long kv_seq = 0;  // cache elements of one sequence in one layer's K (or V) cache
    float lm_c = 0.f;  // the LM head's error-bound constant (lm_bound_c)
    std::vector<void*> owned;
    std::vector<uint16_t*> kcache, vcache;  // per layer: [batch][kv head][max_seq][head_dim]
    PrefillBufs step;  // the decode step's per-token buffers (batch tokens)
    PrefillBufs pf;    // the prompt prefill's buffers
    float* logits = nullptr;              // [batch][vocab]
    float* xn = nullptr;                  // [batch][padded hidden]: final-normed vectors
    float* part_lo = nullptr;             // [batch][lm_grid]: largest lower bound per row block
    float* part_hi = nullptr;             // [batch][lm_grid]: largest upper bound per row block
    float* wnorm = nullptr;               // [vocab]: |LM-head row| (rounded up)
    float* xnorm = nullptr;               // [batch]: |normalised vector| (rounded up)
    int* tokens = nullptr;                // [batch][max_seq + 1]
    float2* rope = nullptr;               // [max_seq][head_dim / 2]
    float2* cur_rope = nullptr;           // [batch][head_dim / 2]
    EngineState* st = nullptr;            // [batch]
    GemmSplit split{};                    // split-K workspace of the step's GEMMs
    std::vector<float2> rope_host;
    hipStream_t stream = nullptr;
    hipStream_t cap_stream = nullptr;
    // Sequence groups (batch_groups): the layers of each group of sequences
    // run as a parallel branch of the step graph (each with its own split-K
    // workspace), joined before the LM head.  aux: the capture streams of
    // groups 1 .. groups - 1; ev[0] forks, ev[g] joins group g.
    int groups = 1;
    std::vector<hipStream_t> aux;
    std::vector<hipEvent_t> ev;
    std::vector<GemmSplit> gsplit;
    // One step graph per bucket of bucket_pos positions: graph k launches
    // the attention on the splits below (k + 1) * bucket_pos only, so the
    // blocks past every sequence's position are not launched at all.  The
    // host replays the graph of pos_hint, an upper bound of the largest
    // position of the live sequences (each advances at most one per step).
    std::vector<hipGraph_t> graphs;
    std::vector<hipGraphExec_t> execs;
    int bucket_pos = 0;
    int pos_hint = 0;

    ~spb_batch_engine() {
        for (hipGraphExec_t x : execs) (void)hipGraphExecDestroy(x);
        for (hipGraph_t g : graphs) (void)hipGraphDestroy(g);
        if (cap_stream) (void)hipStreamDestroy(cap_stream);
        for (hipStream_t a : aux) (void)hipStreamDestroy(a);
        for (hipEvent_t v : ev) (void)hipEventDestroy(v);
        for (void* p : owned) (void)hipFree(p);
    }

    hipError_t launch_step(hipStream_t s) {
        int k = pos_hint / bucket_pos;
        if (k >= static_cast<int>(execs.size())) k = static_cast<int>(execs.size()) - 1;
        const hipError_t err = hipGraphLaunch(execs[k], s);
        pos_hint = pos_hint < max_seq ? pos_hint + 1 : max_seq;
        return err;
    }

    long tok_stride() const { return static_cast<long>(max_seq) + 1; }

    // The layers of sequences b0 .. b0 + nb - 1 on stream s: per layer the
    // producer, GEMM(s) and sink of each projection over their tokens and
    // the batched attention (on the first `splits` splits).  Every per-token
    // buffer is addressed from sequence b0's row.
    hipError_t enqueue_layers(hipStream_t s, int b0, int nb, int splits,
                              const GemmSplit* sp) const {
        const int hd = cfg.head_dim, nh = cfg.num_attention_heads;
        const int nkv = cfg.num_key_value_heads, H = cfg.hidden_size;
        const int I = cfg.intermediate_size, kvdim = nkv * hd, qrows = nh * hd;
        const float eps = cfg.rms_norm_eps;
        const float scale = 1.0f / sqrtf(static_cast<float>(hd));  // inference.cu:182
        const int B = nb;
        const long qkv_row = qrows + 2 * kvdim, hs = static_cast<long>(nh) * S;
        int8_t* const x = step.x + b0 * step.xrow;
        float* const amax = step.amax + b0;
        int32_t* const y[3] = {step.y[0] + b0 * step.yrow0, step.y[1] + b0 * step.yrow,
                               step.y[2] + b0 * step.yrow};
        uint16_t* const qkv = step.qkv + b0 * qkv_row;
        uint16_t* const o = step.o + static_cast<long>(b0) * H;
        uint16_t* const r = step.r + static_cast<long>(b0) * H;
        uint16_t* const r2 = step.r2 + static_cast<long>(b0) * H;
        uint16_t* const gu = step.gu + static_cast<long>(b0) * 2 * I;
        float* const pm = step.pm + b0 * hs;
        float* const pl = step.pl + b0 * hs;
        float* const pacc = step.pacc + b0 * hs * hd;
        EngineState* const stb = st + b0;
        const int* const tok = tokens + b0 * tok_stride();
        float2* const crope = cur_rope + static_cast<long>(b0) * (hd / 2);
        for (size_t l = 0; l < layers.size(); ++l) {
            const spb_transformer_layer& L = layers[l];
            uint16_t* const kc = kcache[l] + b0 * kv_seq;
            uint16_t* const vc = vcache[l] + b0 * kv_seq;
            {
                InputNorm p{r, l == 0 ? embed : nullptr, tok, r, L.input_layernorm, eps, H};
                p.tok_stride = tok_stride();
                launch_prefill_producer(p, H, stb, H, B, x, amax, s);
            }
            const spb_sparse_linear* qkv3[3] = {&L.q_proj, &L.k_proj, &L.v_proj};
            {
                QkvRopeSink sink{};
                sink.out = qkv;
                sink.kc = kc;
                sink.vc = vc;
                sink.cur_rope = crope;
                sink.st = stb;
                sink.g0 = L.q_proj.gamma;
                sink.g1 = L.k_proj.gamma;
                sink.g2 = L.v_proj.gamma;
                sink.end0 = qrows;
                sink.end1 = qrows + kvdim;
                sink.hd = hd;
                sink.hd_log2 = hd == 64 ? 6 : 7;
                sink.max_seq = max_seq;
                sink.rope_tab = nullptr;  // each sequence's own RoPE row (cur_rope)
                sink.kv_stride = kv_seq;
                if (gemm_sink(qkv3, 3, x, amax, sink, qkv_row, y, B, s, sp) != hipSuccess)
                    return hipErrorLaunchFailure;
            }
            launch_attention_batch(hd, nh / nkv, S, splits, nkv, B, s, qkv, kc, vc, pm, pl, pacc,
                                   stb, max_seq, scale, static_cast<int>(qkv_row), kv_seq);
            {
                float* const cb = step.comb + static_cast<long>(b0) * qrows;
                launch_attn_combine(hd, nh, splits, s, pm, pl, pacc, cb, stb, S, B);
                CombinedAttn p{cb, qrows};
                launch_prefill_producer(p, qrows, stb, qrows, B, x, amax, s);
            }
            {
                const spb_sparse_linear* o1[1] = {&L.o_proj};
                SegBf16Sink sink{o, L.o_proj.gamma, L.o_proj.gamma, L.o_proj.gamma, H, H,
                                 0.f, 0.f, 0.f};
                if (gemm_sink(o1, 1, x, amax, sink, H, y, B, s, sp) != hipSuccess)
                    return hipErrorLaunchFailure;
            }
            {
                SubNormResidualNorm p{o, r, r2, L.attn_sub_norm, L.post_attention_layernorm,
                                      eps, H};
                launch_prefill_producer(p, H, stb, H, B, x, amax, s);
            }
            {
                const spb_sparse_linear* gu2[2] = {&L.gate_proj, &L.up_proj};
                SegBf16Sink sink{gu, L.gate_proj.gamma, L.up_proj.gamma, L.up_proj.gamma,
                                 I, 2 * I, 0.f, 0.f, 0.f};
                if (gemm_sink(gu2, 2, x, amax, sink, 2 * I, y, B, s, sp) != hipSuccess)
                    return hipErrorLaunchFailure;
            }
            {
                Relu2Norm p{gu, gu + I, L.ffn_sub_norm,
                            L.ffn_sub_norm ? L.ffn_sub_norm : reinterpret_cast<const float*>(gu),
                            eps, I};
                launch_prefill_producer(p, 2 * I, stb, I, B, x, amax, s);
            }
            {
                const spb_sparse_linear* d1[1] = {&L.down_proj};
                ResidualSink sink{r, r2, L.down_proj.gamma, 0.f};
                if (gemm_sink(d1, 1, x, amax, sink, H, y, B, s, sp) != hipSuccess)
                    return hipErrorLaunchFailure;
            }
        }
        return hipGetLastError();
    }

    // One decode step of every sequence: the layers (the sequence groups in
    // parallel branches), then the final norm and the LM head (the
    // matrix-core logits over every sequence, then the exact candidates and
    // the argmax per sequence).
    hipError_t enqueue_step(hipStream_t s, int splits) const {
        if (groups == 1) {
            const hipError_t err = enqueue_layers(s, 0, batch, splits, &gsplit[0]);
            if (err != hipSuccess) return err;
            return enqueue_head(s);
        }
        if (hipEventRecord(ev[0], s) != hipSuccess) return hipErrorLaunchFailure;
        for (int g = 1; g < groups; ++g)
            if (hipStreamWaitEvent(aux[g - 1], ev[0], 0) != hipSuccess)
                return hipErrorLaunchFailure;
        hipError_t err = hipSuccess;
        for (int g = 0; g < groups && err == hipSuccess; ++g) {
            const int b0 = g * batch / groups, b1 = (g + 1) * batch / groups;
            err = enqueue_layers(g ? aux[g - 1] : s, b0, b1 - b0, splits, &gsplit[g]);
        }
        for (int g = 1; g < groups; ++g)  // rejoin every branch, also after an error
            if (hipEventRecord(ev[g], aux[g - 1]) != hipSuccess ||
                hipStreamWaitEvent(s, ev[g], 0) != hipSuccess)
                err = hipErrorLaunchFailure;
        if (err != hipSuccess) return err;
        return enqueue_head(s);
    }

    hipError_t enqueue_head(hipStream_t s) const {
        const int hd = cfg.head_dim, H = cfg.hidden_size;
        const float eps = cfg.rms_norm_eps;
        const int B = batch;
        const int V = cfg.vocab_size, xstride = lm_head_batch_xstride(H);
        const int nc64 = (H / 8 + kWave - 1) / kWave * kWave;
        hipLaunchKernelGGL(final_norm_batch_kernel<true>, dim3(B), dim3(kLmBlock), 0, s, step.r,
                           final_norm, eps, xn, xnorm, H, nc64, xstride);
        const dim3 grid(lm_grid, (B + kLmMfmaTok - 1) / kLmMfmaTok);
        if (B > 16)
            hipLaunchKernelGGL(lm_head_mfma_kernel<2>, grid, dim3(kLmMfmaBlock), 0, s, lm_head, xn,
                               xstride, wnorm, xnorm, lm_c, logits, part_lo, part_hi, V, H, B,
                               lm_grid);
        else
            hipLaunchKernelGGL(lm_head_mfma_kernel<1>, grid, dim3(kLmMfmaBlock), 0, s, lm_head, xn,
                               xstride, wnorm, xnorm, lm_c, logits, part_lo, part_hi, V, H, B,
                               lm_grid);
        hipLaunchKernelGGL(lm_select_kernel, dim3(B), dim3(kLmSelectBlock), 0, s, lm_head, xn,
                           xstride, wnorm, xnorm, lm_c, logits, part_lo, part_hi, st, tokens,
                           tok_stride(), V, H, rope, cur_rope, hd / 2, max_seq, lm_grid);
        return hipGetLastError();
    }
};

extern "C" int spb_batch_engine_create(const spb_model_config* cfg,
                                       const spb_transformer_layer* layers,
                                       const uint16_t* embed_tokens, const uint16_t* lm_head,
                                       const float* final_norm, int max_seq, int batch,
                                       spb_batch_engine** out) {
    clear_error();
    const char* fn = "spb_batch_engine_create";
    if (!cfg || !layers || !embed_tokens || !final_norm || !out)
        return invalid("%s: null argument", fn);
    *out = nullptr;
    if (int rc = check_model(fn, cfg, layers, embed_tokens, lm_head, max_seq)) return rc;
    if (batch < 1 || batch > kPrefillChunk)
        return invalid("%s: batch must be in [1, %d]", fn, kPrefillChunk);
    const int H = cfg->hidden_size, nh = cfg->num_attention_heads, nkv = cfg->num_key_value_heads;
    const int hd = cfg->head_dim, V = cfg->vocab_size;
    if (H > kLmBatchMaxH)
        return invalid("%s: hidden_size %d exceeds the batched LM head's %d", fn, H, kLmBatchMaxH);
    spb_batch_engine* e = new (std::nothrow) spb_batch_engine();
    if (!e) return invalid("%s: out of host memory", fn);
    e->cfg = *cfg;
    e->layers.assign(layers, layers + cfg->num_hidden_layers);
    e->embed = embed_tokens;
    e->lm_head = lm_head ? lm_head : embed_tokens;
    e->final_norm = final_norm;
    e->max_seq = max_seq;
    e->batch = batch;
    e->S = (max_seq + kAttnSplit - 1) / kAttnSplit;
    e->kv_seq = static_cast<long>(nkv) * max_seq * hd;
    e->lm_c = lm_bound_c(H);
    e->lm_grid = (V + kLmMfmaRows - 1) / kLmMfmaRows;
    if (e->lm_grid > kLmSelMaxBlocks) {
        delete e;
        return invalid("%s: vocabulary %d exceeds the batched LM head's %d rows", fn, V,
                       kLmSelMaxBlocks * kLmMfmaRows);
    }

    auto& own = e->owned;
    const size_t kv = static_cast<size_t>(batch) * e->kv_seq;
    bool ok = true;
    for (int l = 0; l < cfg->num_hidden_layers && ok; ++l) {
        e->kcache.push_back(dev_alloc<uint16_t>(kv, own));
        e->vcache.push_back(dev_alloc<uint16_t>(kv, own));
        ok = e->kcache.back() && e->vcache.back();
    }
    const size_t B = static_cast<size_t>(batch);
    ok = ok && alloc_prefill(e->step, *cfg, e->S, own, batch) &&
         alloc_prefill(e->pf, *cfg, e->S, own) &&
         (e->logits = dev_alloc<float>(B * V, own)) &&
         (e->xn = dev_alloc<float>(B * lm_head_batch_xstride(H), own)) &&
         (e->part_lo = dev_alloc<float>(B * e->lm_grid, own)) &&
         (e->part_hi = dev_alloc<float>(B * e->lm_grid, own)) &&
         (e->wnorm = dev_alloc<float>(static_cast<size_t>(V), own)) &&
         (e->xnorm = dev_alloc<float>(B, own)) &&
         (e->tokens = dev_alloc<int>(B * (max_seq + 1), own)) &&
         (e->rope = dev_alloc<float2>(static_cast<size_t>(max_seq) * (hd / 2), own)) &&
         (e->cur_rope = dev_alloc<float2>(B * (hd / 2), own)) &&
         (e->st = dev_alloc<EngineState>(B, own));
    // split-K workspace of the step's GEMMs (q|k|v, o, gate|up, down over the
    // batch's tokens) and one counter per row x token tile
    {
        const int I = cfg->intermediate_size;
        const int rows_h[3] = {nh * hd + 2 * nkv * hd, H, 2 * I};
        const long w_h = staged_split_words(rows_h, 3, H, batch);
        const long w_i = staged_split_words(&rows_h[1], 1, I, batch);
        e->split.part_words = w_h > w_i ? w_h : w_i;
        e->split.count_words = kGemmSplitCounters;
        if (e->split.part_words > 0)
            ok = ok && (e->split.part = dev_alloc<int32_t>(e->split.part_words, own)) &&
                 (e->split.count = dev_alloc<unsigned>(kGemmSplitCounters, own));
        e->groups = batch_groups(batch);
        e->gsplit.assign(e->groups, e->split);
        for (int g = 1; g < e->groups && e->split.part_words > 0; ++g)
            ok = ok && (e->gsplit[g].part = dev_alloc<int32_t>(e->split.part_words, own)) &&
                 (e->gsplit[g].count = dev_alloc<unsigned>(kGemmSplitCounters, own));
    }
    if (!ok) {
        delete e;
        return invalid("%s: device allocation failed", fn);
    }
    if (gemm_prepare() != 0 || gemm_sink_prepare() != 0) {
        delete e;
        return launch_status(fn);
    }
    // the LM-head rows' norms for the error bounds (the table is the model's,
    // unchanged while the engine lives)
    hipLaunchKernelGGL(lm_row_norm_kernel, dim3((V + 3) / 4), dim3(256), 0, nullptr, e->lm_head,
                       e->wnorm, V, H);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        delete e;
        return launch_status(fn);
    }
    e->rope_host = rope_table(*cfg, max_seq);
    hipError_t err = hipMemcpy(e->rope, e->rope_host.data(), e->rope_host.size() * sizeof(float2),
                               hipMemcpyHostToDevice);
    for (size_t l = 0; l < e->kcache.size() && err == hipSuccess; ++l) {
        err = hipMemset(e->kcache[l], 0, kv * 2);
        if (err == hipSuccess) err = hipMemset(e->vcache[l], 0, kv * 2);
    }
    if (err == hipSuccess) err = hipMemset(e->st, 0, B * sizeof(EngineState));
    if (err == hipSuccess) err = hipMemset(e->tokens, 0, B * (max_seq + 1) * sizeof(int));
    // the split-K tile counters start (and end) at 0
    for (size_t g = 0; g < e->gsplit.size() && err == hipSuccess; ++g)
        if (e->gsplit[g].count)
            err = hipMemset(e->gsplit[g].count, 0, kGemmSplitCounters * sizeof(unsigned));
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&e->cap_stream, hipStreamNonBlocking);
    for (int g = 0; g < e->groups && err == hipSuccess; ++g) {
        hipEvent_t v = nullptr;
        err = hipEventCreateWithFlags(&v, hipEventDisableTiming);
        if (err == hipSuccess) e->ev.push_back(v);
        if (g > 0 && err == hipSuccess) {
            hipStream_t a = nullptr;
            err = hipStreamCreateWithFlags(&a, hipStreamNonBlocking);
            if (err == hipSuccess) e->aux.push_back(a);
        }
    }
    if (err != hipSuccess) {
        delete e;
        return launch_status(fn);
    }
    // the step graphs, one per position bucket (the bs=1 engine's buckets)
    {
        const int per = e->S <= 64 ? kAttnBucketSplits : (e->S + 7) / 8;
        e->bucket_pos = per * kAttnSplit;
        for (int s0 = 0; s0 < e->S && err == hipSuccess; s0 += per) {
            const int splits = s0 + per < e->S ? s0 + per : e->S;
            hipGraph_t g = nullptr;
            hipGraphExec_t x = nullptr;
            err = hipStreamBeginCapture(e->cap_stream, hipStreamCaptureModeThreadLocal);
            if (err == hipSuccess) {
                const hipError_t le = e->enqueue_step(e->cap_stream, splits);
                err = hipStreamEndCapture(e->cap_stream, &g);
                if (err == hipSuccess) e->graphs.push_back(g);
                if (err == hipSuccess && le != hipSuccess) err = le;
            }
            if (err == hipSuccess) err = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
            if (err == hipSuccess) e->execs.push_back(x);
        }
    }
    if (err != hipSuccess) {
        set_error("%s: graph capture failed: %s", fn, hipGetErrorString(err));
        delete e;
        return static_cast<int>(err);
    }
    // every slot done until a generate arms it
    std::vector<EngineState> hs(B);
    for (auto& h : hs) {
        h = EngineState{};
        h.limit = max_seq;
        h.prompt_len = max_seq;
        h.done = 1;
    }
    if (hipMemcpy(e->st, hs.data(), B * sizeof(EngineState), hipMemcpyHostToDevice) !=
        hipSuccess) {
        delete e;
        return launch_status(fn);
    }
    *out = e;
    return 0;
}

extern "C" int spb_batch_engine_destroy(spb_batch_engine* e) {
    clear_error();
    if (e) {
        (void)hipStreamSynchronize(e->stream);
        delete e;
    }
    return 0;
}

extern "C" int spb_batch_engine_set_stream(spb_batch_engine* e, spb_stream_t stream) {
    clear_error();
    if (!e) return invalid("spb_batch_engine_set_stream: null engine");
    e->stream = as_stream(stream);
    return 0;
}

extern "C" int spb_batch_engine_generate(spb_batch_engine* e, const int* prompts,
                                         const int* prompt_lens, int n_seq, int n_new,
                                         int stop_at_eos, int* out_tokens, int* n_generated) {
    clear_error();
    const char* fn = "spb_batch_engine_generate";
    if (!e || !prompts || !prompt_lens || (!out_tokens && n_new > 0))
        return invalid("%s: null argument", fn);
    if (n_seq < 1 || n_seq > e->batch)
        return invalid("%s: n_seq %d outside [1, %d]", fn, n_seq, e->batch);
    if (n_new < 0) return invalid("%s: n_new < 0", fn);
    std::vector<long> off(n_seq + 1, 0);
    for (int b = 0; b < n_seq; ++b) {
        const int n = prompt_lens[b];
        if (n < 1) return invalid("%s: sequence %d has an empty prompt", fn, b);
        if (static_cast<long>(n) + n_new > e->max_seq)
            return invalid("%s: sequence %d: prompt + new tokens (%ld) exceed max_seq %d", fn, b,
                           static_cast<long>(n) + n_new, e->max_seq);
        off[b + 1] = off[b] + n;
    }
    for (long i = 0; i < off[n_seq]; ++i)
        if (prompts[i] < 0 || prompts[i] >= e->cfg.vocab_size)
            return invalid("%s: prompt token %d outside [0, %d)", fn, prompts[i],
                           e->cfg.vocab_size);
    hipStream_t s = e->stream;
    const long ts = e->tok_stride();
    const int half = e->cfg.head_dim / 2;
    // token buffers, then each prompt's positions 0 .. n-2 through the layers
    // (the batched prefill, into the sequence's own KV cache)
    std::vector<int> tok(static_cast<size_t>(n_seq) * ts, 0);
    for (int b = 0; b < n_seq; ++b)
        std::copy(prompts + off[b], prompts + off[b + 1], tok.begin() + b * ts);
    if (hipMemcpyAsync(e->tokens, tok.data(), tok.size() * sizeof(int), hipMemcpyHostToDevice, s) !=
            hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return launch_status(fn);
    for (int b = 0; b < n_seq; ++b) {
        const int pre = prompt_lens[b] - 1;
        const PrefillTarget t{&e->cfg, &e->layers, e->embed, e->rope, e->max_seq, e->S,
                              &e->kcache, &e->vcache, b * e->kv_seq, e->tokens + b * ts};
        for (int p0 = 0; p0 < pre; p0 += e->pf.chunk) {
            const int c = pre - p0 < e->pf.chunk ? pre - p0 : e->pf.chunk;
            if (enqueue_prefill_pass(t, e->pf, p0, c, s) != hipSuccess) return launch_status(fn);
        }
    }
    // decode states: sequence b continues at its last prompt token; unused
    // slots are done
    std::vector<EngineState> hs(e->batch);
    std::vector<float2> cr(static_cast<size_t>(e->batch) * half);
    for (int b = 0; b < e->batch; ++b) {
        EngineState& h = hs[b];
        h = EngineState{};
        h.limit = e->max_seq;
        h.eos = e->cfg.eos_token_id;
        if (b < n_seq) {
            h.pos = prompt_lens[b] - 1;
            h.prompt_len = prompt_lens[b];
            h.stop_eos = stop_at_eos ? 1 : 0;
        } else {
            h.prompt_len = e->max_seq;
            h.done = 1;
        }
        std::copy(e->rope_host.begin() + static_cast<long>(h.pos) * half,
                  e->rope_host.begin() + static_cast<long>(h.pos + 1) * half,
                  cr.begin() + static_cast<long>(b) * half);
    }
    if (hipMemcpyAsync(e->st, hs.data(), hs.size() * sizeof(EngineState), hipMemcpyHostToDevice,
                       s) != hipSuccess ||
        hipMemcpyAsync(e->cur_rope, cr.data(), cr.size() * sizeof(float2), hipMemcpyHostToDevice,
                       s) != hipSuccess)
        return launch_status(fn);
    e->pos_hint = 0;
    for (int b = 0; b < n_seq; ++b)
        if (hs[b].pos > e->pos_hint) e->pos_hint = hs[b].pos;
    for (int i = 0; i < n_new; ++i)
        if (e->launch_step(s) != hipSuccess) return launch_status(fn);
    if (hipMemcpyAsync(hs.data(), e->st, hs.size() * sizeof(EngineState), hipMemcpyDeviceToHost,
                       s) != hipSuccess ||
        hipMemcpyAsync(tok.data(), e->tokens, tok.size() * sizeof(int), hipMemcpyDeviceToHost, s) !=
            hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return launch_status(fn);
    for (int b = 0; b < n_seq; ++b) {
        const int got = hs[b].generated < n_new ? hs[b].generated : n_new;
        for (int i = 0; i < n_new; ++i)
            out_tokens[static_cast<long>(b) * n_new + i] =
                i < got ? tok[b * ts + prompt_lens[b] + i] : -1;
        if (n_generated) n_generated[b] = got;
    }
    return 0;
}

extern "C" int spb_batch_engine_decode_steps(spb_batch_engine* e, int steps) {
    clear_error();
    if (!e) return invalid("spb_batch_engine_decode_steps: null engine");
    if (steps < 0) return invalid("spb_batch_engine_decode_steps: steps < 0");
    for (int i = 0; i < steps; ++i)
        if (e->launch_step(e->stream) != hipSuccess)
            return launch_status("spb_batch_engine_decode_steps");
    return 0;
}

extern "C" int spb_batch_engine_buffers(const spb_batch_engine* e, const float** logits,
                                        const int** tokens) {
    clear_error();
    if (!e) return invalid("spb_batch_engine_buffers: null engine");
    if (logits) *logits = e->logits;
    if (tokens) *tokens = e->tokens;
    return 0;
}

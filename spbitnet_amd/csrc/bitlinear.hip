// bitlinear.hip -- the BitLinear of the reference engine as one call:
// InferenceEngine::bitlinear (src/inference.cu:106-117) runs absmax_reduce_gpu
// into the engine's device scalar d_absmax_, then fused_sparse_bitlinear_gpu.
// Here the scalar (and the activation bit planes) live in a caller workspace:
//   bytes [0, 256)            absmax (float)
//   bytes [256, 256 + P)      bit planes of the quantised activations,
//                             P = 32 * ceil(cols / 32) (the plane layout of
//                             spb_absmax_quantize_planes_*)
// When cols % 8 == 0 and x and the workspace are 16-byte aligned, the planes
// are built once (spb_absmax_quantize_planes_*, one block) and the GEMV reads
// them (spb_fused_sparse_bitlinear_planes_*), instead of every GEMV block
// quantising the vector again; otherwise the reference's pair runs on the
// workspace's absmax.  Both orders give the reference's bits:
//   q = clamp(rint(x * (absmax > 0 ? 127/absmax : 0)), -128, 127),
//   out[r] = 16-bit(float(W q) * ((gamma * absmax) / 127)).
#include <mutex>
#include <string>
#include <type_traits>

#include "bitplane.hpp"
#include "spbitnet_amd.h"

namespace spb {
namespace {

constexpr size_t kAbsmaxBytes = 256;

size_t planes_bytes(int cols) { return 32 * static_cast<size_t>((cols + 31) / 32); }

size_t workspace_bytes(int cols) { return cols > 0 ? kAbsmaxBytes + planes_bytes(cols) : 0; }

// The BitLinear on a workspace already checked to hold workspace_bytes(cols).
template <class T>
int bitlinear_ws(const char* fn, const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                 uint16_t* output, float gamma, int rows, int cols, int ms, int vs,
                 uint8_t* ws, hipStream_t s) {
    float* d_absmax = reinterpret_cast<float*>(ws);
    uint32_t* planes = reinterpret_cast<uint32_t*>(ws + kAbsmaxBytes);
    constexpr bool kBf16 = std::is_same<T, BF16>::value;
    int rc;
    if (cols % 8 == 0 && aligned(x, 16) && aligned(ws, 16)) {
        rc = kBf16 ? spb_absmax_quantize_planes_bf16(x, planes, nullptr, d_absmax, cols, s)
                   : spb_absmax_quantize_planes_f16(x, planes, nullptr, d_absmax, cols, s);
        if (rc == 0)
            rc = kBf16 ? spb_fused_sparse_bitlinear_planes_bf16(meta, values, planes, output,
                                                                d_absmax, gamma, rows, cols, ms,
                                                                vs, s)
                       : spb_fused_sparse_bitlinear_planes_f16(meta, values, planes, output,
                                                               d_absmax, gamma, rows, cols, ms,
                                                               vs, s);
    } else {
        rc = kBf16 ? spb_absmax_reduce_bf16(x, d_absmax, cols, s)
                   : spb_absmax_reduce_f16(x, d_absmax, cols, s);
        if (rc == 0)
            rc = kBf16 ? spb_fused_sparse_bitlinear_bf16(meta, values, x, output, d_absmax, gamma,
                                                         rows, cols, ms, vs, s)
                       : spb_fused_sparse_bitlinear_f16(meta, values, x, output, d_absmax, gamma,
                                                        rows, cols, ms, vs, s);
    }
    if (rc) {
        const std::string inner = last_error();
        set_error("%s: %s", fn, inner.c_str());
    }
    return rc;
}

// Argument checks shared by the entry points (nothing is launched on failure).
int check_bitlinear(const char* fn, const uint32_t* meta, const uint32_t* values,
                    const uint16_t* x, const uint16_t* output, int rows, int cols, int ms,
                    int vs) {
    if (int e = check_weights(fn, meta, values, rows, cols, ms, vs)) return e;
    if (rows && cols && (!x || !output)) return invalid("%s: null activation pointer", fn);
    return 0;
}

template <class T>
int bitlinear(const char* fn, const uint32_t* meta, const uint32_t* values, const uint16_t* x,
              uint16_t* output, float gamma, int rows, int cols, int ms, int vs, void* workspace,
              size_t workspace_bytes_given, spb_stream_t stream) {
    clear_error();
    if (int e = check_bitlinear(fn, meta, values, x, output, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (!workspace) return invalid("%s: null workspace", fn);
    if (!aligned(workspace, 16)) return invalid("%s: workspace must be 16-byte aligned", fn);
    if (workspace_bytes_given < workspace_bytes(cols))
        return invalid("%s: workspace of %zu bytes, %zu needed for %d columns", fn,
                       workspace_bytes_given, workspace_bytes(cols), cols);
    return bitlinear_ws<T>(fn, meta, values, x, output, gamma, rows, cols, ms, vs,
                           static_cast<uint8_t*>(workspace), as_stream(stream));
}

// ---- allocation-free form -------------------------------------------------------
// For callers that cannot allocate (code under HIP graph capture, serving
// loops that forbid hipMalloc): the workspace is `scratch`, a file-scope
// device array of workspace_bytes(kNoAllocMaxCols) bytes.  Each GPU the
// library runs on holds its own copy until the process ends.  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in
// symbol, not a device address): the entry point looks up the copy's device
// address once per device with hipGetSymbolAddress, with that device
// current, and uses that pointer.  Every call on a GPU shares its copy, which
// keeps the last call's contents; nothing in it needs to start at zero (each
// call writes the absmax and every plane word the GEMV reads before reading
// them).  Calls that overlap on one GPU (different streams, host threads)
// race on it.
constexpr int kNoAllocMaxCols = kMaxPlaneCols;  // 32768
constexpr size_t kScratchBytes = kAbsmaxBytes + 32 * (kNoAllocMaxCols / 32);
static_assert(kNoAllocMaxCols % 32 == 0, "planes of the largest vector fill whole groups");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kScratchDevices] = {};

// The device address of the current device's copy of `scratch` (looked up on
// the first call on each device); nullptr with the error recorded on failure.
uint8_t* scratch_on_current_device(const char* fn, int* rc) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("%s: hipGetDevice: %s", fn, hipGetErrorString(e));
        *rc = static_cast<int>(e);
        return nullptr;
    }
    if (dev < 0 || dev >= kScratchDevices) {
        *rc = invalid("%s: device %d beyond the %d devices the scratch table covers", fn, dev,
                      kScratchDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_error("%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
            *rc = static_cast<int>(e != hipSuccess ? e : hipErrorInvalidSymbol);
            return nullptr;
        }
        g_scratch[dev] = static_cast<uint8_t*>(ptr);
    }
    return g_scratch[dev];
}

template <class T>
int bitlinear_noalloc(const char* fn, const uint32_t* meta, const uint32_t* values,
                      const uint16_t* x, uint16_t* output, float gamma, int rows, int cols,
                      int ms, int vs, spb_stream_t stream) {
    clear_error();
    if (int e = check_bitlinear(fn, meta, values, x, output, rows, cols, ms, vs)) return e;
    if (rows == 0 || cols == 0) return 0;
    if (cols > kNoAllocMaxCols)
        return invalid("%s: cols=%d exceeds the %d columns the static scratch holds (use "
                       "spb_bitlinear_* with a workspace)", fn, cols, kNoAllocMaxCols);
    int rc = 0;
    uint8_t* ws = scratch_on_current_device(fn, &rc);
    if (!ws) return rc;
    return bitlinear_ws<T>(fn, meta, values, x, output, gamma, rows, cols, ms, vs, ws,
                           as_stream(stream));
}

}  // namespace
}  // namespace spb

using namespace spb;

extern "C" size_t spb_bitlinear_workspace_size(int cols) { return workspace_bytes(cols); }

extern "C" int spb_bitlinear_f16(const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                                 uint16_t* output, float gamma, int rows, int cols,
                                 int meta_row_stride, int values_row_stride, void* workspace,
                                 size_t workspace_size, spb_stream_t stream) {
    return bitlinear<F16>("spb_bitlinear_f16", meta, values, x, output, gamma, rows, cols,
                          meta_row_stride, values_row_stride, workspace, workspace_size, stream);
}

extern "C" int spb_bitlinear_bf16(const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                                  uint16_t* output, float gamma, int rows, int cols,
                                  int meta_row_stride, int values_row_stride, void* workspace,
                                  size_t workspace_size, spb_stream_t stream) {
    return bitlinear<BF16>("spb_bitlinear_bf16", meta, values, x, output, gamma, rows, cols,
                           meta_row_stride, values_row_stride, workspace, workspace_size, stream);
}

extern "C" int spb_bitlinear_f16_noalloc(const uint32_t* meta, const uint32_t* values,
                                         const uint16_t* x, uint16_t* output, float gamma,
                                         int rows, int cols, int meta_row_stride,
                                         int values_row_stride, spb_stream_t stream) {
    return bitlinear_noalloc<F16>("spb_bitlinear_f16_noalloc", meta, values, x, output, gamma,
                                  rows, cols, meta_row_stride, values_row_stride, stream);
}

extern "C" int spb_bitlinear_bf16_noalloc(const uint32_t* meta, const uint32_t* values,
                                          const uint16_t* x, uint16_t* output, float gamma,
                                          int rows, int cols, int meta_row_stride,
                                          int values_row_stride, spb_stream_t stream) {
    return bitlinear_noalloc<BF16>("spb_bitlinear_bf16_noalloc", meta, values, x, output, gamma,
                                   rows, cols, meta_row_stride, values_row_stride, stream);
}

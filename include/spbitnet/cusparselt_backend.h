// spbitnet/cusparselt_backend.h -- drop-in C++17 replacement for the
// reference's cuSPARSELt backend, over the C ABI in spbitnet_amd.h.
//
// Same namespace, class name, members and argument meaning as the
// reference's include/spbitnet/cusparselt_backend.h:28-77
// (src/cusparselt_backend.cu:38-219):
//
//   CuSparseLtGemm ctx(m, k, n);   // D[m,n] = A[m,k] * B[k,n]
//   ctx.prepare(d_int8_weights);   // prune to 2:4 + compress
//   ctx.execute(d_B, d_D);         // int8 sparse matrix-core product
//   ctx.get_pruned_weights(d_out); // the pruned dense [m x k] int8 matrix
//
// with hipStream_t in place of cudaStream_t.  A is row-major int8 [m x k]
// (any int8 values), B int8 [k x n] column-major, D int32 [m x n]
// column-major, as in the reference.  The object owns the compressed
// operand (device memory, freed by the destructor); it is non-copyable and
// non-movable, as the reference's.
//
// Differences: any n >= 1 is accepted (the reference exits for n < 16,
// src/cusparselt_backend.cu:41-45); the pruning rule is the library's
// documented one (spb_sparse_i8_prune_compress: the two largest |a| of each
// group of four along k, on equal magnitudes the higher index, a group with
// at most two non-zeros kept whole) in place of cuSPARSELt's unspecified
// STRIP selection; get_pruned_weights decompresses the stored operand
// instead of copying a second dense buffer.  Errors print a message and
// exit the process, as the reference's CUSPARSELT_CHECK / CUDA_CHECK do.
//
// The reference compiles this class only under SPBITNET_HAS_CUSPARSELT; the
// macro is defined here so that callers' guarded code paths build.
//
// Link with spbitnet_amd/libspbitnet_amd.so (and libamdhip64).
#pragma once

#ifndef SPBITNET_HAS_CUSPARSELT
#define SPBITNET_HAS_CUSPARSELT 1
#endif

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "spbitnet_amd.h"

namespace spbitnet {

// reference include/spbitnet/cusparselt_backend.h:28-77
class CuSparseLtGemm {
public:
    // m: output rows (weight rows); k: inner dimension (weight cols, a
    // multiple of 4); n: output columns (tokens), n >= 1.
    CuSparseLtGemm(int m, int k, int n) : m_(m), k_(k), n_(n) {
        if (n < 1 || m < 0) fail("CuSparseLtGemm: need m >= 0 and n >= 1");
        const long bytes = spb_sparse_i8_compressed_size(m, k);
        if (bytes < 0) fail("CuSparseLtGemm");
        bytes_ = static_cast<size_t>(bytes);
        if (bytes_ > 0 && hipMalloc(&d_compressed_, bytes_) != hipSuccess)
            fail("CuSparseLtGemm: hipMalloc of the compressed operand failed");
    }
    ~CuSparseLtGemm() {
        if (d_compressed_) (void)hipFree(d_compressed_);
    }

    CuSparseLtGemm(const CuSparseLtGemm&) = delete;
    CuSparseLtGemm& operator=(const CuSparseLtGemm&) = delete;

    // Prune d_weights (device int8 [m x k], row-major) to 2:4 and compress.
    // Synchronises `stream` before returning, as the reference's prepare does
    // (src/cusparselt_backend.cu:117, 164).
    void prepare(const int8_t* d_weights, hipStream_t stream = nullptr) {
        check(spb_sparse_i8_prune_compress(d_weights, nullptr, d_compressed_, m_, k_, stream),
              "CuSparseLtGemm::prepare");
        if (hipStreamSynchronize(stream) != hipSuccess) fail("CuSparseLtGemm::prepare: sync");
        prepared_ = true;
    }

    // D = A_pruned * B (alpha 1, beta 0); d_B int8 [k x n] column-major,
    // d_D int32 [m x n] column-major.
    void execute(const int8_t* d_B, int32_t* d_D, hipStream_t stream = nullptr) {
        if (!prepared_) fail("CuSparseLtGemm::execute() called before prepare()");
        check(spb_sparse_i8_gemm(d_compressed_, d_B, d_D, m_, k_, n_, stream),
              "CuSparseLtGemm::execute");
    }

    // The pruned (uncompressed) weights, device int8 [m x k].
    void get_pruned_weights(int8_t* d_out, hipStream_t stream = nullptr) const {
        if (!prepared_) fail("CuSparseLtGemm::get_pruned_weights() -- not prepared");
        check(spb_sparse_i8_decompress(d_compressed_, d_out, m_, k_, stream),
              "CuSparseLtGemm::get_pruned_weights");
    }

    int m() const { return m_; }
    int k() const { return k_; }
    int n() const { return n_; }

private:
    [[noreturn]] static void fail(const char* what) {
        std::fprintf(stderr, "%s: %s\n", what, spb_last_error_string());
        std::exit(EXIT_FAILURE);
    }
    static void check(int rc, const char* what) {
        if (rc != 0) fail(what);
    }

    int m_, k_, n_;
    bool prepared_ = false;
    void* d_compressed_ = nullptr;
    size_t bytes_ = 0;
};

}  // namespace spbitnet

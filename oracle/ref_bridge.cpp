// ref_bridge.cpp -- C entry points over the reference's own host format code.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile against the
// reference's header-only C++17 format class
// (include/spbitnet/sparse_ternary_tensor.h, used where it lies under the
// reference tree; nothing from it is copied here) into oracle/_ref/.  It lets
// the tests check the C restatement in oracle/spb_oracle.c against the
// reference's own pack/unpack code, and regenerates the exact random inputs of
// the reference's GPU tests (same std::mt19937 seeds and call order as
// tests/test_sparse_ternary.cu:184-402) so their expected outputs can be
// committed as golden vectors.
#include "spbitnet/sparse_ternary_tensor.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

using spbitnet::SparseTernaryTensor;

extern "C" {

int ref_meta_stride(int cols) {
    return static_cast<int>(SparseTernaryTensor(1, cols).meta_row_stride());
}
int ref_values_stride(int cols) {
    return static_cast<int>(SparseTernaryTensor(1, cols).values_row_stride());
}

// SparseTernaryTensor::pack_from_dense (sparse_ternary_tensor.h:58-108).
void ref_pack_from_dense(const int8_t* w, const uint8_t* mask, int rows, int cols,
                         uint32_t* meta, uint32_t* values) {
    auto t = SparseTernaryTensor::pack_from_dense(w, mask, rows, cols);
    std::memcpy(meta, t.meta_data(), t.meta_size() * sizeof(uint32_t));
    std::memcpy(values, t.values_data(), t.values_size() * sizeof(uint32_t));
}

// SparseTernaryTensor::pack_with_pruning (sparse_ternary_tensor.h:123-191).
void ref_pack_with_pruning(const float* latent, int rows, int cols, uint32_t* meta,
                           uint32_t* values) {
    auto t = SparseTernaryTensor::pack_with_pruning(latent, rows, cols);
    std::memcpy(meta, t.meta_data(), t.meta_size() * sizeof(uint32_t));
    std::memcpy(values, t.values_data(), t.values_size() * sizeof(uint32_t));
}

// SparseTernaryTensor::unpack_to_int8 (sparse_ternary_tensor.h:197-232), on
// arrays loaded back into a tensor through pack_from_dense's layout.
void ref_unpack(const uint32_t* meta, const uint32_t* values, int rows, int cols,
                int8_t* out) {
    // Rebuild a tensor holding exactly these words: unpack -> pack is the
    // identity on well-formed data, and the words are then copied verbatim.
    SparseTernaryTensor t(rows, cols);
    auto* m = const_cast<uint32_t*>(t.meta_data());
    auto* v = const_cast<uint32_t*>(t.values_data());
    std::memcpy(m, meta, t.meta_size() * sizeof(uint32_t));
    std::memcpy(v, values, t.values_size() * sizeof(uint32_t));
    t.unpack_to_int8(out);
}

// cpu_sparse_gemv as the reference's tests and benchmark compute it
// (tests/test_sparse_ternary.cu:17-33 = benchmarks/bench_kernels.cu:89-103):
// the reference's own unpack_to_int8, then a dense int32 multiply-accumulate.
// Used as the timed CPU baseline; single thread, like the reference.
void ref_cpu_sparse_gemv(const uint32_t* meta, const uint32_t* values, const int8_t* x,
                         int32_t* y, int rows, int cols) {
    SparseTernaryTensor t(rows, cols);
    std::memcpy(const_cast<uint32_t*>(t.meta_data()), meta, t.meta_size() * sizeof(uint32_t));
    std::memcpy(const_cast<uint32_t*>(t.values_data()), values,
                t.values_size() * sizeof(uint32_t));
    std::vector<int8_t> dense(static_cast<size_t>(rows) * cols);
    t.unpack_to_int8(dense.data());
    for (int r = 0; r < rows; ++r) {
        int32_t sum = 0;
        for (int c = 0; c < cols; ++c)
            sum += static_cast<int32_t>(dense[static_cast<size_t>(r) * cols + c]) *
                   static_cast<int32_t>(x[c]);
        y[r] = sum;
    }
}

// Inputs of tests/test_sparse_ternary.cu: ternary weights from
// uniform_int_distribution(-1,1) and a random 2:4 mask via std::shuffle per
// group (:192-205, :260-271, :338-349), then x from uniform(-5,5) drawn from
// the same engine afterwards (:277-279, :355-357) when want_x is set.
void ref_make_test_case(unsigned seed, int rows, int cols, int want_x, int8_t* w,
                        uint8_t* mask, int8_t* x) {
    const int total = rows * cols;
    std::mt19937 rng(seed);
    std::uniform_int_distribution<int> wdist(-1, 1);
    std::fill(mask, mask + total, 0);
    for (int i = 0; i < total; i += 4) {
        for (int j = 0; j < 4; ++j) w[i + j] = static_cast<int8_t>(wdist(rng));
        int idx[4] = {0, 1, 2, 3};
        std::shuffle(idx, idx + 4, rng);
        mask[i + idx[0]] = 1;
        mask[i + idx[1]] = 1;
    }
    if (want_x) {
        std::uniform_int_distribution<int> xdist(-5, 5);
        for (int c = 0; c < cols; ++c) x[c] = static_cast<int8_t>(xdist(rng));
    }
}

}  // extern "C"

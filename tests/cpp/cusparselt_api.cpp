// Host program with the reference's cuSPARSELt-backend call sequence
// (tests/test_cusparselt.cu:127-201: construct, prepare, execute,
// get_pruned_weights), written against this build's C++ mirror
// include/spbitnet/cusparselt_backend.h.
//
// usage: cusparselt_api DIR M K N
// reads DIR/A.bin (int8 [M][K] row-major) and DIR/B.bin (int8 [K x N]
// column-major); writes DIR/D.bin (int32 [M x N] column-major) and
// DIR/pruned.bin (int8 [M][K]).
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "spbitnet/cusparselt_backend.h"

namespace {

template <class T>
std::vector<T> read_file(const std::string& path, size_t n) {
    std::vector<T> v(n);
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f || std::fread(v.data(), sizeof(T), n, f) != n) {
        std::fprintf(stderr, "cannot read %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
    return v;
}

template <class T>
void write_file(const std::string& path, const std::vector<T>& v) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

#define HIP_OK(call)                                                        \
    do {                                                                    \
        if ((call) != hipSuccess) {                                         \
            std::fprintf(stderr, "%s failed at line %d\n", #call, __LINE__); \
            std::exit(3);                                                   \
        }                                                                   \
    } while (0)

}  // namespace

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s DIR M K N\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const int m = std::atoi(argv[2]), k = std::atoi(argv[3]), n = std::atoi(argv[4]);
    const size_t a_bytes = static_cast<size_t>(m) * k, b_bytes = static_cast<size_t>(k) * n;
    const std::vector<int8_t> A = read_file<int8_t>(dir + "/A.bin", a_bytes);
    const std::vector<int8_t> B = read_file<int8_t>(dir + "/B.bin", b_bytes);
    int8_t *d_weights = nullptr, *d_pruned = nullptr, *d_B = nullptr;
    int32_t* d_D = nullptr;
    HIP_OK(hipMalloc(&d_weights, a_bytes));
    HIP_OK(hipMalloc(&d_pruned, a_bytes));
    HIP_OK(hipMalloc(&d_B, b_bytes));
    HIP_OK(hipMalloc(&d_D, sizeof(int32_t) * m * n));
    HIP_OK(hipMemcpy(d_weights, A.data(), a_bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_B, B.data(), b_bytes, hipMemcpyHostToDevice));
    {
        spbitnet::CuSparseLtGemm ctx(m, k, n);
        ctx.prepare(d_weights);
        ctx.execute(d_B, d_D);
        ctx.get_pruned_weights(d_pruned);
        HIP_OK(hipDeviceSynchronize());
        std::printf("m %d k %d n %d\n", ctx.m(), ctx.k(), ctx.n());
    }
    std::vector<int32_t> D(static_cast<size_t>(m) * n);
    std::vector<int8_t> P(a_bytes);
    HIP_OK(hipMemcpy(D.data(), d_D, sizeof(int32_t) * D.size(), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(P.data(), d_pruned, a_bytes, hipMemcpyDeviceToHost));
    write_file(dir + "/D.bin", D);
    write_file(dir + "/pruned.bin", P);
    HIP_OK(hipFree(d_weights));
    HIP_OK(hipFree(d_pruned));
    HIP_OK(hipFree(d_B));
    HIP_OK(hipFree(d_D));
    return 0;
}

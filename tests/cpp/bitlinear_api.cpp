// Host program with the reference's BitLinear call pair,
// InferenceEngine::bitlinear (src/inference.cu:106-117), written against this
// build's C++ mirror of the reference's kernel headers
// (include/spbitnet/sparse_ternary_kernels.h, inference_kernels.h): the
// absmax reduction into a device scalar, then the fused sparse BitLinear, for
// fp16 (half) and bf16 (__hip_bfloat16) activations.
//
// usage: bitlinear_api DIR ROWS COLS META_STRIDE VALUES_STRIDE GAMMA
// reads DIR/meta.bin, DIR/values.bin (uint32), DIR/x_f16.bin, DIR/x_bf16.bin
// (16-bit bit patterns, COLS each); writes DIR/out_f16.bin, DIR/out_bf16.bin
// (ROWS each).
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "spbitnet/inference_kernels.h"
#include "spbitnet/sparse_ternary_kernels.h"

namespace {

struct SparseLinear {  // the fields InferenceEngine::bitlinear reads (model.h:46-60)
    uint32_t* d_meta;
    uint32_t* d_values;
    float gamma;
    int rows, cols, meta_stride, values_stride;
};

// The reference's engine member, with the engine's absmax scratch.
template <class T>
struct BitLinearCaller {
    float* d_absmax_;
    void bitlinear(const T* input, int input_size, const SparseLinear& layer, T* output) {
        spbitnet::absmax_reduce_gpu(input, d_absmax_, input_size);
        spbitnet::fused_sparse_bitlinear_gpu(layer.d_meta, layer.d_values, input, output,
                                             d_absmax_, layer.gamma, layer.rows, layer.cols,
                                             layer.meta_stride, layer.values_stride);
    }
};

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

template <class T>
void run(const std::string& dir, const char* tag, const SparseLinear& layer, float* d_absmax) {
    const std::vector<uint16_t> x =
        read_file<uint16_t>(dir + "/x_" + tag + ".bin", static_cast<size_t>(layer.cols));
    T *d_x = nullptr, *d_y = nullptr;
    HIP_OK(hipMalloc(&d_x, sizeof(T) * layer.cols));
    HIP_OK(hipMalloc(&d_y, sizeof(T) * layer.rows));
    HIP_OK(hipMemcpy(d_x, x.data(), sizeof(T) * layer.cols, hipMemcpyHostToDevice));
    BitLinearCaller<T>{d_absmax}.bitlinear(d_x, layer.cols, layer, d_y);
    HIP_OK(hipDeviceSynchronize());
    std::vector<uint16_t> y(static_cast<size_t>(layer.rows));
    HIP_OK(hipMemcpy(y.data(), d_y, sizeof(T) * layer.rows, hipMemcpyDeviceToHost));
    write_file(dir + "/out_" + tag + ".bin", y);
    HIP_OK(hipFree(d_x));
    HIP_OK(hipFree(d_y));
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 7) {
        std::fprintf(stderr, "usage: %s DIR ROWS COLS META_STRIDE VALUES_STRIDE GAMMA\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    SparseLinear layer{nullptr, nullptr, std::strtof(argv[6], nullptr), std::atoi(argv[2]),
                       std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5])};
    const size_t nm = static_cast<size_t>(layer.rows) * layer.meta_stride;
    const size_t nv = static_cast<size_t>(layer.rows) * layer.values_stride;
    const std::vector<uint32_t> meta = read_file<uint32_t>(dir + "/meta.bin", nm);
    const std::vector<uint32_t> values = read_file<uint32_t>(dir + "/values.bin", nv);
    HIP_OK(hipMalloc(&layer.d_meta, 4 * nm));
    HIP_OK(hipMalloc(&layer.d_values, 4 * nv));
    HIP_OK(hipMemcpy(layer.d_meta, meta.data(), 4 * nm, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(layer.d_values, values.data(), 4 * nv, hipMemcpyHostToDevice));
    float* d_absmax = nullptr;
    HIP_OK(hipMalloc(&d_absmax, sizeof(float)));
    run<half>(dir, "f16", layer, d_absmax);
    run<__hip_bfloat16>(dir, "bf16", layer, d_absmax);
    HIP_OK(hipFree(layer.d_meta));
    HIP_OK(hipFree(layer.d_values));
    HIP_OK(hipFree(d_absmax));
    std::printf("bitlinear ok %d x %d\n", layer.rows, layer.cols);
    return 0;
}

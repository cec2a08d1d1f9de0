// Host program written against the reference's kernel API names: compiles
// and links against the MI355X library through include/spbitnet/.  Run on a
// machine without a GPU it only makes zero-size calls (the reference's
// no-op rule), which return before touching the HIP runtime.
#include <cstdio>

#include "spbitnet/inference_kernels.h"
#include "spbitnet/sparse_ternary_kernels.h"

int main() {
    uint32_t* meta = nullptr;
    uint32_t* values = nullptr;
    int8_t* x = nullptr;
    int32_t* y = nullptr;
    spbitnet::sparse_ternary_gemv_gpu(meta, values, x, y, /*rows=*/0, /*cols=*/2560, 80, 40);
    spbitnet::sparse_ternary_unpack_gpu(meta, values, x, 0, 2560, 80, 40);
    half* hx = nullptr;
    spbitnet::fused_sparse_bitlinear_gpu(meta, values, hx, hx, nullptr, 1.0f, 0, 2560, 80, 40);
    __hip_bfloat16* bx = nullptr;
    spbitnet::fused_sparse_bitlinear_gpu(meta, values, bx, bx, nullptr, 1.0f, 2560, 0, 0, 0);
    spbitnet::absmax_reduce_gpu(bx, nullptr, 0);
    spbitnet::dequantize_gpu(y, hx, nullptr, 1.0f, 0);
    spbitnet::rms_norm_gpu(hx, nullptr, hx, 0, 1e-5f);
    spbitnet::rope_gpu(bx, 0, 128, 0, 500000.0f);
    spbitnet::relu2_mul_f32_gpu(hx, hx, nullptr, 0);
    spbitnet::residual_add_gpu(bx, bx, bx, 0);
    spbitnet::half_gemv_gpu(hx, hx, nullptr, 0, 2560);
    std::printf("mirror api ok (abi %d)\n", spb_abi_version());
    return 0;
}

/*
 * spbitnet_amd.h -- C ABI of the MI355X (gfx950) sparse-ternary hot path.
 *
 * Plain pointers and sizes; no HIP or torch types.  Every pointer except the
 * scalar arguments is caller-owned DEVICE memory; no entry point allocates
 * or frees.  `stream` is a hipStream_t passed as void* (NULL = the null
 * stream); launches are asynchronous on it, like the reference's wrappers.
 *
 * Return value: 0 on success, otherwise a hipError_t code (1 =
 * hipErrorInvalidValue for rejected arguments); spb_last_error_string()
 * then describes the failure.  Entry points never exit the process (the
 * reference's CUDA_CHECK does, include/spbitnet/cuda_utils.h:13-21; the C++
 * mirror in include/spbitnet/ restores that behaviour for drop-in callers).
 * rows == 0 or cols == 0 (size == 0) is a successful no-op, as in the
 * reference (src/kernels/sparse_ternary.cu:244, 261, 280).
 *
 * Weight layout (reference include/spbitnet/sparse_ternary_tensor.h:12-39):
 *   meta   uint32 [rows][meta_row_stride],   meta_row_stride  >= ceil(cols/32)
 *   values uint32 [rows][values_row_stride], values_row_stride >= ceil(cols/64)
 * cols must be a multiple of 4.  Every 4-bit bitmap must have exactly two
 * bits set (the format's invariant); results for malformed bitmaps are
 * unspecified.
 *
 * 16-bit activations are passed as uint16_t bit patterns (IEEE fp16 for the
 * _f16 entry points, bfloat16 for _bf16).
 */
#ifndef SPBITNET_AMD_H
#define SPBITNET_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* spb_stream_t;

/* Version of this ABI (major*100 + minor). */
int spb_abi_version(void);

/* Message for the last failing call on this host thread ("" if none). */
const char* spb_last_error_string(void);

/* Replaces spbitnet::sparse_ternary_unpack_gpu
 * (reference include/spbitnet/sparse_ternary_kernels.h:16-19,
 *  src/kernels/sparse_ternary.cu:240-254).
 * out: int8 [rows][cols] row-major dense {-1,0,+1}. */
int spb_sparse_ternary_unpack(const uint32_t* meta, const uint32_t* values, int8_t* out,
                              int rows, int cols, int meta_row_stride,
                              int values_row_stride, spb_stream_t stream);

/* Replaces spbitnet::sparse_ternary_gemv_gpu
 * (reference include/spbitnet/sparse_ternary_kernels.h:29-33,
 *  src/kernels/sparse_ternary.cu:256-272).
 * y[r] = sum_c W[r][c] * x[c] as exact int32; x int8 [cols], y int32 [rows]. */
int spb_sparse_ternary_gemv(const uint32_t* meta, const uint32_t* values, const int8_t* x,
                            int32_t* y, int rows, int cols, int meta_row_stride,
                            int values_row_stride, spb_stream_t stream);

/* Replaces spbitnet::fused_sparse_bitlinear_gpu
 * (reference include/spbitnet/sparse_ternary_kernels.h:43-48,
 *  src/kernels/sparse_ternary.cu:181-234, 274-291), fp16 in / fp16 out.
 * q = clamp(rint(x * (absmax>0 ? 127/absmax : 0)), -128, 127) per element,
 * acc = W q (int32), output[r] = fp16(float(acc) * ((gamma*absmax)/127)).
 * d_absmax: device float written by spb_absmax_reduce_* on the same stream. */
int spb_fused_sparse_bitlinear_f16(const uint32_t* meta, const uint32_t* values,
                                   const uint16_t* x, uint16_t* output,
                                   const float* d_absmax, float gamma, int rows, int cols,
                                   int meta_row_stride, int values_row_stride,
                                   spb_stream_t stream);

/* Same as spb_fused_sparse_bitlinear_f16 with bfloat16 input and output
 * (BitNet-2B-4T-shape decode stores activations in bf16). */
int spb_fused_sparse_bitlinear_bf16(const uint32_t* meta, const uint32_t* values,
                                    const uint16_t* x, uint16_t* output,
                                    const float* d_absmax, float gamma, int rows, int cols,
                                    int meta_row_stride, int values_row_stride,
                                    spb_stream_t stream);

/* Replaces spbitnet::absmax_reduce_gpu
 * (reference include/spbitnet/inference_kernels.h:24-25,
 *  src/kernels/inference_kernels.cu:120-148, 549-553): *d_absmax = max|x|. */
int spb_absmax_reduce_f16(const uint16_t* input, float* d_absmax, int size,
                          spb_stream_t stream);
int spb_absmax_reduce_bf16(const uint16_t* input, float* d_absmax, int size,
                           spb_stream_t stream);

/* Replaces spbitnet::absmax_quantize_gpu
 * (reference include/spbitnet/inference_kernels.h:19-20,
 *  src/kernels/inference_kernels.cu:69-114, 543-547). */
int spb_absmax_quantize_f16(const uint16_t* input, int8_t* output, float* d_absmax,
                            int size, spb_stream_t stream);
int spb_absmax_quantize_bf16(const uint16_t* input, int8_t* output, float* d_absmax,
                             int size, spb_stream_t stream);

/* Replaces spbitnet::dequantize_gpu
 * (reference include/spbitnet/inference_kernels.h:29-30,
 *  src/kernels/inference_kernels.cu:162-171, 555-561):
 * output[i] = 16-bit(float(input[i]) * ((gamma * *d_absmax) / 127)). */
int spb_dequantize_f16(const int32_t* input, uint16_t* output, const float* d_absmax,
                       float gamma, int size, spb_stream_t stream);
int spb_dequantize_bf16(const int32_t* input, uint16_t* output, const float* d_absmax,
                        float gamma, int size, spb_stream_t stream);

/* Replaces InferenceEngine::bitlinear (reference src/inference.cu:106-117:
 * absmax_reduce_gpu into the engine's d_absmax_ scratch, then
 * fused_sparse_bitlinear_gpu) as one call; the scratch comes in as a caller
 * workspace of at least spb_bitlinear_workspace_size(cols) bytes, 16-byte
 * aligned (the absmax, then the quantised activations as bit planes, built
 * once instead of in every GEMV workgroup when cols % 8 == 0 and x is 16-byte
 * aligned).  Output bits equal the reference pair's:
 * output[r] = 16-bit(float(W q) * ((gamma * absmax) / 127)),
 * q = clamp(rint(x * (absmax > 0 ? 127/absmax : 0)), -128, 127).
 * Calls that share a workspace must be ordered (same stream). */
size_t spb_bitlinear_workspace_size(int cols);
int spb_bitlinear_f16(const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                      uint16_t* output, float gamma, int rows, int cols, int meta_row_stride,
                      int values_row_stride, void* workspace, size_t workspace_size,
                      spb_stream_t stream);
int spb_bitlinear_bf16(const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                       uint16_t* output, float gamma, int rows, int cols, int meta_row_stride,
                       int values_row_stride, void* workspace, size_t workspace_size,
                       spb_stream_t stream);

/* No counterpart in the reference: spb_bitlinear_* for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  The workspace is a static device array
 * of the library (spb_bitlinear_workspace_size(32768) bytes, one copy per
 * GPU, held until the process ends); cols above 32768 are rejected.  No
 * allocation happens in the call.  Every call on a GPU shares that GPU's
 * copy: calls that overlap on one GPU (several streams or host threads)
 * race and must be serialised by the caller.  Output bits equal
 * spb_bitlinear_*'s. */
int spb_bitlinear_f16_noalloc(const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                              uint16_t* output, float gamma, int rows, int cols,
                              int meta_row_stride, int values_row_stride, spb_stream_t stream);
int spb_bitlinear_bf16_noalloc(const uint32_t* meta, const uint32_t* values, const uint16_t* x,
                               uint16_t* output, float gamma, int rows, int cols,
                               int meta_row_stride, int values_row_stride, spb_stream_t stream);

/* ---- Batched GEMM ---------------------------------------------------------------
 * Replaces the cuSPARSELt path CuSparseLtGemm(m,k,n) + execute
 * (reference include/spbitnet/cusparselt_backend.h:28-77,
 *  src/cusparselt_backend.cu:38-207): Y[t][r] = sum_c W[r][c] * X[t][c] as
 * exact int32 on the packed 2:4 ternary weights (no library pruning or
 * compression step).  X int8 [n][cols] and Y int32 [n][rows] are token-major,
 * which is the column-major B [K x N] / D [M x N] memory of the reference.
 * Any n >= 1 (the reference requires n >= 16, src/cusparselt_backend.cu:41-45).
 * Runs on the int8 structured-sparse matrix cores (v_smfmac_i32_16x16x128_i8)
 * when cols % 128 == 0 and X is 16-byte aligned, else a general kernel. */
int spb_sparse_ternary_gemm(const uint32_t* meta, const uint32_t* values, const int8_t* X,
                            int32_t* Y, int rows, int cols, int n, int meta_row_stride,
                            int values_row_stride, spb_stream_t stream);

/* The same product on the add/sub bit-plane GEMV kernel (tokens on grid.y),
 * kept as the comparator for the matrix-core kernel.  Needs the bit-plane
 * kernel's shape conditions and cols % 16 == 0. */
int spb_sparse_ternary_gemm_addsub(const uint32_t* meta, const uint32_t* values,
                                   const int8_t* X, int32_t* Y, int rows, int cols, int n,
                                   int meta_row_stride, int values_row_stride,
                                   spb_stream_t stream);

/* Which kernel spb_sparse_ternary_gemm would run: 2 the staged matrix-core
 * kernel (cols % 256 == 0, both row strides multiples of 4 words, meta,
 * values and X 16-byte aligned), 1 the direct matrix-core kernel (cols % 128
 * == 0, X 16-byte aligned), 0 the general kernel.  Host-only query; no
 * reference counterpart. */
int spb_sparse_ternary_gemm_kernel_id(const uint32_t* meta, const uint32_t* values,
                                      const int8_t* X, int rows, int cols, int n,
                                      int meta_row_stride, int values_row_stride);

/* ---- 2:4 structured-sparse int8 GEMM (the cuSPARSELt backend) ------------
 * Replaces spbitnet::CuSparseLtGemm (reference include/spbitnet/
 * cusparselt_backend.h:28-77, src/cusparselt_backend.cu:38-219): a dense
 * int8 weight matrix A [m][k] (row-major; any int8 values) is pruned to 2:4
 * along k and compressed once (prepare), then D = A_pruned * B runs on the
 * int8 sparse matrix cores (execute).  Pruning keeps, in every group of
 * four columns, the two largest |a| (on equal magnitudes the higher index);
 * a group with at most two non-zeros is kept whole, so a matrix already in
 * 2:4 form is unchanged (the reference uses cuSPARSELt's STRIP rule, which
 * is not specified there).  The compressed operand is this build's own
 * tile-ordered layout (the library's internal format in the reference):
 * callers size it with spb_sparse_i8_compressed_size and treat it as
 * opaque.  k must be a multiple of 4; m * k < 2^31.  Nothing allocates. */

/* Bytes of the compressed operand of an m x k matrix (the size query of
 * cusparseLtSpMMACompressedSize, src/cusparselt_backend.cu:140-146);
 * -1 for a rejected shape (k % 4 != 0, negative, m * k >= 2^31). */
long spb_sparse_i8_compressed_size(int m, int k);

/* CuSparseLtGemm::prepare (src/cusparselt_backend.cu:107-166): prune A and
 * write the compressed operand; `pruned` (nullable) receives the pruned
 * dense matrix [m][k].  A and pruned 4-byte aligned, compressed 16-byte
 * aligned. */
int spb_sparse_i8_prune_compress(const int8_t* A, int8_t* pruned, void* compressed, int m, int k,
                                 spb_stream_t stream);

/* cusparseLtSpMMAPruneCheck as prepare uses it (src/cusparselt_backend.cu:
 * 123-136): *d_invalid (device int) receives the number of groups of A with
 * more than two non-zeros (0 = A is in 2:4 form). */
int spb_sparse_i8_prune_check(const int8_t* A, int m, int k, int* d_invalid, spb_stream_t stream);

/* CuSparseLtGemm::get_pruned_weights (src/cusparselt_backend.cu:209-217):
 * the pruned dense matrix [m][k] from the compressed operand.  out 4-byte
 * aligned. */
int spb_sparse_i8_decompress(const void* compressed, int8_t* out, int m, int k,
                             spb_stream_t stream);

/* CuSparseLtGemm::execute (src/cusparselt_backend.cu:173-207):
 * D = A_pruned * B with exact int32 accumulation; B int8 [k x n]
 * column-major (= [n][k], token-major), D int32 [m x n] column-major
 * (= [n][m]).  Any n >= 1 (the reference requires n >= 16,
 * src/cusparselt_backend.cu:41-45).  Runs on v_smfmac_i32_16x16x128_i8 when
 * k % 16 == 0 and B is 16-byte aligned, else on a general kernel. */
int spb_sparse_i8_gemm(const void* compressed, const int8_t* B, int32_t* D, int m, int k, int n,
                       spb_stream_t stream);

/* Which kernel spb_sparse_i8_gemm would run: 1 the matrix-core kernel,
 * 0 the general kernel.  Host-only query; no reference counterpart. */
int spb_sparse_i8_gemm_kernel_id(const void* compressed, const int8_t* B, int m, int k, int n);

/* ---- Bit-plane activation layout -------------------------------------------
 * No reference counterpart: an activation layout of this build.  An int8
 * vector of `cols` columns is stored as 8 * ceil(cols/32) uint32 words;
 * word [w*8 + b] holds bit b (two's complement) of columns 32w .. 32w+31,
 * column 32w+j at bit j; columns beyond `cols` are 0.  Same size as the
 * int8 vector.  The GEMV kernel consumes activations in this form; producing
 * it once per activation vector, instead of in every GEMV workgroup, is what
 * these entry points are for.  Buffers must be 16-byte aligned. */

/* int8 x [cols] -> planes.  cols % 8 == 0; x 8-byte aligned. */
int spb_activation_planes(const int8_t* x, uint32_t* planes, int cols, spb_stream_t stream);

/* absmax_quantize (as spb_absmax_quantize_*) writing the plane layout, the
 * absmax, and, when `output` is non-NULL, the int8 vector as well.
 * size % 8 == 0; input 16-byte aligned. */
int spb_absmax_quantize_planes_f16(const uint16_t* input, uint32_t* planes, int8_t* output,
                                   float* d_absmax, int size, spb_stream_t stream);
int spb_absmax_quantize_planes_bf16(const uint16_t* input, uint32_t* planes, int8_t* output,
                                    float* d_absmax, int size, spb_stream_t stream);

/* spb_sparse_ternary_gemv with the weight loads on the default cache policy
 * instead of the non-temporal one: for matrices re-read while they stay in
 * the 256 MB Infinity Cache (a model or a set of layers that fits it), where
 * the streaming hint would evict them.  Same arguments, results and shape
 * rules.  No reference counterpart (the reference has one GEMV). */
int spb_sparse_ternary_gemv_resident(const uint32_t* meta, const uint32_t* values,
                                     const int8_t* x, int32_t* y, int rows, int cols,
                                     int meta_row_stride, int values_row_stride,
                                     spb_stream_t stream);

/* spb_sparse_ternary_gemv with the activations given as planes; results are
 * identical to the int8 entry point on the same activations. */
int spb_sparse_ternary_gemv_planes(const uint32_t* meta, const uint32_t* values,
                                   const uint32_t* planes, int32_t* y, int rows, int cols,
                                   int meta_row_stride, int values_row_stride,
                                   spb_stream_t stream);

/* BitLinear on already-quantised plane activations: the GEMV followed by the
 * reference's dequant epilogue, output[r] = 16-bit(float(acc) * ((gamma *
 * *d_absmax) / 127)); identical to spb_fused_sparse_bitlinear_* when the
 * planes come from spb_absmax_quantize_planes_* of the same input. */
int spb_fused_sparse_bitlinear_planes_f16(const uint32_t* meta, const uint32_t* values,
                                          const uint32_t* planes, uint16_t* output,
                                          const float* d_absmax, float gamma, int rows,
                                          int cols, int meta_row_stride, int values_row_stride,
                                          spb_stream_t stream);
int spb_fused_sparse_bitlinear_planes_bf16(const uint32_t* meta, const uint32_t* values,
                                           const uint32_t* planes, uint16_t* output,
                                           const float* d_absmax, float gamma, int rows,
                                           int cols, int meta_row_stride, int values_row_stride,
                                           spb_stream_t stream);

/* Which GEMV kernel a call with these arguments runs: 1 = the bit-plane
 * kernel (cols % 128 == 0, cols <= 32768, 16-byte aligned meta rows, 8-byte
 * aligned values rows; the int8 / fp16 / bf16 activation pointer must also be
 * 16-byte aligned), 0 = the general kernel.  Host-only query, no launch;
 * no reference counterpart (the reference has a single kernel). */
int spb_sparse_ternary_gemv_kernel_id(const uint32_t* meta, const uint32_t* values,
                                      int rows, int cols, int meta_row_stride,
                                      int values_row_stride);


/* ---- per-op inference kernels ---------------------------------------------
 * The reference's op-by-op wrappers (include/spbitnet/inference_kernels.h:14-87,
 * src/kernels/inference_kernels.cu), each for fp16 (_f16) and bf16 (_bf16)
 * storage; 16-bit tensors are passed as their bit patterns (uint16_t).
 * float32 arithmetic; outputs rounded once to the storage type.  Sizes of 0
 * are no-ops; negative sizes, null pointers and inconsistent shapes return
 * an error (nothing is launched). */

/* rms_norm_gpu (inference_kernels.h:14-15): y = (x * inv) * w,
 * inv = 1 / sqrt(mean(x^2) + eps); x and y may alias. */
int spb_rms_norm_f16(const uint16_t* input, const float* weight, uint16_t* output, int size,
                     float eps, spb_stream_t stream);
int spb_rms_norm_bf16(const uint16_t* input, const float* weight, uint16_t* output, int size,
                      float eps, spb_stream_t stream);
/* rms_norm_f32in_gpu (inference_kernels.h:75-76): float32 input. */
int spb_rms_norm_f32in_f16(const float* input, const float* weight, uint16_t* output, int size,
                           float eps, spb_stream_t stream);
int spb_rms_norm_f32in_bf16(const float* input, const float* weight, uint16_t* output, int size,
                            float eps, spb_stream_t stream);
/* rope_gpu (inference_kernels.h:33-34): in place on (num_heads, head_dim). */
int spb_rope_f16(uint16_t* vec, int num_heads, int head_dim, int pos, float theta,
                 spb_stream_t stream);
int spb_rope_bf16(uint16_t* vec, int num_heads, int head_dim, int pos, float theta,
                  spb_stream_t stream);
/* scatter_kv_gpu (inference_kernels.h:38-40): cache (num_kv_heads,
 * max_seq_len, head_dim); 0 <= pos < max_seq_len. */
int spb_scatter_kv(const uint16_t* src, uint16_t* cache, int num_kv_heads, int head_dim,
                   int max_seq_len, int pos, spb_stream_t stream);
/* attention_scores_gpu (inference_kernels.h:45-48): scores (num_heads,
 * max_seq_len), the first seq_len per head written; kv = h * nkv / nh. */
int spb_attention_scores_f16(const uint16_t* Q, const uint16_t* K_cache, float* scores,
                             int num_heads, int num_kv_heads, int head_dim, int max_seq_len,
                             int seq_len, float scale, spb_stream_t stream);
int spb_attention_scores_bf16(const uint16_t* Q, const uint16_t* K_cache, float* scores,
                              int num_heads, int num_kv_heads, int head_dim, int max_seq_len,
                              int seq_len, float scale, spb_stream_t stream);
/* softmax_gpu (inference_kernels.h:52-53): in place per head. */
int spb_softmax(float* scores, int num_heads, int max_seq_len, int seq_len, spb_stream_t stream);
/* attention_output_gpu (inference_kernels.h:58-61); head_dim <= 256. */
int spb_attention_output_f16(const float* scores, const uint16_t* V_cache, uint16_t* output,
                             int num_heads, int num_kv_heads, int head_dim, int max_seq_len,
                             int seq_len, spb_stream_t stream);
int spb_attention_output_bf16(const float* scores, const uint16_t* V_cache, uint16_t* output,
                              int num_heads, int num_kv_heads, int head_dim, int max_seq_len,
                              int seq_len, spb_stream_t stream);
/* relu2_mul_gpu / relu2_mul_f32_gpu (inference_kernels.h:64-71):
 * out = (max(0, g)^2) * u. */
int spb_relu2_mul_f16(const uint16_t* gate, const uint16_t* up, uint16_t* output, int size,
                      spb_stream_t stream);
int spb_relu2_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* output, int size,
                       spb_stream_t stream);
int spb_relu2_mul_f32_f16(const uint16_t* gate, const uint16_t* up, float* output, int size,
                          spb_stream_t stream);
int spb_relu2_mul_f32_bf16(const uint16_t* gate, const uint16_t* up, float* output, int size,
                           spb_stream_t stream);
/* float_to_half_gpu (inference_kernels.h:79-80). */
int spb_float_to_f16(const float* input, uint16_t* output, int size, spb_stream_t stream);
int spb_float_to_bf16(const float* input, uint16_t* output, int size, spb_stream_t stream);
/* residual_add_gpu (inference_kernels.h:83-84): out = a + b (float32 add). */
int spb_residual_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* output, int size,
                         spb_stream_t stream);
int spb_residual_add_bf16(const uint16_t* a, const uint16_t* b, uint16_t* output, int size,
                          spb_stream_t stream);
/* half_gemv_gpu (inference_kernels.h:87-89): y (float32) = W x, W (rows,
 * cols) 16-bit. */
int spb_gemv_f16(const uint16_t* W, const uint16_t* x, float* y, int rows, int cols,
                 spb_stream_t stream);
int spb_gemv_bf16(const uint16_t* W, const uint16_t* x, float* y, int rows, int cols,
                  spb_stream_t stream);
/* Greedy pick on the device: *out_index = index of max(x) (lowest index among
 * equal maxima); replaces the host std::max_element over copied logits
 * (src/main.cpp:194-200). */
int spb_argmax_f32(const float* x, int n, int* out_index, spb_stream_t stream);

/* ---- decode engine --------------------------------------------------------
 * bs=1 greedy decode of a BitNet b1.58 transformer whose linear layers are
 * 2:4 sparse-ternary, with bf16 activations, bf16 KV cache and a bf16 tied or
 * separate LM head.  One token step is a HIP graph of 5 kernels per layer
 * plus the LM head; greedy generation runs entirely on the device.
 * Replaces the reference's InferenceEngine (include/spbitnet/inference.h:23-70,
 * src/inference.cu:16-283) and its generate loop (src/main.cpp:119-200).
 * Constraints: every projection takes the bit-plane kernel (cols % 128 == 0,
 * meta_stride % 4 == 0, values_stride % 2 == 0, 16/8-byte aligned rows),
 * head_dim even and <= 128, at most 8 query heads per kv head,
 * hidden_size <= 8192. */

/* SparseLinear (reference include/spbitnet/model.h:46-60). */
typedef struct spb_sparse_linear {
    const uint32_t* meta;
    const uint32_t* values;
    float gamma;
    int rows, cols, meta_stride, values_stride;
} spb_sparse_linear;

/* TransformerLayer (reference include/spbitnet/model.h:63-82); norm weights
 * are device float32; attn_sub_norm / ffn_sub_norm may be NULL (skipped, as
 * in src/inference.cu:205-210, 239-245). */
typedef struct spb_transformer_layer {
    spb_sparse_linear q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj;
    const float* input_layernorm;
    const float* post_attention_layernorm;
    const float* attn_sub_norm;
    const float* ffn_sub_norm;
} spb_transformer_layer;

/* ModelConfig (reference include/spbitnet/model.h:23-40), numeric fields. */
typedef struct spb_model_config {
    int hidden_size, num_hidden_layers, num_attention_heads, num_key_value_heads;
    int intermediate_size, vocab_size, max_position_embeddings, head_dim;
    float rms_norm_eps, rope_theta;
    int bos_token_id, eos_token_id;
} spb_model_config;

typedef struct spb_engine spb_engine;

/* InferenceEngine(const Model&) (inference.h:27): borrows the weights (they
 * must outlive the engine), allocates the KV cache for max_seq positions and
 * scratch, and captures the token-step graph.  embed_tokens / lm_head: bf16
 * [vocab][hidden]; lm_head NULL = tied to the embedding. */
int spb_engine_create(const spb_model_config* config, const spb_transformer_layer* layers,
                      const uint16_t* embed_tokens, const uint16_t* lm_head,
                      const float* final_norm, int max_seq, spb_engine** engine);
int spb_engine_destroy(spb_engine* engine);
/* Stream the engine's graphs run on (default: the null stream). */
int spb_engine_set_stream(spb_engine* engine, spb_stream_t stream);
/* InferenceEngine::reset (inference.h:36; inference.cu:92-101). */
int spb_engine_reset(spb_engine* engine);
/* InferenceEngine::forward (inference.h:33; inference.cu:126-283): one token
 * at the next position; *d_logits = device float32 [vocab] (valid until the
 * next call; ordered on the engine stream).  After spb_engine_generate or
 * spb_engine_decode_steps it continues at the position those reached (read
 * back from the device), in forward mode: no EOS stop, no token writes. */
int spb_engine_forward(spb_engine* engine, int token_id, const float** d_logits);
/* InferenceEngine::seq_len (inference.h:38).  After spb_engine_decode_steps
 * it synchronises the engine stream to read the position back (-1 on error). */
int spb_engine_seq_len(const spb_engine* engine);
/* Greedy generation (src/main.cpp:133-155): reset, prefill prompt[0..n-1)
 * one token at a time, then n_new greedy steps starting from the last prompt
 * token (argmax = lowest index among maxima); stops after EOS when
 * stop_at_eos.  All steps are graph launches; the host waits once. */
int spb_engine_generate(spb_engine* engine, const int* prompt, int n_prompt, int n_new,
                        int stop_at_eos, int* out_tokens, int* n_generated);
/* No reference counterpart (the reference feeds a prompt one token at a
 * time).  spb_engine_generate prefills a prompt with at least min_tokens
 * tokens before its last in batches through the layers: per-token
 * producers and sinks of the decode step around the matrix-core GEMM, and a
 * prefill form of the attention kernel.  The KV cache and every generated
 * token are identical to one decode step per prompt token.  0 = always one
 * step per token; default 16. */
int spb_engine_set_prefill_batch(spb_engine* engine, int min_tokens);
/* Launches `steps` more token steps continuing the current state (timing
 * loops); no host synchronisation.  The host learns the new position when
 * spb_engine_seq_len or spb_engine_forward is next called. */
int spb_engine_decode_steps(spb_engine* engine, int steps);
/* Device buffers: logits float32 [vocab], tokens int32 [max_seq + 1]. */
int spb_engine_buffers(const spb_engine* engine, const float** logits, const int** tokens);

/* ---- batched decode engine --------------------------------------------------
 * No reference counterpart: the reference decodes one sequence per engine
 * (InferenceEngine::forward, src/inference.cu:123-283).  BASELINE config 4
 * decodes several sequences at once; this engine steps `batch` independent
 * sequences per HIP-graph replay, each with its own KV cache of max_seq
 * positions, position and token buffer.  Every value of a sequence's step is
 * computed by the same device code, in the same order, as the bs=1 engine,
 * so each sequence's greedy tokens equal those of spb_engine_generate on
 * that sequence alone.  Same model constraints as spb_engine_create, plus
 * hidden_size <= 4096 (the batched LM head keeps 8 normalised vectors in
 * LDS); 1 <= batch <= 1024. */
typedef struct spb_batch_engine spb_batch_engine;
int spb_batch_engine_create(const spb_model_config* config, const spb_transformer_layer* layers,
                            const uint16_t* embed_tokens, const uint16_t* lm_head,
                            const float* final_norm, int max_seq, int batch,
                            spb_batch_engine** engine);
int spb_batch_engine_destroy(spb_batch_engine* engine);
int spb_batch_engine_set_stream(spb_batch_engine* engine, spb_stream_t stream);
/* Greedy generation of n_seq <= batch sequences: prompts concatenated,
 * prompt_lens[n_seq] (each >= 1, prompt + n_new <= max_seq).  Each prompt's
 * tokens before its last are prefilled through the layers into the
 * sequence's cache (the batched prefill of spb_engine_generate); then n_new
 * graph steps each advance every sequence by one token (src/main.cpp:133-155
 * per sequence).  out_tokens [n_seq][n_new] (-1 after a sequence stopped at
 * EOS when stop_at_eos), n_generated [n_seq] (nullable).  The host waits once. */
int spb_batch_engine_generate(spb_batch_engine* engine, const int* prompts,
                              const int* prompt_lens, int n_seq, int n_new, int stop_at_eos,
                              int* out_tokens, int* n_generated);
/* `steps` more batched steps continuing the current states (timing loops);
 * no host synchronisation. */
int spb_batch_engine_decode_steps(spb_batch_engine* engine, int steps);
/* Device buffers: logits float32 [batch][vocab], tokens int32
 * [batch][max_seq + 1]. */
int spb_batch_engine_buffers(const spb_batch_engine* engine, const float** logits,
                             const int** tokens);

/* ---- model loading ----------------------------------------------------------
 * Model::load (reference include/spbitnet/model.h:99-103, src/model.cu:72-311)
 * for the on-disk format of python/convert_model.py (docs/compression_format.md
 * section 4): config.json, manifest.json, .meta/.values uint32 files, float32
 * norm files, fp16 embedding / LM head (converted to bf16 on upload; a
 * manifest dtype "bfloat16" is taken as is).  The model owns its device
 * memory; engines created from spb_model_info borrow it. */
typedef struct spb_model spb_model;
int spb_model_load(const char* model_dir, spb_model** model);
int spb_model_destroy(spb_model* model);
/* Any output pointer may be NULL; *lm_head is NULL for tied weights. */
int spb_model_info(const spb_model* model, spb_model_config* config,
                   const spb_transformer_layer** layers, const uint16_t** embed_tokens,
                   const uint16_t** lm_head, const float** final_norm, size_t* gpu_bytes);

/* ---- random-init weights on the device ------------------------------------
 * Latent W ~ N(0,1) from a counter-based generator (seed, element index),
 * 2:4 top-2 |W| mask (higher index wins ties), kept value sign(W) (W >= 0 ->
 * +1), packed; *d_gamma = mean|W|; latent (nullable) receives W.  The
 * recipe of python/convert_model.py:88-207, 257-316 on a synthetic W.
 * cols % 64 == 0.  Calls on one device must not overlap (they share a
 * 1024-entry partial-sum array). */
int spb_generate_sparse_ternary(uint64_t seed, int rows, int cols, uint32_t* meta,
                                uint32_t* values, int meta_stride, int values_stride,
                                float* d_gamma, float* latent, spb_stream_t stream);
/* out[i] = bf16(std * N(0,1)) from the same generator (embedding init). */
int spb_generate_normal_bf16(uint64_t seed, long n, float std_dev, uint16_t* out,
                             spb_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPBITNET_AMD_H */

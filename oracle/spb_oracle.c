/*
 * spb_oracle.c -- CPU restatement of spbitnet's sparse-ternary hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the spbitnet_amd
 * package, its HIP library, bench.py's GPU leg) links or calls this file.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, and only as the checker.
 *
 * Every function states the reference file:line it restates (paths relative
 * to the reference repository root).  Plain C99, scalar, single thread: the
 * point is to be obviously right, not fast.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   spbo_mask_top2        KATs from tests/test_sparse_ternary.cu:115-141,
 *                         tie cases from convert_model.py's stable argsort,
 *                         brute force over all 4! orderings of a group.
 *   spbo_pack / unpack    KATs (docs/compression_format.md:229-261,
 *                         tests/test_model_loader.cu:95-111), round trips,
 *                         and byte equality with the reference header built
 *                         into oracle/_ref (when /root/reference is present).
 *   spbo_gemv / gemm      golden vectors from the reference tests' own inputs
 *                         (tests/golden), closed forms (all-ones x = row sign
 *                         sum, x = e_j reads column j, bitmap 0x3/sign 0b10
 *                         gives x[4g]-x[4g+1]), linearity in x.
 *   spbo_quantize         closed form, absmax=0, round-half-even ties, clamp.
 *   spbo_dequant / fused  closed form restated with float32 operation order;
 *                         fused == quantize -> gemv -> dequant.
 *   spbo_bf16_round       exhaustive-by-structure checks (ties, NaN, Inf).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define SPBO_GROUP 4
#define SPBO_META_GROUPS_PER_WORD 8    /* sparse_ternary_tensor.h:38 */
#define SPBO_VALUES_GROUPS_PER_WORD 16 /* sparse_ternary_tensor.h:39 */

/* sparse_ternary_tensor.h:254-264 */
int spbo_meta_stride(int cols) {
    int groups = cols / SPBO_GROUP;
    return (groups + SPBO_META_GROUPS_PER_WORD - 1) / SPBO_META_GROUPS_PER_WORD;
}
int spbo_values_stride(int cols) {
    int groups = cols / SPBO_GROUP;
    return (groups + SPBO_VALUES_GROUPS_PER_WORD - 1) / SPBO_VALUES_GROUPS_PER_WORD;
}

/*
 * 2:4 mask from latent magnitudes (python/convert_model.py:88-119).
 * np.argsort(|w|, kind="stable") ascending, keep the last two indices: with
 * equal magnitudes the later (higher) index sorts later, so it wins ties.
 * Equivalently: position i beats j iff |w_i| > |w_j|, or equal and i > j.
 */
void spbo_mask_top2(const float* w, int rows, int cols, uint8_t* mask) {
    for (int r = 0; r < rows; ++r) {
        for (int g = 0; g < cols / 4; ++g) {
            const float* p = w + (size_t)r * cols + 4 * g;
            uint8_t* m = mask + (size_t)r * cols + 4 * g;
            for (int i = 0; i < 4; ++i) {
                /* rank = number of positions that beat i */
                int beaten_by = 0;
                for (int j = 0; j < 4; ++j) {
                    if (j == i) continue;
                    float ai = fabsf(p[i]), aj = fabsf(p[j]);
                    if (aj > ai || (aj == ai && j > i)) ++beaten_by;
                }
                m[i] = (beaten_by < 2) ? 1 : 0;
            }
        }
    }
}

/*
 * Ternary value kept at a masked position (python/convert_model.py:270-283):
 * RoundClip(w/gamma) is +-1 with the sign of w whenever it is non-zero, and a
 * kept zero is forced to +1 if w >= 0 else -1.  Both cases give sign(w) with
 * w >= 0 (including -0.0) mapping to +1, so gamma never changes packed bits.
 */
void spbo_kept_sign(const float* w, const uint8_t* mask, int n, int8_t* out) {
    for (int i = 0; i < n; ++i) out[i] = mask[i] ? (w[i] < 0.0f ? -1 : 1) : 0;
}

/*
 * gamma = mean(|W|) (python/convert_model.py:132).  numpy reduces float32 with
 * pairwise summation; this oracle sums in double, which agrees with numpy to
 * well inside the 1e-3 tolerance applied to dequantised outputs (exact gamma
 * bits are not on the int32 contract).
 */
double spbo_absmean(const float* w, size_t n) {
    double s = 0.0;
    for (size_t i = 0; i < n; ++i) s += fabs((double)w[i]);
    return n ? s / (double)n : 0.0;
}

/* SparseTernaryTensor::pack_from_dense (sparse_ternary_tensor.h:58-108). */
int spbo_pack(const int8_t* w, const uint8_t* mask, int rows, int cols,
              uint32_t* meta, uint32_t* values) {
    if (cols % 4) return -1;
    int ms = spbo_meta_stride(cols), vs = spbo_values_stride(cols);
    memset(meta, 0, (size_t)rows * ms * 4);
    memset(values, 0, (size_t)rows * vs * 4);
    for (int r = 0; r < rows; ++r) {
        for (int g = 0; g < cols / 4; ++g) {
            size_t base = (size_t)r * cols + 4 * g;
            uint32_t bitmap = 0, signs = 0;
            int nz = 0, count = 0;
            for (int i = 0; i < 4; ++i) {
                if (!mask[base + i]) continue;
                ++count;
                bitmap |= 1u << i;
                signs |= (uint32_t)(w[base + i] < 0) << nz;
                ++nz;
            }
            if (count != 2) return -2;
            meta[(size_t)r * ms + g / 8] |= bitmap << ((g % 8) * 4);
            values[(size_t)r * vs + g / 16] |= signs << ((g % 16) * 2);
        }
    }
    return 0;
}

/* SparseTernaryTensor::unpack_to_int8 (sparse_ternary_tensor.h:197-232). */
void spbo_unpack(const uint32_t* meta, const uint32_t* values, int rows, int cols,
                 int ms, int vs, int8_t* out) {
    memset(out, 0, (size_t)rows * cols);
    for (int r = 0; r < rows; ++r) {
        for (int g = 0; g < cols / 4; ++g) {
            uint32_t bitmap = (meta[(size_t)r * ms + g / 8] >> ((g % 8) * 4)) & 0xFu;
            uint32_t signs = (values[(size_t)r * vs + g / 16] >> ((g % 16) * 2)) & 0x3u;
            int nz = 0;
            for (int i = 0; i < 4; ++i) {
                if (!(bitmap & (1u << i))) continue;
                out[(size_t)r * cols + 4 * g + i] = ((signs >> nz) & 1u) ? -1 : 1;
                ++nz;
            }
        }
    }
}

/*
 * cpu_sparse_gemv (tests/test_sparse_ternary.cu:17-33): unpack to dense int8,
 * then a dense int32 multiply-accumulate.  Computed here group by group on
 * the packed words, each group decoded exactly as spbo_unpack decodes it
 * (kept positions ascending, sign bit nz of the group for the nz-th kept
 * position), without the dense copy: the int32 sum is exact, so the result
 * is the unpack-then-MAC value bit for bit.  |acc| <= (cols/2)*128 < 2^31.
 * Rows run in parallel (OpenMP) for large matrices; each row's sum is
 * independent.
 */
void spbo_gemv(const uint32_t* meta, const uint32_t* values, const int8_t* x,
               int32_t* y, int rows, int cols, int ms, int vs) {
    const long work = (long)rows * cols;
#pragma omp parallel for schedule(static) if (work >= (1L << 20))
    for (int r = 0; r < rows; ++r) {
        const uint32_t* mr = meta + (size_t)r * ms;
        const uint32_t* vr = values + (size_t)r * vs;
        int32_t s = 0;
        for (int g = 0; g < cols / 4; ++g) {
            const uint32_t bitmap = (mr[g / 8] >> ((g % 8) * 4)) & 0xFu;
            const uint32_t signs = (vr[g / 16] >> ((g % 16) * 2)) & 0x3u;
            if ((0x1668u >> bitmap) & 1u) { /* two bits set: bitmaps 3, 5, 6, 9, 10, 12 */
                /* the format's case: lower kept position p0 takes sign bit 0,
                 * the higher p1 sign bit 1; -v = (v ^ -1) + 1 */
                const int p0 = __builtin_ctz(bitmap), p1 = __builtin_ctz(bitmap & (bitmap - 1));
                const int32_t m0 = -(int32_t)(signs & 1u), m1 = -(int32_t)(signs >> 1);
                s += (((int32_t)x[4 * g + p0] ^ m0) - m0) + (((int32_t)x[4 * g + p1] ^ m1) - m1);
                continue;
            }
            int nz = 0; /* malformed bitmaps: spbo_unpack's decode, position by position */
            for (int i = 0; i < 4; ++i) {
                if (!(bitmap & (1u << i))) continue;
                const int32_t xv = (int32_t)x[4 * g + i];
                s += ((signs >> nz) & 1u) ? -xv : xv;
                ++nz;
            }
        }
        y[r] = s;
    }
}

/*
 * The multiply-accumulate half of cpu_sparse_gemv (tests/test_sparse_ternary.cu:
 * 26-32) on an already unpacked int8 matrix: the CPU baseline timed without
 * the per-call unpack.
 */
void spbo_dense_mac(const int8_t* dense, const int8_t* x, int32_t* y, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        int32_t s = 0;
        for (int c = 0; c < cols; ++c) s += (int32_t)dense[(size_t)r * cols + c] * (int32_t)x[c];
        y[r] = s;
    }
}

/*
 * cpu_int8_gemm (tests/test_cusparselt.cu:16-28) on the unpacked weights,
 * with the batch in token-major layout: X[n][cols] int8, Y[n][rows] int32.
 * This is cuSPARSELt's column-major B [K x N] / D [M x N]
 * (src/cusparselt_backend.cu:53-62, 83-89) read as row-major [N][.].
 */
void spbo_gemm(const uint32_t* meta, const uint32_t* values, const int8_t* X,
               int32_t* Y, int rows, int cols, int n, int ms, int vs) {
    int8_t* dense = (int8_t*)malloc((size_t)rows * cols + 1);
    spbo_unpack(meta, values, rows, cols, ms, vs, dense);
    for (int t = 0; t < n; ++t) {
        for (int r = 0; r < rows; ++r) {
            int32_t s = 0;
            for (int c = 0; c < cols; ++c)
                s += (int32_t)dense[(size_t)r * cols + c] * (int32_t)X[(size_t)t * cols + c];
            Y[(size_t)t * rows + r] = s;
        }
    }
    free(dense);
}

/* max |x| (src/kernels/inference_kernels.cu:120-148); order-independent. */
float spbo_absmax(const float* x, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; ++i) m = fmaxf(m, fabsf(x[i]));
    return m;
}

/*
 * absmax_quantize_kernel (src/kernels/inference_kernels.cu:69-114):
 * scale = absmax > 0 ? 127.0f/absmax : 0 (float32 divide, correctly rounded),
 * q = clamp(__float2int_rn(x*scale), -128, 127) with round-half-to-even.
 */
float spbo_quant_scale(float absmax) { return absmax > 0.0f ? 127.0f / absmax : 0.0f; }

int32_t spbo_round_clamp(float v) {
    /* __float2int_rn returns INT_MIN for NaN, which the clamp maps to -128 */
    if (isnan(v)) return -128;
    float r = nearbyintf(v); /* default rounding mode: nearest, ties to even */
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int32_t)r;
}

float spbo_quantize(const float* x, int n, int8_t* q) {
    float absmax = spbo_absmax(x, n);
    float scale = spbo_quant_scale(absmax);
    for (int i = 0; i < n; ++i) {
        volatile float prod = x[i] * scale; /* one float32 rounding, no contraction */
        q[i] = (int8_t)spbo_round_clamp(prod);
    }
    return absmax;
}

/*
 * dequantize_kernel (src/kernels/inference_kernels.cu:162-171) and the fused
 * epilogue (src/kernels/sparse_ternary.cu:230-233):
 * out = float(acc) * ((gamma * absmax) / 127.0f), each step rounded to float32.
 * The caller rounds the result to fp16/bf16.
 */
float spbo_dequant_scale(float gamma, float absmax) {
    volatile float ga = gamma * absmax;
    volatile float s = ga / 127.0f;
    return s;
}

void spbo_dequant(const int32_t* acc, int n, float gamma, float absmax, float* out) {
    float s = spbo_dequant_scale(gamma, absmax);
    for (int i = 0; i < n; ++i) {
        volatile float v = (float)acc[i] * s;
        out[i] = v;
    }
}

/*
 * fused_sparse_bitlinear_kernel (src/kernels/sparse_ternary.cu:181-234): the
 * same int32 accumulation as the GEMV on the quantised activations, then the
 * dequant epilogue.  x is the activation already widened to float32.
 */
void spbo_fused_bitlinear(const uint32_t* meta, const uint32_t* values, const float* x,
                          float absmax, float gamma, int rows, int cols, int ms, int vs,
                          float* out, int32_t* acc_out) {
    float scale = spbo_quant_scale(absmax);
    int8_t* q = (int8_t*)malloc((size_t)cols + 1);
    int32_t* acc = (int32_t*)malloc((size_t)rows * 4 + 4);
    for (int i = 0; i < cols; ++i) {
        volatile float prod = x[i] * scale;
        q[i] = (int8_t)spbo_round_clamp(prod);
    }
    spbo_gemv(meta, values, q, acc, rows, cols, ms, vs);
    spbo_dequant(acc, rows, gamma, absmax, out);
    if (acc_out) memcpy(acc_out, acc, (size_t)rows * 4);
    free(q);
    free(acc);
}

/* float32 -> bfloat16 bits, round to nearest even, quiet NaN preserved. */
uint16_t spbo_bf16_round(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}

void spbo_bf16_round_array(const float* in, int n, uint16_t* out) {
    for (int i = 0; i < n; ++i) out[i] = spbo_bf16_round(in[i]);
}

/*
 * Bit-plane activation layout of this build (no reference counterpart):
 * word [w*8 + b] bit j = bit b of the two's-complement byte x[32w + j];
 * columns beyond cols are 0.  Pinned by a round trip (planes -> bytes) and
 * by the GEMV identity sum_j w_j x_j = sum_b c_b sum_j w_j bit_b(x_j).
 */
void spbo_planes(const int8_t* x, int cols, uint32_t* planes) {
    int nw = (cols + 31) / 32;
    memset(planes, 0, (size_t)nw * 8 * 4);
    for (int c = 0; c < cols; ++c) {
        uint32_t byte = (uint8_t)x[c];
        for (int b = 0; b < 8; ++b)
            planes[(c / 32) * 8 + b] |= ((byte >> b) & 1u) << (c % 32);
    }
}

/*
 * 2:4 pruning of a dense int8 matrix A [m][k] along k, the structured-sparse
 * int8 GEMM's prepare (the cuSPARSELt backend, src/cusparselt_backend.cu:
 * 107-166).  The reference leaves the selection to cuSPARSELt's STRIP rule,
 * which it does not specify (its test only checks the 2:4 property and the
 * value range, tests/test_cusparselt.cu:68-117); the build's rule is the one
 * of spbo_mask_top2 on |a|: keep the two largest |a| of each group of four,
 * on equal magnitudes the higher index.  out [m][k] receives the kept
 * values and zeros.
 */
void spbo_prune24_i8(const int8_t* A, int m, int k, int8_t* out) {
    for (long r = 0; r < m; ++r)
        for (int g = 0; g < k / 4; ++g) {
            const int8_t* p = A + r * k + 4 * g;
            int8_t* o = out + r * k + 4 * g;
            for (int i = 0; i < 4; ++i) {
                int beaten_by = 0;
                for (int j = 0; j < 4; ++j) {
                    if (j == i) continue;
                    const int ai = abs((int)p[i]), aj = abs((int)p[j]);
                    if (aj > ai || (aj == ai && j > i)) ++beaten_by;
                }
                o[i] = beaten_by < 2 ? p[i] : 0;
            }
        }
}

/*
 * cpu_int8_gemm (tests/test_cusparselt.cu:16-28): D = A * B in int32, with
 * A [m][k] row-major and B, D in the column-major layouts the backend takes
 * (B [k x n] = [n][k], D [m x n] = [n][m], src/cusparselt_backend.cu:53-78).
 */
void spbo_int8_gemm(const int8_t* A, const int8_t* B, int32_t* D, int m, int k, int n) {
    for (long t = 0; t < n; ++t)
        for (long r = 0; r < m; ++r) {
            int32_t s = 0;
            for (int j = 0; j < k; ++j) s += (int32_t)A[r * k + j] * (int32_t)B[t * k + j];
            D[t * m + r] = s;
        }
}

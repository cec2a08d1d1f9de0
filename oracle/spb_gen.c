/*
 * spb_gen.c -- host restatement of the library's random-init model generator
 * (spb_generate_sparse_ternary / spb_generate_normal_bf16), so that the CPU
 * oracle can rebuild, bit for bit, the models the GPU tests and bench.py
 * decode, and golden tokens for them can be written without a GPU.
 * TEST INFRASTRUCTURE ONLY: imported by tests/ (and the golden-token script
 * under tests/golden), never by the product.
 *
 * The generator is this build's synthetic-input recipe (the reference's
 * models come from checkpoints through python/convert_model.py):
 *   latent W[i] = N(0,1) from the counter (seed, i): z = splitmix64(seed ^
 *     splitmix64(i)); Box-Muller on u1 = ((z >> 40) + 1) / 2^24 and
 *     u2 = ((z >> 16) & 0xFFFFFF) / 2^24 with ln, sqrt and cos evaluated as
 *     fixed sequences of IEEE double adds and multiplies (below), rounded
 *     once to float;
 *   projections: the 2:4 top-2 mask, kept signs and packing of
 *     python/convert_model.py:88-207 on that latent (spb_oracle.c restates
 *     them; the Python wrapper calls those), gamma = mean |W| summed in
 *     double in the device kernel's order (gen_gamma below);
 *   embedding: bf16(float(W[i]) * std).
 *
 * Pinning: the GPU test tests/test_gpu_engine.py::test_generator_matches_host
 * compares the device's packed words, gamma bits and bf16 embedding with this
 * file's output; the CPU tests check the normal against libm's log/sqrt/cos
 * (within 1e-14 relative before the float rounding) and its moments.
 * Build: -ffp-contract=off (oracle/Makefile), as the HIP library, so that no
 * multiply-add is fused on either side.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static const double kLogC[41] = {
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
/* (-1)^i / (2i)! and (-1)^i / (2i+1)! */
static const double kCosC[11] = {
    0x1.0000000000000p+0,  -0x1.0000000000000p-1,  0x1.5555555555555p-5,  -0x1.6c16c16c16c17p-10,
    0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
    0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62};
static const double kSinC[11] = {
    0x1.0000000000000p+0,  -0x1.5555555555555p-3,  0x1.1111111111111p-7,  -0x1.a01a01a01a01ap-13,
    0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41,
    0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57, 0x1.71b8ef6dcf572p-66};

static uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double from_bits(uint64_t b) {
    double d;
    memcpy(&d, &b, 8);
    return d;
}

static uint64_t to_bits(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    return b;
}

/* ln(k / 2^24), k in [1, 2^24]: k / 2^24 = m 2^(e - 24), m in (1/sqrt2, sqrt2],
 * ln(1 + t) = t * sum_{i=0}^{40} (-1)^i t^i / (i + 1), t = m - 1 (Horner). */
double spbo_gen_ln_u24(uint32_t k) {
    int e = 31 - __builtin_clz(k);
    double m = (double)k * from_bits((uint64_t)(1023 - e) << 52);
    if (m > 0x1.6a09e667f3bcdp+0) {
        m = m * 0.5;
        e = e + 1;
    }
    const double t = m - 1.0;
    double p = kLogC[40];
    for (int i = 39; i >= 0; --i) p = p * t + kLogC[i];
    return (double)(e - 24) * 0x1.62e42fefa39efp-1 + t * p;
}

/* sqrt(y) = y * rsqrt(y): bit-pattern guess, four Newton steps. */
double spbo_gen_sqrt(double y) {
    if (!(y > 0.0)) return 0.0;
    double r = from_bits(0x5FE6EB50C7B537A9ull - (to_bits(y) >> 1));
    const double h = 0.5 * y;
    for (int i = 0; i < 4; ++i) r = r * (1.5 - (h * r) * r);
    return y * r;
}

/* cos(2 pi j / 2^24), j in [0, 2^24): octant reduction on the integer, then
 * the Taylor series of cos (degree 20) or sin (degree 21) on [0, pi/4]. */
double spbo_gen_cos_u24(uint32_t j) {
    int neg = 0;
    if (j >= (1u << 23)) j = (1u << 24) - j;
    if (j > (1u << 22)) {
        j = (1u << 23) - j;
        neg = 1;
    }
    const int use_sin = j > (1u << 21);
    const double x = (double)(use_sin ? (1u << 22) - j : j) * 0x1.921fb54442d18p-22;
    const double x2 = x * x;
    double p;
    if (use_sin) {
        p = kSinC[10];
        for (int i = 9; i >= 0; --i) p = p * x2 + kSinC[i];
        p = x * p;
    } else {
        p = kCosC[10];
        for (int i = 9; i >= 0; --i) p = p * x2 + kCosC[i];
    }
    return neg ? -p : p;
}

float spbo_gen_normal(uint64_t seed, uint64_t i) {
    const uint64_t z = splitmix64(seed ^ splitmix64(i));
    const uint32_t k = (uint32_t)(z >> 40) + 1u;
    const uint32_t j = (uint32_t)((z >> 16) & 0xFFFFFFull);
    const double r = spbo_gen_sqrt(-2.0 * spbo_gen_ln_u24(k));
    return (float)(r * spbo_gen_cos_u24(j));
}

/* out[i] = normal(seed, start + i), i < n */
void spbo_gen_normals(uint64_t seed, uint64_t start, long n, float* out) {
#pragma omp parallel for schedule(static) if (n >= 65536)
    for (long i = 0; i < n; ++i) out[i] = spbo_gen_normal(seed, start + (uint64_t)i);
}

uint16_t spbo_bf16_round(float f);

/* out[i] = bf16(float(normal(seed, i)) * std), the embedding generator */
void spbo_gen_normal_bf16(uint64_t seed, long n, float std_, uint16_t* out) {
#pragma omp parallel for schedule(static) if (n >= 65536)
    for (long i = 0; i < n; ++i) out[i] = spbo_bf16_round(spbo_gen_normal(seed, (uint64_t)i) * std_);
}

/*
 * gamma = mean |W| as the device computes it: blocks = min(ceil(units / 256),
 * 1024) blocks of 256 threads, units of 64 columns (unit u = row u / (cols /
 * 64), columns 64 (u % (cols / 64)) ...); thread g of the grid sums |W| in
 * double over its units g, g + 256 blocks, ... (elements in column order);
 * each 64-lane wave combines its sums by the butterfly v[l] += v[l ^ off],
 * off = 32 .. 1, the block as ((w0 + w1) + w2) + w3, then the blocks in
 * order, divided by rows * cols and rounded to float.
 */
float spbo_gen_gamma(const float* latent, int rows, int cols) {
    const long upr = cols / 64;
    const long units = (long)rows * upr;
    long blocks = (units + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    const long nthreads = blocks * 256;
    double* part = (double*)calloc((size_t)blocks, sizeof(double));
#pragma omp parallel for schedule(static)
    for (long b = 0; b < blocks; ++b) {
        double wsum[4];
        for (int w = 0; w < 4; ++w) {
            double v[64];
            for (int l = 0; l < 64; ++l) {
                double s = 0.0;
                for (long u = b * 256 + w * 64 + l; u < units; u += nthreads) {
                    const float* p = latent + (u / upr) * (long)cols + (u % upr) * 64;
                    for (int c = 0; c < 64; ++c) s += fabs((double)p[c]);
                }
                v[l] = s;
            }
            for (int off = 32; off > 0; off >>= 1) {
                double nv[64];
                for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ off];
                memcpy(v, nv, sizeof(v));
            }
            wsum[w] = v[0];
        }
        part[b] = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    }
    double s = 0.0;
    for (long b = 0; b < blocks; ++b) s += part[b];
    free(part);
    return (float)(s / ((double)rows * (double)cols));
}

/*
 * spb_engine_oracle.c -- CPU restatement of one bs=1 decode step of the
 * reference engine, InferenceEngine::forward (src/inference.cu:126-283), for
 * checking the HIP engine.  TEST INFRASTRUCTURE ONLY: imported by tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg, never by the
 * product.
 *
 * Semantics: the reference's layer order and operations (file:line at each
 * function), with bf16 storage of every activation the reference stores in
 * fp16, a bf16 KV cache and a bf16 LM head.
 *
 * Floating-point order: float32 arithmetic in the order the HIP kernels use
 * (fma where they fuse, the same reduction trees), so that logits agree bit
 * for bit and greedy token ids agree exactly:
 *   block sums over T threads: thread t accumulates the 8-element units
 *     t, t+T, ... (fma(v, v, acc) for sums of squares, element order inside
 *     a unit), then per 64-thread wave the pairwise tree over adjacent
 *     lanes, then the wave totals in wave order;
 *   attention scores: four fma chains, one per quarter of the head dim
 *     (d ascending inside a quarter), combined as (a0 + a1) + (a2 + a3), then
 *     times the scale; softmax sums: the 64-lane tree over the positions of a
 *     split;
 *   LM head: lane l accumulates the 8-element chunks l, l+64, ... with fma in
 *     element order, then the 64-lane tree;
 *   1/sqrt with correctly rounded divide and sqrt (reference: rsqrtf);
 *   exp of softmax by exp_neg() below (reference: expf).
 * These differ from the reference's CUDA order only by float32 rounding,
 * which the tests bound separately against float64 evaluations of the same
 * formulas (1e-3 relative).
 *
 * Pinning: the int32 GEMV core is spbo_gemv (spb_oracle.c, pinned there);
 * exp_neg is checked against libm exp; rms_norm / attention / LM head are
 * checked against float64 restatements of the reference formulas, plus
 * closed forms (one-position attention returns v; uniform scores average v;
 * a constant vector normalises to w * sign / sqrt(1 + eps / x^2)).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void spbo_gemv(const uint32_t* meta, const uint32_t* values, const int8_t* x, int32_t* y,
               int rows, int cols, int ms, int vs);
uint16_t spbo_bf16_round(float f);

#define GEMV_THREADS 512 /* threads of the GEMV blocks whose prologues normalise */
#define ATTN_SPLIT 64    /* positions per attention split (one per lane) */
#define LM_THREADS 256

static float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static float bfr(float f) { return bf2f(spbo_bf16_round(f)); }

/* Sum over 64 lanes as the balanced pairwise tree over adjacent lanes
 * (lanes 2i and 2i+1, then pairs of pairs, ...). */
static float tree64(const float* a) {
    float t[64];
    memcpy(t, a, sizeof(t));
    for (int n = 32; n >= 1; n >>= 1)
        for (int i = 0; i < n; ++i) t[i] = t[2 * i] + t[2 * i + 1];
    return t[0];
}

/* Block sum over T threads of per-thread partials p[0..T). */
static float block_sum(float* p, int T) {
    float s = 0.0f;
    for (int w = 0; w < T / 64; ++w) {
        float v = tree64(p + 64 * w);
        s = (w == 0) ? v : s + v;
    }
    return s;
}

/* Sum of squares of v[0..n) in the unit order of T threads: thread t owns
 * the 8-element units t, t+T, ... and accumulates their elements in order
 * with fma; then block_sum. */
static float sumsq(const float* v, int n, int T) {
    float* p = (float*)calloc((size_t)T, sizeof(float));
    const int units = n / 8;
    for (int t = 0; t < T; ++t)
        for (int u = t; u < units; u += T)
            for (int e = 0; e < 8; ++e) p[t] = fmaf(v[8 * u + e], v[8 * u + e], p[t]);
    float s = block_sum(p, T);
    free(p);
    return s;
}

static float inv_rms(float ss, int n, float eps) { return 1.0f / sqrtf(ss / (float)n + eps); }

/* exp(x), x <= 0: Cody-Waite reduction, degree-7 Taylor polynomial (Horner,
 * fma), 2^n scaling; 0 below -86. */
float spbo_exp_neg(float x) {
    if (!(x >= -86.0f)) return 0.0f;
    const float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(-n, 0.693145751953125f, x);
    r = fmaf(-n, 1.42860682030941723e-6f, r);
    float p = 1.98412698412698413e-4f;
    p = fmaf(p, r, 1.38888888888888889e-3f);
    p = fmaf(p, r, 8.33333333333333333e-3f);
    p = fmaf(p, r, 4.16666666666666667e-2f);
    p = fmaf(p, r, 1.66666666666666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

typedef struct {
    const uint32_t* meta;
    const uint32_t* values;
    float gamma;
    int rows, cols, ms, vs;
} lin_t;

typedef struct {
    lin_t p[7]; /* q, k, v, o, gate, up, down */
    const float* norm[4]; /* input_ln, post_ln, attn_sub (nullable), ffn_sub (nullable) */
} layer_t;

typedef struct {
    int H, L, nh, nkv, I, V, hd, max_seq;
    float eps, theta;
    layer_t* layers;
    const uint16_t* embed;
    const uint16_t* lm;
    const float* final_norm;
    float* rope;       /* [max_seq][hd/2][2] */
    uint16_t** kc;     /* [L] of [nkv][max_seq][hd] */
    uint16_t** vc;
    int pos;
    /* scratch */
    float *x, *xb, *vec, *qkv, *o, *gu, *attn, *h_in, *m_in;
    int8_t* q8;
    int32_t* acc;
    float* logit_buf; /* [V] */
} spbo_engine;

/* absmax, quantise (spb_oracle.c rules), GEMV, dequantise to bf16 with gamma;
 * fused_sparse_bitlinear (src/kernels/sparse_ternary.cu:181-234) on a vector
 * that is already bf16-rounded. */
float spbo_quantize(const float* x, int n, int8_t* q);
float spbo_dequant_scale(float gamma, float absmax);

static float bitlinear_raw(spbo_engine* e, const lin_t* w, const float* in, int32_t* acc) {
    const float amax = spbo_quantize(in, w->cols, e->q8);
    spbo_gemv(w->meta, w->values, e->q8, acc, w->rows, w->cols, w->ms, w->vs);
    return amax;
}

/* rms_norm_kernel (src/kernels/inference_kernels.cu:15-56): y = bf16((x*inv)*w) */
static void rmsnorm(const float* x, const float* w, int n, float eps, int T, float* y) {
    const float inv = inv_rms(sumsq(x, n, T), n, eps);
    for (int i = 0; i < n; ++i) y[i] = bfr((x[i] * inv) * w[i]);
}

void spbo_engine_free(spbo_engine* e);

spbo_engine* spbo_engine_new(const int* icfg, const float* fcfg, const uint32_t** metas,
                             const uint32_t** values, const float* gammas, const int* ms,
                             const int* vs, const float** norms, const uint16_t* embed,
                             const uint16_t* lm_head, const float* final_norm) {
    spbo_engine* e = (spbo_engine*)calloc(1, sizeof(spbo_engine));
    e->H = icfg[0];
    e->L = icfg[1];
    e->nh = icfg[2];
    e->nkv = icfg[3];
    e->I = icfg[4];
    e->V = icfg[5];
    e->hd = icfg[6];
    e->max_seq = icfg[7];
    e->eps = fcfg[0];
    e->theta = fcfg[1];
    const int H = e->H, I = e->I, hd = e->hd, kvd = e->nkv * hd;
    const int rows[7] = {H, kvd, kvd, H, I, I, H};
    const int cols[7] = {H, H, H, H, H, H, I};
    e->layers = (layer_t*)calloc((size_t)e->L, sizeof(layer_t));
    for (int l = 0; l < e->L; ++l) {
        for (int k = 0; k < 7; ++k) {
            lin_t* p = &e->layers[l].p[k];
            p->meta = metas[7 * l + k];
            p->values = values[7 * l + k];
            p->gamma = gammas[7 * l + k];
            p->rows = rows[k];
            p->cols = cols[k];
            p->ms = ms[7 * l + k];
            p->vs = vs[7 * l + k];
        }
        for (int k = 0; k < 4; ++k) e->layers[l].norm[k] = norms[4 * l + k];
    }
    e->embed = embed;
    e->lm = lm_head ? lm_head : embed;
    e->final_norm = final_norm;
    /* RoPE table (inference_kernels.cu:195-198) */
    e->rope = (float*)malloc(sizeof(float) * (size_t)e->max_seq * hd);
    for (int p = 0; p < e->max_seq; ++p)
        for (int i = 0; i < hd / 2; ++i) {
            const float freq = 1.0f / powf(e->theta, (float)(2 * i) / (float)hd);
            const float angle = (float)p * freq;
            e->rope[((size_t)p * (hd / 2) + i) * 2] = (float)cos((double)angle);
            e->rope[((size_t)p * (hd / 2) + i) * 2 + 1] = (float)sin((double)angle);
        }
    e->kc = (uint16_t**)calloc((size_t)e->L, sizeof(uint16_t*));
    e->vc = (uint16_t**)calloc((size_t)e->L, sizeof(uint16_t*));
    for (int l = 0; l < e->L; ++l) {
        e->kc[l] = (uint16_t*)calloc((size_t)kvd * e->max_seq, 2);
        e->vc[l] = (uint16_t*)calloc((size_t)kvd * e->max_seq, 2);
    }
    const int mx = (H > I ? H : I) + 2 * kvd + I;
    e->x = (float*)calloc((size_t)H, 4);
    e->xb = (float*)calloc((size_t)H, 4);
    e->vec = (float*)calloc((size_t)mx, 4);
    e->qkv = (float*)calloc((size_t)(H + 2 * kvd), 4);
    e->o = (float*)calloc((size_t)H, 4);
    e->gu = (float*)calloc((size_t)2 * I, 4);
    e->attn = (float*)calloc((size_t)H, 4);
    e->h_in = (float*)calloc((size_t)H, 4);
    e->m_in = (float*)calloc((size_t)I, 4);
    e->q8 = (int8_t*)calloc((size_t)mx, 1);
    e->acc = (int32_t*)calloc((size_t)mx, 4);
    e->logit_buf = (float*)calloc((size_t)e->V, 4);
    e->pos = 0;
    return e;
}

void spbo_engine_free(spbo_engine* e) {
    if (!e) return;
    for (int l = 0; l < e->L; ++l) {
        free(e->kc[l]);
        free(e->vc[l]);
    }
    free(e->kc);
    free(e->vc);
    free(e->layers);
    free(e->rope);
    free(e->x);
    free(e->xb);
    free(e->vec);
    free(e->qkv);
    free(e->o);
    free(e->gu);
    free(e->attn);
    free(e->h_in);
    free(e->m_in);
    free(e->q8);
    free(e->acc);
    free(e->logit_buf);
    free(e);
}

void spbo_engine_reset(spbo_engine* e) {
    const size_t kv = (size_t)e->nkv * e->hd * e->max_seq * 2;
    for (int l = 0; l < e->L; ++l) {
        memset(e->kc[l], 0, kv);
        memset(e->vc[l], 0, kv);
    }
    e->pos = 0;
}

/* attention of one layer (inference.cu:166-202; inference_kernels.cu:185-371)
 * in 64-position splits, combined as in the o-projection prologue. */
static void attention(spbo_engine* e, int l) {
    const int nh = e->nh, nkv = e->nkv, hd = e->hd, G = nh / nkv, half = hd / 2;
    const int pos = e->pos, S = pos / ATTN_SPLIT + 1;
    const float scale = 1.0f / sqrtf((float)hd);
    const float* rp = e->rope + (size_t)pos * hd;
    float* pm = (float*)malloc(sizeof(float) * nh * S);
    float* pl = (float*)malloc(sizeof(float) * nh * S);
    float* pacc = (float*)malloc(sizeof(float) * nh * S * hd);
    /* RoPE of k and the cache writes at pos (every kv head) */
    for (int kvh = 0; kvh < nkv; ++kvh) {
        const float* kh = e->qkv + nh * hd + kvh * hd;
        const float* vh = e->qkv + (nh + nkv) * hd + kvh * hd;
        uint16_t* kc = e->kc[l] + (size_t)kvh * e->max_seq * hd;
        uint16_t* vc = e->vc[l] + (size_t)kvh * e->max_seq * hd;
        for (int i = 0; i < half; ++i) {
            const float x0 = kh[2 * i], x1 = kh[2 * i + 1], c = rp[2 * i], s = rp[2 * i + 1];
            kc[(size_t)pos * hd + 2 * i] = spbo_bf16_round(x0 * c - x1 * s);
            kc[(size_t)pos * hd + 2 * i + 1] = spbo_bf16_round(x0 * s + x1 * c);
        }
        for (int d = 0; d < hd; ++d) vc[(size_t)pos * hd + d] = spbo_bf16_round(vh[d]);
    }
    /* the partials of every (kv head, split): independent, so they run in
     * parallel (OpenMP) for long contexts */
#pragma omp parallel for schedule(dynamic) if (S * nkv >= 16)
    for (int task = 0; task < nkv * S; ++task) {
        const int kvh = task / S, s = task % S;
        float qs[8][128];
        float sc[8][ATTN_SPLIT];
        for (int g = 0; g < G; ++g)
            for (int i = 0; i < half; ++i) {
                const float* qh = e->qkv + (kvh * G + g) * hd;
                const float x0 = qh[2 * i], x1 = qh[2 * i + 1], c = rp[2 * i], sn = rp[2 * i + 1];
                qs[g][2 * i] = bfr(x0 * c - x1 * sn);
                qs[g][2 * i + 1] = bfr(x0 * sn + x1 * c);
            }
        const uint16_t* kc = e->kc[l] + (size_t)kvh * e->max_seq * hd;
        const uint16_t* vc = e->vc[l] + (size_t)kvh * e->max_seq * hd;
        {
            const int j0 = s * ATTN_SPLIT;
            const int jn = (pos + 1 - j0) < ATTN_SPLIT ? (pos + 1 - j0) : ATTN_SPLIT;
            for (int jj = 0; jj < jn; ++jj) {
                const uint16_t* kj = kc + (size_t)(j0 + jj) * hd;
                for (int g = 0; g < G; ++g) {
                    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    for (int d = 0; d < hd; ++d) {
                        const int k = d / (hd / 4);
                        a[k] = fmaf(qs[g][d], bf2f(kj[d]), a[k]);
                    }
                    sc[g][jj] = ((a[0] + a[1]) + (a[2] + a[3])) * scale;
                }
            }
            for (int g = 0; g < G; ++g) {
                float m = -INFINITY;
                for (int jj = 0; jj < jn; ++jj) m = fmaxf(m, sc[g][jj]);
                float p[64];
                for (int t = 0; t < 64; ++t) {
                    p[t] = t < jn ? spbo_exp_neg(sc[g][t] - m) : 0.0f;
                    if (t < jn) sc[g][t] = p[t];
                }
                const float lsum = tree64(p);
                const int h = kvh * G + g;
                pm[h * S + s] = m;
                pl[h * S + s] = lsum;
                for (int d = 0; d < hd; ++d) {
                    float a = 0.0f;
                    for (int jj = 0; jj < jn; ++jj)
                        a = fmaf(sc[g][jj], bf2f(vc[(size_t)(j0 + jj) * hd + d]), a);
                    pacc[((size_t)h * S + s) * hd + d] = a;
                }
            }
        }
    }
    for (int i = 0; i < nh * hd; ++i) {
        const int h = i / hd, d = i % hd;
        float M = pm[h * S];
        for (int s = 1; s < S; ++s) M = fmaxf(M, pm[h * S + s]);
        float lsum = 0.0f, a = 0.0f;
        for (int s = 0; s < S; ++s) {
            const float w = spbo_exp_neg(pm[h * S + s] - M);
            lsum = fmaf(w, pl[h * S + s], lsum);
            a = fmaf(w, pacc[((size_t)h * S + s) * hd + d], a);
        }
        e->attn[i] = bfr(a / lsum);
    }
    free(pm);
    free(pl);
    free(pacc);
}

static int engine_step(spbo_engine* e, int token, float* logits, int with_head);

/* One token: returns argmax(logits) (lowest index among maxima), or -1 when
 * the KV cache is full or the token id is out of range; logits (nullable)
 * receives the float32 logits. */
int spbo_engine_step(spbo_engine* e, int token, float* logits) {
    return engine_step(e, token, logits, 1);
}

/* A prompt token before the last (src/main.cpp:133-143): the same step
 * without the LM head, whose logits the generate loop does not use; the KV
 * cache and position are those spbo_engine_step leaves.  Returns 0, or -1
 * as spbo_engine_step. */
int spbo_engine_prefill(spbo_engine* e, int token) { return engine_step(e, token, NULL, 0); }

static int engine_step(spbo_engine* e, int token, float* logits, int with_head) {
    if (e->pos >= e->max_seq || token < 0 || token >= e->V) return -1; /* cache full / bad id */
    const int H = e->H, I = e->I, hd = e->hd, kvd = e->nkv * hd;
    const float eps = e->eps;
    float* vec = e->vec;
    int32_t* acc = e->acc;
    for (int i = 0; i < H; ++i) e->x[i] = bf2f(e->embed[(size_t)token * H + i]); /* :134-138 */
    for (int l = 0; l < e->L; ++l) {
        const layer_t* L = &e->layers[l];
        /* input RMSNorm and q/k/v (inference.cu:147-160, 171-177) */
        rmsnorm(e->x, L->norm[0], H, eps, GEMV_THREADS, vec);
        memcpy(e->h_in, vec, sizeof(float) * H);
        const float a0 = bitlinear_raw(e, &L->p[0], vec, acc);
        {
            const int R[3] = {H, kvd, kvd};
            int off = 0;
            for (int k = 0; k < 3; ++k) {
                const float dq = spbo_dequant_scale(L->p[k].gamma, a0);
                spbo_gemv(L->p[k].meta, L->p[k].values, e->q8, acc, R[k], H, L->p[k].ms,
                          L->p[k].vs);
                for (int r = 0; r < R[k]; ++r) e->qkv[off + r] = bfr((float)acc[r] * dq);
                off += R[k];
            }
        }
        attention(e, l);
        /* o projection (inference.cu:198-202) */
        const float a1 = bitlinear_raw(e, &L->p[3], e->attn, acc);
        const float dq1 = spbo_dequant_scale(L->p[3].gamma, a1);
        for (int r = 0; r < H; ++r) e->o[r] = bfr((float)acc[r] * dq1);
        /* attn sub-norm, residual, post-attention norm (:205-230) */
        if (L->norm[2]) {
            rmsnorm(e->o, L->norm[2], H, eps, GEMV_THREADS, vec);
            memcpy(e->o, vec, sizeof(float) * H);
        }
        for (int i = 0; i < H; ++i) e->xb[i] = bfr(e->o[i] + e->x[i]);
        rmsnorm(e->xb, L->norm[1], H, eps, GEMV_THREADS, vec);
        /* gate / up (:233-236) */
        const float a2 = bitlinear_raw(e, &L->p[4], vec, acc);
        for (int k = 4; k < 6; ++k) {
            const float dq = spbo_dequant_scale(L->p[k].gamma, a2);
            spbo_gemv(L->p[k].meta, L->p[k].values, e->q8, acc, I, H, L->p[k].ms, L->p[k].vs);
            for (int r = 0; r < I; ++r) e->gu[(k - 4) * I + r] = bfr((float)acc[r] * dq);
        }
        /* relu^2 * up in fp32, ffn sub-norm (:238-251) */
        for (int i = 0; i < I; ++i) {
            const float rr = fmaxf(0.0f, e->gu[i]);
            vec[i] = (rr * rr) * e->gu[I + i];
        }
        if (L->norm[3]) {
            const float inv = inv_rms(sumsq(vec, I, GEMV_THREADS), I, eps);
            for (int i = 0; i < I; ++i) vec[i] = bfr((vec[i] * inv) * L->norm[3][i]);
        } else {
            for (int i = 0; i < I; ++i) vec[i] = bfr(vec[i]);
        }
        /* down projection and residual (:253-262) */
        memcpy(e->m_in, vec, sizeof(float) * I);
        const float a3 = bitlinear_raw(e, &L->p[6], vec, acc);
        const float dq3 = spbo_dequant_scale(L->p[6].gamma, a3);
        for (int r = 0; r < H; ++r) e->x[r] = bfr(bfr((float)acc[r] * dq3) + e->xb[r]);
    }
    if (!with_head) {
        e->pos += 1;
        return 0;
    }
    /* final norm and LM head (:268-277; half_gemv_kernel :488-531); rows are
     * independent, so they run in parallel (OpenMP) and the argmax follows */
    rmsnorm(e->x, e->final_norm, H, eps, LM_THREADS, vec);
    const int nch = H / 8;
    float* lg = e->logit_buf;
#pragma omp parallel for schedule(static) if ((long)e->V * H >= (1L << 22))
    for (int r = 0; r < e->V; ++r) {
        const uint16_t* w = e->lm + (size_t)r * H;
        float lanes[64];
        for (int ln = 0; ln < 64; ++ln) {
            float a = 0.0f;
            for (int c = ln; c < nch; c += 64)
                for (int k = 0; k < 8; ++k) a = fmaf(bf2f(w[8 * c + k]), vec[8 * c + k], a);
            lanes[ln] = a;
        }
        lg[r] = tree64(lanes);
    }
    int best = -1;
    float bv = -INFINITY;
    for (int r = 0; r < e->V; ++r) {
        if (logits) logits[r] = lg[r];
        if (lg[r] > bv) {
            bv = lg[r];
            best = r;
        }
    }
    e->pos += 1;
    return best < 0 ? 0 : best;
}

/* Hidden state after the last step (float values of the bf16 residual). */
void spbo_engine_hidden(const spbo_engine* e, float* out) { memcpy(out, e->x, sizeof(float) * e->H); }

/* Internal vectors of the last step's last layer, for checking the checker
 * itself: 0 = q|k|v (pre-RoPE), 1 = attention output, 2 = o (after the
 * sub-norm), 3 = mid-layer residual, 4 = gate|up, 5 = normalised layer input,
 * 6 = normalised down-projection input, 7 = final-normed hidden state (after
 * a step with the LM head). */
int spbo_engine_debug(const spbo_engine* e, int which, float* out) {
    const int H = e->H, kvd = e->nkv * e->hd, I = e->I;
    switch (which) {
        case 0: memcpy(out, e->qkv, sizeof(float) * (H + 2 * kvd)); return H + 2 * kvd;
        case 1: memcpy(out, e->attn, sizeof(float) * H); return H;
        case 2: memcpy(out, e->o, sizeof(float) * H); return H;
        case 3: memcpy(out, e->xb, sizeof(float) * H); return H;
        case 4: memcpy(out, e->gu, sizeof(float) * 2 * I); return 2 * I;
        case 5: memcpy(out, e->h_in, sizeof(float) * H); return H;
        case 6: memcpy(out, e->m_in, sizeof(float) * I); return I;
        case 7: memcpy(out, e->vec, sizeof(float) * H); return H;
        default: return 0;
    }
}

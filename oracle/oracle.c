/*
 * The oracle: CPU restatement of the reference's encoder-block arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it (as oracle/build/liboracle.so) to check or to time
 * against; the product library never links, loads or calls it.
 *
 * Every function cites the reference file and lines it restates. Build with
 * -ffp-contract=off so f32 expressions round as written, like the reference's
 * Rust (which never contracts) and its WGSL without FMA contraction.
 *
 * How each part is pinned (tests/test_oracle.py):
 *  - generators: the reference's LCG formula, first values checked by hand
 *    arithmetic and statistics (mean/variance of 1e6 draws);
 *  - blo_erf: the reference's Abramowitz & Stegun table 7.1 values to 1e-12
 *    (reference.rs:760-776) and libm's erf over a grid;
 *  - gelu_erf / gelu_tanh / softmax / matmul / attention / layernorm /
 *    patch_embed / prepend_token: the reference's known-answer tests
 *    (reference.rs:723-855) and torch's CPU F.gelu / F.softmax /
 *    F.layer_norm / F.scaled_dot_product_attention / F.conv2d on random
 *    inputs (a library, not the reference);
 *  - blo_ref_vit_block: composed from the pinned ops, and checked against a
 *    torch CPU float64 forward pass of the same block;
 *  - blo_wg_*: against the f64 ops within the reference's own tolerance, and
 *    blo_wg_gelu_erf1 within GELU_ERF_MAX_ERROR = 5e-7 of GELU through f64 erf
 *    over the reference's grid (reference.rs:790-812).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* generators                                                                */
/* ------------------------------------------------------------------------ */

/* One step of the reference's 64-bit LCG and its value in [0, 1): the top 24
 * bits over 2^24, exact in f32 (net.rs:183-194). */
static float lcg_next(uint64_t *state) {
    *state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
    return (float)(*state >> 40) / 16777216.0f;
}

/* net.rs:197-203: low + (high - low) * u, in f32. */
void blo_uniform(uint64_t seed, size_t count, float low, float high, float *out) {
    uint64_t s = seed;
    float span = high - low;
    for (size_t i = 0; i < count; i++) {
        float u = lcg_next(&s);
        float scaled = span * u;
        out[i] = low + scaled;
    }
}

/* Box-Muller (G. E. P. Box and M. E. Muller, 1958) on pairs of the LCG's
 * uniforms, the cosine branch only: z = sqrt(-2 ln(1 - u1)) cos(2 pi u2).
 * 1 - u1 is in (0, 1], so the logarithm is finite. */
void blo_normal(uint64_t seed, size_t count, float mean, float std, float *out) {
    uint64_t s = seed;
    for (size_t i = 0; i < count; i++) {
        double u1 = lcg_next(&s);
        double u2 = lcg_next(&s);
        double z = sqrt(-2.0 * log(1.0 - u1)) * cos(6.283185307179586 * u2);
        out[i] = (float)(mean + std * z);
    }
}

/* ------------------------------------------------------------------------ */
/* 1. f64 reference ops                                                      */
/* ------------------------------------------------------------------------ */

/* reference.rs:337-360: the Maclaurin series of erf below 3 and the continued
 * fraction of erfc from 3 (60 levels, evaluated from the tail), odd in x. */
double blo_erf(double x) {
    double z = fabs(x);
    double v;
    if (z < 3.0) {
        /* erf z = 2/sqrt(pi) sum_n (-1)^n z^(2n+1) / (n! (2n+1)) */
        double term = z, sum = z, n = 0.0;
        while (fabs(term) > 1e-17 * fabs(sum)) {
            n += 1.0;
            term *= -z * z / n;
            sum += term / (2.0 * n + 1.0);
        }
        v = sum * 2.0 / sqrt(M_PI);
    } else {
        /* erfc z = exp(-z^2)/sqrt(pi) / (z + (1/2)/(z + 1/(z + (3/2)/(z + ...)))) */
        double tail = z;
        for (int k = 60; k >= 1; k--) tail = z + (double)k / 2.0 / tail;
        v = 1.0 - exp(-z * z) / sqrt(M_PI) / tail;
    }
    return copysign(v, x);
}

/* reference.rs:247-270: two-pass mean and biased variance in f64. */
void blo_ref_layernorm(const float *x, const float *gamma, const float *beta,
                       size_t rows, size_t c, float eps, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * c;
        double mean = 0.0;
        for (size_t i = 0; i < c; i++) mean += row[i];
        mean /= (double)c;
        double var = 0.0;
        for (size_t i = 0; i < c; i++) {
            double dv = row[i] - mean;
            var += dv * dv;
        }
        var /= (double)c;
        double inv = 1.0 / sqrt(var + (double)eps);
        for (size_t i = 0; i < c; i++)
            out[r * c + i] = (float)((row[i] - mean) * inv * gamma[i] + beta[i]);
    }
}

/* reference.rs:273-298: C = A B + bias, f64 accumulators seeded with the
 * bias, summed over k in increasing order. */
void blo_ref_matmul(const float *a, const float *b, const float *bias,
                    size_t m, size_t k, size_t n, float *out) {
    #pragma omp parallel
    {
        double *acc = (double *)malloc(n * sizeof(double));
        #pragma omp for schedule(static)
        for (size_t i = 0; i < m; i++) {
            for (size_t j = 0; j < n; j++) acc[j] = bias ? (double)bias[j] : 0.0;
            for (size_t l = 0; l < k; l++) {
                double av = a[i * k + l];
                const float *brow = b + l * n;
                for (size_t j = 0; j < n; j++) acc[j] += av * (double)brow[j];
            }
            for (size_t j = 0; j < n; j++) out[i * n + j] = (float)acc[j];
        }
        free(acc);
    }
}

void blo_ref_add(const float *a, const float *b, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = (float)((double)a[i] + (double)b[i]);
}

void blo_ref_relu(const float *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* reference.rs:314-322: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in f64. */
void blo_ref_gelu_tanh(const float *x, size_t n, float *out) {
    double k = sqrt(2.0 / M_PI);
    for (size_t i = 0; i < n; i++) {
        double v = x[i];
        out[i] = (float)(0.5 * v * (1.0 + tanh(k * (v + 0.044715 * v * v * v))));
    }
}

void blo_ref_scale(const float *x, size_t n, float f, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = (float)((double)x[i] * (double)f);
}

/* reference.rs:369-376: 0.5 x (1 + erf(x / sqrt 2)) through blo_erf. */
void blo_ref_gelu_erf(const float *x, size_t n, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) {
        double v = x[i];
        out[i] = (float)(0.5 * v * (1.0 + blo_erf(v / M_SQRT2)));
    }
}

/* reference.rs:379-384: element i times scale[i % channels]. */
void blo_ref_channel_scale(const float *x, const float *s, size_t n,
                           size_t channels, float *out) {
    for (size_t i = 0; i < n; i++)
        out[i] = (float)((double)x[i] * (double)s[i % channels]);
}

/* reference.rs:437-455: S[i][hd][j] = Q[i][hd] . K[j][hd] from qkv
 * [t][3][h][d]; result [t][h][t]. */
void blo_ref_attention_scores(const float *qkv, size_t t, size_t h, size_t d,
                              float *out) {
    size_t row = 3 * h * d;
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < t; i++)
        for (size_t hd = 0; hd < h; hd++) {
            const float *q = qkv + i * row + hd * d;
            for (size_t j = 0; j < t; j++) {
                const float *kk = qkv + j * row + h * d + hd * d;
                double dot = 0.0;
                for (size_t e = 0; e < d; e++) dot += (double)q[e] * (double)kk[e];
                out[(i * h + hd) * t + j] = (float)dot;
            }
        }
}

/* reference.rs:459-470: exp(x - rowmax) / sum, in f64. */
void blo_ref_softmax(const float *x, size_t rows, size_t cols, float *out) {
    #pragma omp parallel
    {
        double *e = (double *)malloc(cols * sizeof(double));
        #pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            const float *row = x + r * cols;
            double m = -INFINITY;
            for (size_t j = 0; j < cols; j++) m = fmax(m, (double)row[j]);
            double sum = 0.0;
            for (size_t j = 0; j < cols; j++) {
                e[j] = exp((double)row[j] - m);
                sum += e[j];
            }
            for (size_t j = 0; j < cols; j++) out[r * cols + j] = (float)(e[j] / sum);
        }
        free(e);
    }
}

/* reference.rs:474-494: O[i][hd][:] = sum_j P[i][hd][j] V[j][hd][:]; result
 * [t][h*d], heads side by side. */
void blo_ref_attention_values(const float *probs, const float *qkv, size_t t,
                              size_t h, size_t d, float *out) {
    size_t row = 3 * h * d;
    #pragma omp parallel
    {
        double *acc = (double *)malloc(d * sizeof(double));
        #pragma omp for schedule(static)
        for (size_t i = 0; i < t; i++)
            for (size_t hd = 0; hd < h; hd++) {
                for (size_t e = 0; e < d; e++) acc[e] = 0.0;
                const float *p = probs + (i * h + hd) * t;
                for (size_t j = 0; j < t; j++) {
                    const float *v = qkv + j * row + 2 * h * d + hd * d;
                    double w = p[j];
                    for (size_t e = 0; e < d; e++) acc[e] += w * (double)v[e];
                }
                for (size_t e = 0; e < d; e++) out[i * h * d + hd * d + e] = (float)acc[e];
            }
        free(acc);
    }
}

/* The three attention ops of reference.rs:526-528 composed per query row in
 * f64, without storing the [t][h][t] scores or probabilities. */
void blo_ref_attention(const float *qkv, size_t t, size_t h, size_t d,
                       float scale, float *out) {
    size_t row = 3 * h * d;
    #pragma omp parallel
    {
        double *s = (double *)malloc(t * sizeof(double));
        double *acc = (double *)malloc(d * sizeof(double));
        #pragma omp for schedule(static)
        for (size_t i = 0; i < t; i++)
            for (size_t hd = 0; hd < h; hd++) {
                const float *q = qkv + i * row + hd * d;
                double m = -INFINITY;
                for (size_t j = 0; j < t; j++) {
                    const float *kk = qkv + j * row + h * d + hd * d;
                    double dot = 0.0;
                    for (size_t e = 0; e < d; e++) dot += (double)q[e] * (double)kk[e];
                    s[j] = dot * (double)scale;
                    m = fmax(m, s[j]);
                }
                double sum = 0.0;
                for (size_t j = 0; j < t; j++) {
                    s[j] = exp(s[j] - m);
                    sum += s[j];
                }
                for (size_t e = 0; e < d; e++) acc[e] = 0.0;
                for (size_t j = 0; j < t; j++) {
                    const float *v = qkv + j * row + 2 * h * d + hd * d;
                    double w = s[j] / sum;
                    for (size_t e = 0; e < d; e++) acc[e] += w * (double)v[e];
                }
                for (size_t e = 0; e < d; e++) out[i * h * d + hd * d + e] = (float)acc[e];
            }
        free(s);
        free(acc);
    }
}

/* reference.rs:388-420: image [gh*p][gw*p][cin] by HWIO weights
 * [p][p][cin][cout] plus bias; result [gh*gw][cout]. */
void blo_ref_patch_embed(const float *image, const float *w, const float *bias,
                         size_t gh, size_t gw, size_t p, size_t cin, size_t cout,
                         float *out) {
    size_t width = gw * p;
    #pragma omp parallel
    {
        double *acc = (double *)malloc(cout * sizeof(double));
        #pragma omp for schedule(static)
        for (size_t patch = 0; patch < gh * gw; patch++) {
            size_t gy = patch / gw, gx = patch % gw;
            for (size_t co = 0; co < cout; co++) acc[co] = bias ? (double)bias[co] : 0.0;
            for (size_t ky = 0; ky < p; ky++)
                for (size_t kx = 0; kx < p; kx++) {
                    size_t pixel = ((gy * p + ky) * width + gx * p + kx) * cin;
                    for (size_t ci = 0; ci < cin; ci++) {
                        double xv = image[pixel + ci];
                        const float *wr = w + ((ky * p + kx) * cin + ci) * cout;
                        for (size_t co = 0; co < cout; co++) acc[co] += xv * (double)wr[co];
                    }
                }
            for (size_t co = 0; co < cout; co++) out[patch * cout + co] = (float)acc[co];
        }
        free(acc);
    }
}

/* reference.rs:43-81: every output pixel centred on input (y s, x s); a tap
 * outside the image reads zero. Sum in f64 in (ky, kx, ci) order after the bias. */
void blo_ref_conv3x3(const float *in, const float *w, const float *bias, size_t h,
                     size_t wd, size_t cin, size_t cout, size_t stride, float *out) {
    const size_t oh = (h - 1) / stride + 1, ow = (wd - 1) / stride + 1;
    #pragma omp parallel for schedule(static)
    for (size_t px = 0; px < oh * ow; px++) {
        const size_t y = px / ow, x = px % ow;
        for (size_t co = 0; co < cout; co++) {
            double acc = bias ? (double)bias[co] : 0.0;
            for (size_t ky = 0; ky < 3; ky++)
                for (size_t kx = 0; kx < 3; kx++) {
                    if (y * stride + ky < 1 || x * stride + kx < 1) continue;
                    const size_t iy = y * stride + ky - 1, ix = x * stride + kx - 1;
                    if (iy >= h || ix >= wd) continue;
                    const float *a = in + (iy * wd + ix) * cin;
                    const float *b = w + (ky * 3 + kx) * cin * cout + co;
                    for (size_t ci = 0; ci < cin; ci++) acc += (double)a[ci] * (double)b[ci * cout];
                }
            out[px * cout + co] = (float)acc;
        }
    }
}

/* reference.rs:87-106. */
void blo_ref_conv1x1(const float *in, const float *w, const float *bias, size_t pixels,
                     size_t cin, size_t cout, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t p = 0; p < pixels; p++)
        for (size_t co = 0; co < cout; co++) {
            double acc = bias ? (double)bias[co] : 0.0;
            for (size_t ci = 0; ci < cin; ci++) acc += (double)in[p * cin + ci] * (double)w[ci * cout + co];
            out[p * cout + co] = (float)acc;
        }
}

/* reference.rs:114-144: every input pixel adds its channels times each tap
 * into the output pixel the tap reaches, accumulated in f64; then the bias. */
void blo_ref_conv_transpose(const float *in, const float *w, const float *bias, size_t h,
                            size_t wd, size_t cin, size_t cout, size_t f, float *out) {
    const size_t ow = wd * f, total = h * f * ow * cout;
    double *acc = (double *)calloc(total, sizeof(double));
    for (size_t y = 0; y < h; y++)
        for (size_t x = 0; x < wd; x++)
            for (size_t ky = 0; ky < f; ky++)
                for (size_t kx = 0; kx < f; kx++) {
                    double *o = acc + ((y * f + ky) * ow + x * f + kx) * cout;
                    for (size_t ci = 0; ci < cin; ci++) {
                        const double v = in[(y * wd + x) * cin + ci];
                        const float *taps = w + ((ky * f + kx) * cin + ci) * cout;
                        for (size_t co = 0; co < cout; co++) o[co] += v * (double)taps[co];
                    }
                }
    for (size_t i = 0; i < total; i++) out[i] = (float)(acc[i] + (bias ? (double)bias[i % cout] : 0.0));
    free(acc);
}

/* reference.rs:151-179: position o (in - 1) / (out - 1) (zero for one output),
 * the floor and the next index clamped to the last, weights in f64. */
static void resize_axis(size_t o, size_t in, size_t outn, size_t *i0, size_t *i1, double *l) {
    const double pos = outn > 1 ? (double)o * (double)(in - 1) / (double)(outn - 1) : 0.0;
    size_t f = (size_t)floor(pos);
    if (f > in - 1) f = in - 1;
    *i0 = f;
    *i1 = f + 1 < in ? f + 1 : in - 1;
    *l = pos - (double)f;
}
void blo_ref_resize_bilinear(const float *in, size_t ih, size_t iw, size_t oh, size_t ow,
                             size_t c, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t oy = 0; oy < oh; oy++) {
        size_t y0, y1;
        double ly;
        resize_axis(oy, ih, oh, &y0, &y1, &ly);
        for (size_t ox = 0; ox < ow; ox++) {
            size_t x0, x1;
            double lx;
            resize_axis(ox, iw, ow, &x0, &x1, &lx);
            for (size_t ch = 0; ch < c; ch++) {
                const double a = in[(y0 * iw + x0) * c + ch], b = in[(y0 * iw + x1) * c + ch];
                const double cc = in[(y1 * iw + x0) * c + ch], d = in[(y1 * iw + x1) * c + ch];
                const double top = (1.0 - lx) * a + lx * b, bottom = (1.0 - lx) * cc + lx * d;
                out[(oy * ow + ox) * c + ch] = (float)((1.0 - ly) * top + ly * bottom);
            }
        }
    }
}

/* reference.rs:423-425. */
void blo_ref_prepend_token(const float *token, const float *tokens, size_t rows,
                           size_t c, float *out) {
    memcpy(out, token, c * sizeof(float));
    memcpy(out + c, tokens, rows * c * sizeof(float));
}

/* reference.rs:520-544, written as its forward pass. */
void blo_ref_vit_block(const float *x, const blo_block_weights *w, size_t t,
                       size_t h, size_t d, size_t mlp, float eps,
                       int attention_rounded, float *out) {
    size_t width = h * d;
    size_t td = t * width;
    float *n1 = (float *)malloc(td * sizeof(float));
    float *qkv = (float *)malloc(3 * td * sizeof(float));
    float *values = (float *)malloc(td * sizeof(float));
    float *proj = (float *)malloc(td * sizeof(float));
    float *x1 = (float *)malloc(td * sizeof(float));
    float *hidden = (float *)malloc(t * mlp * sizeof(float));
    float scale = 1.0f / sqrtf((float)d);

    blo_ref_layernorm(x, w->norm1_g, w->norm1_b, t, width, eps, n1);
    blo_ref_matmul(n1, w->qkv_w, w->qkv_b, t, width, 3 * width, qkv);
    if (attention_rounded) {
        size_t ns = t * h * t;
        float *s = (float *)malloc(ns * sizeof(float));
        float *p = (float *)malloc(ns * sizeof(float));
        blo_ref_attention_scores(qkv, t, h, d, s);
        blo_ref_scale(s, ns, scale, s);
        blo_ref_softmax(s, t * h, t, p);
        blo_ref_attention_values(p, qkv, t, h, d, values);
        free(s);
        free(p);
    } else {
        blo_ref_attention(qkv, t, h, d, scale, values);
    }
    blo_ref_matmul(values, w->proj_w, w->proj_b, t, width, width, proj);
    blo_ref_channel_scale(proj, w->ls1, td, width, proj);
    blo_ref_add(x, proj, td, x1);
    blo_ref_layernorm(x1, w->norm2_g, w->norm2_b, t, width, eps, n1);
    blo_ref_matmul(n1, w->fc1_w, w->fc1_b, t, width, mlp, hidden);
    blo_ref_gelu_erf(hidden, t * mlp, hidden);
    blo_ref_matmul(hidden, w->fc2_w, w->fc2_b, t, mlp, width, proj);
    blo_ref_channel_scale(proj, w->ls2, td, width, proj);
    blo_ref_add(x1, proj, td, out);

    free(n1); free(qkv); free(values); free(proj); free(x1); free(hidden);
}

/* ------------------------------------------------------------------------ */
/* 2. WGSL-order emulation                                                   */
/* ------------------------------------------------------------------------ */

/* The A&S 7.1.26 constants the reference's kernels evaluate
 * (crates/beatlm-core/src/kernel.rs:355-364). */
static const float GELU_P = 0.3275911f;
static const float GELU_A1 = 0.254829592f, GELU_A2 = -0.284496736f,
                   GELU_A3 = 1.421413741f, GELU_A4 = -1.453152027f,
                   GELU_A5 = 1.061405429f;

/* wgsl.rs:331-353: x * Phi(x) with Phi from erfc(|x|/sqrt 2)/2, in f32. */
float blo_wg_gelu_erf1(float x) {
    float z = fabsf(x) * 0.70710678118654752f;
    float t = 1.0f / (1.0f + GELU_P * z);
    float poly = t * (GELU_A1 + t * (GELU_A2 + t * (GELU_A3 + t * (GELU_A4 + t * GELU_A5))));
    float q = 0.5f * poly * expf(-z * z);
    return x * (x >= 0.0f ? 1.0f - q : q);
}

/* In-place halving tree over `lanes` partials (a power of two), as the
 * workgroup-memory reductions of wgsl.rs:529-541 and :600-629 do. */
static float tree_sum(float *s, unsigned lanes) {
    for (unsigned stride = lanes / 2; stride > 0; stride >>= 1)
        for (unsigned l = 0; l < stride; l++) s[l] = s[l] + s[l + stride];
    return s[0];
}
static float tree_max(float *s, unsigned lanes) {
    for (unsigned stride = lanes / 2; stride > 0; stride >>= 1)
        for (unsigned l = 0; l < stride; l++) s[l] = fmaxf(s[l], s[l + stride]);
    return s[0];
}

static void wg_layernorm_row(const float *x, const float *gamma, const float *beta,
                             size_t c, float eps, float *y) {
    enum { LANES = 64 };
    float part[LANES];
    for (unsigned l = 0; l < LANES; l++) {
        float s = 0.0f;
        for (size_t i = l; i < c; i += LANES) s = s + x[i];
        part[l] = s;
    }
    float mean = tree_sum(part, LANES) / (float)c;
    for (unsigned l = 0; l < LANES; l++) {
        float s = 0.0f;
        for (size_t i = l; i < c; i += LANES) {
            float dv = x[i] - mean;
            s = s + dv * dv;
        }
        part[l] = s;
    }
    float inv = 1.0f / sqrtf(tree_sum(part, LANES) / (float)c + eps);
    for (size_t i = 0; i < c; i++) y[i] = (x[i] - mean) * inv * gamma[i] + beta[i];
}

/* wgsl.rs:519-585: 64 lane-strided f32 partials, a halving tree, mean; then
 * the same for sum (x - mean)^2; inverseSqrt(var + eps). */
void blo_wg_layernorm(const float *x, const float *gamma, const float *beta,
                      size_t rows, size_t c, float eps, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++)
        wg_layernorm_row(x + r * c, gamma, beta, c, eps, out + r * c);
}

static void wg_softmax_row(const float *x, size_t cols, float *y) {
    enum { LANES = 256 };
    float part[LANES];
    for (unsigned l = 0; l < LANES; l++) {
        float m = -3.40282347e38f; /* f32::MIN, wgsl.rs:640 */
        for (size_t i = l; i < cols; i += LANES) m = fmaxf(m, x[i]);
        part[l] = m;
    }
    float row_max = tree_max(part, LANES);
    for (unsigned l = 0; l < LANES; l++) {
        float s = 0.0f;
        for (size_t i = l; i < cols; i += LANES) s = s + expf(x[i] - row_max);
        part[l] = s;
    }
    float inv = 1.0f / tree_sum(part, LANES);
    for (size_t i = 0; i < cols; i++) y[i] = expf(x[i] - row_max) * inv;
}

/* wgsl.rs:590-669. */
void blo_wg_softmax(const float *x, size_t rows, size_t cols, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++) wg_softmax_row(x + r * cols, cols, out + r * cols);
}

/* wgsl.rs:835-846, :920-932: every output a sequential f32 sum over k from
 * zero, then + bias. Rows handed to threads; within a row the accumulators
 * run along n so each one still sums k in increasing order. */
static void wg_matmul_rows(const float *a, const float *b, const float *bias,
                           size_t r0, size_t r1, size_t k, size_t n, float *out) {
    for (size_t i = r0; i < r1; i++) {
        float *o = out + i * n;
        for (size_t j = 0; j < n; j++) o[j] = 0.0f;
        for (size_t l = 0; l < k; l++) {
            float av = a[i * k + l];
            const float *brow = b + l * n;
            for (size_t j = 0; j < n; j++) o[j] = o[j] + av * brow[j];
        }
        if (bias)
            for (size_t j = 0; j < n; j++) o[j] = o[j] + bias[j];
    }
}

void blo_wg_matmul(const float *a, const float *b, const float *bias,
                   size_t m, size_t k, size_t n, float *out) {
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < m; i++) wg_matmul_rows(a, b, bias, i, i + 1, k, n, out);
}

size_t blo_wg_block_scratch_floats(size_t t, size_t h, size_t d, size_t mlp) {
    size_t width = h * d;
    return t * width            /* n1 / n2 */
         + 3 * t * width        /* qkv */
         + 2 * t * h * t        /* scores, probabilities */
         + t * width            /* values */
         + t * width            /* x1 */
         + t * mlp;             /* hidden */
}

/* The reference's 9 fused kernels of one block (kernel.rs:3798-3811), each as
 * its WGSL template computes it: layernorm; matmul; attention_scores+scale;
 * softmax; attention_values; matmul+channel_scale+add; layernorm;
 * matmul+gelu_erf; matmul+channel_scale+add. */
void blo_wg_vit_block(const float *x, const blo_block_weights *w, size_t t,
                      size_t h, size_t d, size_t mlp, float eps, int threads,
                      float *scratch, float *out) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    size_t width = h * d, row3 = 3 * width;
    float *n1 = scratch;
    float *qkv = n1 + t * width;
    float *s = qkv + 3 * t * width;
    float *p = s + t * h * t;
    float *values = p + t * h * t;
    float *x1 = values + t * width;
    float *hidden = x1 + t * width;
    const float scale = 1.0f / sqrtf((float)d); /* Scale(0.125) at d = 64 */

    blo_wg_layernorm(x, w->norm1_g, w->norm1_b, t, width, eps, n1);
    blo_wg_matmul(n1, w->qkv_w, w->qkv_b, t, width, row3, qkv);
    /* attention_scores + scale (wgsl.rs:975-988): sum over d, then * scale. */
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < t; i++)
        for (size_t hd = 0; hd < h; hd++) {
            const float *q = qkv + i * row3 + hd * d;
            float *srow = s + (i * h + hd) * t;
            for (size_t j = 0; j < t; j++) {
                const float *kk = qkv + j * row3 + width + hd * d;
                float acc = 0.0f;
                for (size_t e = 0; e < d; e++) acc = acc + q[e] * kk[e];
                srow[j] = acc * scale;
            }
        }
    blo_wg_softmax(s, t * h, t, p);
    /* attention_values (wgsl.rs:992-1010): sum over keys in order. */
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < t; i++)
        for (size_t hd = 0; hd < h; hd++) {
            float *o = values + i * width + hd * d;
            const float *prow = p + (i * h + hd) * t;
            for (size_t e = 0; e < d; e++) o[e] = 0.0f;
            for (size_t j = 0; j < t; j++) {
                const float *v = qkv + j * row3 + 2 * width + hd * d;
                float pw = prow[j];
                for (size_t e = 0; e < d; e++) o[e] = o[e] + pw * v[e];
            }
        }
    /* matmul + channel_scale + add: out-proj into x1. */
    blo_wg_matmul(values, w->proj_w, w->proj_b, t, width, width, x1);
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < t * width; i++) x1[i] = x1[i] * w->ls1[i % width] + x[i];
    blo_wg_layernorm(x1, w->norm2_g, w->norm2_b, t, width, eps, n1);
    blo_wg_matmul(n1, w->fc1_w, w->fc1_b, t, width, mlp, hidden);
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < t * mlp; i++) hidden[i] = blo_wg_gelu_erf1(hidden[i]);
    blo_wg_matmul(hidden, w->fc2_w, w->fc2_b, t, mlp, width, out);
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < t * width; i++) out[i] = out[i] * w->ls2[i % width] + x1[i];
}

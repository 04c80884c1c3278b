/*
 * The oracle: a CPU restatement of the reference's algorithm for the pre-LN
 * ViT encoder block. TEST INFRASTRUCTURE ONLY — tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg use it as the checker or the CPU baseline;
 * the product (libbeatlm_hip.so) never links or calls it.
 *
 * Two halves:
 *
 *  1. `blo_ref_*`: the reference's CPU reference ops, f64 accumulation, each
 *     result rounded to f32 (crates/beatlm-bench/src/reference.rs). These are
 *     the values a kernel is compared against, within
 *     |got - want| <= 1e-4 + 1e-4 |want| for f32 (reference.rs:22-24).
 *
 *  2. `blo_wg_*`: the reference's generated WGSL kernels' arithmetic, f32 in
 *     the same summation order (crates/beatlm/src/codegen/wgsl.rs), i.e. what
 *     the reference's own wgpu path computes up to FMA contraction and
 *     exp/inverseSqrt ulps. Timed as the CPU baseline, multi-threaded over row
 *     ranges.
 *
 * Plus the seeded generators the reference's tests and the configurations use
 * (crates/beatlm-bench/src/net.rs:183-203).
 */
#ifndef BEATLM_ORACLE_H
#define BEATLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- generators (net.rs:183-203, harness.rs:80-84) ---- */

/* `count` values uniform in [low, high): the reference's LCG, top 24 bits. */
void blo_uniform(uint64_t seed, size_t count, float low, float high, float *out);
/* `count` standard normals: Box-Muller over the same LCG's uniforms. */
void blo_normal(uint64_t seed, size_t count, float mean, float std, float *out);

/* ---- 1. f64 reference ops (reference.rs) ---- */

double blo_erf(double x);                                       /* :337-360 */
void blo_ref_layernorm(const float *x, const float *gamma, const float *beta,
                       size_t rows, size_t c, float eps, float *out); /* :247-270 */
void blo_ref_matmul(const float *a, const float *b, const float *bias,
                    size_t m, size_t k, size_t n, float *out);   /* :273-298 */
void blo_ref_add(const float *a, const float *b, size_t n, float *out); /* :301-306 */
void blo_ref_relu(const float *x, size_t n, float *out);              /* :309-311 */
void blo_ref_gelu_tanh(const float *x, size_t n, float *out);         /* :314-322 */
void blo_ref_scale(const float *x, size_t n, float f, float *out);    /* :325-329 */
void blo_ref_gelu_erf(const float *x, size_t n, float *out);          /* :369-376 */
void blo_ref_channel_scale(const float *x, const float *s, size_t n,
                           size_t channels, float *out);              /* :379-384 */
void blo_ref_attention_scores(const float *qkv, size_t t, size_t h, size_t d,
                              float *out);                            /* :437-455 */
void blo_ref_softmax(const float *x, size_t rows, size_t cols, float *out); /* :459-470 */
void blo_ref_attention_values(const float *probs, const float *qkv, size_t t,
                              size_t h, size_t d, float *out);        /* :474-494 */
/* scores -> scale -> softmax -> values in f64 one query row at a time, the
 * three ops of reference.rs:526-528 without rounding the two [t][h][t]
 * intermediates to f32 (for sequence lengths whose scores do not fit). */
void blo_ref_attention(const float *qkv, size_t t, size_t h, size_t d,
                       float scale, float *out);
void blo_ref_patch_embed(const float *image, const float *w, const float *bias,
                         size_t gh, size_t gw, size_t p, size_t cin, size_t cout,
                         float *out);                                 /* :388-420 */
void blo_ref_prepend_token(const float *token, const float *tokens, size_t rows,
                           size_t c, float *out);                     /* :423-425 */

/* The DPT head's operations, NHWC maps and HWIO weights (reference.rs:26-191). */
/* 3x3 convolution, zero padding 1, at `stride`: output [oh][ow][cout] with
 * oh = (h - 1) / stride + 1; bias may be NULL.                    :31-81 */
void blo_ref_conv3x3(const float *in, const float *w, const float *bias, size_t h,
                     size_t wd, size_t cin, size_t cout, size_t stride, float *out);
/* 1x1 convolution: [pixels][cin] times [cin][cout], per pixel.        :87-106 */
void blo_ref_conv1x1(const float *in, const float *w, const float *bias, size_t pixels,
                     size_t cin, size_t cout, float *out);
/* Transposed convolution, kernel = stride = f, no padding, written as its
 * scatter definition: output [h f][w f][cout].                       :114-144 */
void blo_ref_conv_transpose(const float *in, const float *w, const float *bias, size_t h,
                            size_t wd, size_t cin, size_t cout, size_t f, float *out);
/* Bilinear resampling with aligned corners, f64 positions.          :151-179 */
void blo_ref_resize_bilinear(const float *in, size_t ih, size_t iw, size_t oh, size_t ow,
                             size_t c, float *out);

/* The weights of one block in the IR's layouts (reference.rs:497-516). */
typedef struct {
    const float *norm1_g, *norm1_b;
    const float *qkv_w, *qkv_b;      /* [D][3D], [3D] */
    const float *proj_w, *proj_b;    /* [D][D], [D] */
    const float *ls1;
    const float *norm2_g, *norm2_b;
    const float *fc1_w, *fc1_b;      /* [D][M], [M] */
    const float *fc2_w, *fc2_b;      /* [M][D], [D] */
    const float *ls2;
} blo_block_weights;

/* One pre-norm DINOv2 block (reference.rs:520-544). `attention_rounded`
 * selects the reference's own path (scores and probabilities rounded to f32
 * as the unfused program stores them) when nonzero, blo_ref_attention when 0. */
void blo_ref_vit_block(const float *x, const blo_block_weights *w, size_t t,
                       size_t h, size_t d, size_t mlp, float eps,
                       int attention_rounded, float *out);

/* ---- 2. WGSL-order emulation (wgsl.rs), f32 ---- */

float blo_wg_gelu_erf1(float x);                                      /* wgsl.rs:331-353 */
void blo_wg_layernorm(const float *x, const float *gamma, const float *beta,
                      size_t rows, size_t c, float eps, float *out);  /* :519-585 */
void blo_wg_softmax(const float *x, size_t rows, size_t cols, float *out); /* :590-669 */
/* tiled matmul: each output a sequential f32 sum over k, then +bias (:835-846). */
void blo_wg_matmul(const float *a, const float *b, const float *bias,
                   size_t m, size_t k, size_t n, float *out);
/* The fused block, as the reference's 9 kernels compute it, over `threads`
 * threads (0 = one per online CPU). `scratch` holds at least
 * blo_wg_block_scratch_floats(t, h, d, mlp) floats. */
size_t blo_wg_block_scratch_floats(size_t t, size_t h, size_t d, size_t mlp);
void blo_wg_vit_block(const float *x, const blo_block_weights *w, size_t t,
                      size_t h, size_t d, size_t mlp, float eps, int threads,
                      float *scratch, float *out);

#ifdef __cplusplus
}
#endif
#endif

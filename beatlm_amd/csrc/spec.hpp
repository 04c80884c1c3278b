// Internal: the launch arguments of each device kernel and the host-side
// launchers the backend dispatches a kernel spec to.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/beatlm_hip.h"

namespace bl {

struct DevEpilogue;

// How an f32 or f16 product is computed on the matrix cores.
enum class Math : int {
    F32 = 0,    // f32 storage, v_mfma_f32_16x16x4_f32
    SPLIT = 1,  // f32 storage, each operand hi + lo bf16, three v_mfma_f32_16x16x32_bf16
    F16 = 2,    // f16 storage, v_mfma_f32_16x16x32_f16, f32 accumulate
};

struct EpilogueArgs {
    int n;
    int kind[BL_MAX_EPILOGUE];
    float factor[BL_MAX_EPILOGUE];
    uint32_t channels[BL_MAX_EPILOGUE];
    const void *operand[BL_MAX_EPILOGUE];
};

struct LayerNormArgs {
    const void *x, *gamma, *beta;
    void *y;
    uint32_t rows, channels;
    uint32_t row0, row1;  // the part's rows
    float eps;
    EpilogueArgs epi;
    uint64_t y_planes;    // y kept as hi and lo bf16 planes this many elements apart (0: as T)
};

struct GemmArgs {
    const void *a;
    const void *b;        // the packed B: [planes][n_pad][k_pad]
    const void *bias;
    void *c;
    uint32_t m, n, k;
    uint32_t n_pad, k_pad;
    uint32_t row0, row1;
    int load;             // A: 0 rows of whole vectors, 1 element by element, 2 patches of an image
    int epi_mode;         // 0 none, 1 gelu_erf, 2 channel_scale(over n) + add, 3 any steps
    int pipeline;         // 1: the LDS-ring kernel with direct loads (k a multiple of 32)
    uint32_t kgroups;     // pipelined kernel: groups of 4 waves splitting the k-steps (1, 2 or 4)
    uint32_t stages;      // pipelined kernel: ring depth per group (2 .. 4)
    uint32_t kslices;     // pipelined kernel: 32-wide k-slices per ring stage (1 or 2)
    uint32_t p0, p1, p2, p3;  // patches: grid_w, patch, cin, image width; conv3x3: height, width, cin, stride
    uint32_t p4, p5;          // conv3x3: output width, ReLU prologue (1) or none (0)
    // Split k (the non-pipelined kernel, gathered A only): ksplit > 1
    // workgroups per tile (blockIdx.y) each multiply a contiguous run of the
    // k-steps and write their raw sums to partials [ksplit][row1 - row0][n];
    // gemm_reduce_kernel then adds them in split order, adds the bias and
    // runs the epilogue.
    uint32_t ksplit;
    float *partials;
    EpilogueArgs epi;
    // The QKV projection of a flash attention kernel also writes that
    // kernel's K [planes][H][t_pad][64] and Vt [planes][H][64][t_pad]
    // operands (its prep step, fused) when flash_ops is set; with 2, qkv
    // itself receives the queries alone (its first third of columns).
    int flash_ops;
    void *fl_kp, *fl_vt;
    uint32_t fl_tpad;
    // bf16x3 math: A, or C, kept as hi and lo bf16 planes this many elements
    // apart (0: f32).
    uint64_t a_planes, c_planes;
    // A LayerNorm over this product's output folded into the product that
    // reads the LayerNorm's output (this product is the fold's producer):
    // ln_out [m][n / 32] of (mean, sum of squared deviations from that mean)
    // of each row's 32-column blocks of the output as stored; ln_shadow (f32
    // storage) the output once more, centred per block (each value less its
    // block's mean), as hi and lo bf16 planes m * n elements apart for
    // bf16x3 or as f32 for the f32 matrix cores: the consumer's A. Null: none.
    float *ln_out;
    void *ln_shadow;
    // A LayerNorm folded into this product (the fold's consumer): A is the
    // LayerNorm's input x; ln_stats holds x's block statistics as ln_out
    // does; the packed B holds gamma (.) B row by row, ln_c [n] its column
    // sums and ln_d [n] = beta . B[:, n] + bias[n], so that
    // LN(x) B + bias = rstd (x (gamma B) - mean c) + d (f16 storage). With
    // ln_cb (f32 storage) A is x centred per block (the producer's shadow) and
    // ln_cb [n][32] holds the column sums of gamma (.) B over each 32-row
    // block of k: LN(x) B + bias = rstd (A (gamma B) + sum_b (mean_b - mean)
    // cb[b]) + d, where the correction is one more product on the matrix cores
    // and no term carries x's common offset.
    const float *ln_stats, *ln_c, *ln_d, *ln_cb;
    uint32_t ln_blocks;   // 32-column blocks of x (k / 32)
    float ln_eps;
    // The ring kernel's per-lane epilogue in place of the one through LDS.
    uint32_t lane_epilogue;
    // The ring kernel with B in registers: B packed fragment-major
    // (packed_at), each wave loading its columns' fragments straight into
    // registers STAGES k-steps ahead; A alone goes through the LDS ring.
    uint32_t breg;
    // The direct 3x3 convolution: workgroups of its persistent grid (each
    // takes every cd_grid-th tile of its XCD's share), and whether they keep
    // every input-channel chunk's weights in LDS (staged once) or stage one
    // chunk's per tile.
    uint32_t cd_grid, cd_resident;
    // ln_shadow's plane distance in elements (0: m * n).
    uint64_t ln_plane;
    // The class-token prepend fused into this product (a patch embedding,
    // the plain kernel): c is x's second row, so that the product's rows are
    // x's rows 1 .. m, and the epilogue's added tensors are read one row on
    // likewise; the workgroups of the first row band also write x's first
    // row, cls_epi applied to cls_token [n], at cls_out (x itself), with its
    // block statistics at cls_ln_out and its planes at cls_shadow when the
    // product is a fold's producer. Null cls_out: none.
    const void *cls_token;
    void *cls_out;
    float *cls_ln_out;
    void *cls_shadow;
    EpilogueArgs cls_epi;
};

hipError_t launch_gemm_reduce(const GemmArgs &a, bool f16, hipStream_t s);

// B [k][n] -> the GEMM's packed operand (transposed, padded, converted).
struct PackArgs {
    const void *src;
    void *dst;
    uint32_t k, n, k_pad, n_pad;
    // A folded LayerNorm's weights (null: a plain pack): row k of B is packed
    // scaled by gamma[k], and vec [2][n_pad] receives c[n] (the column sums of
    // the packed B as the matrix cores read it) and d[n] = beta . B[:, n] +
    // bias[n] (bias may be null).
    const void *gamma, *beta, *bias;
    float *vec;
    uint32_t frag;  // pack fragment-major (packed_at) for the B-in-registers kernel
};

// Where element (n, k) of a packed B plane lies. Row layout: [n_pad][k_pad].
// Fragment-major: 16-column, 32-deep blocks of 512 elements, column block
// major, each block in the order the 16 x 16 x 32 MFMA's 64 lanes take their
// B operand (lane = n % 16 + 16 * (k % 32 / 8), 8 consecutive k a lane), so
// one 16-byte load per lane is one whole 1 KB block.
__host__ __device__ inline uint64_t packed_at(uint32_t n, uint32_t k, uint32_t k_pad, bool frag) {
    if (!frag) return (uint64_t)n * k_pad + k;
    const uint64_t block = (uint64_t)(n / 16) * (k_pad / 32) + k / 32;
    return block * 512 + ((k % 32) / 8 * 16 + n % 16) * 8 + k % 8;
}

// A folded LayerNorm's statistics made from x itself (when the fold's
// producer has not written them since x last changed): x [rows][cols]
// (cols a multiple of 32) -> stats [rows][cols / 32] of (mean, sum of squared
// deviations), and (f32 x, shadow non-null) x centred per block, as hi and
// lo bf16 planes `planes` elements apart, or as f32 (planes 0).
struct LnStatsArgs {
    const void *x;
    float *stats;
    void *shadow;
    uint32_t rows, cols;
    uint64_t planes;
};
hipError_t launch_ln_stats(const LnStatsArgs &a, bool f16, hipStream_t s);

// The tiled products whose operands are gathered (the unfused attention
// products and the patch embedding), on the vector ALUs.
enum class Gather : int { SCORES = 0, VALUES = 1, PATCH = 2 };

struct GatherArgs {
    const void *a, *b, *bias;
    void *c;
    uint32_t n, k, layers;          // output columns per layer, reduction, layers
    uint32_t row0, row1;
    // attention: tokens, heads, head_dim; patch: grid_w, patch, cin, image width
    uint32_t p0, p1, p2, p3;
    EpilogueArgs epi;
};

struct SoftmaxArgs {
    const void *x;
    void *y;
    uint32_t cols;
    uint32_t row0, row1;
    EpilogueArgs epi;
};

struct FlashArgs {
    const void *qkv;
    void *out;
    void *kp;             // keys [planes][heads][t_pad][64] in the operand type
    void *vt;             // values transposed [planes][heads][64][t_pad]
    float *partial;       // partial outputs of key ranges (unnormalised, f32)
    float *stats;         // their (max, sum) pairs
    uint32_t tokens, heads, t_pad;
    uint32_t row0, row1;  // query rows of the part
    uint32_t splits;      // f32 math: key ranges per query tile
    float scale;          // softmax scale (the Scale epilogue of the scores)
    // f16 and bf16x3 math: the (head, query tile, key tile) units are dealt
    // out in equal contiguous runs to `wgs` workgroups.
    uint32_t qtiles, wgs;
    uint64_t units;
    uint32_t merge;       // 1 when some query tile's key tiles span two runs
    uint32_t prepped;     // 1 when the QKV projection already wrote K and Vt
    uint64_t out_planes;  // bf16x3 math: out kept as hi and lo bf16 planes this many elements apart (0: f32)
    // f16 and bf16x3 math: 1 when the runs that split a query tile combine
    // its partial results themselves (no merge launch). One arrival counter
    // per (head, query tile) pair; every counter is zero between launches.
    uint32_t merge_inline;
    uint32_t *counters;
};

// How a flash attention spec is launched: its grid and the scratch it needs
// (operands, then partial outputs and statistics).
struct FlashPlan {
    uint32_t splits = 1, qtiles = 0, wgs = 0, merge = 0;
    uint64_t units = 0;
    // Operands, partial results and statistics. The arrival counters of the
    // in-kernel merge (`counters` words, one per (head, query tile) pair) are
    // not counted: they sit in a region of their own in front, shared by every
    // flash kernel of the scratch and zero between launches.
    uint64_t scratch_bytes = 0;
    uint32_t counters = 0;
    uint64_t counter_bytes = 0;  // the counters' bytes (each on a line of its own)
    // False when the shape's unit runs would overflow the kernels' 32-bit
    // run arithmetic (units of one XCD times its runs, 2^32 or more): the
    // backend refuses such a kernel.
    bool fits = true;
};
// Host check of plan_flash's unit runs for a shape (f16 and bf16x3 math):
// every XCD's units [0, U) are covered by its G runs in order, each unit by
// exactly one (run_begin monotone from 0 to U, run_of agreeing at every
// run's ends). BL_OK, BL_ERR_TOO_LARGE when the plan refuses the shape, or
// BL_ERR_KERNEL when the runs are wrong.
int flash_plan_check(uint32_t tokens, uint32_t heads, uint32_t compute_units, bool f16, uint64_t *units);

// The DPT head's gathers: each output element from a few input values.
enum class Dpt : int { CONV_TRANSPOSE = 0, RESIZE = 1 };

struct DptArgs {
    const void *x, *w, *bias;
    void *y;
    uint32_t d[6];        // conv transpose: height, width, cin, cout, factor, has_bias;
                          // resize: in_height, in_width, out_height, out_width, channels
    float ry, rx;         // resize: input rows (columns) per output row (column), as PyTorch computes them
    uint64_t start, end;  // output elements of the part
    EpilogueArgs epi;
};

// One element per invocation: the standalone map, the token copies.
enum class PerElement : int { MAP = 0, PREPEND = 1, DROP_FIRST = 2 };

struct ElementArgs {
    const void *a, *b;
    void *y;
    uint64_t start, end;  // output elements of the part
    uint32_t channels;
    EpilogueArgs epi;
    // The prepend as a folded LayerNorm's producer (GemmArgs::ln_out and
    // ln_shadow mean the same): the output's rows are ln_cols elements, a
    // multiple of 32, and the part is whole rows; ln_shadow's planes are
    // ln_plane elements apart (0: the shadow is f32). Null: none.
    float *ln_out = nullptr;
    void *ln_shadow = nullptr;
    uint32_t ln_cols = 0;
    uint64_t ln_plane = 0;
};

// A product with at most 4 output columns (the depth head's 1x1 convolution
// to one channel): rows [row0, row1) of C [m][n] = A [m][k] B [k][n] + bias,
// then the epilogue; B as the plan holds it, k a multiple of 4.
struct GemvArgs {
    const void *a, *b, *bias;
    void *c;
    uint32_t k, n, row0, row1;
    EpilogueArgs epi;
};

// ---- launchers (one per kernel family), defined with their kernels ----

hipError_t launch_layernorm(const LayerNormArgs &a, bool f16, hipStream_t s);
hipError_t launch_gemv(const GemvArgs &a, bool f16, hipStream_t s);
hipError_t launch_gemm_f32(const GemmArgs &a, int tile, hipStream_t s);
hipError_t launch_gemm_split(const GemmArgs &a, int tile, hipStream_t s);
hipError_t launch_gemm_f16(const GemmArgs &a, int tile, hipStream_t s);
hipError_t launch_pack_f32(const PackArgs &a, hipStream_t s);
hipError_t launch_pack_split(const PackArgs &a, hipStream_t s);
hipError_t launch_pack_f16(const PackArgs &a, hipStream_t s);
inline hipError_t launch_gemm(const GemmArgs &a, Math m, int tile, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    return m == Math::F32 ? launch_gemm_f32(a, tile, s)
         : m == Math::SPLIT ? launch_gemm_split(a, tile, s) : launch_gemm_f16(a, tile, s);
}
inline hipError_t launch_pack(const PackArgs &a, Math m, hipStream_t s) {
    return m == Math::F32 ? launch_pack_f32(a, s) : m == Math::SPLIT ? launch_pack_split(a, s) : launch_pack_f16(a, s);
}
// Bytes of a packed B.
inline uint64_t packed_bytes(Math m, uint32_t k_pad, uint32_t n_pad) {
    return (uint64_t)k_pad * n_pad * (m == Math::F16 ? 2 : 4);
}
hipError_t launch_gather(const GatherArgs &a, Gather g, bool f16, hipStream_t s);
hipError_t launch_softmax(const SoftmaxArgs &a, bool f16, hipStream_t s);
hipError_t launch_flash(const FlashArgs &a, Math m, hipStream_t s);
FlashPlan plan_flash(Math m, uint32_t tokens, uint32_t heads, uint32_t row0, uint32_t row1, uint32_t compute_units);
// Points a planned FlashArgs at its scratch: the counter region of
// counter_bytes (at least the plan's counter_bytes, zero) at `base`, then
// plan.scratch_bytes of operands and partial results.
void bind_flash_scratch(FlashArgs &a, Math m, void *base, uint64_t counter_bytes);
hipError_t launch_element(const ElementArgs &a, PerElement p, bool f16, hipStream_t s);
hipError_t launch_spin(uint64_t ticks, uint32_t blocks, hipStream_t s);
hipError_t launch_dpt(const DptArgs &a, Dpt k, bool f16, hipStream_t s);

// The direct 3x3 convolution (k_conv_direct.inc): output rows, columns and
// channels per workgroup, input channels per staged chunk.
constexpr int CD_TH = 2, CD_TW = 64, CD_NB = 32, CD_CC = 32;
constexpr int CD_HR = CD_TH + 2, CD_HC = CD_TW + 2;
constexpr int CD_HALO = CD_HR * CD_HC * 64, CD_WTS = 9 * CD_NB * 64;  // bytes per plane

struct ConvTile {
    uint32_t oy0, ox0, n0;
};
// The part's tiles: the first output row, and tile rows, columns and channel
// blocks.
__host__ __device__ inline void conv_direct_tiles(const GemmArgs &a, uint32_t &oy_first, uint32_t &rows,
                                                  uint32_t &cols, uint32_t &nbs) {
    const uint32_t W = a.p1;
    oy_first = a.row0 / W;
    const uint32_t oy_last = (a.row1 - 1) / W;
    rows = (oy_last - oy_first + CD_TH) / CD_TH;
    cols = (W + CD_TW - 1) / CD_TW;
    nbs = (a.n + CD_NB - 1) / CD_NB;
}
// Whether the direct kernel takes this convolution: stride 1 (output the
// input's size), whole 8-channel groups in and whole 32-channel blocks out,
// one pass (no split k), A as stored (not split planes), no fold.
__host__ inline bool conv_direct_fits(const GemmArgs &a) {
    return a.load == 3 && a.p3 == 1 && a.p4 == a.p1 && a.m == a.p0 * a.p1 && a.p2 % 8 == 0 && a.n % CD_NB == 0 &&
           a.k == 9 * a.p2 && a.ksplit <= 1 && a.a_planes == 0 && !a.ln_stats && !a.ln_out && !a.flash_ops &&
           a.row0 < a.row1 && a.row1 <= a.m && (a.epi_mode == 0 || a.epi_mode == 3) && (uint64_t)a.p0 * a.p1 * a.p2 < (1ull << 40);
}

// Bytes of LDS the kernel holds: the window and `chunks_held` (at least one) chunks
// of weights, per plane.
__host__ inline uint32_t conv_direct_lds(Math m, uint32_t chunks_held) {
    const uint32_t planes = m == Math::SPLIT ? 2 : 1;
    return planes * (CD_HALO + (chunks_held ? chunks_held : 1) * CD_WTS);
}

// GEMM tile shapes the dispatcher can pick from: BM x BN.
// TILE_CONV3: the direct 3x3 convolution (2 output rows x 64 columns x 32
// channels per workgroup; its rows and columns below are the pixels and
// channels of one tile).
enum GemmTile : int { TILE_64x64 = 0, TILE_32x64 = 1, TILE_64x128 = 2, TILE_128x64 = 3, TILE_128x32 = 4, TILE_64x96 = 5, TILE_CONV3 = 6, TILE_COUNT = 7 };
inline int gemm_tile_rows(int t) { const int r[] = {64, 32, 64, 128, 128, 64, 128}; return r[t]; }
inline int gemm_tile_cols(int t) { const int c[] = {64, 64, 128, 64, 32, 96, 32}; return c[t]; }
// K and N of a packed B are padded to these.
constexpr uint32_t PACK_K = 32, PACK_N = 128;

constexpr uint32_t FLASH_HEAD_DIM = 64;

}  // namespace bl

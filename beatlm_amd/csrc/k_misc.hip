// The bandwidth-bound and vector-ALU kernels: layer norm, the standalone
// softmax, the tiled products with gathered operands (unfused attention
// scores and values, the patch embedding), one-element-per-invocation kernels
// (standalone map, class-token prepend, token drop) and a fixed-time spin.
#include <cstdlib>

#include "device_common.hpp"

namespace bl {
namespace {

// ------------------------------------------------------------------------
// Layer norm (MainOp::LayerNorm, kernel.rs:643-659; reference arithmetic
// wgsl.rs:519-585): (x - mean) * rsqrt(var + eps) * gamma + beta per row,
// mean first, then the biased variance of (x - mean).
//
// One wave per row, four rows per workgroup. A lane keeps its share of the
// row in registers (16-byte loads, the row read from HBM once), so the two
// passes and the store cost one read and one write of the row.
// ------------------------------------------------------------------------
template <typename T, int NV>
__global__ __launch_bounds__(256) void layernorm_kernel(LayerNormArgs a) {
    constexpr int VEC = 16 / sizeof(T);
    using V = typename std::conditional<sizeof(T) == 4, f32x4, f16x8>::type;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row = a.row0 + blockIdx.x * 4 + wave;
    if (row >= a.row1) return;
    const uint32_t C = a.channels, nch = C / VEC;
    const T *x = (const T *)a.x + (uint64_t)row * C;
    float v[NV][VEC];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        uint32_t c = lane + 64 * i;
        V chunk = {};
        if (c < nch) chunk = *(const V *)(x + c * VEC);
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            v[i][e] = to_f32(chunk[e]);
            sum += v[i][e];
        }
    }
    const float mean = wave_sum(sum) / (float)C;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        if (lane + 64 * i < nch) {
#pragma unroll
            for (int e = 0; e < VEC; e++) {
                float d = v[i][e] - mean;
                sq += d * d;
            }
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)C + a.eps);
    const T *gamma = (const T *)a.gamma, *beta = (const T *)a.beta;
    T *y = (T *)a.y + (uint64_t)row * C;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        uint32_t c = lane + 64 * i;
        if (c >= nch) continue;
        V gv = *(const V *)(gamma + c * VEC), bv = *(const V *)(beta + c * VEC);
        V out;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            float r = (v[i][e] - mean) * inv * to_f32(gv[e]) + to_f32(bv[e]);
            if (a.epi.n) r = apply_epilogue<T>(a.epi, r, (uint64_t)row * C + c * VEC + e);
            out[e] = from_f32<T>(r);
        }
        if constexpr (sizeof(T) == 4) {
            if (a.y_planes) {
                store_f32x4((float *)a.y, (uint64_t)row * C + c * VEC, out, a.y_planes);
                continue;
            }
        }
        *(V *)(y + c * VEC) = out;
    }
}

// Rows of 3 * LPR 16-byte chunks (384 f32 or f16 channels and the like):
// LPR lanes per row, three chunks per lane, 64 / LPR rows per wave, so every
// lane loads and every reduction stays inside its row's lanes. The row is
// read once into registers. With NT (input and output larger than the
// 256 MB Infinity Cache) the loads and stores are streaming (non-temporal);
// otherwise they stay cached for the next kernel, which reads the output.
template <typename T, int LPR, bool NT>
__global__ __launch_bounds__(256) void layernorm3_kernel(LayerNormArgs a) {
    constexpr int VEC = 16 / sizeof(T), RPW = 64 / LPR;
    using V = typename std::conditional<sizeof(T) == 4, f32x4, f16x8>::type;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LPR, l = lane % LPR;
    const uint32_t row = a.row0 + (blockIdx.x * 4 + wave) * RPW + sub;
    const bool ok = row < a.row1;
    const uint32_t C = a.channels;
    const T *x = (const T *)a.x + (uint64_t)(ok ? row : a.row0) * C;
    float v[3][VEC];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const V *src = (const V *)(x + (l + LPR * i) * VEC);
        const V chunk = NT ? __builtin_nontemporal_load(src) : *src;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            v[i][e] = to_f32(chunk[e]);
            sum += v[i][e];
        }
    }
    const float mean = row_sum<LPR>(sum) / (float)C;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            const float d = v[i][e] - mean;
            sq += d * d;
        }
    const float inv = 1.0f / sqrtf(row_sum<LPR>(sq) / (float)C + a.eps);
    if (!ok) return;
    const T *gamma = (const T *)a.gamma, *beta = (const T *)a.beta;
    T *y = (T *)a.y + (uint64_t)row * C;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const uint32_t c = l + LPR * i;
        const V gv = *(const V *)(gamma + c * VEC), bv = *(const V *)(beta + c * VEC);
        V out;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            float r = (v[i][e] - mean) * inv * to_f32(gv[e]) + to_f32(bv[e]);
            if (a.epi.n) r = apply_epilogue<T>(a.epi, r, (uint64_t)row * C + c * VEC + e);
            out[e] = from_f32<T>(r);
        }
        if constexpr (sizeof(T) == 4) {
            if (a.y_planes) {
                store_f32x4((float *)a.y, (uint64_t)row * C + c * VEC, out, a.y_planes);
                continue;
            }
        }
        if constexpr (NT) __builtin_nontemporal_store(out, (V *)(y + c * VEC));
        else *(V *)(y + c * VEC) = out;
    }
}

// Any width: three passes over the row in memory, one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void layernorm_any_kernel(LayerNormArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row = a.row0 + blockIdx.x * 4 + wave;
    if (row >= a.row1) return;
    const uint32_t C = a.channels;
    const T *x = (const T *)a.x + (uint64_t)row * C;
    float sum = 0.0f;
    for (uint32_t c = lane; c < C; c += 64) sum += to_f32(x[c]);
    const float mean = wave_sum(sum) / (float)C;
    float sq = 0.0f;
    for (uint32_t c = lane; c < C; c += 64) {
        float d = to_f32(x[c]) - mean;
        sq += d * d;
    }
    const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)C + a.eps);
    const T *gamma = (const T *)a.gamma, *beta = (const T *)a.beta;
    for (uint32_t c = lane; c < C; c += 64) {
        float r = (to_f32(x[c]) - mean) * inv * to_f32(gamma[c]) + to_f32(beta[c]);
        r = apply_epilogue<T>(a.epi, r, (uint64_t)row * C + c);
        store_elem<T>((T *)a.y, (uint64_t)row * C + c, r, a.y_planes);
    }
}

template <typename T>
hipError_t ln_launch(const LayerNormArgs &a, hipStream_t s) {
    constexpr uint32_t VEC = 16 / sizeof(T);
    dim3 grid((a.row1 - a.row0 + 3) / 4), block(256);
    const uint32_t nch = a.channels / VEC;
    if (a.channels % VEC == 0 && nch % 3 == 0 && !getenv("BL_LN_WAVE_ROW")) {
        const uint32_t lpr = nch / 3, rows = a.row1 - a.row0;
        auto grid3 = [&](uint32_t rpw) { return dim3((rows + 4 * rpw - 1) / (4 * rpw)); };
        const bool nt = 2ull * rows * a.channels * sizeof(T) > (256ull << 20);
#define BL_LN3(L, RPW)                                                                                 \
    if (lpr == L) {                                                                                    \
        if (nt) hipLaunchKernelGGL((layernorm3_kernel<T, L, true>), grid3(RPW), block, 0, s, a);       \
        else hipLaunchKernelGGL((layernorm3_kernel<T, L, false>), grid3(RPW), block, 0, s, a);        \
        return hipGetLastError();                                                                      \
    }
        BL_LN3(16, 4)
        BL_LN3(32, 2)
        BL_LN3(64, 1)
#undef BL_LN3
    }
    if (a.channels % VEC == 0) {
        if (nch <= 64) { hipLaunchKernelGGL((layernorm_kernel<T, 1>), grid, block, 0, s, a); return hipGetLastError(); }
        if (nch <= 128) { hipLaunchKernelGGL((layernorm_kernel<T, 2>), grid, block, 0, s, a); return hipGetLastError(); }
        if (nch <= 256) { hipLaunchKernelGGL((layernorm_kernel<T, 4>), grid, block, 0, s, a); return hipGetLastError(); }
    }
    hipLaunchKernelGGL(layernorm_any_kernel<T>, grid, block, 0, s, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------------
// Softmax over rows (MainOp::Softmax, kernel.rs:748-756; wgsl.rs:590-669):
// exp(x - rowmax) / sum exp(x - rowmax). One workgroup per row; the unfused
// attention path only (the block runs the flash kernel).
// ------------------------------------------------------------------------
__device__ __forceinline__ float block_reduce(float v, bool is_max, float *scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < (int)(blockDim.x / 64); w++) r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
    return r;
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_kernel(SoftmaxArgs a) {
    __shared__ float scratch[4];
    const uint32_t row = a.row0 + blockIdx.x;
    if (row >= a.row1) return;
    const uint32_t C = a.cols;
    const T *x = (const T *)a.x + (uint64_t)row * C;
    float m = -INFINITY;
    for (uint32_t c = threadIdx.x; c < C; c += 256) m = fmaxf(m, to_f32(x[c]));
    m = block_reduce(m, true, scratch);
    float sum = 0.0f;
    for (uint32_t c = threadIdx.x; c < C; c += 256) sum += __expf(to_f32(x[c]) - m);
    sum = block_reduce(sum, false, scratch);
    const float inv = 1.0f / sum;
    T *y = (T *)a.y + (uint64_t)row * C;
    for (uint32_t c = threadIdx.x; c < C; c += 256) {
        uint64_t i = (uint64_t)row * C + c;
        y[c] = from_f32<T>(apply_epilogue<T>(a.epi, __expf(to_f32(x[c]) - m) * inv, i));
    }
}

// ------------------------------------------------------------------------
// Tiled products with gathered operands on the vector ALUs: the unfused
// attention scores (one product per head, kernel.rs:731-741), the unfused
// weighted sum of the values (kernel.rs:765-777) and the patch embedding as a
// product of the gathered patches by the HWIO weights (kernel.rs:661-687).
// 64 x 64 output tile, 16 reduction indices staged per step, 4 x 4 outputs
// per invocation; each output summed over k in increasing order.
// ------------------------------------------------------------------------
template <Gather G, typename T>
__device__ __forceinline__ float gather_a(const GatherArgs &a, uint32_t row, uint32_t kk, uint32_t layer) {
    const T *A = (const T *)a.a;
    if constexpr (G == Gather::SCORES) {
        const uint32_t H = a.p1, D = a.p2;
        return to_f32(A[(uint64_t)row * 3 * H * D + layer * D + kk]);
    } else if constexpr (G == Gather::VALUES) {
        const uint32_t Tn = a.p0, H = a.p1;
        return to_f32(A[((uint64_t)row * H + layer) * Tn + kk]);
    } else {
        const uint32_t gw = a.p0, p = a.p1, cin = a.p2, width = a.p3;
        uint32_t gy = row / gw, gx = row % gw;
        uint32_t ky = kk / (p * cin), kx = (kk / cin) % p, ci = kk % cin;
        return to_f32(A[((uint64_t)(gy * p + ky) * width + gx * p + kx) * cin + ci]);
    }
}
template <Gather G, typename T>
__device__ __forceinline__ float gather_b(const GatherArgs &a, uint32_t kk, uint32_t col, uint32_t layer) {
    const T *B = (const T *)a.b;
    if constexpr (G == Gather::SCORES) {
        const uint32_t H = a.p1, D = a.p2;
        return to_f32(B[(uint64_t)col * 3 * H * D + H * D + layer * D + kk]);
    } else if constexpr (G == Gather::VALUES) {
        const uint32_t H = a.p1, D = a.p2;
        return to_f32(B[(uint64_t)kk * 3 * H * D + 2 * H * D + layer * D + col]);
    } else {
        return to_f32(B[(uint64_t)kk * a.n + col]);
    }
}
template <Gather G>
__device__ __forceinline__ uint64_t gather_out(const GatherArgs &a, uint32_t row, uint32_t col, uint32_t layer) {
    if constexpr (G == Gather::SCORES) {
        return ((uint64_t)row * a.p1 + layer) * a.p0 + col;
    } else if constexpr (G == Gather::VALUES) {
        return (uint64_t)row * a.p1 * a.p2 + layer * a.p2 + col;
    } else {
        return (uint64_t)row * a.n + col;
    }
}

template <Gather G, typename T>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
    constexpr int TR = 64, TC = 64, TD = 16;
    __shared__ float As[TD][TR + 4];
    __shared__ float Bs[TD][TC + 4];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const uint32_t row0 = a.row0 + blockIdx.y * TR, col0 = blockIdx.x * TC, layer = blockIdx.z;
    float acc[4][4] = {};
    for (uint32_t k0 = 0; k0 < a.k; k0 += TD) {
        for (int e = threadIdx.x; e < TR * TD; e += 256) {
            int kk = e % TD, r = e / TD;
            uint32_t row = row0 + r, k = k0 + kk;
            As[kk][r] = (row < a.row1 && k < a.k) ? gather_a<G, T>(a, row, k, layer) : 0.0f;
        }
        for (int e = threadIdx.x; e < TD * TC; e += 256) {
            int kk, c;
            if (G == Gather::SCORES) { kk = e % TD; c = e / TD; }  // keys: k contiguous
            else { c = e % TC; kk = e / TC; }
            uint32_t col = col0 + c, k = k0 + kk;
            Bs[kk][c] = (col < a.n && k < a.k) ? gather_b<G, T>(a, k, col, layer) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < TD; kk++) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] += av[i] * bv[j];
        }
        __syncthreads();
    }
    const T *bias = (const T *)a.bias;
    T *C = (T *)a.c;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t row = row0 + ty * 4 + i;
        if (row >= a.row1) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t col = col0 + tx * 4 + j;
            if (col >= a.n) continue;
            float v = acc[i][j] + (bias ? to_f32(bias[col]) : 0.0f);
            uint64_t idx = gather_out<G>(a, row, col, layer);
            C[idx] = from_f32<T>(apply_epilogue<T>(a.epi, v, idx));
        }
    }
}

// ------------------------------------------------------------------------
// One output element per invocation over the part's elements.
// ------------------------------------------------------------------------
template <PerElement P, typename T>
__global__ __launch_bounds__(256) void element_kernel(ElementArgs a) {
    const T *A = (const T *)a.a, *B = (const T *)a.b;
    T *Y = (T *)a.y;
    for (uint64_t i = a.start + (uint64_t)blockIdx.x * 256 + threadIdx.x; i < a.end;
         i += (uint64_t)gridDim.x * 256) {
        float v;
        if constexpr (P == PerElement::MAP) v = to_f32(A[i]);
        else if constexpr (P == PerElement::PREPEND) v = i < a.channels ? to_f32(A[i]) : to_f32(B[i - a.channels]);
        else v = to_f32(A[i + a.channels]);
        Y[i] = from_f32<T>(apply_epilogue<T>(a.epi, v, i));
    }
}

// The class-token prepend (with its epilogue) as the producer of a folded
// LayerNorm over its output: eight consecutive elements of one row per
// invocation, so that a quad of invocations is one 32-column block (rows of
// ln_cols elements, a multiple of 32, and a part of whole rows: a block lies
// in one row, and in the token or in the rows after it). Stores y, the
// block's (mean, sum of squared deviations from that mean) of the values as
// stored at ln_out [row][ln_cols / 32], and for f32 storage y once more as hi
// and lo bf16 planes (ln_shadow, ln_plane elements apart) or as f32
// (ln_plane 0), each value less its block's mean.
// Eight consecutive values v[e] of element i + e (i a multiple of 8) from
// 16-byte loads, f32 or f16.
template <typename T>
__device__ __forceinline__ void load8(const T *p, float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 x = *(const f32x4 *)p, y = *(const f32x4 *)(p + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = x[e];
            v[4 + e] = y[e];
        }
    } else {
        const f16x8 x = *(const f16x8 *)p;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)x[e];
    }
}

template <typename T>
__global__ __launch_bounds__(256) void prepend_stats_kernel(ElementArgs a) {
    const T *A = (const T *)a.a, *B = (const T *)a.b;
    T *Y = (T *)a.y;
    const uint64_t chunks = (a.end - a.start) / 8;  // a multiple of 4: whole rows of whole blocks
    const uint32_t nblk = a.ln_cols / 32;
    for (uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (uint64_t)gridDim.x * 256) {
        const uint64_t i = a.start + 8 * c;
        float v[8], s = 0.0f;
        load8<T>(i < a.channels ? A + i : B + (i - a.channels), v);
        // The epilogue step by step over the eight values; an added tensor
        // as 16-byte loads.
        for (int k = 0; k < a.epi.n; k++) {
            if (a.epi.kind[k] == BL_EPI_ADD) {
                float w[8];
                load8<T>((const T *)a.epi.operand[k] + i, w);
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] += w[e];
            } else {
                EpilogueArgs one = a.epi;
                one.n = 1;
                one.kind[0] = a.epi.kind[k];
                one.factor[0] = a.epi.factor[k];
                one.channels[0] = a.epi.channels[k];
                one.operand[0] = a.epi.operand[k];
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = apply_epilogue<T>(one, v[e], i + e);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            v[e] = to_f32(from_f32<T>(v[e]));  // as stored
            s += v[e];
        }
        if constexpr (sizeof(T) == 4) {
            *(f32x4 *)(Y + i) = f32x4{v[0], v[1], v[2], v[3]};
            *(f32x4 *)(Y + i + 4) = f32x4{v[4], v[5], v[6], v[7]};
        } else {
            f16x8 w;
#pragma unroll
            for (int e = 0; e < 8; e++) w[e] = (_Float16)v[e];
            *(f16x8 *)(Y + i) = w;
        }
        const float mean = quad_sum(s) * (1.0f / 32.0f);
        float m2 = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) m2 += (v[e] - mean) * (v[e] - mean);
        m2 = quad_sum(m2);
        if (c % 4 == 0) {
            const uint64_t row = i / a.ln_cols;
            *(f32x2 *)(a.ln_out + 2 * (row * nblk + (i % a.ln_cols) / 32)) = f32x2{mean, m2};
        }
        if constexpr (sizeof(T) == 4) {
            if (a.ln_shadow) {
                // The consumer's A: the values less their block's mean.
                float dv[8];
#pragma unroll
                for (int e = 0; e < 8; e++) dv[e] = v[e] - mean;
                if (a.ln_plane) {
                    bf16x8 hi, lo;
                    split8_bf16(dv, hi, lo);
                    *(bf16x8 *)((__bf16 *)a.ln_shadow + i) = hi;
                    *(bf16x8 *)((__bf16 *)a.ln_shadow + a.ln_plane + i) = lo;
                } else {
                    *(f32x4 *)((float *)a.ln_shadow + i) = f32x4{dv[0], dv[1], dv[2], dv[3]};
                    *(f32x4 *)((float *)a.ln_shadow + i + 4) = f32x4{dv[4], dv[5], dv[6], dv[7]};
                }
            }
        }
    }
}

// ------------------------------------------------------------------------
// The DPT head's gathers, V consecutive channels of one output pixel per
// invocation (V = 4 when the channel count is a multiple of 4, else 1).
//
// Transposed convolution, kernel = stride = f (ConvTranspose2d,
// kernel.rs:547-597): output pixel (Y, X) lies in the f x f block of input
// pixel (Y / f, X / f) at tap (Y % f, X % f), and no other input pixel reaches
// it, so each output element is the bias plus one dot product over the input
// channels (the reference's own kernel gathers the same way). An input value
// serves the V channels; the HWIO weights of V channels are one vector load.
//
// Bilinear resampling with aligned corners (ResizeBilinear,
// kernel.rs:599-631): positions as PyTorch's interpolate computes them in f32,
// ratio * index, the floor and the next index clamped to the last row or
// column, weights 1 - l and l; each corner one vector load.
// ------------------------------------------------------------------------
template <typename T, int V> struct VecOf { typedef T type __attribute__((ext_vector_type(V))); };
template <typename T> struct VecOf<T, 1> { typedef T type; };

template <typename T, int V>
__device__ __forceinline__ void load_vec(const T *p, float (&v)[V]) {
    if constexpr (V == 1) {
        v[0] = to_f32(*p);
    } else {
        const typename VecOf<T, V>::type x = *(const typename VecOf<T, V>::type *)p;
#pragma unroll
        for (int e = 0; e < V; e++) v[e] = to_f32(x[e]);
    }
}
template <typename T, int V>
__device__ __forceinline__ void store_vec(T *p, const float (&v)[V]) {
    if constexpr (V == 1) {
        *p = from_f32<T>(v[0]);
    } else {
        typename VecOf<T, V>::type x;
#pragma unroll
        for (int e = 0; e < V; e++) x[e] = from_f32<T>(v[e]);
        *(typename VecOf<T, V>::type *)p = x;
    }
}

template <Dpt K, typename T, int V>
__global__ __launch_bounds__(256) void dpt_kernel(DptArgs a) {
    const T *X = (const T *)a.x;
    T *Y = (T *)a.y;
    const uint64_t groups = (a.end - a.start) / V;
    for (uint64_t gi = (uint64_t)blockIdx.x * 256 + threadIdx.x; gi < groups; gi += (uint64_t)gridDim.x * 256) {
        const uint64_t i = a.start + gi * V;
        float v[V];
        if constexpr (K == Dpt::CONV_TRANSPOSE) {
            const uint32_t w = a.d[1], cin = a.d[2], cout = a.d[3], f = a.d[4];
            const uint64_t pixel = i / cout;
            const uint32_t co = (uint32_t)(i % cout);
            const uint32_t ow = w * f;
            const uint32_t oy = (uint32_t)(pixel / ow), ox = (uint32_t)(pixel % ow);
            const uint32_t y = oy / f, ky = oy % f, x = ox / f, kx = ox % f;
            const T *in = X + ((uint64_t)y * w + x) * cin;
            const T *wt = (const T *)a.w + ((uint64_t)(ky * f + kx) * cin) * cout + co;
            float acc[V];
#pragma unroll
            for (int e = 0; e < V; e++) acc[e] = 0.0f;
            uint32_t ci = 0;
            if (cin % 4 == 0) {
                // Input channels four at a time (one vector load), summed in order.
                for (; ci < cin; ci += 4) {
                    float xv[4];
                    load_vec<T, 4>(in + ci, xv);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float wv[V];
                        load_vec<T, V>(wt + (uint64_t)(ci + q) * cout, wv);
#pragma unroll
                        for (int e = 0; e < V; e++) acc[e] += xv[q] * wv[e];
                    }
                }
            }
            for (; ci < cin; ci++) {
                const float xv = to_f32(in[ci]);
                float wv[V];
                load_vec<T, V>(wt + (uint64_t)ci * cout, wv);
#pragma unroll
                for (int e = 0; e < V; e++) acc[e] += xv * wv[e];
            }
            float b[V];
            if (a.d[5]) load_vec<T, V>((const T *)a.bias + co, b);
#pragma unroll
            for (int e = 0; e < V; e++) v[e] = acc[e] + (a.d[5] ? b[e] : 0.0f);
        } else {
            const uint32_t ih = a.d[0], iw = a.d[1], ow = a.d[3], c = a.d[4];
            const uint64_t pixel = i / c;
            const uint32_t ch = (uint32_t)(i % c);
            const uint32_t oy = (uint32_t)(pixel / ow), ox = (uint32_t)(pixel % ow);
            const float py = a.ry * (float)oy, px = a.rx * (float)ox;
            const uint32_t y0 = min((uint32_t)py, ih - 1), x0 = min((uint32_t)px, iw - 1);
            const uint32_t y1 = min(y0 + 1, ih - 1), x1 = min(x0 + 1, iw - 1);
            const float ly = py - (float)y0, lx = px - (float)x0;
            float p00[V], p01[V], p10[V], p11[V];
            load_vec<T, V>(X + ((uint64_t)y0 * iw + x0) * c + ch, p00);
            load_vec<T, V>(X + ((uint64_t)y0 * iw + x1) * c + ch, p01);
            load_vec<T, V>(X + ((uint64_t)y1 * iw + x0) * c + ch, p10);
            load_vec<T, V>(X + ((uint64_t)y1 * iw + x1) * c + ch, p11);
#pragma unroll
            for (int e = 0; e < V; e++) {
                const float top = (1.0f - lx) * p00[e] + lx * p01[e];
                const float bottom = (1.0f - lx) * p10[e] + lx * p11[e];
                v[e] = (1.0f - ly) * top + ly * bottom;
            }
        }
#pragma unroll
        for (int e = 0; e < V; e++) v[e] = apply_epilogue<T>(a.epi, v[e], i + e);
        store_vec<T, V>(Y + i, v);
    }
}

// ------------------------------------------------------------------------
// Products with at most 4 output columns, on the vector ALUs: 8 lanes per row
// read its k as 16-byte runs (a row of 32 f32 is one coalesced 128-byte
// read), each lane summing its chunks k = 4 (lane % 8) + 32 j in order; the
// 8 partial sums meet by shuffles, then bias and epilogue as the GEMM's.
// ------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    const uint32_t sub = threadIdx.x & 7, N = a.n, K = a.k;
    const T *B = (const T *)a.b;
    for (uint64_t row = a.row0 + ((uint64_t)blockIdx.x * 256 + threadIdx.x) / 8; row < a.row1;
         row += (uint64_t)gridDim.x * 32) {
        const T *x = (const T *)a.a + row * K;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (uint32_t k = 4 * sub; k < K; k += 32) {
            float xv[4];
            load_vec<T, 4>(x + k, xv);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if ((uint32_t)c < N) acc[c] += xv[e] * to_f32(B[(uint64_t)(k + e) * N + c]);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            acc[c] += __shfl_xor(acc[c], 1, 8);
            acc[c] += __shfl_xor(acc[c], 2, 8);
            acc[c] += __shfl_xor(acc[c], 4, 8);
        }
        if (sub == 0) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if ((uint32_t)c < N) {
                    const uint64_t idx = row * N + c;
                    const float v = acc[c] + (a.bias ? to_f32(((const T *)a.bias)[c]) : 0.0f);
                    ((T *)a.c)[idx] = from_f32<T>(apply_epilogue<T>(a.epi, v, idx));
                }
            }
        }
    }
}

// ------------------------------------------------------------------------
// The second pass of a split-k GEMM: output element i of the part (row
// row0 + i / n, column i % n) is the sum of its ksplit partial sums in split
// order, plus the bias, through the epilogue steps in order — what the
// unsplit kernel's store does with one sum.
// ------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs a) {
    const uint32_t N = a.n;
    const uint64_t total = (uint64_t)(a.row1 - a.row0) * N;
    const T *bias = (const T *)a.bias;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (uint64_t)gridDim.x * 256) {
        // Four partials in flight at a time, added in split order.
        const float *p = a.partials + i;
        float v = 0.0f;
        uint32_t z = 0;
        for (; z + 4 <= a.ksplit; z += 4) {
            const float p0 = p[z * total], p1 = p[(z + 1) * total], p2 = p[(z + 2) * total], p3 = p[(z + 3) * total];
            v += p0;
            v += p1;
            v += p2;
            v += p3;
        }
        for (; z < a.ksplit; z++) v += p[z * total];
        if (bias) v += to_f32(bias[i % N]);
        const uint64_t idx = (uint64_t)a.row0 * N + i;
        store_elem<T>((T *)a.c, idx, apply_epilogue<T>(a.epi, v, idx), a.c_planes);
    }
}

// Spins until `ticks` of the device's constant-rate wall clock have passed.
__global__ void spin_kernel(uint64_t ticks) {
    const uint64_t t0 = wall_clock64();
    while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(1);
}

// A folded LayerNorm's statistics of x made from x itself: one invocation
// per (row, 32-column block), the block's mean and then its sum of squared
// deviations from it, as the fold's producer computes them in its epilogue;
// f32 x also goes to the shadow less its block's mean, as hi and lo bf16
// planes (a.planes apart) or as f32 (a.planes 0).
template <typename T>
__global__ __launch_bounds__(256) void ln_stats_kernel(LnStatsArgs a) {
    const uint32_t nblk = a.cols / 32;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)a.rows * nblk) return;
    const uint32_t row = (uint32_t)(i / nblk), blk = (uint32_t)(i % nblk);
    const uint64_t base = (uint64_t)row * a.cols + blk * 32;
    const T *x = (const T *)a.x + base;
    float v[32];
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) {
        v[e] = to_f32(x[e]);
        sum += v[e];
    }
    const float mean = sum * (1.0f / 32.0f);
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; e++) sq += (v[e] - mean) * (v[e] - mean);
    *(f32x2 *)(a.stats + 2 * i) = f32x2{mean, sq};
    if constexpr (sizeof(T) == 4) {
        if (a.shadow) {
#pragma unroll
            for (int e = 0; e < 32; e += 4)
                store_f32x4((float *)a.shadow, base + e,
                            f32x4{v[e] - mean, v[e + 1] - mean, v[e + 2] - mean, v[e + 3] - mean}, a.planes);
        }
    }
}

}  // namespace

hipError_t launch_ln_stats(const LnStatsArgs &a, bool f16, hipStream_t s) {
    const uint64_t n = (uint64_t)a.rows * (a.cols / 32);
    const dim3 grid((uint32_t)((n + 255) / 256));
    if (f16) hipLaunchKernelGGL(ln_stats_kernel<_Float16>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(ln_stats_kernel<float>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_layernorm(const LayerNormArgs &a, bool f16, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    return f16 ? ln_launch<_Float16>(a, s) : ln_launch<float>(a, s);
}

hipError_t launch_softmax(const SoftmaxArgs &a, bool f16, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    dim3 grid(a.row1 - a.row0);
    if (f16) hipLaunchKernelGGL(softmax_kernel<_Float16>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(softmax_kernel<float>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gather(const GatherArgs &a, Gather g, bool f16, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    dim3 grid((a.n + 63) / 64, (a.row1 - a.row0 + 63) / 64, a.layers);
#define BL_GATHER(G)                                                                     \
    if (f16) hipLaunchKernelGGL((gather_kernel<G, _Float16>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((gather_kernel<G, float>), grid, dim3(256), 0, s, a);
    switch (g) {
    case Gather::SCORES: BL_GATHER(Gather::SCORES) break;
    case Gather::VALUES: BL_GATHER(Gather::VALUES) break;
    default: BL_GATHER(Gather::PATCH) break;
    }
#undef BL_GATHER
    return hipGetLastError();
}

hipError_t launch_element(const ElementArgs &a, PerElement p, bool f16, hipStream_t s) {
    if (a.end <= a.start) return hipSuccess;
    if (a.ln_out) {
        // Whole rows of whole 32-column blocks, the token whole blocks too.
        if (p != PerElement::PREPEND || a.ln_cols == 0 || a.ln_cols % 32 != 0 || a.start % a.ln_cols != 0 ||
            a.end % a.ln_cols != 0 || a.channels % 32 != 0)
            return hipErrorInvalidValue;
        // 16-byte loads and stores of eight elements.
        auto aligned = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
        bool ok = aligned(a.a) && aligned(a.b) && aligned(a.y) && (!a.ln_shadow || aligned(a.ln_shadow));
        for (int k = 0; k < a.epi.n; k++)
            if (a.epi.kind[k] == BL_EPI_ADD) ok = ok && aligned(a.epi.operand[k]);
        if (!ok) return hipErrorInvalidValue;
        uint64_t blocks = ((a.end - a.start) / 8 + 255) / 256;
        if (blocks > 65535) blocks = 65535;
        if (f16) hipLaunchKernelGGL((prepend_stats_kernel<_Float16>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
        else hipLaunchKernelGGL((prepend_stats_kernel<float>), dim3((uint32_t)blocks), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    uint64_t blocks = (a.end - a.start + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    dim3 grid((uint32_t)blocks);
#define BL_ELEM(P)                                                                        \
    if (f16) hipLaunchKernelGGL((element_kernel<P, _Float16>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((element_kernel<P, float>), grid, dim3(256), 0, s, a);
    switch (p) {
    case PerElement::MAP: BL_ELEM(PerElement::MAP) break;
    case PerElement::PREPEND: BL_ELEM(PerElement::PREPEND) break;
    default: BL_ELEM(PerElement::DROP_FIRST) break;
    }
#undef BL_ELEM
    return hipGetLastError();
}

hipError_t launch_dpt(const DptArgs &a, Dpt k, bool f16, hipStream_t s) {
    if (a.end <= a.start) return hipSuccess;
    // Channels per pixel: the part's range is whole pixels of them.
    const uint32_t channels = k == Dpt::CONV_TRANSPOSE ? a.d[3] : a.d[4];
    const int v = channels % 4 == 0 ? 4 : 1;
    uint64_t blocks = ((a.end - a.start) / v + 255) / 256;
    if (blocks > 65535) blocks = 65535;
    dim3 grid((uint32_t)blocks);
#define BL_DPT(K, V)                                                                       \
    if (f16) hipLaunchKernelGGL((dpt_kernel<K, _Float16, V>), grid, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((dpt_kernel<K, float, V>), grid, dim3(256), 0, s, a);
    if (k == Dpt::CONV_TRANSPOSE) {
        if (v == 4) { BL_DPT(Dpt::CONV_TRANSPOSE, 4) } else { BL_DPT(Dpt::CONV_TRANSPOSE, 1) }
    } else {
        if (v == 4) { BL_DPT(Dpt::RESIZE, 4) } else { BL_DPT(Dpt::RESIZE, 1) }
    }
#undef BL_DPT
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs &a, bool f16, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    if (a.n == 0 || a.n > 4 || a.k % 4 != 0) return hipErrorInvalidValue;
    uint64_t blocks = ((uint64_t)(a.row1 - a.row0) + 31) / 32;
    if (blocks > 65535) blocks = 65535;
    if (f16) hipLaunchKernelGGL(gemv_kernel<_Float16>, dim3((uint32_t)blocks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(gemv_kernel<float>, dim3((uint32_t)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gemm_reduce(const GemmArgs &a, bool f16, hipStream_t s) {
    const uint64_t total = (uint64_t)(a.row1 - a.row0) * a.n;
    if (total == 0) return hipSuccess;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (f16) hipLaunchKernelGGL(gemm_reduce_kernel<_Float16>, dim3((uint32_t)blocks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(gemm_reduce_kernel<float>, dim3((uint32_t)blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_spin(uint64_t ticks, uint32_t blocks, hipStream_t s) {
    hipLaunchKernelGGL(spin_kernel, dim3(blocks), dim3(64), 0, s, ticks);
    return hipGetLastError();
}

}  // namespace bl

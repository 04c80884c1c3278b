// Fused multi-head self-attention for one qkv tensor: the reference's three
// kernels attention_scores+scale -> softmax -> attention_values
// (crates/beatlm-core/src/kernel.rs:731-777; codegen/wgsl.rs:590-669,
// :975-1010) as one flash-style kernel with an online softmax, so the
// [T][H][T] scores and probabilities never exist.
//
//   qkv  [T][3][H][64]  (queries, keys, values of each token, heads side by side)
//   out  [T][H * 64]    (heads side by side, as the output projection reads them)
//
// Workgroup: 4 waves, 64 query rows of one head; wave w owns queries
// 16w .. 16w + 15. Keys and values stream through LDS in tiles of 64 keys,
// shared by the four waves. Each wave computes the transposed scores
// S^T = K Q^T on the matrix cores, so a lane's accumulators hold 16 keys of
// ONE query (query = lane % 16): the row maximum and row sum of the online
// softmax are per-lane values plus two cross-lane steps (lanes 16 and 32
// apart), and the probabilities are already laid out as the B operand of
// O^T = V^T P^T, which accumulates the output transposed with the same query
// per lane, so rescaling by exp(m_old - m_new) is one multiply per register.
//
// Softmax in base 2: s * scale * log2(e) and exp2, the same function.
//
// When T gives fewer than ~512 workgroups, the keys are split into `splits`
// ranges; each writes its unnormalised output and (max, sum) to scratch and a
// second kernel merges them. Query rows outside the part are not stored.
#include "device_common.hpp"

namespace bl {
namespace {

constexpr int THREADS = 256;
constexpr int KT = 64;   // keys per tile
constexpr int HD = 64;   // head width
constexpr float LOG2E = 1.4426950408889634f;

template <Math M> struct FlashTraits;
template <> struct FlashTraits<Math::F16> {
    using T = _Float16;
    using L = _Float16;
    static constexpr int VEC = 8;
    static constexpr int ROW = HD + 8;  // LDS row (elements)
    static constexpr int COPIES = 1;
};
template <> struct FlashTraits<Math::SPLIT> {
    using T = float;
    using L = __bf16;
    static constexpr int VEC = 4;
    static constexpr int ROW = HD + 8;
    static constexpr int COPIES = 2;
};
template <> struct FlashTraits<Math::F32> {
    using T = float;
    using L = float;
    static constexpr int VEC = 4;
    static constexpr int ROW = HD + 4;
    static constexpr int COPIES = 1;
};

template <typename T, int VEC> struct FChunk;
template <> struct FChunk<float, 4> { using V = f32x4; };
template <> struct FChunk<_Float16, 8> { using V = f16x8; };

template <Math M>
__global__ __launch_bounds__(THREADS) void flash_kernel(FlashArgs args) {
    using Tr = FlashTraits<M>;
    using T = typename Tr::T;
    using L = typename Tr::L;
    constexpr int VEC = Tr::VEC;
    constexpr int ROW = Tr::ROW;
    using V = typename FChunk<T, VEC>::V;
    constexpr int CHUNKS = KT * HD / VEC;      // per operand tile
    constexpr int PER = CHUNKS / THREADS;      // per thread
    static_assert(CHUNKS % THREADS == 0, "tile chunks");

    // K [key][d] and V^T [d][key], k-contiguous for the MFMA operands.
    __shared__ __attribute__((aligned(16))) L Ks[Tr::COPIES][KT * ROW];
    __shared__ __attribute__((aligned(16))) L Vt[Tr::COPIES][HD * ROW];

    const T *__restrict__ qkv = (const T *)args.qkv;
    const uint32_t Tn = args.tokens, H = args.heads;
    const uint32_t row_stride = 3 * H * HD;
    const uint32_t head = blockIdx.y, split = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const uint32_t q0 = args.row0 + blockIdx.x * 64;
    const uint32_t q = q0 + 16 * wave + l16;
    const bool q_ok = q < args.row1;

    // This split's key tiles.
    const uint32_t ntiles = (Tn + KT - 1) / KT;
    const uint32_t t_begin = split * ntiles / args.splits;
    const uint32_t t_end = (split + 1) * ntiles / args.splits;

    // ---- the wave's queries as the B operand of S^T = K Q^T ----
    const T *qrow = qkv + (uint64_t)q * row_stride + head * HD;
    f16x8 qf16[2];
    bf16x8 qhi[2], qlo[2];
    float qf32[16];
    if constexpr (M == Math::F16) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            f16x8 v = {};
            if (q_ok) v = *(const f16x8 *)(qrow + 32 * c + 8 * g);
            qf16[c] = v;
        }
    } else if constexpr (M == Math::SPLIT) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            f32x4 a = {}, b = {};
            if (q_ok) {
                a = *(const f32x4 *)(qrow + 32 * c + 8 * g);
                b = *(const f32x4 *)(qrow + 32 * c + 8 * g + 4);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                __bf16 h, l;
                split_bf16(e < 4 ? a[e] : b[e - 4], h, l);
                qhi[c][e] = h;
                qlo[c][e] = l;
            }
        }
    } else {
        // Lane group g, step (h, s) of the 16 x 16 x 4 products reads d = 16h + 4g + s.
#pragma unroll
        for (int h = 0; h < 4; h++) {
            f32x4 a = {};
            if (q_ok) a = *(const f32x4 *)(qrow + 16 * h + 4 * g);
#pragma unroll
            for (int s = 0; s < 4; s++) qf32[4 * h + s] = a[s];
        }
    }

    // ---- K/V tile staging: HBM -> registers -> LDS ----
    V rk[PER], rv[PER];
    auto load_tile = [&](uint32_t t) {
        const uint32_t kbase = t * KT;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int c = tid + i * THREADS;
            int r = c / (HD / VEC), dc = (c % (HD / VEC)) * VEC;
            uint32_t key = kbase + r;
            V kv = {}, vv = {};
            if (key < Tn) {
                const T *base = qkv + (uint64_t)key * row_stride + head * HD + dc;
                kv = *(const V *)(base + H * HD);
                vv = *(const V *)(base + 2 * H * HD);
            }
            rk[i] = kv;
            rv[i] = vv;
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int c = tid + i * THREADS;
            int r = c / (HD / VEC), dc = (c % (HD / VEC)) * VEC;
            if constexpr (M == Math::SPLIT) {
                bf16x4 kh, kl;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    __bf16 h, l;
                    split_bf16(rk[i][e], h, l);
                    kh[e] = h;
                    kl[e] = l;
                    split_bf16(rv[i][e], h, l);
                    Vt[0][(dc + e) * ROW + r] = h;
                    Vt[1][(dc + e) * ROW + r] = l;
                }
                *(bf16x4 *)&Ks[0][r * ROW + dc] = kh;
                *(bf16x4 *)&Ks[1][r * ROW + dc] = kl;
            } else {
                *(V *)&Ks[0][r * ROW + dc] = rk[i];
#pragma unroll
                for (int e = 0; e < VEC; e++) Vt[0][(dc + e) * ROW + r] = rv[i][e];
            }
        }
    };

    f32x4 o[4];  // O^T: d = 16 dt + 4g + r, query l16
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32x4{0, 0, 0, 0};
    float m_run = -INFINITY, l_run = 0.0f;
    const float sl2 = args.scale * LOG2E;

    if (t_begin < t_end) load_tile(t_begin);
    for (uint32_t t = t_begin; t < t_end; t++) {
        store_tile();
        __syncthreads();
        if (t + 1 < t_end) load_tile(t + 1);

        // S^T tiles: keys 16 kt + 4g + r of this tile, query l16.
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            f32x4 acc = {0, 0, 0, 0};
            const int krow = (16 * kt + l16) * ROW;
            if constexpr (M == Math::F16) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    f16x8 a = *(const f16x8 *)&Ks[0][krow + 32 * c + 8 * g];
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf16[c], acc, 0, 0, 0);
                }
            } else if constexpr (M == Math::SPLIT) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    bf16x8 ah = *(const bf16x8 *)&Ks[0][krow + 32 * c + 8 * g];
                    bf16x8 al = *(const bf16x8 *)&Ks[1][krow + 32 * c + 8 * g];
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, qhi[c], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, qlo[c], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, qhi[c], acc, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    f32x4 a = *(const f32x4 *)&Ks[0][krow + 16 * h + 4 * g];
#pragma unroll
                    for (int st = 0; st < 4; st++)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], qf32[4 * h + st], acc, 0, 0, 0);
                }
            }
            s[kt] = acc;
        }

        // Online softmax for query l16 over this tile's keys.
        const uint32_t kbase = t * KT;
        float tmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                uint32_t key = kbase + 16 * kt + 4 * g + r;
                float v = key < Tn ? s[kt][r] * sl2 : -INFINITY;
                s[kt][r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);  // finite: every tile has a key < T
        const float alpha = exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float p = exp2f(s[kt][r] - m_new);
                s[kt][r] = p;
                psum += p;
            }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;

        // O^T += V^T P^T.
        if constexpr (M == Math::F32) {
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const int vrow = (16 * dt + l16) * ROW;
#pragma unroll
                for (int kt = 0; kt < 4; kt++) {
                    f32x4 a = *(const f32x4 *)&Vt[0][vrow + 16 * kt + 4 * g];
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], s[kt][r], o[dt], 0, 0, 0);
                }
            }
        } else {
            // 32 keys per step: slots 0..3 are keys 32m + 4g + e, slots 4..7 keys
            // 32m + 16 + 4g + e, for A (V^T) and B (P^T) alike.
#pragma unroll
            for (int mh = 0; mh < 2; mh++) {
                if constexpr (M == Math::F16) {
                    f16x8 b;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        b[e] = (_Float16)s[2 * mh][e];
                        b[4 + e] = (_Float16)s[2 * mh + 1][e];
                    }
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) {
                        const int vrow = (16 * dt + l16) * ROW + 32 * mh + 4 * g;
                        f16x4 lo = *(const f16x4 *)&Vt[0][vrow];
                        f16x4 hi = *(const f16x4 *)&Vt[0][vrow + 16];
                        f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, o[dt], 0, 0, 0);
                    }
                } else {
                    bf16x8 bh, bl;
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        __bf16 h, l;
                        split_bf16(e < 4 ? s[2 * mh][e] : s[2 * mh + 1][e - 4], h, l);
                        bh[e] = h;
                        bl[e] = l;
                    }
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) {
                        const int vrow = (16 * dt + l16) * ROW + 32 * mh + 4 * g;
                        bf16x4 h0 = *(const bf16x4 *)&Vt[0][vrow];
                        bf16x4 h1 = *(const bf16x4 *)&Vt[0][vrow + 16];
                        bf16x4 l0 = *(const bf16x4 *)&Vt[1][vrow];
                        bf16x4 l1 = *(const bf16x4 *)&Vt[1][vrow + 16];
                        bf16x8 ah = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                        bf16x8 al = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, o[dt], 0, 0, 0);
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, o[dt], 0, 0, 0);
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, o[dt], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    }

    // The row sum over the four lane groups of query l16.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (!q_ok) return;

    if (args.splits == 1) {
        const float inv = 1.0f / l_run;
        T *out = (T *)args.out + (uint64_t)q * H * HD + head * HD;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
            const int d = 16 * dt + 4 * g;
            if constexpr (M == Math::F16) {
                f16x4 v;
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = (_Float16)(o[dt][r] * inv);
                *(f16x4 *)(out + d) = v;
            } else {
                *(f32x4 *)(out + d) = o[dt] * inv;
            }
        }
    } else {
        const uint64_t slot = ((uint64_t)split * Tn + q) * H + head;
        float *part = args.partial + slot * HD;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) *(f32x4 *)(part + 16 * dt + 4 * g) = o[dt];
        if (g == 0) {
            args.stats[2 * slot] = m_run;
            args.stats[2 * slot + 1] = l_run;
        }
    }
}

// Merges the key splits: O = sum_s 2^(m_s - m) O_s / sum_s 2^(m_s - m) l_s.
// One invocation per (query, head, 4 output columns).
template <typename T>
__global__ __launch_bounds__(256) void flash_merge_kernel(FlashArgs args) {
    const uint32_t H = args.heads, Tn = args.tokens;
    const uint64_t per_row = (uint64_t)H * (HD / 4);
    const uint64_t total = (uint64_t)(args.row1 - args.row0) * per_row;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t q = args.row0 + (uint32_t)(i / per_row);
        const uint32_t rem = (uint32_t)(i % per_row);
        const uint32_t head = rem / (HD / 4), d = (rem % (HD / 4)) * 4;
        float m = -INFINITY;
        for (uint32_t s = 0; s < args.splits; s++)
            m = fmaxf(m, args.stats[2 * (((uint64_t)s * Tn + q) * H + head)]);
        f32x4 acc = {0, 0, 0, 0};
        float l = 0.0f;
        for (uint32_t s = 0; s < args.splits; s++) {
            const uint64_t slot = ((uint64_t)s * Tn + q) * H + head;
            const float ms = args.stats[2 * slot];
            if (ms == -INFINITY) continue;  // a split with no keys
            const float w = exp2f(ms - m);
            l += w * args.stats[2 * slot + 1];
            acc += w * *(const f32x4 *)(args.partial + slot * HD + d);
        }
        const float inv = 1.0f / l;
        T *out = (T *)args.out + (uint64_t)q * H * HD + head * HD + d;
#pragma unroll
        for (int r = 0; r < 4; r++) out[r] = from_f32<T>(acc[r] * inv);
    }
}

template <Math M>
hipError_t launch_m(const FlashArgs &a, hipStream_t s) {
    using T = typename FlashTraits<M>::T;
    dim3 grid((a.row1 - a.row0 + 63) / 64, a.heads, a.splits);
    hipLaunchKernelGGL(flash_kernel<M>, grid, dim3(THREADS), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1) return e;
    uint64_t work = (uint64_t)(a.row1 - a.row0) * a.heads * (HD / 4);
    uint32_t blocks = (uint32_t)((work + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(flash_merge_kernel<T>, dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_flash(const FlashArgs &a, Math m, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    switch (m) {
    case Math::F16: return launch_m<Math::F16>(a, s);
    case Math::SPLIT: return launch_m<Math::SPLIT>(a, s);
    default: return launch_m<Math::F32>(a, s);
    }
}

}  // namespace bl

// Fused multi-head self-attention for one qkv tensor: the reference's three
// kernels attention_scores+scale -> softmax -> attention_values
// (crates/beatlm-core/src/kernel.rs:731-777; codegen/wgsl.rs:590-669,
// :975-1010) as one flash-style kernel with an online softmax, so the
// [T][H][T] scores and probabilities never exist.
//
//   qkv  [T][3][H][64]  (queries, keys, values of each token, heads side by side)
//   out  [T][H * 64]    (heads side by side, as the output projection reads them)
//
// Three launches per spec:
//  1. flash_prep_kernel writes the keys as K [H][T_pad][64] and the values
//     transposed as Vt [H][64][T_pad], once, in the matrix cores' operand type
//     (f16, f32, or hi and lo bf16 planes), zero-padded to whole 64-key tiles;
//  2. flash_kernel: a workgroup of 4 waves owns 64 query rows of one head and
//     one range of key tiles; K and Vt tiles stream through a ring of LDS
//     stages filled by direct 16-byte loads. Each wave computes the transposed
//     scores S^T = K Q^T for its 16 queries, so a lane's accumulators hold 16
//     keys of ONE query (query = lane % 16): the online softmax's row max and
//     row sum are per-lane values plus two cross-lane steps, and the
//     probabilities are already laid out as the B operand of O^T = V^T P^T,
//     whose accumulators hold the same query per lane, so the rescale by
//     exp(m_old - m_new) is one multiply per register. Softmax in base 2:
//     s * scale * log2(e) and exp2;
//  3. when the key range was split across workgroups (too few query tiles to
//     fill 256 CUs), flash_merge_kernel combines the splits' (max, sum,
//     unnormalised output).
// Query rows outside the part are not stored.
#include <type_traits>

#include "device_common.hpp"

namespace bl {
namespace {

constexpr int THREADS = 256;
constexpr int KT = 64;  // keys per tile
constexpr int HD = 64;  // head width
constexpr float LOG2E = 1.4426950408889634f;

template <Math M> struct FlashTraits;
template <> struct FlashTraits<Math::F16> {
    using T = _Float16;   // storage of qkv and out
    using L = _Float16;   // operand element of K / Vt
    static constexpr int PLANES = 1;
    static constexpr int CPR = 8;     // 16-byte chunks per 64-element row
    static constexpr int STAGES = 3;
};
template <> struct FlashTraits<Math::SPLIT> {
    using T = float;
    using L = __bf16;
    static constexpr int PLANES = 2;
    static constexpr int CPR = 8;
    static constexpr int STAGES = 2;
};
template <> struct FlashTraits<Math::F32> {
    using T = float;
    using L = float;
    static constexpr int PLANES = 1;
    static constexpr int CPR = 16;
    static constexpr int STAGES = 2;
};

// ---- 1. K and Vt in operand layout ----
// One workgroup per 64 keys of one head: 16-byte loads of the key and value
// rows, keys written as they are, values transposed through LDS and written
// as rows of 64 keys.
template <Math M>
__global__ __launch_bounds__(THREADS) void flash_prep_kernel(FlashArgs a) {
    using Tr = FlashTraits<M>;
    using T = typename Tr::T;
    using L = typename Tr::L;
    constexpr int V = 16 / sizeof(T);          // elements per 16-byte load
    constexpr int CHUNKS = KT * HD / V;        // per tile
    using VT = typename std::conditional<sizeof(T) == 4, f32x4, f16x8>::type;
    __shared__ float vt[HD][KT + 4];
    const uint32_t Tn = a.tokens, H = a.heads, tpad = a.t_pad;
    const uint32_t head = blockIdx.y, kbase = blockIdx.x * KT;
    const uint32_t row_stride = 3 * H * HD;
    const T *qkv = (const T *)a.qkv;
    L *kp = (L *)a.kp, *vp = (L *)a.vt;
    const uint64_t plane = (uint64_t)H * tpad * HD;
    for (int c = threadIdx.x; c < CHUNKS; c += THREADS) {
        const int r = c / (HD / V), d = (c % (HD / V)) * V;
        const uint32_t key = kbase + r;
        VT kv = {}, vv = {};
        if (key < Tn) {
            const T *base = qkv + (uint64_t)key * row_stride + head * HD + d;
            kv = *(const VT *)(base + H * HD);
            vv = *(const VT *)(base + 2 * H * HD);
        }
        const uint64_t ki = ((uint64_t)head * tpad + key) * HD + d;
        if constexpr (M == Math::SPLIT) {
            bf16x4 h, l;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                __bf16 hh, ll;
                split_bf16(kv[e], hh, ll);
                h[e] = hh;
                l[e] = ll;
            }
            *(bf16x4 *)(kp + ki) = h;
            *(bf16x4 *)(kp + plane + ki) = l;
        } else {
            *(VT *)(kp + ki) = kv;
        }
#pragma unroll
        for (int e = 0; e < V; e++) vt[d + e][r] = to_f32(vv[e]);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < HD * KT / 4; c += THREADS) {
        const int d = c / (KT / 4), r = (c % (KT / 4)) * 4;
        const uint64_t vi = ((uint64_t)head * HD + d) * tpad + kbase + r;
        if constexpr (M == Math::SPLIT) {
            bf16x4 h, l;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                __bf16 hh, ll;
                split_bf16(vt[d][r + e], hh, ll);
                h[e] = hh;
                l[e] = ll;
            }
            *(bf16x4 *)(vp + vi) = h;
            *(bf16x4 *)(vp + plane + vi) = l;
        } else if constexpr (M == Math::F16) {
            f16x4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (_Float16)vt[d][r + e];
            *(f16x4 *)(vp + vi) = h;
        } else {
            *(f32x4 *)(vp + vi) = f32x4{vt[d][r], vt[d][r + 1], vt[d][r + 2], vt[d][r + 3]};
        }
    }
}

// ---- 2. the attention ----
template <Math M>
__global__ __launch_bounds__(THREADS) void flash_kernel(FlashArgs args) {
    using Tr = FlashTraits<M>;
    using T = typename Tr::T;
    using L = typename Tr::L;
    constexpr int CPR = Tr::CPR, PLANES = Tr::PLANES, STAGES = Tr::STAGES;
    constexpr int TILE_BYTES = 64 * CPR * 16;  // one plane of a K or Vt tile
    constexpr int K_BYTES = PLANES * TILE_BYTES;
    constexpr int STAGE_BYTES = 2 * K_BYTES;
    constexpr int LPS = 2 * PLANES * loads_per_wave<64, CPR>();

    __shared__ __attribute__((aligned(16))) char smem[STAGES * STAGE_BYTES];

    const T *__restrict__ qkv = (const T *)args.qkv;
    const uint32_t Tn = args.tokens, H = args.heads, tpad = args.t_pad;
    const uint32_t row_stride = 3 * H * HD;
    const uint32_t head = blockIdx.y, split = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const uint32_t q = args.row0 + blockIdx.x * 64 + 16 * wave + l16;
    const bool q_ok = q < args.row1;

    const uint32_t ntiles = tpad / KT;
    const uint32_t t_begin = split * ntiles / args.splits;
    const uint32_t t_end = (split + 1) * ntiles / args.splits;

    // This head's K [tpad][64] and Vt [64][tpad], per plane.
    constexpr int ESZ = sizeof(L);
    const uint64_t plane_bytes = (uint64_t)H * tpad * HD * ESZ;
    const char *kbase = (const char *)args.kp + (uint64_t)head * tpad * HD * ESZ;
    const char *vbase = (const char *)args.vt + (uint64_t)head * HD * tpad * ESZ;

    const RowLoader<64, CPR> kload(HD * ESZ, 63, wave, lane);
    const RowLoader<64, CPR> vload(tpad * ESZ, 63, wave, lane);
    auto issue = [&](uint32_t t, int slot) {
        char *st = smem + slot * STAGE_BYTES;
#pragma unroll
        for (int p = 0; p < PLANES; p++) {
            // K rows: 64 keys of 64 d; Vt rows: 64 d of 64 keys, from key t*64.
            kload.issue(kbase + p * plane_bytes + (uint64_t)t * KT * HD * ESZ, st + p * TILE_BYTES);
            vload.issue(vbase + p * plane_bytes + (uint64_t)t * KT * ESZ, st + K_BYTES + p * TILE_BYTES);
        }
    };

    // Fragment offsets inside a staged tile: row 16 j + l16 has the same
    // swizzle for every j, so only the lane's own part is computed here.
    constexpr int ROWB = CPR * 16;  // bytes per staged row
    const int lrow = l16 * ROWB;
    const int x = (CPR == 16) ? l16 : ((l16 >> 1) & 7);

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
        // Step (h, s) of the 16 x 16 x 4 products: lane group g reads d = 16h + 4g + s.
#pragma unroll
        for (int h = 0; h < 4; h++) {
            f32x4 a = {};
            if (q_ok) a = *(const f32x4 *)(qrow + 16 * h + 4 * g);
#pragma unroll
            for (int s = 0; s < 4; s++) qf32[4 * h + s] = a[s];
        }
    }

    f32x4 o[4];  // O^T: d = 16 dt + 4g + r, query l16
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = f32x4{0, 0, 0, 0};
    float m_run = -INFINITY, l_run = 0.0f;
    const float sl2 = args.scale * LOG2E;

#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if (t_begin + s < t_end) issue(t_begin + s, s);

    for (uint32_t t = t_begin; t < t_end; t++) {
        const uint32_t i = t - t_begin;
        if (t + STAGES - 2 < t_end) wait_vmcnt<(STAGES - 2) * LPS>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (t + STAGES - 1 < t_end) issue(t + STAGES - 1, (i + STAGES - 1) % STAGES);
        const char *st = smem + (i % STAGES) * STAGE_BYTES;
        const char *ks = st, *vs = st + K_BYTES;

        // S^T tiles: keys 16 kt + 4g + r of this tile, query l16.
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            f32x4 acc = {0, 0, 0, 0};
            const char *krow = ks + kt * 16 * ROWB + lrow;
            if constexpr (M == Math::F16) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    f16x8 a = *(const f16x8 *)(krow + (((4 * c + g) ^ x) << 4));
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf16[c], acc, 0, 0, 0);
                }
            } else if constexpr (M == Math::SPLIT) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const int off = ((4 * c + g) ^ x) << 4;
                    bf16x8 ah = *(const bf16x8 *)(krow + off);
                    bf16x8 al = *(const bf16x8 *)(krow + TILE_BYTES + off);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, qhi[c], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, qlo[c], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, qhi[c], acc, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    f32x4 a = *(const f32x4 *)(krow + (((4 * h + g) ^ x) << 4));
#pragma unroll
                    for (int st2 = 0; st2 < 4; st2++)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st2], qf32[4 * h + st2], acc, 0, 0, 0);
                }
            }
            s[kt] = acc;
        }

        // Online softmax for query l16 over this tile's keys; only a tile
        // reaching past the last token masks.
        const uint32_t kb = t * KT;
        float tmax = -INFINITY;
        if (kb + KT <= Tn) {
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    s[kt][r] *= sl2;
                    tmax = fmaxf(tmax, s[kt][r]);
                }
        } else {
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t key = kb + 16 * kt + 4 * g + r;
                    const float v = key < Tn ? s[kt][r] * sl2 : -INFINITY;
                    s[kt][r] = v;
                    tmax = fmaxf(tmax, v);
                }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);  // finite: every tile has a key < T
        // 2^x on v_exp_f32: arguments are <= 0, results in (0, 1]; an
        // underflow to zero is a probability below 2^-126.
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(s[kt][r] - m_new);
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
                const char *vrow = vs + dt * 16 * ROWB + lrow;
#pragma unroll
                for (int kt = 0; kt < 4; kt++) {
                    f32x4 a = *(const f32x4 *)(vrow + (((4 * kt + g) ^ x) << 4));
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
                // The 4-key runs at 32mh + 4g and 32mh + 16 + 4g: chunks
                // 4mh + g/2 and 4mh + 2 + g/2, half (g & 1) of each.
                const int o0 = (((4 * mh + (g >> 1)) ^ x) << 4) + (g & 1) * 8;
                const int o1 = (((4 * mh + 2 + (g >> 1)) ^ x) << 4) + (g & 1) * 8;
                if constexpr (M == Math::F16) {
                    f16x8 b;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        b[e] = (_Float16)s[2 * mh][e];
                        b[4 + e] = (_Float16)s[2 * mh + 1][e];
                    }
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) {
                        const char *vrow = vs + dt * 16 * ROWB + lrow;
                        const f16x4 lo = *(const f16x4 *)(vrow + o0);
                        const f16x4 hi = *(const f16x4 *)(vrow + o1);
                        const f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
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
                        const char *vrow = vs + dt * 16 * ROWB + lrow;
                        const bf16x4 h0 = *(const bf16x4 *)(vrow + o0), h1 = *(const bf16x4 *)(vrow + o1);
                        const bf16x4 l0 = *(const bf16x4 *)(vrow + TILE_BYTES + o0), l1 = *(const bf16x4 *)(vrow + TILE_BYTES + o1);
                        const bf16x8 ah = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                        const bf16x8 al = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, o[dt], 0, 0, 0);
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, o[dt], 0, 0, 0);
                        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, o[dt], 0, 0, 0);
                    }
                }
            }
        }
        asm volatile("" ::: "memory");
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
        if (g == 0) *(f32x2 *)(args.stats + 2 * slot) = f32x2{m_run, l_run};
    }
}

// ---- 3. merging the key splits ----
// O = sum_s 2^(m_s - m) O_s / sum_s 2^(m_s - m) l_s, one invocation per
// (query, head, 4 output columns).
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
        f32x2 st[8];
        float m = -INFINITY;
        for (uint32_t s = 0; s < args.splits; s++) {
            st[s] = *(const f32x2 *)(args.stats + 2 * (((uint64_t)s * Tn + q) * H + head));
            m = fmaxf(m, st[s][0]);
        }
        f32x4 acc = {0, 0, 0, 0};
        float l = 0.0f;
        for (uint32_t s = 0; s < args.splits; s++) {
            if (st[s][0] == -INFINITY) continue;  // a split with no keys
            const uint64_t slot = ((uint64_t)s * Tn + q) * H + head;
            const float w = exp2f(st[s][0] - m);
            l += w * st[s][1];
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
    hipLaunchKernelGGL(flash_prep_kernel<M>, dim3(a.t_pad / KT, a.heads), dim3(THREADS), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    dim3 grid((a.row1 - a.row0 + 63) / 64, a.heads, a.splits);
    hipLaunchKernelGGL(flash_kernel<M>, grid, dim3(THREADS), 0, s, a);
    e = hipGetLastError();
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

uint64_t flash_operand_bytes(Math m, uint32_t heads, uint32_t t_pad) {
    const uint64_t per = (uint64_t)heads * t_pad * HD;
    return 2 * per * (m == Math::F16 ? 2 : 4);  // K and Vt; SPLIT's two bf16 planes are 4 bytes together
}

}  // namespace bl

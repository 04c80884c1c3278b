// Fused multi-head self-attention for one qkv tensor: the reference's three
// kernels attention_scores+scale -> softmax -> attention_values
// (crates/beatlm-core/src/kernel.rs:731-777; codegen/wgsl.rs:590-669,
// :975-1010) as one flash-style pass with an online softmax, so the
// [T][H][T] scores and probabilities never exist.
//
//   qkv  [T][3][H][64]  (queries, keys, values of each token, heads side by side)
//   out  [T][H * 64]    (heads side by side, as the output projection reads them)
//
// Launches per spec (the prep only when no projection wrote K and Vt):
//  1. flash_prep_kernel writes the keys as K [H][T_pad][64] and the values
//     transposed as Vt [H][64][T_pad], once, in the matrix cores' operand type
//     (f16, f32, or hi and lo bf16 planes), zero-padded to whole 64-key tiles.
//     When the qkv tensor comes straight from a QKV projection, that GEMM's
//     epilogue writes these operands instead and this launch is skipped.
//     For the 32 x 32 kernel each 16-key group of a Vt row is stored in the
//     order 0-3, 8-11, 4-7, 12-15 (bits 2 and 3 of the key swapped), which is
//     the order in which that kernel's probabilities come out of its score
//     accumulators.
//  2. attn_kernel (f16 and bf16x3 math): the (head, NW x 32 query rows,
//     64-key tile) units are dealt out in equal contiguous runs to a fixed
//     grid of workgroups (one per CU), so every CU gets the same amount of
//     work whatever T and H are. A workgroup walks its run as segments of one
//     (head, query tile) each; its NW = 8 waves own 32 queries each and
//     share the K and Vt tiles, which stream through an LDS ring filled by
//     direct 16-byte loads. Each wave computes the transposed scores
//     S^T = K Q^T with v_mfma_f32_32x32x16, so a lane's accumulators hold 16
//     keys of ONE query: the row max is lane-local plus one exchange with the
//     lane 32 away. Eight consecutive accumulators are then exactly the
//     B operand of O^T = V^T P^T for one 16-key step. The running max is only
//     raised when a tile's max exceeds it by more than 8 (in log2 units), so
//     most tiles skip the rescale of O; probabilities stay <= 2^8.
//     The (head, query tile) pairs are dealt to the 8 XCDs in 8 contiguous
//     blocks, so an XCD's pairs share one or two heads and its L2 fetches
//     their keys and values once, and each XCD's units to its own workgroups
//     (workgroup g runs on XCD g % 8), so every query tile is computed and
//     merged inside one XCD and its L2.
//     A segment that covers all keys of its query tile writes the output; one
//     that covers part of them writes (max, sum, unnormalised output) to
//     scratch. The runs that split a tile then combine it themselves at the
//     end of the kernel: each adds one to the tile's arrival counter once its
//     partial result is stored (agent-coherent stores), one wave per
//     workgroup waits until all the tile's runs have arrived, and run j of r
//     combines rows [256 j / r, 256 (j + 1) / r) (agent-coherent loads). The
//     grid is one workgroup per CU, all resident at once, so every wait ends;
//     it is bounded all the same. attn_merge_kernel, a launch of its own,
//     does the same combination when BL_FLASH_MERGE_LAUNCH is set.
//  3. flash16_kernel (f32 math, v_mfma_f32_16x16x4_f32): a workgroup owns 64
//     queries of one head and one range of key tiles (split when there are
//     too few query tiles to fill the chip); merged by flash16_merge_kernel.
// Query rows outside the part are not stored.
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <vector>

#include "device_common.hpp"

namespace bl {
namespace {

constexpr int THREADS = 256;
constexpr int KT = 64;  // keys per tile
constexpr int HD = 64;  // head width
constexpr float LOG2E = 1.4426950408889634f;
constexpr int NW = 8;   // waves per workgroup of the 32 x 32 kernel (two per SIMD)
constexpr int THREADS32 = NW * 64;
// A tile's max must exceed the running max by more than this (log2 units)
// before the running max moves: probabilities are then at most 2^RESCALE.
constexpr float RESCALE = 8.0f;

template <Math M> struct FlashTraits;
template <> struct FlashTraits<Math::F16> {
    using T = _Float16;   // storage of qkv and out
    using L = _Float16;   // operand element of K / Vt
    static constexpr int PLANES = 1;  // operand planes (hi and lo for bf16x3)
    static constexpr int STAGES = 4;  // LDS ring depth
    static constexpr int QB = 1;      // 32-query blocks per wave
};
template <> struct FlashTraits<Math::SPLIT> {
    using T = float;
    using L = __bf16;
    static constexpr int PLANES = 2;
    static constexpr int STAGES = 4;
    static constexpr int QB = 1;
};
template <> struct FlashTraits<Math::F32> {
    using T = float;
    using L = float;
    static constexpr int CPR = 16;    // 16-byte chunks per 64-element row
    static constexpr int STAGES = 2;
};

// Query rows of one unit (a workgroup's tile) of the 32 x 32 kernel.
template <Math M> constexpr uint32_t query_rows() { return NW * FlashTraits<M>::QB * 32; }

// ---- 1. K and Vt in operand layout ----
// One workgroup per 64 keys of one head: 16-byte loads of the key and value
// rows, keys written as they are, values transposed through LDS and written
// as rows of 64 keys (in vt_pos order when PERM).
template <Math M, bool PERM>
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
        const uint64_t vi = ((uint64_t)head * HD + d) * tpad + kbase + (PERM ? vt_pos(r) : r);
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

// ---- 2. the 32 x 32 kernel (f16, bf16x3) ----

template <Math M> struct Op32;
template <> struct Op32<Math::F16> {
    using V = f16x8;
    static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Op32<Math::SPLIT> {
    using V = bf16x8;
    static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

// The bias product that starts each score chain. Key side (A, lane l32 =
// key, slots of lanes 0-31 only): [1, mask], mask = BIG for a key past the
// last token. Query side (B): [-m, -1]. The result is -m, or -m - BIG.
template <Math M> struct BiasBig;
template <> struct BiasBig<Math::F16> { static constexpr float value = 60000.0f; };
template <> struct BiasBig<Math::SPLIT> { static constexpr float value = 1e30f; };

template <Math M>
__device__ __forceinline__ typename Op32<M>::V bias_a(bool low_lanes, bool masked) {
    using V8 = typename Op32<M>::V;
    using E = std::remove_cv_t<std::remove_reference_t<decltype(V8{}[0])>>;
    V8 a = {};
    a[0] = (E)(low_lanes ? 1.0f : 0.0f);
    a[1] = (E)(low_lanes && masked ? BiasBig<M>::value : 0.0f);
    return a;
}
template <Math M>
__device__ __forceinline__ typename Op32<M>::V bias_b(float m, int h) {
    using V8 = typename Op32<M>::V;
    using E = std::remove_cv_t<std::remove_reference_t<decltype(V8{}[0])>>;
    V8 b = {};
    b[0] = (E)(h == 0 ? -m : 0.0f);
    b[1] = (E)(h == 0 ? -1.0f : 0.0f);
    return b;
}
// The nearest value of the operand type (kept within f16's range), so the
// bias product subtracts exactly the offset o and l carry.
template <Math M> __device__ __forceinline__ float representable(float v);
template <> __device__ __forceinline__ float representable<Math::F16>(float v) {
    return (float)(_Float16)fminf(fmaxf(v, -30000.0f), 30000.0f);
}
template <> __device__ __forceinline__ float representable<Math::SPLIT>(float v) { return (float)(__bf16)v; }

// The run of units [begin, end) of virtual workgroup v out of G: equal
// contiguous shares of U. The planner refuses shapes with U * G of 2^32 or
// more (FlashPlan::fits).
__host__ __device__ inline uint32_t run_begin(uint32_t v, uint32_t U, uint32_t G) { return v * U / G; }
// The virtual workgroup whose run holds unit u.
__host__ __device__ inline uint32_t run_of(uint32_t u, uint32_t U, uint32_t G) { return ((u + 1) * G - 1) / U; }

// XCD x's share of the `pairs` (head, query tile) pairs: the n pairs from
// run_begin(x, pairs, 8) on (the 8 XCDs' contiguous blocks; run_of(p, pairs,
// 8) is pair p's XCD), as n * kt units (pair after pair, key tiles
// inner) dealt in equal contiguous runs to the first G of the XCD's wgs / 8
// workgroups (local index g / 8 of workgroup g). When every pair can have two
// runs, the runs are counted so that each lies inside one pair: s per pair,
// the fewest that keep the longest run as short as floor(wgs / 8 / n) runs
// would. G is 0 when the XCD has no pair.
struct XcdShare {
    uint32_t n, U, G;
};
__host__ __device__ inline XcdShare xcd_share(uint32_t pairs, uint32_t kt, uint32_t wgs, uint32_t x) {
    XcdShare sh;
    const uint32_t gx = wgs / 8;
    sh.n = run_begin(x + 1, pairs, 8) - run_begin(x, pairs, 8);
    sh.U = sh.n * kt;
    sh.G = gx;
    if (sh.n && 2 * sh.n <= gx) {
        const uint32_t s0 = gx / sh.n, longest = (kt + s0 - 1) / s0, s = (kt + longest - 1) / longest;
        sh.G = sh.n * s;
    }
    if (sh.G > sh.U) sh.G = sh.U;
    return sh;
}

// The pairs (local indices within the XCD's share) of a run's first and last
// segments, and whether each is split, i.e. the run covers only part of its
// key tiles. The last is reported only when it differs from the first.
struct RunSplits {
    uint32_t first, last;
    bool first_split, last_split;
};
__host__ __device__ inline RunSplits run_splits(uint32_t u_begin, uint32_t u_end, uint32_t kt) {
    RunSplits r;
    r.first = u_begin / kt;
    r.last = (u_end - 1) / kt;
    r.first_split = u_begin % kt != 0 || u_end < (r.first + 1) * kt;
    r.last_split = r.last != r.first && u_end % kt != 0;
    return r;
}

// Partial results of workgroup g's segments: slot 0 holds its run's first
// segment, slot 1 its last (segments between them cover whole query tiles and
// write the output). Row r of a slot: QROWS rows of 64 floats, (max, sum)
// pairs beside.
template <Math M> __device__ __forceinline__ uint64_t partial_row(uint32_t g, uint32_t slot, uint32_t r) {
    return ((uint64_t)g * 2 + slot) * query_rows<M>() + r;
}

// Partial results that other workgroups of the same launch read (the
// in-kernel merge) are stored and loaded with the cache policy of agent-scope
// atomics (sc1: coherent across the device's XCDs and their L2s), so they
// are visible once the writer's stores have completed, with no L2 write-back
// between. Buffer descriptors over the partial and statistics arrays give
// 16- and 8-byte accesses with that policy.
constexpr int CPOL_AGENT = 16;  // sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7fffffff, 0x00020000);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x4 coherent_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte, 0, CPOL_AGENT));
}
__device__ __forceinline__ f32x2 coherent_load2(__amdgpu_buffer_rsrc_t r, uint32_t byte) {
    return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte, 0, CPOL_AGENT));
}
__device__ __forceinline__ void coherent_store4(__amdgpu_buffer_rsrc_t r, uint32_t byte, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte, 0, CPOL_AGENT);
}
__device__ __forceinline__ void coherent_store2(__amdgpu_buffer_rsrc_t r, uint32_t byte, f32x2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, byte, 0, CPOL_AGENT);
}

// The in-kernel merge's arrival counter of one pair, one 128-byte line per
// counter: every run that wrote a partial result of the pair adds 1 once all
// its waves' stores have completed; every run adds 1 more once it has seen
// all the runs arrive, and the last of those resets the counter to zero for
// the next launch. One wave per workgroup polls. Waiting is bounded (a
// fraction of a second): every workgroup of the grid is resident at once
// (one per CU, as many as CUs), so the arrivals come unless the device runs
// fewer workgroups at a time; a wait that runs out writes NaN for its rows,
// so that such a result can never pass for a right one, instead of waiting
// for ever.
constexpr uint32_t COUNTER_STRIDE = 32;  // words
constexpr uint32_t ARRIVAL_SPIN_LIMIT = 1u << 18;
__device__ __forceinline__ void arrive_count(uint32_t *ctr) {
    __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Whether the count reached `target` within the bound.
__device__ __forceinline__ bool await_count(const uint32_t *ctr, uint32_t target) {
    bool reached = false;
    for (uint32_t i = 0; i < ARRIVAL_SPIN_LIMIT && !reached; i++) {
        reached = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target;
        if (!reached) __builtin_amdgcn_s_sleep(8);
    }
    asm volatile("" ::: "memory");
    return reached;
}
__device__ __forceinline__ void depart_count(uint32_t *ctr, uint32_t total) {
    if (__hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1)
        __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Combines rows [r0, r1) of pair `item` (head item / qtiles, query tile
// item % qtiles) from the partial results of the XCD-local runs vf .. vl that
// split its key tiles:
//   O = sum_r 2^(m_r - m) O_r / sum_r 2^(m_r - m) l_r,
// folded run by run with a running max, BATCH runs at a time. One invocation
// per (row, 4 columns) out of `nthreads`, ITEMS of them at a time, every load
// of an iteration's items and batch issued before the first is used.
// COHERENT: the partial results were written in this launch (loads with the
// agent-coherent policy).
constexpr uint32_t MERGE_BATCH = 8;
template <Math M, bool COHERENT, uint32_t ITEMS, uint32_t BATCH>
__device__ __forceinline__ void merge_rows(const FlashArgs &a, uint32_t item, uint32_t r0, uint32_t r1, uint32_t tid,
                                           uint32_t nthreads, bool poison = false) {
    using T = typename FlashTraits<M>::T;
    constexpr uint32_t QROWS = query_rows<M>();
    const uint32_t kt = a.t_pad / KT, H = a.heads, pairs = a.qtiles * H;
    const uint32_t x = run_of(item, pairs, 8);
    const XcdShare sh = xcd_share(pairs, kt, a.wgs, x);
    const uint32_t u0 = (item - run_begin(x, pairs, 8)) * kt;
    const uint32_t vf = run_of(u0, sh.U, sh.G), vl = run_of(u0 + kt - 1, sh.U, sh.G);
    const uint32_t head = item / a.qtiles, qt = item % a.qtiles;
    // The first run holds this tile in its second slot unless the run starts with it.
    const uint32_t first_slot = run_begin(vf, sh.U, sh.G) < u0 ? 1 : 0;
    const uint32_t n = (r1 - r0) * (HD / 4);
    for (uint32_t w0 = tid; w0 < n; w0 += ITEMS * nthreads) {
        float m[ITEMS], l[ITEMS];
        f32x4 acc[ITEMS];
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; i++) {
            m[i] = -INFINITY;
            l[i] = 0.0f;
            acc[i] = f32x4{0, 0, 0, 0};
        }
        for (uint32_t v0 = vf; v0 <= vl; v0 += BATCH) {
            f32x2 st[ITEMS][BATCH];
            f32x4 ov[ITEMS][BATCH];
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; i++) {
                const uint32_t w = w0 + i * nthreads;
                const uint32_t r = r0 + w / (HD / 4), d = (w % (HD / 4)) * 4;
#pragma unroll
                for (uint32_t b = 0; b < BATCH; b++) {
                    const uint32_t v = v0 + b;
                    st[i][b] = f32x2{-INFINITY, 0.0f};
                    ov[i][b] = f32x4{0, 0, 0, 0};
                    if (v <= vl && w < n) {
                        const uint64_t row = partial_row<M>(v * 8 + x, v == vf ? first_slot : 0, r);
                        if constexpr (COHERENT) {
                            st[i][b] = coherent_load2(coherent_rsrc(a.stats), (uint32_t)(row * 8));
                            ov[i][b] = coherent_load4(coherent_rsrc(a.partial), (uint32_t)((row * HD + d) * 4));
                        } else {
                            st[i][b] = *(const f32x2 *)(a.stats + 2 * row);
                            ov[i][b] = *(const f32x4 *)(a.partial + row * HD + d);
                        }
                    }
                }
            }
#pragma unroll
            for (uint32_t i = 0; i < ITEMS; i++) {
                float m_new = m[i];
#pragma unroll
                for (uint32_t b = 0; b < BATCH; b++) m_new = fmaxf(m_new, st[i][b][0]);
                const float wa = __builtin_amdgcn_exp2f(m[i] - m_new);
                l[i] *= wa;
                acc[i] *= wa;
#pragma unroll
                for (uint32_t b = 0; b < BATCH; b++) {
                    const float wb = __builtin_amdgcn_exp2f(st[i][b][0] - m_new);  // 0 for a run past vl
                    l[i] += st[i][b][1] * wb;
                    acc[i] += ov[i][b] * wb;
                }
                m[i] = m_new;
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < ITEMS; i++) {
            const uint32_t w = w0 + i * nthreads;
            const uint32_t r = r0 + w / (HD / 4), d = (w % (HD / 4)) * 4;
            const uint32_t q = a.row0 + qt * QROWS + r;
            if (w >= n || q >= a.row1) continue;
            const float inv = poison ? __builtin_nanf("") : 1.0f / l[i];
            if constexpr (M == Math::SPLIT) {
                store_f32x4((float *)a.out, ((uint64_t)q * H + head) * HD + d, acc[i] * inv, a.out_planes);
            } else {
                f16x4 w4;
#pragma unroll
                for (int e = 0; e < 4; e++) w4[e] = (_Float16)(acc[i][e] * inv);
                *(f16x4 *)((T *)a.out + ((uint64_t)q * H + head) * HD + d) = w4;
            }
        }
    }
}

template <Math M>
__global__ __launch_bounds__(THREADS32, 2) void attn_kernel(FlashArgs args) {
    using Tr = FlashTraits<M>;
    using T = typename Tr::T;
    using Op = Op32<M>;
    using V8 = typename Op::V;
    constexpr int PLANES = Tr::PLANES, STAGES = Tr::STAGES;
    constexpr int CPR = 8;
    constexpr int ROWB = CPR * 16;             // 128 bytes per staged row
    constexpr int TILE_BYTES = 64 * ROWB;      // one plane of a K or Vt tile
    constexpr int K_BYTES = PLANES * TILE_BYTES;
    constexpr int STAGE_BYTES = 2 * K_BYTES;
    constexpr int LPS = 2 * PLANES * loads_per_wave<64, CPR, NW>();
    constexpr uint32_t QROWS = query_rows<M>();
    constexpr bool SPLIT = M == Math::SPLIT;
    static_assert(Tr::QB == 1, "one 32-query block per wave");
    static_assert(STAGES >= 3, "two tiles are read while the next is loaded");

    __shared__ __attribute__((aligned(16))) char smem[STAGES * STAGE_BYTES];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const uint32_t H = args.heads, tpad = args.t_pad, Tn = args.tokens;
    const uint32_t kt = tpad / KT;
    const uint32_t pairs = args.qtiles * H;
    // This workgroup's XCD (g % 8: workgroups are dealt to the XCDs round
    // robin) and its run among that XCD's workgroups.
    const uint32_t g = blockIdx.x, xg = g % 8, v = g / 8;
    const XcdShare sh = xcd_share(pairs, kt, args.wgs, xg);
    const uint32_t u_begin = v < sh.G ? run_begin(v, sh.U, sh.G) : 0;
    const uint32_t u_end = v < sh.G ? run_begin(v + 1, sh.U, sh.G) : 0;

    constexpr int ESZ = 2;
    const uint64_t plane_bytes = (uint64_t)H * tpad * HD * ESZ;
    const RowLoader<64, CPR, NW> kload(HD * ESZ, 63, wave, lane);
    const RowLoader<64, CPR, NW> vload(tpad * ESZ, 63, wave, lane);
    const float c = args.scale * LOG2E;
    const uint32_t row_stride = 3 * H * HD;
    // Fragment reads: staged row 32 b + l32 carries the swizzle of l32.
    const int x = (l32 >> 1) & 7;
    const int lrow = l32 * ROWB;

    uint32_t u = u_begin;
    bool first = true;
    while (u < u_end) {
        const uint32_t item = run_begin(xg, pairs, 8) + u / kt;
        const uint32_t k0 = u % kt;
        const uint32_t left = u_end - u;
        const uint32_t k1 = left < kt - k0 ? k0 + left : kt;
        const uint32_t head = item / args.qtiles, qt = item % args.qtiles;
        const uint32_t q = args.row0 + qt * QROWS + wave * 32 + l32;

        const char *kbase = (const char *)args.kp + (uint64_t)head * tpad * HD * ESZ;
        const char *vbase = (const char *)args.vt + (uint64_t)head * HD * tpad * ESZ;
        auto issue = [&](uint32_t t) {
            char *st = smem + ((t - k0) % STAGES) * STAGE_BYTES;
#pragma unroll
            for (int p = 0; p < PLANES; p++) {
                kload.issue(kbase + p * plane_bytes + (uint64_t)t * KT * HD * ESZ, st + p * TILE_BYTES);
                vload.issue(vbase + p * plane_bytes + (uint64_t)t * KT * ESZ, st + K_BYTES + p * TILE_BYTES);
            }
        };
        // Tile t has landed for every wave once this wave's loads up to it are
        // done (at most the later tiles' loads outstanding) and all waves met.
        auto arrive = [&](uint32_t t) {
            if (t + STAGES - 3 <= k1 - 1) wait_vmcnt<(STAGES - 3) * LPS>();
            else wait_vmcnt<0>();
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        };

        // The wave's 32 queries as they are stored: lane (l32, h) loads d =
        // 16 ds + 8 h + e of query q. Issued before the segment's first K and Vt
        // tiles, so one wait covers both.
        f32x4 qa[4], qb[4];
        f16x8 q16[4];
        {
            const bool ok = q < args.row1;
            const T *qrow = (const T *)args.qkv + (uint64_t)q * row_stride + head * HD + 8 * h;
#pragma unroll
            for (int ds = 0; ds < 4; ds++) {
                if constexpr (SPLIT) {
                    qa[ds] = f32x4{0, 0, 0, 0};
                    qb[ds] = f32x4{0, 0, 0, 0};
                    if (ok) {
                        qa[ds] = *(const f32x4 *)(qrow + 16 * ds);
                        qb[ds] = *(const f32x4 *)(qrow + 16 * ds + 4);
                    }
                } else {
                    q16[ds] = f16x8{};
                    if (ok) q16[ds] = *(const f16x8 *)(qrow + 16 * ds);
                }
            }
        }
        for (uint32_t t = k0; t < k0 + STAGES - 1 && t < k1; t++) issue(t);
        arrive(k0);
        // The queries pre-scaled by scale * log2(e), as the B operand of
        // S^T = K Q^T.
        V8 qh[4], ql[4];
#pragma unroll
        for (int ds = 0; ds < 4; ds++) {
            if constexpr (SPLIT) {
                float qv[8];
#pragma unroll
                for (int e = 0; e < 8; e++) qv[e] = (e < 4 ? qa[ds][e] : qb[ds][e - 4]) * c;
                split8_bf16(qv, qh[ds], ql[ds]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) qh[ds][e] = (_Float16)((float)q16[ds][e] * c);
            }
        }

        // S^T - bias for tile t: keys 32 mb + 8 (i/4) + 4 h + i%4, query q. Each
        // chain starts with the bias product: key slots [1, mask] (mask = BIG
        // for a key past the last token) times query slots [-bias, -1] in the
        // k-slots of lanes 0-31.
        auto scores = [&](uint32_t t, const V8 &bq, f32x16 (&s)[2]) {
            const char *ks = smem + ((t - k0) % STAGES) * STAGE_BYTES + lrow;
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const uint32_t key = t * KT + 32 * mb + l32;
                s[mb] = Op::mma(bias_a<M>(h == 0, key >= Tn), bq, f32x16{});
#pragma unroll
                for (int ds = 0; ds < 4; ds++) {
                    const int off = mb * 32 * ROWB + (((2 * ds + h) ^ x) << 4);
                    const V8 kh = *(const V8 *)(ks + off);
                    if constexpr (SPLIT) {
                        const V8 kl = *(const V8 *)(ks + TILE_BYTES + off);
                        s[mb] = Op::mma(kl, qh[ds], s[mb]);
                        s[mb] = Op::mma(kh, ql[ds], s[mb]);
                        s[mb] = Op::mma(kh, qh[ds], s[mb]);
                    } else {
                        s[mb] = Op::mma(kh, qh[ds], s[mb]);
                    }
                }
            }
        };

        f32x16 o[2] = {f32x16{}, f32x16{}};  // O^T: d = 32 db + 8 (i/4) + 4 h + i%4, query q
        // m_run: the exponent offset of o and l_run (log2 units), always a value
        // of the operand type. bias_q: the offset the bias operand bq carries,
        // i.e. the offset of scores computed from now on; bias_cur: that of the
        // tile being finished (0 for the first tile).
        float m_run = -INFINITY, l_run = 0.0f, bias_cur = 0.0f, bias_q = 0.0f;
        V8 bq = bias_b<M>(0.0f, h);

        // One key tile: finish tile t from s_cur (softmax, O^T += V^T P^T) while
        // tile t + 1's scores go into s_next, interleaved on the matrix cores.
        auto step = [&](uint32_t t, f32x16 (&s_cur)[2], f32x16 (&s_next)[2]) {
            const bool more = t + 1 < k1;
            if (more) {
                arrive(t + 1);  // also: every wave is past tile t - 1, whose slot is reloaded next
                if (t + STAGES - 1 < k1) issue(t + STAGES - 1);
            }
            // The running max only moves when the tile's max exceeds it by more
            // than RESCALE; the scores already carry the offset unless it moved
            // since they were computed.
            float tmax = -INFINITY;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) tmax = fmaxf(tmax, s_cur[mb][r]);
            const float top = max_xor32(tmax) + bias_cur;  // finite: every tile holds a key < T
            const bool up = top > m_run + RESCALE;
            if (__any(up)) {
                const float m_new = up ? representable<M>(top) : m_run;
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
                o[0] *= alpha;
                o[1] *= alpha;
                m_run = m_new;
                bq = bias_b<M>(m_new, h);
                bias_q = m_new;
            }
            const float shift = m_run - bias_cur;
            if (__any(shift != 0.0f)) {
#pragma unroll
                for (int mb = 0; mb < 2; mb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) s_cur[mb][r] -= shift;
            }
            bias_cur = bias_q;

            const char *vs = smem + ((t - k0) % STAGES) * STAGE_BYTES + K_BYTES + lrow;
            float psum = 0.0f;
            if constexpr (!SPLIT) {
                // f16: an explicit schedule. The tile's 16 LDS fragments are read
                // first; then each score product of tile t + 1 is followed by
                // four of this tile's exponentials, and each value product by
                // the conversions and row sums that feed the next.
                typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
                const char *ks = smem + ((t + 1 - k0) % STAGES) * STAGE_BYTES + lrow;
                V8 kf[8], vf[8];
                if (more) {
#pragma unroll
                    for (int i = 0; i < 8; i++) kf[i] = *(const V8 *)(ks + (i / 4) * 32 * ROWB + (((2 * (i % 4) + h) ^ x) << 4));
                }
#pragma unroll
                for (int i = 0; i < 8; i++) vf[i] = *(const V8 *)(vs + (i % 2) * 32 * ROWB + (((2 * (i / 2) + h) ^ x) << 4));
                auto exp4 = [&](int c) {
#pragma unroll
                    for (int r = 0; r < 4; r++) s_cur[c / 4][4 * (c % 4) + r] = __builtin_amdgcn_exp2f(s_cur[c / 4][4 * (c % 4) + r]);
                };
                __builtin_amdgcn_sched_barrier(0);
                if (more) {
#pragma unroll
                    for (int mb = 0; mb < 2; mb++) {
                        const uint32_t key = (t + 1) * KT + 32 * mb + l32;
                        s_next[mb] = Op::mma(bias_a<M>(h == 0, key >= Tn), bq, f32x16{});
                        exp4(mb);
                        __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int ds = 0; ds < 4; ds++)
#pragma unroll
                        for (int mb = 0; mb < 2; mb++) {
                            s_next[mb] = Op::mma(kf[4 * mb + ds], qh[ds], s_next[mb]);
                            if (2 + 2 * ds + mb < 8) exp4(2 + 2 * ds + mb);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                } else {
#pragma unroll
                    for (int c = 0; c < 8; c++) exp4(c);
                }
#pragma unroll
                for (int st2 = 0; st2 < 4; st2++) {
                    const int mb = st2 >> 1, hf = st2 & 1;
                    V8 ph;
#pragma unroll
                    for (int e = 0; e < 8; e++) ph[e] = (_Float16)s_cur[mb][8 * hf + e];
                    o[0] = Op::mma(vf[2 * st2], ph, o[0]);
                    psum = __builtin_amdgcn_fdot2(h2{ph[0], ph[1]}, one, psum, false);
                    psum = __builtin_amdgcn_fdot2(h2{ph[2], ph[3]}, one, psum, false);
                    __builtin_amdgcn_sched_barrier(0);
                    o[1] = Op::mma(vf[2 * st2 + 1], ph, o[1]);
                    psum = __builtin_amdgcn_fdot2(h2{ph[4], ph[5]}, one, psum, false);
                    psum = __builtin_amdgcn_fdot2(h2{ph[6], ph[7]}, one, psum, false);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                // bf16x3: tile t + 1's scores on the matrix cores while this
                // tile's probabilities are made on the vector ALUs.
                if (more) scores(t + 1, bq, s_next);
#pragma unroll
                for (int mb = 0; mb < 2; mb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) s_cur[mb][r] = __builtin_amdgcn_exp2f(s_cur[mb][r]);
                // O^T += V^T P^T, 16 keys a step: the step's probabilities are
                // accumulators 8 (st%2) .. +7 of key block st/2, keys 16 st + 4 h + 0..3
                // and 16 st + 8 + 4 h + 0..3, the order the Vt row holds them in.
#pragma unroll
                for (int st2 = 0; st2 < 4; st2++) {
                    const int mb = st2 >> 1, hf = st2 & 1;
                    V8 ph, pl;
                    float pv[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        pv[e] = s_cur[mb][8 * hf + e];
                        psum += pv[e];
                    }
                    split8_bf16(pv, ph, pl);
#pragma unroll
                    for (int db = 0; db < 2; db++) {
                        const int off = db * 32 * ROWB + (((2 * st2 + h) ^ x) << 4);
                        const V8 vh = *(const V8 *)(vs + off);
                        const V8 vl = *(const V8 *)(vs + TILE_BYTES + off);
                        o[db] = Op::mma(vl, ph, o[db]);
                        o[db] = Op::mma(vh, pl, o[db]);
                        o[db] = Op::mma(vh, ph, o[db]);
                    }
                }
            }
            l_run += psum;
            asm volatile("" ::: "memory");
        };

        f32x16 sa[2], sb[2];
        scores(k0, bq, sa);
        uint32_t t = k0;
        for (; t + 1 < k1; t += 2) {
            step(t, sa, sb);
            step(t + 1, sb, sa);
        }
        if (t < k1) step(t, sa, sb);

        // The segment's result: the output itself when it covered every key
        // tile, else (max, sum, unnormalised output) in the run's slot.
        const float l_tot = sum_xor32(l_run);
        if (q < args.row1) {
            if (k0 == 0 && k1 == kt) {
                const float inv = 1.0f / l_tot;
                T *out = (T *)args.out + ((uint64_t)q * H + head) * HD;
#pragma unroll
                for (int db = 0; db < 2; db++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int d = 32 * db + 8 * j + 4 * h;
                        if constexpr (SPLIT) {
                            store_f32x4((float *)args.out, ((uint64_t)q * H + head) * HD + d,
                                        f32x4{o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]} * inv,
                                        args.out_planes);
                        } else {
                            f16x4 w;
#pragma unroll
                            for (int r = 0; r < 4; r++) w[r] = (_Float16)(o[db][4 * j + r] * inv);
                            *(f16x4 *)(out + d) = w;
                        }
                    }
            } else {
                const uint64_t row = partial_row<M>(g, first ? 0 : 1, wave * 32 + l32);
                if (args.merge_inline) {
                    const __amdgpu_buffer_rsrc_t pr = coherent_rsrc(args.partial);
#pragma unroll
                    for (int db = 0; db < 2; db++)
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            coherent_store4(pr, (uint32_t)((row * HD + 32 * db + 8 * j + 4 * h) * 4),
                                            f32x4{o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]});
                    if (h == 0) coherent_store2(coherent_rsrc(args.stats), (uint32_t)(row * 8), f32x2{m_run, l_tot});
                } else {
                    float *part = args.partial + row * HD;
#pragma unroll
                    for (int db = 0; db < 2; db++)
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            *(f32x4 *)(part + 32 * db + 8 * j + 4 * h) =
                                f32x4{o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]};
                    if (h == 0) *(f32x2 *)(args.stats + 2 * row) = f32x2{m_run, l_tot};
                }
            }
        }
        const bool partial = !(k0 == 0 && k1 == kt);
        u += k1 - k0;
        first = false;
        // Every wave is done with the ring before the next segment refills it,
        // and no store is left outstanding under the next segment's load counts
        // (nor, for a partial result merged in this launch, before its arrival).
        wait_vmcnt<0>();
        __syncthreads();
        if (partial && args.merge_inline && tid == 0) arrive_count(args.counters + item * COUNTER_STRIDE);
    }

    // The in-kernel merge: this workgroup's share of each query tile it
    // computed part of (at most its first and its last segment). Run j of the
    // r runs vf .. vl that split the tile combines rows [QROWS j / r,
    // QROWS (j + 1) / r) once all r runs' waves have arrived.
    if (args.merge_inline && u_begin < u_end) {
        const RunSplits rs = run_splits(u_begin, u_end, kt);
        for (uint32_t s = 0; s < 2; s++) {
            if (!(s == 0 ? rs.first_split : rs.last_split)) continue;
            const uint32_t local = s == 0 ? rs.first : rs.last;
            const uint32_t item = run_begin(xg, pairs, 8) + local;
            const uint32_t u0 = local * kt;
            const uint32_t vf = run_of(u0, sh.U, sh.G), vl = run_of(u0 + kt - 1, sh.U, sh.G);
            const uint32_t r = vl - vf + 1, j = v - vf;
            uint32_t *ctr = args.counters + item * COUNTER_STRIDE;
            bool missed = false;
            if (wave == 0) missed = !await_count(ctr, r);
            missed = __syncthreads_or(missed);
            if (tid == 0) depart_count(ctr, 2 * r);
            if (r <= 2) merge_rows<M, true, 4, 2>(args, item, QROWS * j / r, QROWS * (j + 1) / r, tid, THREADS32, missed);
            else merge_rows<M, true, 2, MERGE_BATCH>(args, item, QROWS * j / r, QROWS * (j + 1) / r, tid, THREADS32, missed);
        }
    }
}

// Combines the split pairs' partial results: a workgroup takes MERGE_ROWS
// rows of one pair, one invocation per (row, 4 columns). Workgroup b runs on
// XCD b % 8 and takes a pair of that XCD's block, whose partial results its
// L2 may still hold.
constexpr uint32_t MERGE_ROWS = 16;
template <Math M>
__global__ __launch_bounds__(256) void attn_merge_kernel(FlashArgs a) {
    constexpr uint32_t GROUPS = query_rows<M>() / MERGE_ROWS;
    const uint32_t x = blockIdx.x % 8, k = blockIdx.x / 8;
    const uint32_t pairs = a.qtiles * a.heads;
    const uint32_t local = k / GROUPS, r0 = (k % GROUPS) * MERGE_ROWS;
    if (local >= run_begin(x + 1, pairs, 8) - run_begin(x, pairs, 8)) return;
    const uint32_t item = run_begin(x, pairs, 8) + local;
    const uint32_t kt = a.t_pad / KT;
    const XcdShare sh = xcd_share(pairs, kt, a.wgs, x);
    const uint32_t u0 = local * kt;
    if (run_of(u0, sh.U, sh.G) == run_of(u0 + kt - 1, sh.U, sh.G)) return;  // written by attn_kernel
    merge_rows<M, false, 1, MERGE_BATCH>(a, item, r0, r0 + MERGE_ROWS, threadIdx.x, 256);
}

// ---- 3. the 16 x 16 kernel (f32 math) ----
__global__ __launch_bounds__(THREADS) void flash16_kernel(FlashArgs args) {
    using Tr = FlashTraits<Math::F32>;
    constexpr int CPR = Tr::CPR, STAGES = Tr::STAGES;
    constexpr int TILE_BYTES = 64 * CPR * 16;
    constexpr int K_BYTES = TILE_BYTES;
    constexpr int STAGE_BYTES = 2 * K_BYTES;
    constexpr int LPS = 2 * loads_per_wave<64, CPR>();

    __shared__ __attribute__((aligned(16))) char smem[STAGES * STAGE_BYTES];

    const float *__restrict__ qkv = (const float *)args.qkv;
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

    constexpr int ESZ = 4;
    const char *kbase = (const char *)args.kp + (uint64_t)head * tpad * HD * ESZ;
    const char *vbase = (const char *)args.vt + (uint64_t)head * HD * tpad * ESZ;
    const RowLoader<64, CPR> kload(HD * ESZ, 63, wave, lane);
    const RowLoader<64, CPR> vload(tpad * ESZ, 63, wave, lane);
    auto issue = [&](uint32_t t, int slot) {
        char *st = smem + slot * STAGE_BYTES;
        kload.issue(kbase + (uint64_t)t * KT * HD * ESZ, st);
        vload.issue(vbase + (uint64_t)t * KT * ESZ, st + K_BYTES);
    };

    constexpr int ROWB = CPR * 16;
    const int lrow = l16 * ROWB;
    const int x = l16;

    // Step (h, s) of the 16 x 16 x 4 products: lane group g reads d = 16h + 4g + s.
    const float *qrow = qkv + (uint64_t)q * row_stride + head * HD;
    float qf32[16];
#pragma unroll
    for (int hh = 0; hh < 4; hh++) {
        f32x4 a = {};
        if (q_ok) a = *(const f32x4 *)(qrow + 16 * hh + 4 * g);
#pragma unroll
        for (int s = 0; s < 4; s++) qf32[4 * hh + s] = a[s];
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

        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            f32x4 acc = {0, 0, 0, 0};
            const char *krow = ks + kt * 16 * ROWB + lrow;
#pragma unroll
            for (int hh = 0; hh < 4; hh++) {
                f32x4 a = *(const f32x4 *)(krow + (((4 * hh + g) ^ x) << 4));
#pragma unroll
                for (int st2 = 0; st2 < 4; st2++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st2], qf32[4 * hh + st2], acc, 0, 0, 0);
            }
            s[kt] = acc;
        }

        const uint32_t kb = t * KT;
        float tmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t key = kb + 16 * kt + 4 * g + r;
                const float v = key < Tn ? s[kt][r] * sl2 : -INFINITY;
                s[kt][r] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
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
        asm volatile("" ::: "memory");
    }

    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (!q_ok) return;

    if (args.splits == 1) {
        const float inv = 1.0f / l_run;
        float *out = (float *)args.out + (uint64_t)q * H * HD + head * HD;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) *(f32x4 *)(out + 16 * dt + 4 * g) = o[dt] * inv;
    } else {
        const uint64_t slot = ((uint64_t)split * Tn + q) * H + head;
        float *part = args.partial + slot * HD;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) *(f32x4 *)(part + 16 * dt + 4 * g) = o[dt];
        if (g == 0) *(f32x2 *)(args.stats + 2 * slot) = f32x2{m_run, l_run};
    }
}

__global__ __launch_bounds__(256) void flash16_merge_kernel(FlashArgs args) {
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
            const float w = exp2f(args.stats[2 * slot] - m);
            l += w * args.stats[2 * slot + 1];
            acc += w * *(const f32x4 *)(args.partial + slot * HD + d);
        }
        const float inv = 1.0f / l;
        float *out = (float *)args.out + (uint64_t)q * H * HD + head * HD + d;
        *(f32x4 *)out = acc * inv;
    }
}

constexpr uint32_t FLASH16_MAX_SPLITS = 8;

uint64_t operand_bytes(Math m, uint32_t heads, uint32_t t_pad) {
    const uint64_t per = (uint64_t)heads * t_pad * HD;
    return 2 * per * (m == Math::F16 ? 2 : 4);  // K and Vt; SPLIT's two bf16 planes are 4 bytes together
}

template <Math M>
hipError_t launch_32(const FlashArgs &a, hipStream_t s) {
    hipError_t e;
    if (!a.prepped) {
        hipLaunchKernelGGL((flash_prep_kernel<M, true>), dim3(a.t_pad / KT, a.heads), dim3(THREADS), 0, s, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(attn_kernel<M>, dim3(a.wgs), dim3(THREADS32), 0, s, a);
    e = hipGetLastError();
    if (e != hipSuccess || !a.merge || a.merge_inline) return e;
    const uint32_t blocks = 8 * ((a.qtiles * a.heads + 7) / 8) * (query_rows<M>() / MERGE_ROWS);
    hipLaunchKernelGGL(attn_merge_kernel<M>, dim3(blocks), dim3(MERGE_ROWS * (HD / 4)), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_16(const FlashArgs &a, hipStream_t s) {
    hipLaunchKernelGGL((flash_prep_kernel<Math::F32, false>), dim3(a.t_pad / KT, a.heads), dim3(THREADS), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    dim3 grid((a.row1 - a.row0 + 63) / 64, a.heads, a.splits);
    hipLaunchKernelGGL(flash16_kernel, grid, dim3(THREADS), 0, s, a);
    e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1) return e;
    uint64_t work = (uint64_t)(a.row1 - a.row0) * a.heads * (HD / 4);
    uint32_t blocks = (uint32_t)std::min<uint64_t>((work + 255) / 256, 4096);
    hipLaunchKernelGGL(flash16_merge_kernel, dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_flash(const FlashArgs &a, Math m, hipStream_t s) {
    if (a.row1 <= a.row0) return hipSuccess;
    switch (m) {
    case Math::F16: return launch_32<Math::F16>(a, s);
    case Math::SPLIT: return launch_32<Math::SPLIT>(a, s);
    default: return launch_16(a, s);
    }
}

FlashPlan plan_flash(Math m, uint32_t tokens, uint32_t heads, uint32_t row0, uint32_t row1, uint32_t compute_units) {
    FlashPlan p;
    const uint32_t rows = row1 > row0 ? row1 - row0 : 0;
    const uint32_t t_pad = (tokens + KT - 1) / KT * KT;
    const uint32_t kt = t_pad / KT;
    uint64_t extra = 0;
    if (m == Math::F32) {
        const uint32_t wgs = (rows + 63) / 64 * heads;
        // Enough workgroups for two per CU, each split keeping two key tiles or more.
        uint32_t splits = wgs ? (2 * compute_units + wgs - 1) / wgs : 1;
        p.splits = std::max<uint32_t>(1, std::min<uint32_t>({splits, kt / 2, FLASH16_MAX_SPLITS}));
        if (p.splits > 1) extra = (uint64_t)p.splits * tokens * heads * (HD + 2) * sizeof(float);
    } else {
        const uint32_t qrows = m == Math::F16 ? query_rows<Math::F16>() : query_rows<Math::SPLIT>();
        p.qtiles = (rows + qrows - 1) / qrows;
        p.units = (uint64_t)heads * p.qtiles * kt;
        // One workgroup per CU, the same number on each XCD (its 8 waves are
        // two per SIMD); the pairs and their units are shared out per XCD.
        p.wgs = std::max<uint32_t>(8, compute_units / 8 * 8);
        // The run arithmetic is 32-bit: (pairs + 1) * 8, and each XCD's
        // units times its runs, stay below 2^32.
        const uint64_t pairs64 = (uint64_t)heads * p.qtiles;
        if ((pairs64 + 1) * 8 >= (1ull << 32)) {
            p.fits = false;
            return p;
        }
        const uint32_t pairs = (uint32_t)pairs64;
        for (uint32_t x = 0; x < 8; x++) {
            const uint64_t n = run_begin(x + 1, pairs, 8) - run_begin(x, pairs, 8);
            if ((n * kt + 1) * (p.wgs / 8) >= (1ull << 32)) {
                p.fits = false;
                return p;
            }
        }
        for (uint32_t item = 0; item < pairs && !p.merge; item++) {
            const uint32_t x = run_of(item, pairs, 8);
            const XcdShare sh = xcd_share(pairs, kt, p.wgs, x);
            const uint32_t u0 = (item - run_begin(x, pairs, 8)) * kt;
            p.merge = run_of(u0, sh.U, sh.G) != run_of(u0 + kt - 1, sh.U, sh.G);
        }
        // Two result slots per workgroup: its first and its last segment.
        extra = (uint64_t)p.wgs * 2 * qrows * (HD + 2) * sizeof(float);
        p.counters = p.merge ? pairs : 0;
        p.counter_bytes = (uint64_t)p.counters * COUNTER_STRIDE * sizeof(uint32_t);
    }
    p.scratch_bytes = operand_bytes(m, heads, t_pad) + extra;
    return p;
}

int flash_plan_check(uint32_t tokens, uint32_t heads, uint32_t compute_units, bool f16, uint64_t *units) {
    const FlashPlan p = plan_flash(f16 ? Math::F16 : Math::SPLIT, tokens, heads, 0, tokens, compute_units);
    if (!p.fits) return BL_ERR_TOO_LARGE;
    const uint32_t kt = (tokens + KT - 1) / KT, pairs = heads * p.qtiles;
    uint64_t total = 0;
    for (uint32_t x = 0; x < 8; x++) {
        const XcdShare sh = xcd_share(pairs, kt, p.wgs, x);
        total += sh.U;
        if (sh.U == 0) continue;
        if (sh.G == 0 || sh.G > p.wgs / 8 || run_begin(0, sh.U, sh.G) != 0 || run_begin(sh.G, sh.U, sh.G) != sh.U)
            return BL_ERR_KERNEL;
        for (uint32_t v = 0; v < sh.G; v++) {
            const uint32_t b = run_begin(v, sh.U, sh.G), e = run_begin(v + 1, sh.U, sh.G);
            if (e < b) return BL_ERR_KERNEL;
            if (e > b && (run_of(b, sh.U, sh.G) != v || run_of(e - 1, sh.U, sh.G) != v)) return BL_ERR_KERNEL;
        }
        // The in-kernel merge: the runs vf .. vl of every split pair, and
        // only they, name the pair among their split segments (each arrives
        // and waits for r runs), and their row shares cover the tile once.
        std::vector<uint32_t> named(sh.n, 0);
        for (uint32_t v = 0; v < sh.G; v++) {
            const uint32_t b = run_begin(v, sh.U, sh.G), e = run_begin(v + 1, sh.U, sh.G);
            if (e <= b) continue;
            const RunSplits rs = run_splits(b, e, kt);
            for (uint32_t s = 0; s < 2; s++) {
                if (!(s == 0 ? rs.first_split : rs.last_split)) continue;
                const uint32_t local = s == 0 ? rs.first : rs.last;
                const uint32_t vf = run_of(local * kt, sh.U, sh.G), vl = run_of(local * kt + kt - 1, sh.U, sh.G);
                if (local >= sh.n || v < vf || v > vl || vf == vl) return BL_ERR_KERNEL;
                named[local]++;
            }
        }
        const uint32_t qrows = f16 ? query_rows<Math::F16>() : query_rows<Math::SPLIT>();
        for (uint32_t local = 0; local < sh.n; local++) {
            const uint32_t vf = run_of(local * kt, sh.U, sh.G), vl = run_of(local * kt + kt - 1, sh.U, sh.G);
            const uint32_t r = vl - vf + 1;
            if (named[local] != (r > 1 ? r : 0)) return BL_ERR_KERNEL;
            for (uint32_t j = 0; j < r; j++)
                if (qrows * j / r > qrows * (j + 1) / r || (j + 1 == r && qrows * (j + 1) / r != qrows)) return BL_ERR_KERNEL;
        }
    }
    if (units) *units = total;
    return total == p.units ? BL_OK : BL_ERR_KERNEL;
}

void bind_flash_scratch(FlashArgs &a, Math m, void *base, uint64_t counter_bytes) {
    const uint64_t ops = operand_bytes(m, a.heads, a.t_pad);
    a.counters = (uint32_t *)base;
    char *b = (char *)base + counter_bytes;
    a.kp = b;
    a.vt = b + ops / 2;
    a.partial = (float *)(b + ops);
    if (m == Math::F32) {
        a.stats = a.partial + (uint64_t)a.splits * a.tokens * a.heads * HD;
    } else {
        const uint32_t qrows = m == Math::F16 ? query_rows<Math::F16>() : query_rows<Math::SPLIT>();
        a.stats = a.partial + (uint64_t)a.wgs * 2 * qrows * HD;
    }
}

}  // namespace bl

// Test hook (no GPU work): flash_plan_check for a shape.
extern "C" int bl_flash_plan_check(uint32_t tokens, uint32_t heads, uint32_t compute_units, uint32_t dtype,
                                   uint64_t *units) {
    if (tokens == 0 || heads == 0 || compute_units == 0 || (dtype != BL_F32 && dtype != BL_F16))
        return BL_ERR_INVALID_ARGUMENT;
    return bl::flash_plan_check(tokens, heads, compute_units, dtype == BL_F16, units);
}

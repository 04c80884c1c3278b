// Device-side helpers shared by the CDNA4 (gfx950) kernels: vector and MFMA
// operand types, 64-lane wave reductions, the epilogue steps of a kernel spec
// and GELU through erf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "spec.hpp"

namespace bl {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;

// ---- loads/stores of one element as f32 ----

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }

// ---- 64-lane reductions (butterfly over the whole wave) ----

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// The sum over the LPR consecutive lanes that hold one row (LPR a power of 2).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// v plus v of the lane DPP control CTRL names (row and bank masks full).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// The sum over the 16 lanes of v's DPP row (lanes 16r .. 16r + 15), in every
// one of them: swaps of neighbours and of pairs inside each quad, then the
// mirror images inside each half row and each row (gfx9 DPP has no xor mask
// beyond a quad): after each step the lanes of the next larger group hold
// equal sums. No LDS round trip, unlike a shuffle.
__device__ __forceinline__ float row16_sum(float v) {
    v = dpp_add<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v = dpp_add<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v = dpp_add<0x141>(v);  // row_half_mirror
    return dpp_add<0x140>(v);  // row_mirror
}
// The sum over the 4 lanes of v's quad, in each of them.
__device__ __forceinline__ float quad_sum(float v) { return dpp_add<0x4E>(dpp_add<0xB1>(v)); }

// ---- the attention's value operand layout ----
// Position of key k inside a row of the transposed values Vt for the 32 x 32
// flash kernel: bits 2 and 3 of k swapped, so each 16-key group is stored in
// the order 0-3, 8-11, 4-7, 12-15 in which that kernel's probabilities come
// out of its score accumulators.
__host__ __device__ constexpr uint32_t vt_pos(uint32_t k) { return (k & ~12u) | ((k & 4u) << 1) | ((k & 8u) >> 1); }

// ---- lane l and lane l ^ 32 (v_permlane32_swap: no LDS round trip) ----
// The swap exchanges lanes 32-63 of its first operand with lanes 0-31 of its
// second; with v in both, the two results hold (v[l], v[l ^ 32]) in some order.
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- GELU through erf ----
//
// x * Phi(x) with Phi from erfc(|x| / sqrt 2) / 2, erfc by Abramowitz and
// Stegun, Handbook of Mathematical Functions, formula 7.1.26 (|error| <=
// 1.5e-7), the method and constants the reference's kernels use
// (crates/beatlm-core/src/kernel.rs:335-372, codegen/wgsl.rs:331-353). The
// negative side is a product, so nothing cancels.
__device__ __forceinline__ float gelu_erf(float x) {
    const float p = 0.3275911f;
    const float a1 = 0.254829592f, a2 = -0.284496736f, a3 = 1.421413741f,
                a4 = -1.453152027f, a5 = 1.061405429f;
    float z = fabsf(x) * 0.70710678118654752f;
    float t = __builtin_amdgcn_rcpf(1.0f + p * z);  // 1 ulp; 1 + p z >= 1, no denormals
    float poly = t * (a1 + t * (a2 + t * (a3 + t * (a4 + t * a5))));
    float q = 0.5f * poly * __expf(-z * z);
    return x * (x >= 0.0f ? 1.0f - q : q);
}

// GELU, tanh approximation (OpKind::Gelu, kernel.rs:934-942).
__device__ __forceinline__ float gelu_tanh(float x) {
    float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    u = fminf(fmaxf(u, -15.0f), 15.0f);
    return 0.5f * x * (1.0f + tanhf(u));
}

// ---- epilogue: the spec's element-wise steps, in order, at an output index ----



template <typename T>
__device__ __forceinline__ float apply_epilogue(const EpilogueArgs &e, float v, uint64_t index) {
    for (int s = 0; s < e.n; s++) {
        switch (e.kind[s]) {
        case BL_EPI_ADD: v = v + to_f32(((const T *)e.operand[s])[index]); break;
        case BL_EPI_RELU: v = fmaxf(v, 0.0f); break;
        case BL_EPI_GELU: v = gelu_tanh(v); break;
        case BL_EPI_GELU_ERF: v = gelu_erf(v); break;
        case BL_EPI_SCALE: v = v * e.factor[s]; break;
        case BL_EPI_CHANNEL_SCALE:
            v = v * to_f32(((const T *)e.operand[s])[index % e.channels[s]]);
            break;
        default: break;
        }
    }
    return v;
}

// ---- splitting an f32 into two bf16s (hi + lo) ----
//
// hi = bf16(x), lo = bf16(x - hi): x - hi - lo is within 2^-16 |x|, so the
// three products hi*hi + hi*lo + lo*hi of two split operands reproduce an f32
// product to about 2^-15 relative (Henry, Tang and Heinecke, "Leveraging the
// bfloat16 artificial intelligence datatype for higher-precision
// computations", ARITH 2019).
__device__ __forceinline__ void split_bf16(float x, __bf16 &hi, __bf16 &lo) {
    hi = (__bf16)x;
    lo = (__bf16)(x - (float)hi);
}
// The same split for two values at once: each conversion then rounds a pair
// (v_cvt_pk_bf16_f32), the same roundings as two split_bf16 calls.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split2_bf16(float a, float b, bf16x2 &hi, bf16x2 &lo) {
    const f32x2 v = {a, b};
    hi = __builtin_convertvector(v, bf16x2);
    lo = __builtin_convertvector(v - __builtin_convertvector(hi, f32x2), bf16x2);
}
// Eight values (v[0..7]) into hi and lo bf16x8 operands.
__device__ __forceinline__ void split8_bf16(const float (&v)[8], bf16x8 &hi, bf16x8 &lo) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        bf16x2 h, l;
        split2_bf16(v[e], v[e + 1], h, l);
        hi[e] = h[0];
        hi[e + 1] = h[1];
        lo[e] = l[0];
        lo[e + 1] = l[1];
    }
}


// ---- f32 activations kept as hi and lo bf16 planes ----
//
// An activation the host never reads and that bf16x3 GEMMs read only as their
// A operand is stored split, as the GEMM would split it: element i's hi part
// at ((__bf16 *)base)[i] and its lo part `planes` elements further on
// (planes = the tensor's element count, so the two planes fill the f32
// tensor's bytes). planes == 0: plain f32 (or f16) storage.
template <typename T>
__device__ __forceinline__ void store_elem(T *base, uint64_t i, float v, uint64_t planes) {
    if constexpr (sizeof(T) == 4) {
        if (planes) {
            __bf16 h, l;
            split_bf16(v, h, l);
            ((__bf16 *)base)[i] = h;
            ((__bf16 *)base)[planes + i] = l;
            return;
        }
    }
    base[i] = from_f32<T>(v);
}
__device__ __forceinline__ void store_f32x4(float *base, uint64_t i, f32x4 v, uint64_t planes) {
    if (planes) {
        bf16x4 h, l;
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
            bf16x2 hh, ll;
            split2_bf16(v[e], v[e + 1], hh, ll);
            h[e] = hh[0];
            h[e + 1] = hh[1];
            l[e] = ll[0];
            l[e + 1] = ll[1];
        }
        *(bf16x4 *)((__bf16 *)base + i) = h;
        *(bf16x4 *)((__bf16 *)base + planes + i) = l;
    } else {
        *(f32x4 *)(base + i) = v;
    }
}

// ---- direct HBM/L2 -> LDS staging (global_load_lds_dwordx4) ----

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt in [3:0] and
// [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// The slot a chunk occupies in its staged row.
//
// LDS serves 64 banks of 4 bytes; a 16-byte read by 16 lanes is conflict-free
// when their (row, slot) pairs cover 256 distinct bytes modulo 256. Rows of
// 4 chunks (64 B) repeat every 4 rows, rows of 8 every 2, rows of 16 every
// row, so the slot is XORed with the row bits above that period.
template <int CPR>
__device__ __forceinline__ int swz(int row, int chunk) {
    if constexpr (CPR == 4) return chunk ^ ((row >> 2) & 3);
    else if constexpr (CPR == 8) return chunk ^ ((row >> 1) & 7);
    else return chunk ^ (row & 15);
}

// One operand's direct loads for one stage: ROWS rows of CPR 16-byte chunks,
// spread over the NWAVES waves of the workgroup in lane order. The lane's byte offsets from the
// operand's tile base (its row, clamped to `row_limit`, and its swizzled
// chunk) are computed once; a stage then costs one address add per load.
//
// With `halves` set (the bytes from one plane to another), a staged row is
// two planes side by side: its chunks 0 .. CPR/2-1 come from the first plane
// and CPR/2 .. CPR-1 from the same row of the second.
template <int ROWS, int CPR, int NWAVES = 4>
struct RowLoader {
    static constexpr int TOTAL = ROWS * CPR;
    static constexpr int PER_WAVE = TOTAL / NWAVES;
    static constexpr int INSTR = (PER_WAVE + 63) / 64;
    static_assert(TOTAL % NWAVES == 0, "chunks per wave");
    uint32_t off[INSTR];
    bool active[INSTR];
    int wave;

    __device__ __forceinline__ RowLoader(uint32_t row_stride_bytes, uint32_t row_limit, int wave_, int lane,
                                         uint32_t halves = 0)
        : wave(wave_) {
#pragma unroll
        for (int q = 0; q < INSTR; q++) {
            const int li = q * 64 + lane;
            const int i = wave * PER_WAVE + li;
            const int row = i / CPR, slot = i % CPR;
            const uint32_t r = min((uint32_t)row, row_limit);
            const int c = swz<CPR>(row, slot);
            off[q] = r * row_stride_bytes + (halves ? (c % (CPR / 2)) * 16 + (c / (CPR / 2)) * halves : c * 16);
            active[q] = li < PER_WAVE;
        }
    }
    __device__ __forceinline__ void issue(const char *base, char *lds) const {
#pragma unroll
        for (int q = 0; q < INSTR; q++) {
            if (active[q])
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(base + off[q]),
                                                 (__attribute__((address_space(3))) void *)(lds + (wave * PER_WAVE + q * 64) * 16),
                                                 16, 0, 0);
        }
    }
};

template <int ROWS, int CPR, int NWAVES = 4>
constexpr int loads_per_wave() { return ((ROWS * CPR / NWAVES) + 63) / 64; }

}  // namespace bl

// Device-side building blocks shared by the gfx950 attention kernels: storage dtypes, 16-byte operand loads,
// MFMA wrappers, cross-lane reductions and the key-attendance predicate.
//
// MFMA fragment conventions (CDNA 16x16x32, wave64). For D = A * B with A [16 x 32], B [32 x 16]:
//   A: lane l holds A[l % 16][8 * (l / 16) + e], e = 0..7   (one 16-byte register quad)
//   B: lane l holds B[8 * (l / 16) + e][l % 16]
//   D: lane l holds D[4 * (l / 16) + i][l % 16], i = 0..3
// The kernels compute S^T = K * Q^T (keys on M, query rows on N) and O^T = V^T * P^T (head dims on M, rows on N),
// so a query row always lives in lanes with l % 16 == row: its softmax statistics, its P fragment and its output
// accumulator sit in the same lanes and never move across lanes except for the 4-way row reduction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dgx {

enum DType : int { DT_FP32 = 0, DT_F16 = 1, DT_BF16 = 2 };   // same codes as KV_FP32/KV_F16/KV_BF16

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// Element storage type of a dtype code.
template <int DT> struct Elem;
template <> struct Elem<DT_FP32> { using T = float; };
template <> struct Elem<DT_F16> { using T = uint16_t; };
template <> struct Elem<DT_BF16> { using T = uint16_t; };

// MFMA operand precision for a KV dtype: an f16 cache runs f16 MFMA with its own bits, a bf16 cache bf16 MFMA,
// an fp32 cache is rounded (RN-even) to bf16 as the reference's flash path does (attention_flash.cuh:126-128).
template <int KVT> struct OpIsF16 { static constexpr bool value = (KVT == DT_F16); };

__device__ __forceinline__ uint16_t f32_to_op(float x, bool f16) {
    if (f16) { _Float16 h = (_Float16)x; return __builtin_bit_cast(uint16_t, h); }
    __bf16 b = (__bf16)x; return __builtin_bit_cast(uint16_t, b);
}
template <bool F16> __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)f32_to_op(a, F16) | ((uint32_t)f32_to_op(b, F16) << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
template <int DT> __device__ __forceinline__ float elem_to_f32(typename Elem<DT>::T v) {
    if constexpr (DT == DT_FP32) return v;
    else if constexpr (DT == DT_F16) return f16_bits_to_f32(v);
    else return bf16_bits_to_f32(v);
}

// 8 consecutive elements of a DT array -> one 16-byte MFMA operand of precision F16 (f16) or !F16 (bf16).
template <int DT, bool F16>
__device__ __forceinline__ u32x4 load8_op(const typename Elem<DT>::T *p) {
    if constexpr (DT == DT_FP32) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(p), b = *(reinterpret_cast<const f32x4 *>(p) + 1);
        u32x4 r;
        r.x = pack2<F16>(a.x, a.y); r.y = pack2<F16>(a.z, a.w);
        r.z = pack2<F16>(b.x, b.y); r.w = pack2<F16>(b.z, b.w);
        return r;
    } else if constexpr ((DT == DT_F16) == F16) {
        return *reinterpret_cast<const u32x4 *>(p);                       // same 16-bit format: raw bits
    } else {
        const u32x4 raw = *reinterpret_cast<const u32x4 *>(p);            // the other 16-bit format: convert
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = raw[i];
            const float lo = elem_to_f32<DT>((uint16_t)(w & 0xffffu)), hi = elem_to_f32<DT>((uint16_t)(w >> 16));
            r[i] = pack2<F16>(lo, hi);
        }
        return r;
    }
}

template <bool F16>
__device__ __forceinline__ f32x4 mfma16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <bool F16>
__device__ __forceinline__ f32x16 mfma32(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Reductions across the four 16-lane groups that hold one query row (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float max_over_groups(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}
__device__ __forceinline__ float sum_over_groups(float v) {
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}
// Reductions across the two 32-lane halves (32x32 MFMA layout: a row lives in lanes l and l^32).
__device__ __forceinline__ float max_over_halves(float v) { return fmaxf(v, __shfl_xor(v, 32)); }
__device__ __forceinline__ float sum_over_halves(float v) { return v + __shfl_xor(v, 32); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Per-row attendance rule. Keys [lo, pos] with lo = max(0, pos - window + 1) (attention_decode_split.cuh:51);
// with a tree mask, key j >= tb is attended iff j - tb < 32 and bit (j - tb) of anc is set
// (attention_flash.cuh:177-178; there tb = base, the first tree node's position).
struct RowMask {
    int lo, pos, tb;
    uint32_t anc;
    bool tree, valid;
    __device__ __forceinline__ bool attends(int j) const {
        if (!valid || j < lo || j > pos) return false;
        if (!tree || j < tb) return true;
        const int d = j - tb;
        return d < 32 && ((anc >> d) & 1u);
    }
};

}  // namespace dgx

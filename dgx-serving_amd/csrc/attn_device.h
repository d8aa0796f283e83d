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
#include <type_traits>

namespace dgx {

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): compile-time indices into register arrays.
template <int I, int N, class F> __device__ __forceinline__ void static_for_(F &&f) {
    if constexpr (I < N) { f(std::integral_constant<int, I>{}); static_for_<I + 1, N>(f); }
}
template <int N, class F> __device__ __forceinline__ void static_for(F &&f) { static_for_<0, N>(f); }

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
constexpr float kPosInf = __builtin_inff();

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
// Two floats -> one packed pair (RN-even; a single v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32 on gfx950).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <bool F16> __device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (F16) { const f16x2 v = {(_Float16)a, (_Float16)b}; return __builtin_bit_cast(uint32_t, v); }
    else { const bf16x2 v = {(__bf16)a, (__bf16)b}; return __builtin_bit_cast(uint32_t, v); }
}
// Probabilities as the B operand of the PV MFMA. An f16 operand carries p to 11 significant bits (relative error
// <= 2^-12). A bf16 operand would carry 8 (2^-9: 4.5e-3 on an output of magnitude 2.5 from a two-key row), so for
// bf16 p is split into hi = RN_bf16(p) and lo = RN_bf16(p - hi) (p - hi is exact in fp32), fed to two MFMAs:
// hi + lo carries p to about 16 bits (relative error <= 2^-17).
template <bool F16> struct PFrag { u32x2 hi, lo; };
template <bool F16> __device__ __forceinline__ PFrag<F16> p_frag(float p0, float p1, float p2, float p3) {
    PFrag<F16> f;
    f.hi = u32x2{pack2<F16>(p0, p1), pack2<F16>(p2, p3)};
    if constexpr (!F16) {
        const float h0 = __uint_as_float(f.hi[0] << 16), h1 = __uint_as_float(f.hi[0] & 0xffff0000u);
        const float h2 = __uint_as_float(f.hi[1] << 16), h3 = __uint_as_float(f.hi[1] & 0xffff0000u);
        f.lo = u32x2{pack2<F16>(p0 - h0, p1 - h1), pack2<F16>(p2 - h2, p3 - h3)};
    } else {
        f.lo = u32x2{0u, 0u};
    }
    return f;
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

// The same from a streamed-once source (K/V in decode): non-temporal loads, which keep the caches for data that is
// reused and sustain a higher HBM read rate.
template <int DT, bool F16>
__device__ __forceinline__ u32x4 load8_op_stream(const typename Elem<DT>::T *p) {
    if constexpr (DT == DT_FP32) {
        const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
        const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p) + 1);
        u32x4 r;
        r.x = pack2<F16>(a.x, a.y); r.y = pack2<F16>(a.z, a.w);
        r.z = pack2<F16>(b.x, b.y); r.w = pack2<F16>(b.z, b.w);
        return r;
    } else if constexpr ((DT == DT_F16) == F16) {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    } else {
        const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
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

// 16x16x16 MFMA: A lane l holds A[l % 16][4 * (l / 16) + e], B lane l holds B[4 * (l / 16) + e][l % 16], e = 0..3;
// D as for 16x16x32.
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
template <bool F16>
__device__ __forceinline__ f32x4 mfma16k16(const u32x2 &a, const u32x2 &b, const f32x4 &c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}


// acc += V^T P^T over 16 keys with the P fragment split as above. f16: one 16x16x16 MFMA. bf16: hi and lo share one
// 16x16x32 MFMA, whose reduction runs over (the lane's 4 keys with hi, the same 4 keys with lo) against the V
// fragment given twice: on gfx950 a 16x16x32 issues in the time of a 16x16x16, so the lo products cost nothing.
// PACK = false keeps two 16x16x16 MFMAs (fewer live operand registers, for kernels at the register limit).
template <bool F16, bool PACK = true>
__device__ __forceinline__ f32x4 mfma_pv16(const u32x2 &v, const PFrag<F16> &p, f32x4 c) {
    if constexpr (F16) return mfma16k16<F16>(v, p.hi, c);
    else if constexpr (PACK) return mfma16<F16>(u32x4{v[0], v[1], v[0], v[1]}, u32x4{p.hi[0], p.hi[1], p.lo[0], p.lo[1]}, c);
    else return mfma16k16<F16>(v, p.lo, mfma16k16<F16>(v, p.hi, c));
}
// The 16x16x32 form over two sub-tiles: B = (P of sub-tile 0, P of sub-tile 1) in k-groups of 4 keys.
template <bool F16>
__device__ __forceinline__ f32x4 mfma_pv32(const u32x4 &v, const PFrag<F16> &p0, const PFrag<F16> &p1, f32x4 c) {
    c = mfma16<F16>(v, u32x4{p0.hi[0], p0.hi[1], p1.hi[0], p1.hi[1]}, c);
    if constexpr (!F16) c = mfma16<F16>(v, u32x4{p0.lo[0], p0.lo[1], p1.lo[0], p1.lo[1]}, c);
    return c;
}
// The hi and lo halves of mfma_pv32 on their own (the same two products in the same order), so that a batch of
// independent accumulators can issue all hi products before the lo products that depend on them.
template <bool F16>
__device__ __forceinline__ f32x4 mfma_pv32_hi(const u32x4 &v, const PFrag<F16> &p0, const PFrag<F16> &p1, f32x4 c) {
    return mfma16<F16>(v, u32x4{p0.hi[0], p0.hi[1], p1.hi[0], p1.hi[1]}, c);
}
template <bool F16>
__device__ __forceinline__ f32x4 mfma_pv32_lo(const u32x4 &v, const PFrag<F16> &p0, const PFrag<F16> &p1, f32x4 c) {
    if constexpr (!F16) c = mfma16<F16>(v, u32x4{p0.lo[0], p0.lo[1], p1.lo[0], p1.lo[1]}, c);
    return c;
}

// LDS transpose read (gfx950 ds_read_b64_tr_b16). Within each 16-lane group g, lane i passes the address of
// row 4g + i/4, columns 4*(i%4)..+3 of a row-major 16-bit tile; lane n of the group receives column n of
// rows 4g..4g+3. With rows = keys and columns = head dims this is the A fragment of O^T += V^T P^T for a
// 16x16x16 MFMA, straight from a row-major V tile.
typedef short lds_s4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t *p) {
    const lds_s4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) lds_s4 *)(reinterpret_cast<uintptr_t>(p)));
    return __builtin_bit_cast(u32x2, r);
}

// Buffer resource of a raw byte range [base, base + bytes) (no stride, no swizzle): buffer loads at vector
// offsets past `bytes` return zeros instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    // wave-uniform operands (readfirstlane), so the resource lives in SGPRs and no waterfall loop is generated
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(u), (short)0,
                                             __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000);
}
// 16 bytes per lane from buffer offset voffset into LDS at lds + 16 * lane (gfx950 buffer_load_dwordx4 ... lds).
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void *lds, int voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(reinterpret_cast<uintptr_t>(lds)),
                                             16, voffset, 0, 0, 0);
}

// Online-softmax rescale threshold (log2 units): the running reference max of a row moves only when a new score
// exceeds it by more than this, so unnormalised probabilities stay <= 2^8 and the accumulator is rescaled on a
// handful of tiles instead of every tile.
constexpr float kRescaleThreshold = 8.0f;

// Reductions across the four 16-lane groups that hold one query row (lanes l, l^16, l^32, l^48), on the VALU:
// gfx950's v_permlane16_swap / v_permlane32_swap hand every lane the (even row, odd row) and (low half,
// high half) pair of a value, so each step is one op and all four lanes combine the operands in the same order
// (bit-identical results).
__device__ __forceinline__ float max_over_groups(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
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

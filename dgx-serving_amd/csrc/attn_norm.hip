// Per-head RMSNorm (+ RoPE) (+ store in the KV dtype) on gfx950: the producer side of the KV cache.
//
// Replaces launch_norm_rope_store<TO> / norm_rope_store_kernel (kernels/norm_fused.cuh:84-133), which the Gemma4
// decoders call for q (into scratch), k (norm + RoPE into the cache) and v (norm without scale into the cache)
// (models/gemma4_decode.cu:340,353-354; models/gemma4_batch.cu:142,153,477,486).
//
// Row r = (token s = r / NH, head h = r % NH) of hd fp32 values. One wave64 per row, four rows per workgroup:
// lane l holds the float4 chunks l, l + 64, ... of the row (hd / 4 chunks), so the whole row lives in registers
// (LDS holds a row only for the rotation partners of head dims whose partner is not in a register, see RoPE).
//   * RMS: each lane sums the squares of its chunks in order, the wave adds the 64 lane sums with a fixed
//     butterfly; the order depends only on hd, so a row's bits do not depend on how many rows share the launch.
//     inv = rsqrt(ss / hd + eps); y = (x * inv) * W (two roundings, as the reference's norm_par_mul).
//   * RoPE (rotate-half): element e < hd/2 pairs with e + hd/2. For hd 512 and 1024 the partner chunk sits in the
//     same lane (chunk index + hd/512); for power-of-two hd up to 256 it sits in lane l ^ (hd/8), one cross-lane
//     swap; any other hd (a multiple of 4) takes its partners from the row staged in the wave's LDS slice. The
//     products and the difference / sum are rounded separately: o = t1*c - t2*s, o' = t2*c + t1*s with cos/sin
//     from the row p of the tables (entries [p*hd, p*hd + hd/2)). This is a deliberate choice, not a copy of the
//     reference's rounding: the reference writes the same expressions (norm_fused.cuh:119-120) but its compiler
//     may contract one product into an FMA, so its fp32 results can differ from these by about one ulp; the
//     tests compare against the fp64 oracle.
//   * Store: p = pos_arr ? pos_arr[s] : base + s * pos_step, row at Y + s*slot_stride + p*row_stride + h*hd, in
//     fp32 or rounded to nearest-even f16 / bf16 (as kv_store_kernel converts).
#include "attn_device.h"
#include "attn_internal.h"

namespace dgx {

__device__ __forceinline__ float wave_sum64(float v) {
    // butterfly over the 64 lanes (bit-identical result in every lane)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int DT, bool ROPE, int NV, bool GEN = false>
__global__ void __launch_bounds__(256) norm_rope_store_kernel(const float *X, const float *W, void *Y, int rows, int NH,
                                                              int hd, float eps, const float *cosT, const float *sinT,
                                                              int base, int pos_step, const int *pos_arr,
                                                              long slot_stride, long row_stride) {
    const int lane = threadIdx.x & 63;
    const int r = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (r >= rows) return;                                             // wave-uniform
    const int s = r / NH, h = r % NH, n4 = hd >> 2;
    const float *xr = X + (size_t)r * hd;
    const long p = pos_arr ? (long)pos_arr[s] : (long)base + (long)s * pos_step;
    // every load of the row goes out before any arithmetic: x, the scale W and this lane's cos / sin entries
    // (element e takes table entry e mod hd/2; four consecutive elements, one 16-byte load each)
    const int half = hd >> 1;
    f32x4 v[NV], wv[NV], cv[NV], sv[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int c = lane + 64 * k;
        v[k] = wv[k] = cv[k] = sv[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (c < n4) {
            v[k] = *reinterpret_cast<const f32x4 *>(xr + 4 * c);
            if (W) wv[k] = *reinterpret_cast<const f32x4 *>(W + 4 * c);
            if constexpr (ROPE && !GEN) {
                const int t = (4 * c) % half;
                cv[k] = *reinterpret_cast<const f32x4 *>(cosT + p * hd + t);
                sv[k] = *reinterpret_cast<const f32x4 *>(sinT + p * hd + t);
            }
            if constexpr (ROPE && GEN) {                           // a chunk may straddle the halves: per element
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int e = 4 * c + q, t = e < half ? e : e - half;
                    cv[k][q] = cosT[p * hd + t];
                    sv[k][q] = sinT[p * hd + t];
                }
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        ss += v[k].x * v[k].x; ss += v[k].y * v[k].y; ss += v[k].z * v[k].z; ss += v[k].w * v[k].w;
    }
    ss = wave_sum64(ss);
    const float inv = rsqrtf(ss / (float)hd + eps);
    f32x4 y[NV];
#pragma unroll
    for (int k = 0; k < NV; k++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float t = __fmul_rn(v[k][q], inv);
            y[k][q] = W ? __fmul_rn(t, wv[k][q]) : t;
        }
    f32x4 o[NV];
    if constexpr (ROPE && GEN) {
        // partners through this wave's slice of the row buffer (hd floats per wave)
        __shared__ float ys[4][1024];
        float *yw = ys[threadIdx.x >> 6];
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int c = lane + 64 * k;
            if (c < n4) *reinterpret_cast<f32x4 *>(yw + 4 * c) = y[k];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");          // the wave's row is in LDS before any lane
        __builtin_amdgcn_wave_barrier();                             // reads its partner (no workgroup barrier:
                                                                     // waves past the last row have returned)
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int c = lane + 64 * k;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int e = 4 * c + q;
                const bool lo = e < half;
                const float pr = c < n4 ? yw[lo ? e + half : e - half] : 0.f;
                o[k][q] = lo ? __fsub_rn(__fmul_rn(y[k][q], cv[k][q]), __fmul_rn(pr, sv[k][q]))
                             : __fadd_rn(__fmul_rn(y[k][q], cv[k][q]), __fmul_rn(pr, sv[k][q]));
            }
        }
    } else if constexpr (ROPE) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            f32x4 pr;                                                  // the partner chunk's values
            if constexpr (NV >= 2) {
                constexpr int KH = NV / 2;                             // hd >= 512: chunk index +- hd/512, same lane
                pr = y[k < KH ? k + KH : k - KH];
            } else {
                const int m = hd >> 3;                                 // hd <= 256: lane l ^ (hd / 8)
#pragma unroll
                for (int q = 0; q < 4; q++) pr[q] = __shfl_xor(y[0][q], m);
            }
            const bool lo = 4 * (lane + 64 * k) < half;                // the chunk lies in one half (half % 4 == 0)
#pragma unroll
            for (int q = 0; q < 4; q++)
                o[k][q] = lo ? __fsub_rn(__fmul_rn(y[k][q], cv[k][q]), __fmul_rn(pr[q], sv[k][q]))
                             : __fadd_rn(__fmul_rn(y[k][q], cv[k][q]), __fmul_rn(pr[q], sv[k][q]));
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV; k++) o[k] = y[k];
    }
    const size_t ob = (size_t)((long)s * slot_stride + p * row_stride + (long)h * hd);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int c = lane + 64 * k;
        if (c >= n4) continue;
        if constexpr (DT == DT_FP32) {
            *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(Y) + ob + 4 * c) = o[k];
        } else {
            constexpr bool F16 = DT == DT_F16;
            *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(Y) + ob + 4 * c) =
                u32x2{pack2<F16>(o[k].x, o[k].y), pack2<F16>(o[k].z, o[k].w)};
        }
    }
}

bool norm_rope_shape_ok(int hd, bool rope) {
    (void)rope;                                      // every hd below has a rotate-half partner layout
    return hd > 0 && hd % 4 == 0 && hd <= 1024;
}

// Rotate-half partners in registers: the same lane (hd 512, 1024) or a lane XOR (power-of-two hd up to 256).
static bool rope_in_registers(int hd) { return hd == 512 || hd == 1024 || (hd >= 8 && hd <= 256 && (hd & (hd - 1)) == 0); }

template <int DT, bool ROPE>
static hipError_t launch_nrs_t(const float *X, const float *W, void *Y, int rows, int NH, int hd, float eps,
                               const float *cosT, const float *sinT, int base, int pos_step, const int *pos_arr,
                               long slot_stride, long row_stride, hipStream_t st) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (ROPE && !rope_in_registers(hd)) {
        if (hd <= 256)
            hipLaunchKernelGGL((norm_rope_store_kernel<DT, ROPE, 1, true>), grid, dim3(256), 0, st, X, W, Y, rows, NH, hd,
                               eps, cosT, sinT, base, pos_step, pos_arr, slot_stride, row_stride);
        else if (hd <= 512)
            hipLaunchKernelGGL((norm_rope_store_kernel<DT, ROPE, 2, true>), grid, dim3(256), 0, st, X, W, Y, rows, NH, hd,
                               eps, cosT, sinT, base, pos_step, pos_arr, slot_stride, row_stride);
        else
            hipLaunchKernelGGL((norm_rope_store_kernel<DT, ROPE, 4, true>), grid, dim3(256), 0, st, X, W, Y, rows, NH, hd,
                               eps, cosT, sinT, base, pos_step, pos_arr, slot_stride, row_stride);
        return hipGetLastError();
    }
    if (hd <= 256)
        hipLaunchKernelGGL((norm_rope_store_kernel<DT, ROPE, 1>), grid, dim3(256), 0, st, X, W, Y, rows, NH, hd, eps, cosT,
                           sinT, base, pos_step, pos_arr, slot_stride, row_stride);
    else if (hd <= 512)
        hipLaunchKernelGGL((norm_rope_store_kernel<DT, ROPE, 2>), grid, dim3(256), 0, st, X, W, Y, rows, NH, hd, eps, cosT,
                           sinT, base, pos_step, pos_arr, slot_stride, row_stride);
    else
        hipLaunchKernelGGL((norm_rope_store_kernel<DT, ROPE, 4>), grid, dim3(256), 0, st, X, W, Y, rows, NH, hd, eps, cosT,
                           sinT, base, pos_step, pos_arr, slot_stride, row_stride);
    return hipGetLastError();
}

hipError_t launch_norm_rope_store(const float *X, const float *W, void *Y, int y_dtype, int rows, int NH, int hd,
                                  float eps, const float *cosT, const float *sinT, int base, int pos_step,
                                  const int *pos_arr, long slot_stride, long row_stride, bool rope, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    if (rows < 0 || NH <= 0 || !X || !Y || !norm_rope_shape_ok(hd, rope) || (rope && (!cosT || !sinT)))
        return hipErrorInvalidValue;
    if (rows > 0x7ffffff0) return hipErrorInvalidConfiguration;
#define DGX_NRS(DT)                                                                                                     \
    return rope ? launch_nrs_t<DT, true>(X, W, Y, rows, NH, hd, eps, cosT, sinT, base, pos_step, pos_arr, slot_stride,  \
                                         row_stride, st)                                                                \
                : launch_nrs_t<DT, false>(X, W, Y, rows, NH, hd, eps, cosT, sinT, base, pos_step, pos_arr, slot_stride, \
                                          row_stride, st)
    switch (y_dtype) {
    case DT_FP32: DGX_NRS(DT_FP32);
    case DT_F16: DGX_NRS(DT_F16);
    case DT_BF16: DGX_NRS(DT_BF16);
    default: return hipErrorInvalidValue;
    }
#undef DGX_NRS
}

}  // namespace dgx

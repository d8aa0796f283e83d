// fp32 attention for fp32 KV caches, and the KV storage conversion kernel.
//
// Replaces attn_kernel / attn_decode_kernel / attn_decode_batch_kernel (kernels/attention.cuh:33-187) and
// serves launch_attn_decode_split on an fp32 cache (attention_decode_split.cuh:228), where the reference
// computes in fp32 FMA and its gate asks for a 1e-5 normalised error (tests/test_attn_decode_split.cu:87).
// Unlike the reference kernels this one keeps no full score row in shared memory: keys are consumed in
// 256-key chunks with an online softmax, so there is no context-length limit and no shared-memory guard
// (attention.cuh:13-24) is needed.
//
// One workgroup (256 threads) per (query row, q-head). Per chunk: thread j scores key j0+j (fp32 FMA over the
// head dims in increasing order, q in LDS), the chunk max and sum are workgroup reductions, then thread d
// accumulates sum_j p_j V[j][d] over the chunk's keys in increasing (or, with reverse, decreasing) order.
#include "attn_device.h"
#include "attn_internal.h"
#include <cfloat>

namespace dgx {

struct ScalarArgs {
    const float *Q, *K, *V;
    float *O;
    int nseq, T, NQ, NKV, HD;
    long kv_stride;
    int pos_mode, base, pos_step;   // as Problem
    const int *pos_arr;
    float scale;
    int window, reverse;
};

__device__ __forceinline__ int scalar_pos(const ScalarArgs &a, int s, int t) {
    if (a.pos_mode == 0) { const int r = s * a.T + t; return a.pos_arr ? a.pos_arr[r] : a.base + r * a.pos_step; }
    return (a.pos_arr ? a.pos_arr[s] : a.base) + t;
}

__device__ __forceinline__ float block_max(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6, ln = threadIdx.x & 63;
    __syncthreads();
    if (ln == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmaxf(r, red[i]);
    return r;
}
__device__ __forceinline__ float block_sum(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6, ln = threadIdx.x & 63;
    __syncthreads();
    if (ln == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r += red[i];
    return r;
}

__global__ void __launch_bounds__(256) scalar_attn_kernel(const ScalarArgs a) {
    constexpr int CH = 256;
    __shared__ float qs[512], ps[CH], red[4];
    const int r = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int s = r / a.T, t = r % a.T, HD = a.HD;
    const int GRP = a.NQ / a.NKV, kvh = h / GRP;
    const int pos = scalar_pos(a, s, t);
    const int lo = (a.window > 0 && pos - a.window + 1 > 0) ? pos - a.window + 1 : 0;
    const float *K = a.K + (size_t)s * a.kv_stride + (size_t)kvh * HD;
    const float *V = a.V + (size_t)s * a.kv_stride + (size_t)kvh * HD;
    const size_t krow = (size_t)a.NKV * HD;
    for (int d = tid; d < HD; d += 256) qs[d] = a.Q[((size_t)r * a.NQ + h) * HD + d];
    __syncthreads();
    float m = -FLT_MAX, l = 0.f, acc0 = 0.f, acc1 = 0.f;
    const int nch = (pos - lo) / CH + 1;
    for (int ci = 0; ci < nch; ci++) {
        const int c = a.reverse ? nch - 1 - ci : ci;
        const int j0 = lo + c * CH, j1 = min(pos + 1, j0 + CH);
        const int j = j0 + tid;
        float sc = -FLT_MAX;
        if (j < j1) {
            const float *kp = K + (size_t)j * krow;
            float dot = 0.f;
            for (int d = 0; d < HD; d++) dot = fmaf(qs[d], kp[d], dot);
            sc = dot * a.scale;
        }
        const float mc = block_max(sc, red);
        const float mn = fmaxf(m, mc), alpha = expf(m - mn);
        const float p = (j < j1) ? expf(sc - mn) : 0.f;
        ps[tid] = p;
        const float sum = block_sum(p, red);
        l = l * alpha + sum; m = mn; acc0 *= alpha; acc1 *= alpha;
        __syncthreads();
        const int n = j1 - j0;
        if (tid < HD) {
            if (a.reverse) for (int k = n - 1; k >= 0; k--) acc0 = fmaf(ps[k], V[(size_t)(j0 + k) * krow + tid], acc0);
            else for (int k = 0; k < n; k++) acc0 = fmaf(ps[k], V[(size_t)(j0 + k) * krow + tid], acc0);
        }
        if (tid + 256 < HD) {
            if (a.reverse) for (int k = n - 1; k >= 0; k--) acc1 = fmaf(ps[k], V[(size_t)(j0 + k) * krow + tid + 256], acc1);
            else for (int k = 0; k < n; k++) acc1 = fmaf(ps[k], V[(size_t)(j0 + k) * krow + tid + 256], acc1);
        }
        __syncthreads();
    }
    float *o = a.O + ((size_t)r * a.NQ + h) * HD;
    if (tid < HD) o[tid] = acc0 / l;
    if (tid + 256 < HD) o[tid + 256] = acc1 / l;
}

static hipError_t launch_scalar(const ScalarArgs &a, hipStream_t st) {
    if (a.HD <= 0 || a.HD > 512 || a.NQ % a.NKV) return hipErrorInvalidValue;
    dim3 grid(a.nseq * a.T, a.NQ);
    if (grid.y > 65535u) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(scalar_attn_kernel, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_scalar_prefill(const float *Q, const float *K, const float *V, float *O, int S, int NQ, int NKV,
                                 int HD, float scale, int window, hipStream_t st) {
    ScalarArgs a{Q, K, V, O, 1, S, NQ, NKV, HD, 0, 1, 0, 1, nullptr, scale, window, 0};
    return launch_scalar(a, st);
}

// nseq sequences x Sq tokens; token t of sequence s sits at (base_b ? base_b[s] : base) + t.
hipError_t launch_scalar_decode(const float *Q, const float *Kc, const float *Vc, float *O, int nseq, int Sq,
                                int NQ, int NKV, int HD, int base, long kv_stride, const int *base_b, float scale,
                                int window, int reverse, hipStream_t st) {
    ScalarArgs a{Q, Kc, Vc, O, nseq, Sq, NQ, NKV, HD, kv_stride, 1, base, 1, base_b, scale, window, reverse};
    return launch_scalar(a, st);
}

// Decode-split rows on an fp32 cache: pos_mode 0 (pos_arr[r] or base + r*pos_step), KV of row r at r*kv_stride.
hipError_t launch_scalar_rows(const float *Q, const float *Kc, const float *Vc, float *O, int rows, int NQ, int NKV,
                              int HD, int base, int pos_step, const int *pos_arr, long kv_stride, float scale,
                              int window, int reverse, hipStream_t st) {
    ScalarArgs a{Q, Kc, Vc, O, rows, 1, NQ, NKV, HD, kv_stride, 0, base, pos_step, pos_arr, scale, window, reverse};
    return launch_scalar(a, st);
}

// ---------------------------------------------------------------- KV storage conversion (kv_store.cuh:76-113)
// stats[0] / [1]: non-finite stored K / V values; [2] / [3]: bits of max |stored K| / |stored V|.
__device__ unsigned int g_kv_stats[4];

template <bool F16>
__global__ void __launch_bounds__(256) kv_store_kernel(const float *src, uint16_t *dst, size_t n, int stats, int which) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint16_t out = f32_to_op(src[i], F16);
    dst[i] = out;
    if (stats) {
        const float back = F16 ? f16_bits_to_f32(out) : bf16_bits_to_f32(out);
        if (!isfinite(back)) atomicAdd(&g_kv_stats[which], 1u);
        else atomicMax(&g_kv_stats[2 + which], __float_as_uint(fabsf(back)));
    }
}

// y[i] *= sigmoid(gate[i]) in place, fp32, with the factor 1 / (1 + 2^(-g log2 e)) of the fused output gate of the
// split path (the same float operations, so a separately gated output equals the fused one bit for bit). Four
// elements per thread with 16-byte accesses when both arrays are 16-byte aligned, else one.
template <bool VEC>
__global__ void __launch_bounds__(256) gate_sigmoid_kernel(float *y, const float *gate, size_t n) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * (VEC ? 4 : 1);
    if (i >= n) return;
    if (VEC && i + 4 <= n) {
        f32x4 v = *reinterpret_cast<const f32x4 *>(y + i);
        const f32x4 g = *reinterpret_cast<const f32x4 *>(gate + i);
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] *= 1.f / (1.f + fast_exp2(-g[e] * kLog2e));
        *reinterpret_cast<f32x4 *>(y + i) = v;
    } else {
        for (size_t j = i; j < n && j < i + (VEC ? 4 : 1); j++) y[j] *= 1.f / (1.f + fast_exp2(-gate[j] * kLog2e));
    }
}

hipError_t launch_gate_sigmoid(float *y, const float *gate, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const bool vec = ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(gate)) & 15) == 0;
    const size_t threads = vec ? (n + 3) / 4 : n;
    if ((threads + 255) / 256 > 0x7fffffffu) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (vec) hipLaunchKernelGGL(gate_sigmoid_kernel<true>, grid, dim3(256), 0, st, y, gate, n);
    else hipLaunchKernelGGL(gate_sigmoid_kernel<false>, grid, dim3(256), 0, st, y, gate, n);
    return hipGetLastError();
}

hipError_t launch_kv_store(const float *src, void *dst, size_t n, int kv_dtype, int which, int stats, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (which < 0 || which > 1) return hipErrorInvalidValue;
    if (kv_dtype == DT_FP32) return hipMemcpyAsync(dst, src, n * 4, hipMemcpyDeviceToDevice, st);
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (kv_dtype == DT_F16) hipLaunchKernelGGL(kv_store_kernel<true>, dim3(blocks), dim3(256), 0, st, src, (uint16_t *)dst, n, stats, which);
    else if (kv_dtype == DT_BF16) hipLaunchKernelGGL(kv_store_kernel<false>, dim3(blocks), dim3(256), 0, st, src, (uint16_t *)dst, n, stats, which);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// Ragged KV append: token t of sequence b (source row b*T + t of [nseq*T][row] fp32 K and V) goes to cache row
// pos(b) + t of sequence b (cache element b*kv_stride + (pos(b) + t)*row), converted as kv_store_kernel does.
// One thread per 4 consecutive elements (a 16-byte fp32 read); grid.y = 0 for K, 1 for V.
template <int DT>
__global__ void __launch_bounds__(256) kv_append_kernel(const float *ks, const float *vs, void *Kc, void *Vc, int T,
                                                        long kv_stride, int row, const int *pos_b, int base,
                                                        size_t groups, int stats) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= groups) return;
    const int which = blockIdx.y;
    const int gpr = row / 4;
    const size_t r = i / gpr, c = (i % gpr) * 4;
    const int b = (int)(r / T), t = (int)(r % T);
    const size_t o = (size_t)b * kv_stride + (size_t)((pos_b ? pos_b[b] : base) + t) * row + c;
    const f32x4 v = *reinterpret_cast<const f32x4 *>((which ? vs : ks) + r * row + c);
    void *dst = which ? Vc : Kc;
    if constexpr (DT == DT_FP32) {
        *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(dst) + o) = v;
    } else {
        constexpr bool F16 = DT == DT_F16;
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) h[e] = f32_to_op(v[e], F16);
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(dst) + o) =
            u32x2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
        if (stats) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float back = F16 ? f16_bits_to_f32(h[e]) : bf16_bits_to_f32(h[e]);
                if (!isfinite(back)) atomicAdd(&g_kv_stats[which], 1u);
                else atomicMax(&g_kv_stats[2 + which], __float_as_uint(fabsf(back)));
            }
        }
    }
}

hipError_t launch_kv_append(const float *ks, const float *vs, void *Kc, void *Vc, int kv_dtype, int nseq, int T,
                            long kv_stride, int row, const int *pos_b, int base, int stats, hipStream_t st) {
    if (nseq == 0 || T == 0) return hipSuccess;
    if (nseq < 0 || T < 0 || row <= 0 || row % 4 || kv_stride % 4 || kv_stride < 0 || base < 0)
        return hipErrorInvalidValue;
    const size_t groups = (size_t)nseq * T * (row / 4);
    const size_t blocks = (groups + 255) / 256;
    if (blocks > 0x7fffffffu) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)blocks, 2);
    switch (kv_dtype) {
    case DT_FP32: hipLaunchKernelGGL(kv_append_kernel<DT_FP32>, grid, dim3(256), 0, st, ks, vs, Kc, Vc, T, kv_stride, row, pos_b, base, groups, 0); break;
    case DT_F16: hipLaunchKernelGGL(kv_append_kernel<DT_F16>, grid, dim3(256), 0, st, ks, vs, Kc, Vc, T, kv_stride, row, pos_b, base, groups, stats); break;
    case DT_BF16: hipLaunchKernelGGL(kv_append_kernel<DT_BF16>, grid, dim3(256), 0, st, ks, vs, Kc, Vc, T, kv_stride, row, pos_b, base, groups, stats); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t read_kv_stats(unsigned out[4]) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_kv_stats), sizeof(unsigned) * 4, 0, hipMemcpyDeviceToHost);
}

}  // namespace dgx

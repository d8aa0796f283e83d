// Streaming split-KV GQA decode on gfx950: one query token per sequence, HD 128 or 256, up to 16 q-heads per KV
// head (the decode rows of kernels/attention_decode_split.cuh:43-145 and of the per-slot flash decode at
// models/qwen35_batch.cu:165-167).
//
// Grid: (kv head, key chunk of C keys, sequence). A workgroup owns the GRP query rows of one KV head and one
// chunk; its 4 wave64s take the chunk's 16-key tiles round-robin (wave w: tiles w, w+4, ...) and run fully
// independent online softmaxes, merged in wave order at the end. The main loop touches no LDS and has no
// barrier:
//   * K is read straight into MFMA A fragments (lane = key, 16 bytes of head dims per load),
//   * S^T = K Q^T on 16x16x32 MFMA (Q fragments come from LDS, staged once),
//   * V rows are read coalesced, staged in the wave's private LDS slice and read back with the gfx950 transpose
//     read (ds_read_b64_tr_b16) as the A fragments of O^T += V^T P^T on 16x16x16 MFMA; P^T comes straight from
//     the softmax registers. LDS carries 16 KB per 16-key tile and wave (V in and out) and needs no barrier.
//
// Chunk boundaries and tile positions are absolute and the wave that owns a tile depends only on its position,
// so a row's result is identical whatever the batch, grid or maximum position (batch row == single row).
#include "attn_device.h"
#include "attn_internal.h"
#include <climits>

namespace dgx {

struct DecodeArgs {
    Problem p;
    Partials part;
    int C;
    float sl2;
};

template <int HD>
struct DecodeCfg {
    static constexpr int NW = 4, KT = 16;
    static constexpr int KS = HD / 32;                 // 32-dim blocks (QK k-steps, V fragment loads)
    static constexpr int DB = HD / 16;                 // 16-dim output blocks
    static constexpr int QSTR = HD + 8;                // Q row stride in LDS (16-bit elements)
    static constexpr int BSTR = HD + 4;                // merge buffer row stride (floats)
    static constexpr int VSTR = HD + 8;                // V tile row stride in LDS (16-bit elements)
    static constexpr int VCH = KT * HD / 8 / 64;       // 16-byte V chunks per lane per tile
    static constexpr size_t LDS_Q = (size_t)16 * QSTR * 2;
    static constexpr size_t LDS_V = (size_t)NW * KT * VSTR * 2;     // one private V tile per wave
    static constexpr size_t LDS_MERGE = ((size_t)2 * NW * 16 + (size_t)16 * BSTR) * 4;
    static constexpr size_t LDS = LDS_Q + (LDS_V > LDS_MERGE ? LDS_V : LDS_MERGE);
};

#ifdef DGX_TRACE
__device__ unsigned long long g_dtrace[1 << 16][4];
__device__ unsigned long long g_ptrace[64][16][5];   // [wave slot][tile][phase] shader-clock stamps
extern "C" hipError_t dgx_dtrace_read(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_dtrace), bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" hipError_t dgx_ptrace_read(void *host, size_t bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_ptrace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

template <int HD, int KVT, int QT>
__global__ void __launch_bounds__(256) decode_stream_kernel(const DecodeArgs a) {
#ifdef DGX_TRACE
    const unsigned long long t_start = __builtin_amdgcn_s_memrealtime();
#endif
    using Cf = DecodeCfg<HD>;
    constexpr int NW = Cf::NW, KT = Cf::KT;
    constexpr bool F16 = OpIsF16<KVT>::value;
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];

    const Problem &p = a.p;
    const int kvh = blockIdx.x, c = blockIdx.y, seq = blockIdx.z;
    const int GRP = p.NQ / p.NKV;
    const int pos = tok_pos(p, seq, 0), lo = win_lo(pos, p.window), hi = pos + 1;
    const int C = a.C;
    const int j_lo = max(c * C, lo), j_hi = min(c * C + C, hi);
    if (j_lo >= j_hi) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, ln = lane & 15;
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = reinterpret_cast<const KE *>(p.K) + (size_t)seq * p.kv_stride + (size_t)kvh * HD;
    const KE *Vb = reinterpret_cast<const KE *>(p.V) + (size_t)seq * p.kv_stride + (size_t)kvh * HD;
    uint16_t *qs = reinterpret_cast<uint16_t *>(smem);
    float *redm = reinterpret_cast<float *>(smem + Cf::LDS_Q), *redl = redm + NW * 16, *buf = redl + NW * 16;
    uint16_t *vs = reinterpret_cast<uint16_t *>(smem + Cf::LDS_Q) + (size_t)wave * KT * Cf::VSTR;   // reused by the merge

    for (int i = tid; i < 16 * (HD / 8); i += NW * 64) {
        const int row = i / (HD / 8), col = (i % (HD / 8)) * 8;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (row < GRP)
            v = load8_op<QT, F16>(reinterpret_cast<const QE *>(p.Q) + ((size_t)seq * p.NQ + kvh * GRP + row) * HD + col);
        *reinterpret_cast<u32x4 *>(qs + row * Cf::QSTR + col) = v;
    }
    RowMask rm;
    rm.pos = pos; rm.lo = lo; rm.valid = ln < GRP; rm.tree = p.anc != nullptr;
    rm.anc = p.anc ? p.anc[seq] : 0u; rm.tb = pos;
    __syncthreads();

    float m = kNegInf, l = 0.f;
    f32x4 acc[Cf::DB];
#pragma unroll
    for (int db = 0; db < Cf::DB; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t *qrow = qs + ln * Cf::QSTR + 8 * g;
    // This wave's tiles: k = k0 .. k1-1 with tile k at key c*C + KT*(wave + NW*k), the ones meeting [j_lo, j_hi).
    const int tb0 = j_lo / KT - c * (C / KT), tb1 = (j_hi - 1) / KT - c * (C / KT);   // tile range in the chunk
    const int k0 = tb0 <= wave ? 0 : (tb0 - wave + NW - 1) / NW;
    const int k1 = tb1 < wave ? 0 : (tb1 - wave) / NW + 1;
    // Keys of a tile are attended without per-key tests when the tile lies inside [j_lo, j_hi) and below the tree.
    const int full_hi = min(j_hi, p.anc ? pos : INT_MAX);
    const KE *kp = Kb + (size_t)(c * C + KT * (wave + NW * k0) + ln) * krow + 8 * g;
    const KE *vp = Vb + (size_t)(c * C + KT * (wave + NW * k0) + ln) * krow + 8 * g;
    const size_t kstep = (size_t)KT * NW * krow;
#ifdef DGX_TRACE
    const int tslot = (blockIdx.z == 3 && blockIdx.x == 1 && blockIdx.y < 16) ? (int)blockIdx.y * 4 + wave : -1;
#define PT(ph) if (tslot >= 0 && lane == 0 && k - k0 < 16) g_ptrace[tslot][k - k0][ph] = __builtin_amdgcn_s_memtime();
#else
#define PT(ph)
#endif
    for (int k = k0; k < k1; k++, kp += kstep, vp += kstep) {
        const int jt = c * C + KT * (wave + NW * k);
        PT(0)
        const KE *kq = kp;
        if (jt + KT > hi) kq = Kb + (size_t)min(jt + ln, hi - 1) * krow + 8 * g;   // last tile: clamp to the last key
        u32x4 kf[Cf::KS], vr[Cf::VCH];
#pragma unroll
        for (int ks = 0; ks < Cf::KS; ks++) kf[ks] = load8_op<KVT, F16>(kq + 32 * ks);
        // V tile rows, coalesced (HD/8 lanes per key row), for the private LDS transpose.
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            vr[u] = load8_op<KVT, F16>(Vb + (size_t)min(jt + key, hi - 1) * krow + col);
        }
        // S^T[key jt + 4g + i][row ln], two independent MFMA chains.
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int ks = 0; ks < Cf::KS; ks++) {
            const u32x4 qf = *reinterpret_cast<const u32x4 *>(qrow + 32 * ks);
            if (ks & 1) s1 = mfma16<F16>(kf[ks], qf, s1);
            else s0 = mfma16<F16>(kf[ks], qf, s0);
        }
        const f32x4 s = (s0 + s1) * a.sl2;
        PT(1)
        // Online softmax (log2 domain), lazily moved reference max; l is this lane's share of the row sum.
        float tv[4];
        if (jt >= j_lo && jt + KT <= full_hi) {
#pragma unroll
            for (int i = 0; i < 4; i++) tv[i] = s[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = jt + 4 * g + i;
                const bool in = (key >= j_lo) & (key < j_hi) & rm.attends(key);
                tv[i] = in ? s[i] : kNegInf;
            }
        }
        float mx = fmaxf(fmaxf(tv[0], tv[1]), fmaxf(tv[2], tv[3]));
        mx = max_over_groups(mx);
        const float mnew = (mx > m + kRescaleThreshold) ? mx : m;
        if (__any(mnew != m)) {
            const float alpha = (mnew == m) ? 1.f : fast_exp2(m - mnew);
            l *= alpha; m = mnew;
#pragma unroll
            for (int db = 0; db < Cf::DB; db++) acc[db] *= alpha;
        }
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pv[i] = fast_exp2(tv[i] - m);   // exp2(-inf) = 0; m is finite once a key is seen
        if (m == kNegInf) pv[0] = pv[1] = pv[2] = pv[3] = 0.f;
        l += (pv[0] + pv[1]) + (pv[2] + pv[3]);
        const u32x2 pop = u32x2{pack2<F16>(pv[0], pv[1]), pack2<F16>(pv[2], pv[3])};
        PT(2)
        // O^T += V^T P^T (16x16x16): stage the V tile in this wave's LDS slice, read it back transposed.
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(vs + key * Cf::VSTR + col) = vr[u];
        }
        __builtin_amdgcn_wave_barrier();
        const uint16_t *vt = vs + (4 * g + (ln >> 2)) * Cf::VSTR + 4 * (ln & 3);
#pragma unroll
        for (int db = 0; db < Cf::DB; db++) acc[db] = mfma16k16<F16>(lds_read_tr16(vt + 16 * db), pop, acc[db]);
        __builtin_amdgcn_wave_barrier();
        PT(3)
    }
#undef PT
    l = sum_over_groups(l);
#ifdef DGX_TRACE
    if (lane == 0) {
        const size_t bid = (((size_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 4 + wave;
        unsigned xcc, hwid;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
        g_dtrace[bid & 0xffff][0] = t_start;
        g_dtrace[bid & 0xffff][1] = __builtin_amdgcn_s_memrealtime();
        g_dtrace[bid & 0xffff][2] = (j_hi - j_lo + 15) / 16;
        g_dtrace[bid & 0xffff][3] = (xcc & 0xf) | (((hwid >> 8) & 0xf) << 4) | (((hwid >> 12) & 0x7) << 8) | (((hwid >> 4) & 3) << 12);
    }
#endif

    // Merge the four wave states in wave order (LDS, over the V slices), then write the chunk partial of each row.
    __syncthreads();
    if (g == 0) { redm[wave * 16 + ln] = m; redl[wave * 16 + ln] = l; }
    __syncthreads();
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; w++) M = fmaxf(M, redm[w * 16 + ln]);
    const float f = (m == kNegInf) ? 0.f : fast_exp2(m - M);
    for (int w = 0; w < NW; w++) {
        if (wave == w && ln < GRP) {
#pragma unroll
            for (int db = 0; db < Cf::DB; db++) {
                f32x4 *dst = reinterpret_cast<f32x4 *>(buf + ln * Cf::BSTR + 16 * db + 4 * g);
                f32x4 v = acc[db] * f;
                if (w > 0) v += *dst;
                *dst = v;
            }
        }
        __syncthreads();
    }
    const int ns = a.part.ns_cap;
    for (int idx = tid; idx < GRP * (HD / 4); idx += NW * 64) {
        const int row = idx / (HD / 4), d4 = idx % (HD / 4);
        const size_t pi = ((size_t)seq * p.NQ + kvh * GRP + row) * ns + c;
        *reinterpret_cast<f32x4 *>(a.part.acc + pi * HD + 4 * d4) = *reinterpret_cast<const f32x4 *>(buf + row * Cf::BSTR + 4 * d4);
    }
    if (tid < GRP) {
        float Mr = kNegInf;
        for (int w = 0; w < NW; w++) Mr = fmaxf(Mr, redm[w * 16 + tid]);
        float L = 0.f;
        if (Mr != kNegInf)
            for (int w = 0; w < NW; w++) {
                const float mw = redm[w * 16 + tid];
                if (mw != kNegInf) L += redl[w * 16 + tid] * fast_exp2(mw - Mr);
            }
        const size_t pi = ((size_t)seq * p.NQ + kvh * GRP + tid) * ns + c;
        a.part.m[pi] = Mr; a.part.l[pi] = L;
    }
}

template <int HD, int KVT, int QT>
static hipError_t launch_dec_t(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((decode_stream_kernel<HD, KVT, QT>), grid, dim3(256), DecodeCfg<HD>::LDS, st, a);
    return hipGetLastError();
}

template <int KVT, int QT>
static hipError_t dec_dispatch_hd(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return launch_dec_t<128, KVT, QT>(a, grid, st);
    case 256: return launch_dec_t<256, KVT, QT>(a, grid, st);
    default: return hipErrorNotSupported;
    }
}

bool decode_stream_supported(const Problem &p) {
    return p.T == 1 && (p.HD == 128 || p.HD == 256) && p.NQ % p.NKV == 0 && p.NQ / p.NKV <= 16 &&
           p.kv_dtype != DT_FP32;
}

hipError_t launch_decode_stream(const Problem &p, int chunk, const Partials &part, hipStream_t st) {
    if (!decode_stream_supported(p)) return hipErrorNotSupported;
    if (chunk <= 0 || chunk % 16) return hipErrorInvalidValue;
    if (p.max_pos / chunk + 1 > part.ns_cap) return hipErrorInvalidValue;
    DecodeArgs a{p, part, chunk, p.scale * kLog2e};
    dim3 grid(p.NKV, p.max_pos / chunk + 1, p.nseq);
    if (grid.z > 65535u || grid.y > 65535u) return hipErrorInvalidConfiguration;
    const int kv = p.kv_dtype, q = p.q_dtype;
    if (kv == DT_F16 && q == DT_FP32) return dec_dispatch_hd<DT_F16, DT_FP32>(a, grid, st);
    if (kv == DT_F16 && q == DT_F16) return dec_dispatch_hd<DT_F16, DT_F16>(a, grid, st);
    if (kv == DT_BF16 && q == DT_FP32) return dec_dispatch_hd<DT_BF16, DT_FP32>(a, grid, st);
    if (kv == DT_BF16 && q == DT_BF16) return dec_dispatch_hd<DT_BF16, DT_BF16>(a, grid, st);
    return hipErrorNotSupported;
}

}  // namespace dgx

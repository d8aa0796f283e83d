// Split-KV GQA attention for decode, verify and speculative tree verify on gfx950.
//
// Replaces the reference's attn_split_p1_kernel / attn_split_combine_kernel
// (kernels/attention_decode_split.cuh:43-165) and, for short query runs, flash_attn2bs_p1(_custom)_kernel /
// flash_attn2bs_p2_kernel (kernels/attention_flash.cuh:28-227).
//
// Grid: (chunk c, kv head, sequence x query-token tile). One workgroup = NW wave64s. It owns the query rows
// (token, head) of one KV head (GQA group, rows token-major) for a token tile and the keys
// [c*C, (c+1)*C) of its sequence, and writes one LSE partial per (row, chunk). Inside the chunk the keys are
// cut into 32-key tiles at absolute positions; wave w takes tiles w, w+NW, ... and keeps its own online
// softmax state in registers, so waves never synchronise until the end, where their states are merged in wave
// order through LDS. Per tile a wave:
//   * streams K (16 bytes per lane, straight into MFMA A fragments) and V (16-byte coalesced rows) from HBM,
//   * computes S^T = K Q^T on 16x16x32 MFMA (Q fragments live in registers for the whole chunk),
//   * applies the causal / sliding-window / tree mask and the online softmax on the S^T fragment (a query row
//     sits in 4 lanes; row max and row sum are two xor shuffles),
//   * stages the V tile in its private LDS slice and reads it back transposed as the A fragment of
//     O^T += V^T P^T (P^T comes straight from the softmax registers, no LDS round trip).
// Every K/V byte of a chunk is read once per workgroup and serves all GRP query heads of the KV head.
//
// Invariants (kept from the reference, attention_decode_split.cuh:8-12): chunk and tile boundaries are absolute
// key positions; which wave owns a tile depends only on the tile's position; the partial merge and the chunk
// combine run in fixed order. A row's result therefore does not depend on the batch, the other rows of its tile,
// the grid size or the maximum position: a row is bit-identical alone (S=1), as a verify row or as a batch row.
#include "attn_device.h"
#include "attn_internal.h"
#include <climits>

namespace dgx {

struct SplitArgs {
    Problem p;
    Partials part;
    int C;          // chunk (keys), multiple of 32
    int tpb;        // query tokens per workgroup
    int nchunks;    // token tiles per sequence
    float sl2;      // scale * log2(e)
};

template <int HD, int RB, int NW>
struct SplitCfg {
    static constexpr int KS = HD / 32;        // QK k-steps
    static constexpr int DB = HD / 16;        // PV output dim blocks
    static constexpr int VSTR = HD + 8;       // V tile LDS row stride (16-bit elements)
    static constexpr int VCH = HD / 16;       // 16-byte V chunks per lane per 32-key tile
    static constexpr int RR = RB * 16;        // rows per workgroup
    static constexpr int BSTR = HD + 4;       // merge buffer row stride (floats)
    static constexpr size_t LDS_TILES = (size_t)NW * 32 * VSTR * 2;
    static constexpr size_t LDS_MERGE = ((size_t)2 * NW * RR + (size_t)RR * BSTR) * 4;
    static constexpr size_t LDS = LDS_TILES > LDS_MERGE ? LDS_TILES : LDS_MERGE;
};

template <int HD, int RB, int KVT, int QT, int NW>
__global__ void __launch_bounds__(NW * 64) split_kernel(const SplitArgs a) {
    using Cf = SplitCfg<HD, RB, NW>;
    constexpr bool F16 = OpIsF16<KVT>::value;
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];

    const Problem &p = a.p;
    const int c = blockIdx.x, kvh = blockIdx.y;
    const int seq = blockIdx.z / a.nchunks, tchunk = blockIdx.z % a.nchunks;
    const int GRP = p.NQ / p.NKV;
    const int tok0 = tchunk * a.tpb, tok1 = min(p.T, tok0 + a.tpb);
    const int nrows = (tok1 - tok0) * GRP;
    int lo_b = INT_MAX, hi_b = 0;
    for (int t = tok0; t < tok1; t++) {
        const int ps = tok_pos(p, seq, t);
        lo_b = min(lo_b, win_lo(ps, p.window));
        hi_b = max(hi_b, ps + 1);
    }
    const int C = a.C;
    const int j_lo = max(c * C, lo_b), j_hi = min(c * C + C, hi_b);
    if (j_lo >= j_hi) return;                                  // chunk outside every row's key range

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, ln = lane & 15;
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = reinterpret_cast<const KE *>(p.K) + (size_t)seq * p.kv_stride + (size_t)kvh * HD;
    const KE *Vb = reinterpret_cast<const KE *>(p.V) + (size_t)seq * p.kv_stride + (size_t)kvh * HD;

    RowMask rm[RB];
    u32x4 qop[RB][Cf::KS];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int rho = rb * 16 + ln;
        const bool valid = rho < nrows;
        const int t = tok0 + (valid ? rho / GRP : 0), h = kvh * GRP + (valid ? rho % GRP : 0);
        const int ps = tok_pos(p, seq, t);
        rm[rb].pos = ps; rm[rb].lo = win_lo(ps, p.window); rm[rb].valid = valid;
        rm[rb].tree = p.anc != nullptr;
        rm[rb].anc = p.anc ? p.anc[seq * p.T + t] : 0u;
        rm[rb].tb = p.anc ? tok_pos(p, seq, 0) : 0;
        const QE *qrow = reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + t) * p.NQ + h) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < Cf::KS; ks++)
            qop[rb][ks] = valid ? load8_op<QT, F16>(qrow + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
    }

    float m[RB], l[RB];
    f32x4 acc[RB][Cf::DB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        m[rb] = kNegInf; l[rb] = 0.f;
#pragma unroll
        for (int db = 0; db < Cf::DB; db++) acc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    uint16_t *vs = reinterpret_cast<uint16_t *>(smem) + (size_t)wave * 32 * Cf::VSTR;
    const int ntiles = C / 32;
    for (int it = wave; it < ntiles; it += NW) {
        const int jt = c * C + 32 * it;
        if (jt + 32 <= j_lo || jt >= j_hi) continue;
        // K fragments: lane (key ln of block kb, group g) holds dims 32*ks + 8*g .. +8.
        u32x4 kop[2][Cf::KS];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const int key = min(jt + 16 * kb + ln, hi_b - 1);
            const KE *kp = Kb + (size_t)key * krow + 8 * g;
#pragma unroll
            for (int ks = 0; ks < Cf::KS; ks++) kop[kb][ks] = load8_op<KVT, F16>(kp + 32 * ks);
        }
        // V tile rows, coalesced: HD/8 lanes per key row.
        u32x4 vr[Cf::VCH];
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            const int kc = min(jt + key, hi_b - 1);
            vr[u] = load8_op<KVT, F16>(Vb + (size_t)kc * krow + col);
        }
        f32x4 s[RB][2];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < Cf::KS; ks++) x = mfma16<F16>(kop[kb][ks], qop[rb][ks], x);
                s[rb][kb] = x;
            }
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(vs + key * Cf::VSTR + col) = vr[u];
        }
        // Online softmax (log2 domain). Lane holds keys jt + 16*kb + 4*g + i of row ln.
        u32x4 pop[RB];
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            float tv[8], mx = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = jt + 16 * kb + 4 * g + i;
                    const float v = rm[rb].attends(key) ? s[rb][kb][i] * a.sl2 : kNegInf;
                    tv[kb * 4 + i] = v; mx = fmaxf(mx, v);
                }
            mx = max_over_groups(mx);
            const float mnew = fmaxf(m[rb], mx);
            const float alpha = (mnew == kNegInf) ? 1.f : fast_exp2(m[rb] - mnew);
            float pv[8], ps = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) { pv[e] = (tv[e] == kNegInf) ? 0.f : fast_exp2(tv[e] - mnew); ps += pv[e]; }
            ps = sum_over_groups(ps);
            l[rb] = l[rb] * alpha + ps; m[rb] = mnew;
#pragma unroll
            for (int db = 0; db < Cf::DB; db++) acc[rb][db] *= alpha;
            pop[rb] = u32x4{pack2<F16>(pv[0], pv[1]), pack2<F16>(pv[2], pv[3]), pack2<F16>(pv[4], pv[5]), pack2<F16>(pv[6], pv[7])};
        }
        __builtin_amdgcn_wave_barrier();
        // O^T += V^T P^T. A fragment: lane (dim 16*db + ln, group g) holds V[key(g, e)][dim] with
        // key(g, e) = 4g + e (e < 4) or 16 + 4g + e - 4 (e >= 4): the same key order as the P^T registers.
#pragma unroll
        for (int db = 0; db < Cf::DB; db++) {
            const uint16_t *vc = vs + 16 * db + ln;
            uint16_t x[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int key = (e < 4) ? 4 * g + e : 16 + 4 * g + (e - 4);
                x[e] = vc[key * Cf::VSTR];
            }
            const u32x4 vop = u32x4{(uint32_t)x[0] | ((uint32_t)x[1] << 16), (uint32_t)x[2] | ((uint32_t)x[3] << 16),
                                    (uint32_t)x[4] | ((uint32_t)x[5] << 16), (uint32_t)x[6] | ((uint32_t)x[7] << 16)};
#pragma unroll
            for (int rb = 0; rb < RB; rb++) acc[rb][db] = mfma16<F16>(vop, pop[rb], acc[rb][db]);
        }
        __builtin_amdgcn_wave_barrier();
    }

    // Merge the NW wave states in wave order, then write the chunk partial.
    __syncthreads();
    float *redm = reinterpret_cast<float *>(smem), *redl = redm + NW * Cf::RR, *buf = redl + NW * Cf::RR;
    if (g == 0) {
#pragma unroll
        for (int rb = 0; rb < RB; rb++) { redm[wave * Cf::RR + rb * 16 + ln] = m[rb]; redl[wave * Cf::RR + rb * 16 + ln] = l[rb]; }
    }
    __syncthreads();
    float f[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int row = rb * 16 + ln;
        float M = kNegInf;
        for (int w = 0; w < NW; w++) M = fmaxf(M, redm[w * Cf::RR + row]);
        f[rb] = (m[rb] == kNegInf) ? 0.f : fast_exp2(m[rb] - M);
    }
    for (int w = 0; w < NW; w++) {
        if (wave == w) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                const int row = rb * 16 + ln;
                if (row < nrows) {
#pragma unroll
                    for (int db = 0; db < Cf::DB; db++) {
                        f32x4 *dst = reinterpret_cast<f32x4 *>(buf + row * Cf::BSTR + 16 * db + 4 * g);
                        f32x4 v = acc[rb][db] * f[rb];
                        if (w > 0) v += *dst;
                        *dst = v;
                    }
                }
            }
        }
        __syncthreads();
    }
    const int NQ = p.NQ, ns = a.part.ns_cap;
    for (int idx = threadIdx.x; idx < nrows * (HD / 4); idx += NW * 64) {
        const int row = idx / (HD / 4), d4 = idx % (HD / 4);
        const int r = seq * p.T + tok0 + row / GRP, h = kvh * GRP + row % GRP;
        const size_t pi = ((size_t)r * NQ + h) * ns + c;
        *reinterpret_cast<f32x4 *>(a.part.acc + pi * HD + 4 * d4) = *reinterpret_cast<const f32x4 *>(buf + row * Cf::BSTR + 4 * d4);
    }
    for (int row = threadIdx.x; row < nrows; row += NW * 64) {
        float M = kNegInf;
        for (int w = 0; w < NW; w++) M = fmaxf(M, redm[w * Cf::RR + row]);
        float L = 0.f;
        if (M != kNegInf)
            for (int w = 0; w < NW; w++) {
                const float mw = redm[w * Cf::RR + row];
                if (mw != kNegInf) L += redl[w * Cf::RR + row] * fast_exp2(mw - M);
            }
        const int r = seq * p.T + tok0 + row / GRP, h = kvh * GRP + row % GRP;
        const size_t pi = ((size_t)r * NQ + h) * ns + c;
        a.part.m[pi] = M; a.part.l[pi] = L;
    }
}

// LSE combine over the row's valid chunks [lo/C, pos/C] in ascending order
// (attention_decode_split.cuh:147-165): O = sum w_c acc_c / sum w_c l_c, w_c = 2^(m_c - max m).
template <int OT>
__global__ void __launch_bounds__(256) combine_kernel(const Problem p, const Partials part, int C) {
    const int r = blockIdx.x, h = blockIdx.y;
    const int s = r / p.T, t = r % p.T;
    const int pos = tok_pos(p, s, t), lo = win_lo(pos, p.window);
    const int c_lo = lo / C, c_hi = pos / C;
    const size_t base = ((size_t)r * p.NQ + h) * part.ns_cap;
    float mg = kNegInf;
    for (int c = c_lo; c <= c_hi; c++) mg = fmaxf(mg, part.m[base + c]);
    float L = 0.f;
    if (mg != kNegInf)
        for (int c = c_lo; c <= c_hi; c++) {
            const float mc = part.m[base + c];
            if (mc != kNegInf) L += part.l[base + c] * fast_exp2(mc - mg);
        }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int HD = p.HD;
    for (int d = threadIdx.x; d < HD; d += blockDim.x) {
        float acc = 0.f;
        if (mg != kNegInf)
            for (int c = c_lo; c <= c_hi; c++) {
                const float mc = part.m[base + c];
                if (mc != kNegInf) acc += part.acc[(base + c) * HD + d] * fast_exp2(mc - mg);
            }
        const float o = acc * inv;
        const size_t oi = ((size_t)r * p.NQ + h) * HD + d;
        if constexpr (OT == DT_FP32) reinterpret_cast<float *>(p.O)[oi] = o;
        else reinterpret_cast<uint16_t *>(p.O)[oi] = f32_to_op(o, OT == DT_F16);
    }
    if (p.lse && threadIdx.x == 0)
        p.lse[(size_t)r * p.NQ + h] = (L > 0.f) ? (mg + log2f(L)) * kLn2 : kNegInf;
}

// ---------------------------------------------------------------- host side
template <int HD, int RB, int KVT, int QT, int NW>
static hipError_t launch_split_t(const SplitArgs &a, dim3 grid, hipStream_t st) {
    using Cf = SplitCfg<HD, RB, NW>;
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&split_kernel<HD, RB, KVT, QT, NW>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL((split_kernel<HD, RB, KVT, QT, NW>), grid, dim3(NW * 64), Cf::LDS, st, a);
    return hipGetLastError();
}

template <int HD, int KVT, int QT>
static hipError_t dispatch_rb(const SplitArgs &a, int RB, dim3 grid, hipStream_t st) {
    constexpr int NW = HD >= 512 ? 2 : 4;
    switch (RB) {
    case 1: return launch_split_t<HD, 1, KVT, QT, NW>(a, grid, st);
    case 2: return launch_split_t<HD, 2, KVT, QT, NW>(a, grid, st);
    case 3: if constexpr (HD <= 256) return launch_split_t<HD, 3, KVT, QT, NW>(a, grid, st); else return hipErrorInvalidValue;
    case 4: if constexpr (HD <= 256) return launch_split_t<HD, 4, KVT, QT, NW>(a, grid, st); else return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

template <int KVT, int QT>
static hipError_t dispatch_hd(const SplitArgs &a, int RB, dim3 grid, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return dispatch_rb<128, KVT, QT>(a, RB, grid, st);
    case 256: return dispatch_rb<256, KVT, QT>(a, RB, grid, st);
    case 512: return dispatch_rb<512, KVT, QT>(a, RB, grid, st);
    default: return hipErrorInvalidValue;
    }
}

static void split_tiling(const Problem &p, int &RB, int &tpb, int &nchunks) {
    const int GRP = p.NQ / p.NKV;
    const int maxrb = p.HD >= 512 ? 2 : 4;
    const int rows = p.T * GRP;
    RB = (rows + 15) / 16;
    if (RB > maxrb) RB = maxrb;
    if (RB * 16 < GRP) RB = (GRP + 15) / 16;
    tpb = (RB * 16) / GRP;
    if (tpb < 1) tpb = 1;
    nchunks = (p.T + tpb - 1) / tpb;
}

size_t partial_rows(const Problem &p, int chunk) {
    return (size_t)p.nseq * p.T * p.NQ * (size_t)(p.max_pos / chunk + 1);
}

hipError_t launch_split(const Problem &p, int chunk, const Partials &part, hipStream_t st) {
    if (chunk <= 0 || chunk % 32) return hipErrorInvalidValue;
    if (p.NQ % p.NKV) return hipErrorInvalidValue;
    const int GRP = p.NQ / p.NKV;
    int RB, tpb, nchunks;
    split_tiling(p, RB, tpb, nchunks);
    if (RB * 16 < GRP || RB > (p.HD >= 512 ? 2 : 4)) return hipErrorInvalidValue;
    if (p.max_pos / chunk + 1 > part.ns_cap) return hipErrorInvalidValue;
    SplitArgs a{p, part, chunk, tpb, nchunks, p.scale * kLog2e};
    dim3 grid(p.max_pos / chunk + 1, p.NKV, p.nseq * nchunks);
    if (grid.z > 65535u || grid.y > 65535u) return hipErrorInvalidConfiguration;
    const int kv = p.kv_dtype, q = p.q_dtype;
    if (kv == DT_F16 && q == DT_FP32) return dispatch_hd<DT_F16, DT_FP32>(a, RB, grid, st);
    if (kv == DT_F16 && q == DT_F16) return dispatch_hd<DT_F16, DT_F16>(a, RB, grid, st);
    if (kv == DT_BF16 && q == DT_FP32) return dispatch_hd<DT_BF16, DT_FP32>(a, RB, grid, st);
    if (kv == DT_BF16 && q == DT_BF16) return dispatch_hd<DT_BF16, DT_BF16>(a, RB, grid, st);
    if (kv == DT_FP32 && q == DT_FP32) return dispatch_hd<DT_FP32, DT_FP32>(a, RB, grid, st);
    return hipErrorInvalidValue;
}

hipError_t launch_combine(const Problem &p, int chunk, const Partials &part, hipStream_t st) {
    dim3 grid(p.nseq * p.T, p.NQ);
    const int threads = p.HD >= 256 ? 256 : p.HD;
    switch (p.o_dtype) {
    case DT_FP32: hipLaunchKernelGGL(combine_kernel<DT_FP32>, grid, dim3(threads), 0, st, p, part, chunk); break;
    case DT_F16: hipLaunchKernelGGL(combine_kernel<DT_F16>, grid, dim3(threads), 0, st, p, part, chunk); break;
    case DT_BF16: hipLaunchKernelGGL(combine_kernel<DT_BF16>, grid, dim3(threads), 0, st, p, part, chunk); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dgx

// Flash prefill / chunked prefill attention on gfx950 (causal, sliding window, optional tree mask).
//
// Replaces the reference's fav2::flash_v2_kernel (kernels/attention_flash_v2.cuh:104-259) and, for long query
// runs, flash_attn2bs_p1(_custom)_kernel (kernels/attention_flash.cuh:28-217).
//
// Grid: (query-row tile, kv head, sequence x key split). A workgroup owns NW*RB*16 query rows (tokens x the GRP
// q-heads of one KV head, token-major, so every K/V tile is fetched once for the whole GQA group); wave w owns
// rows [w*RB*16, (w+1)*RB*16). The key range is walked in 32-key tiles at absolute positions; each tile of K and
// V is fetched from HBM by the whole workgroup (16-byte coalesced loads, prefetched into registers one tile
// ahead) into a double-buffered LDS ring, so there is one barrier per tile. Per tile a wave
//   * reads K fragments from LDS (one 16-byte read per MFMA) and computes S^T = K Q^T on 16x16x32 MFMA with its
//     Q fragments held in registers,
//   * masks (causal / window / tree) and runs the online softmax on the S^T fragment in registers,
//   * computes O^T += V^T P^T with V^T read transposed from LDS and P^T straight from registers.
// Waves skip the MFMA work of tiles that no row of theirs attends (the causal upper triangle, keys left of the
// window). Query tiles are scheduled latest-first (they carry the most keys).
//
// Key splits (kv_split > 0) cut the keys at absolute multiples of kv_split: a row whose whole key range lies in
// one split is normalised and written here; other rows write an LSE partial per split for the combine kernel.
// Either way a row's arithmetic depends only on its own query, position and keys (tile and split boundaries are
// absolute, tiles are visited in increasing order and a tile the row does not attend leaves its state exactly
// unchanged), so prefill is bit-invariant to how the prompt is chunked (attention_flash_v2.cuh:13-18).
#include "attn_device.h"
#include "attn_internal.h"
#include <climits>

namespace dgx {

struct PrefArgs {
    Problem p;
    Partials part;
    int kv_split;      // 0: no split
    int nqt;           // query-row tiles per sequence
    int nsplit;        // key splits per sequence (grid.z = nseq * nsplit)
    int tq;            // tokens per query tile
    float sl2;         // scale * log2(e)
};

template <int HD, int RB, int NW>
struct PrefCfg {
    static constexpr int KS = HD / 32;
    static constexpr int DB = HD / 16;
    static constexpr int STR = HD + 8;                  // LDS row stride (16-bit elements) of K and V tiles
    static constexpr int RW = NW * RB * 16;             // rows per workgroup
    static constexpr int NT = NW * 64;
    static constexpr int CPT = 32 * HD / 8 / NT;        // 16-byte chunks per thread per tile (K and V each)
    static constexpr size_t TILE = (size_t)32 * STR;    // elements of one K or V tile
    static constexpr size_t LDS = 4 * TILE * 2;         // K, V x double buffer
    static_assert((32 * HD / 8) % NT == 0, "tile chunks");
};

template <int HD, int RB, int NW, int KVT, int QT, int OT>
__global__ void __launch_bounds__(NW * 64) prefill_kernel(const PrefArgs a) {
    using Cf = PrefCfg<HD, RB, NW>;
    constexpr bool F16 = OpIsF16<KVT>::value;
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t *lds = reinterpret_cast<uint16_t *>(smem);

    const Problem &p = a.p;
    const int qt = a.nqt - 1 - (int)blockIdx.x;              // latest query tile first
    const int kvh = blockIdx.y;
    const int seq = blockIdx.z / a.nsplit, sp = blockIdx.z % a.nsplit;
    const int GRP = p.NQ / p.NKV;
    const int tok0 = qt * a.tq, tok1 = min(p.T, tok0 + a.tq);
    const int nrows = (tok1 - tok0) * GRP;
    int lo_b = INT_MAX, hi_b = 0;
    for (int t = tok0; t < tok1; t++) {
        const int ps = tok_pos(p, seq, t);
        lo_b = min(lo_b, win_lo(ps, p.window));
        hi_b = max(hi_b, ps + 1);
    }
    int j_lo = lo_b, j_hi = hi_b;
    if (a.kv_split > 0) { j_lo = max(j_lo, sp * a.kv_split); j_hi = min(j_hi, (sp + 1) * a.kv_split); }
    if (j_lo >= j_hi) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, ln = lane & 15;
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = reinterpret_cast<const KE *>(p.K) + (size_t)seq * p.kv_stride + (size_t)kvh * HD;
    const KE *Vb = reinterpret_cast<const KE *>(p.V) + (size_t)seq * p.kv_stride + (size_t)kvh * HD;

    // This wave's rows.
    RowMask rm[RB];
    u32x4 qop[RB][Cf::KS];
    int wlo = INT_MAX, whi = -1;                               // key span attended by any row of the wave
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int rho = (wave * RB + rb) * 16 + ln;
        const bool valid = rho < nrows;
        const int t = tok0 + (valid ? rho / GRP : 0), h = kvh * GRP + (valid ? rho % GRP : 0);
        const int ps = tok_pos(p, seq, t);
        rm[rb].pos = ps; rm[rb].lo = win_lo(ps, p.window); rm[rb].valid = valid;
        rm[rb].tree = p.anc != nullptr;
        rm[rb].anc = p.anc ? p.anc[seq * p.T + t] : 0u;
        rm[rb].tb = p.anc ? tok_pos(p, seq, 0) : 0;
        if (valid) { wlo = min(wlo, rm[rb].lo); whi = max(whi, ps); }
        const QE *qrow = reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + t) * p.NQ + h) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < Cf::KS; ks++)
            qop[rb][ks] = valid ? load8_op<QT, F16>(qrow + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
    }
    // wave-uniform span
    for (int o = 1; o < 64; o <<= 1) { wlo = min(wlo, __shfl_xor(wlo, o)); whi = max(whi, __shfl_xor(whi, o)); }

    float m[RB], l[RB];
    f32x4 acc[RB][Cf::DB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        m[rb] = kNegInf; l[rb] = 0.f;
#pragma unroll
        for (int db = 0; db < Cf::DB; db++) acc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int jb = (j_lo / 32) * 32;
    const int ntile = (j_hi - jb + 31) / 32;
    // Cooperative tile fetch: chunk q = tid + NT*u -> key q / (HD/8), column (q % (HD/8)) * 8.
    u32x4 kr[Cf::CPT], vr[Cf::CPT];
    auto fetch = [&](int jt) {
#pragma unroll
        for (int u = 0; u < Cf::CPT; u++) {
            const int q = tid + Cf::NT * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            const size_t off = (size_t)min(jt + key, hi_b - 1) * krow + col;
            kr[u] = load8_op<KVT, F16>(Kb + off);
            vr[u] = load8_op<KVT, F16>(Vb + off);
        }
    };
    auto stash = [&](int buf) {
        uint16_t *ks = lds + (size_t)buf * 2 * Cf::TILE, *vsb = ks + Cf::TILE;
#pragma unroll
        for (int u = 0; u < Cf::CPT; u++) {
            const int q = tid + Cf::NT * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(ks + key * Cf::STR + col) = kr[u];
            *reinterpret_cast<u32x4 *>(vsb + key * Cf::STR + col) = vr[u];
        }
    };
    fetch(jb);
    stash(0);
    __syncthreads();
    for (int it = 0; it < ntile; it++) {
        const int jt = jb + 32 * it, buf = it & 1;
        const bool more = it + 1 < ntile;
        if (more) fetch(jt + 32);
        if (jt <= whi && jt + 31 >= wlo) {
            const uint16_t *ks = lds + (size_t)buf * 2 * Cf::TILE, *vsb = ks + Cf::TILE;
            f32x4 s[RB][2];
#pragma unroll
            for (int rb = 0; rb < RB; rb++) s[rb][0] = s[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                const uint16_t *kp = ks + (16 * kb + ln) * Cf::STR + 8 * g;
#pragma unroll
                for (int kk = 0; kk < Cf::KS; kk++) {
                    const u32x4 kf = *reinterpret_cast<const u32x4 *>(kp + 32 * kk);
#pragma unroll
                    for (int rb = 0; rb < RB; rb++) s[rb][kb] = mfma16<F16>(kf, qop[rb][kk], s[rb][kb]);
                }
            }
            u32x4 pop[RB];
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                float tv[8], mx = kNegInf;
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = jt + 16 * kb + 4 * g + i;
                        const bool in = key >= j_lo && key < j_hi && rm[rb].attends(key);
                        const float v = in ? s[rb][kb][i] * a.sl2 : kNegInf;
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
#pragma unroll
            for (int db = 0; db < Cf::DB; db++) {
                const uint16_t *vc = vsb + 16 * db + ln;
                uint16_t x[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int key = (e < 4) ? 4 * g + e : 16 + 4 * g + (e - 4);
                    x[e] = vc[key * Cf::STR];
                }
                const u32x4 vop = u32x4{(uint32_t)x[0] | ((uint32_t)x[1] << 16), (uint32_t)x[2] | ((uint32_t)x[3] << 16),
                                        (uint32_t)x[4] | ((uint32_t)x[5] << 16), (uint32_t)x[6] | ((uint32_t)x[7] << 16)};
#pragma unroll
                for (int rb = 0; rb < RB; rb++) acc[rb][db] = mfma16<F16>(vop, pop[rb], acc[rb][db]);
            }
        }
        if (more) stash(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: a row whose key range lies in this split alone is final; otherwise it leaves a partial.
    const int NQ = p.NQ;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int rho = (wave * RB + rb) * 16 + ln;
        if (rho >= nrows) continue;
        const int r = seq * p.T + tok0 + rho / GRP, h = kvh * GRP + rho % GRP;
        const bool direct = a.kv_split <= 0 || (rm[rb].lo / a.kv_split == rm[rb].pos / a.kv_split);
        if (direct) {
            const float inv = l[rb] > 0.f ? 1.f / l[rb] : 0.f;
            const size_t ob = ((size_t)r * NQ + h) * HD;
#pragma unroll
            for (int db = 0; db < Cf::DB; db++) {
                const f32x4 o = acc[rb][db] * inv;
                const int d = 16 * db + 4 * g;
                if constexpr (OT == DT_FP32) *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.O) + ob + d) = o;
                else {
                    const u32x2 w = u32x2{pack2<OT == DT_F16>(o.x, o.y), pack2<OT == DT_F16>(o.z, o.w)};
                    *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(p.O) + ob + d) = w;
                }
            }
            if (p.lse && g == 0) p.lse[(size_t)r * NQ + h] = (l[rb] > 0.f) ? (m[rb] + log2f(l[rb])) * kLn2 : kNegInf;
        } else {
            const size_t pi = ((size_t)r * NQ + h) * a.part.ns_cap + sp;
#pragma unroll
            for (int db = 0; db < Cf::DB; db++)
                *reinterpret_cast<f32x4 *>(a.part.acc + pi * HD + 16 * db + 4 * g) = acc[rb][db];
            if (g == 0) { a.part.m[pi] = m[rb]; a.part.l[pi] = l[rb]; }
        }
    }
}

// Combine for prefill splits: rows whose key range spans more than one split (the others were written directly).
template <int OT>
__global__ void __launch_bounds__(256) prefill_combine_kernel(const Problem p, const Partials part, int C) {
    const int r = blockIdx.x, h = blockIdx.y;
    const int s = r / p.T, t = r % p.T;
    const int pos = tok_pos(p, s, t), lo = win_lo(pos, p.window);
    const int c_lo = lo / C, c_hi = pos / C;
    if (c_lo == c_hi) return;
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
template <int HD, int RB, int NW, int KVT, int QT, int OT>
static hipError_t launch_pref_t(const PrefArgs &a, dim3 grid, hipStream_t st) {
    using Cf = PrefCfg<HD, RB, NW>;
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&prefill_kernel<HD, RB, NW, KVT, QT, OT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL((prefill_kernel<HD, RB, NW, KVT, QT, OT>), grid, dim3(NW * 64), Cf::LDS, st, a);
    return hipGetLastError();
}

template <int HD> struct PrefTile;                       // rows per wave (RB*16) and waves per workgroup
template <> struct PrefTile<128> { static constexpr int RB = 2, NW = 4; };
template <> struct PrefTile<256> { static constexpr int RB = 2, NW = 4; };
template <> struct PrefTile<512> { static constexpr int RB = 1, NW = 4; };

template <int KVT, int QT, int OT>
static hipError_t pref_dispatch_hd(const PrefArgs &a, dim3 grid, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return launch_pref_t<128, PrefTile<128>::RB, PrefTile<128>::NW, KVT, QT, OT>(a, grid, st);
    case 256: return launch_pref_t<256, PrefTile<256>::RB, PrefTile<256>::NW, KVT, QT, OT>(a, grid, st);
    case 512: return launch_pref_t<512, PrefTile<512>::RB, PrefTile<512>::NW, KVT, QT, OT>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

static int pref_rows(int HD) {
    switch (HD) {
    case 128: return PrefTile<128>::RB * PrefTile<128>::NW * 16;
    case 256: return PrefTile<256>::RB * PrefTile<256>::NW * 16;
    case 512: return PrefTile<512>::RB * PrefTile<512>::NW * 16;
    default: return 0;
    }
}

hipError_t launch_prefill(const Problem &p, int kv_split, const Partials &part, hipStream_t st) {
    if (p.NQ % p.NKV) return hipErrorInvalidValue;
    const int GRP = p.NQ / p.NKV, RW = pref_rows(p.HD);
    if (RW == 0 || GRP > RW) return hipErrorInvalidValue;
    if (kv_split < 0 || (kv_split > 0 && kv_split % 32)) return hipErrorInvalidValue;
    const int tq = RW / GRP;
    const int nqt = (p.T + tq - 1) / tq;
    const int nsplit = kv_split > 0 ? p.max_pos / kv_split + 1 : 1;
    if (kv_split > 0 && nsplit > part.ns_cap) return hipErrorInvalidValue;
    PrefArgs a{p, part, kv_split, nqt, nsplit, tq, p.scale * kLog2e};
    dim3 grid(nqt, p.NKV, p.nseq * nsplit);
    if (grid.z > 65535u || grid.y > 65535u) return hipErrorInvalidConfiguration;
    hipError_t e = hipErrorInvalidValue;
    const int kv = p.kv_dtype, q = p.q_dtype, o = p.o_dtype;
#define DGX_PREF(KV, Q, O) if (kv == KV && q == Q && o == O) e = pref_dispatch_hd<KV, Q, O>(a, grid, st); else
    DGX_PREF(DT_F16, DT_FP32, DT_FP32)
    DGX_PREF(DT_BF16, DT_FP32, DT_FP32)
    DGX_PREF(DT_FP32, DT_FP32, DT_FP32)
    DGX_PREF(DT_F16, DT_F16, DT_F16)
    DGX_PREF(DT_BF16, DT_BF16, DT_BF16)
    return hipErrorInvalidValue;
#undef DGX_PREF
    if (e != hipSuccess || kv_split <= 0) return e;
    dim3 cg(p.nseq * p.T, p.NQ);
    const int threads = p.HD >= 256 ? 256 : p.HD;
    switch (o) {
    case DT_FP32: hipLaunchKernelGGL(prefill_combine_kernel<DT_FP32>, cg, dim3(threads), 0, st, p, part, kv_split); break;
    case DT_F16: hipLaunchKernelGGL(prefill_combine_kernel<DT_F16>, cg, dim3(threads), 0, st, p, part, kv_split); break;
    default: hipLaunchKernelGGL(prefill_combine_kernel<DT_BF16>, cg, dim3(threads), 0, st, p, part, kv_split); break;
    }
    return hipGetLastError();
}

}  // namespace dgx

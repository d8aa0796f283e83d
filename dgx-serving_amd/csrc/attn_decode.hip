// Streaming split-KV GQA decode on gfx950: up to 16 query rows (tokens x q-heads) per KV head and sequence, HD
// 128 or 256, 16-bit caches (the decode rows of kernels/attention_decode_split.cuh:43-145 and of the per-slot flash
// decode at models/qwen35_batch.cu:165-167).
//
// Grid: one workgroup per (sequence, key chunk of C keys, kv head) that holds keys, enumerated on the device from
// the positions, so the launched workgroups with work come first and spread over all CUs. A workgroup owns the
// query rows of one KV head and one chunk (RW blocks of 16 rows, token-major); its NKL key lanes of wave64s take
// the chunk's 16-key tiles round-robin (lane kl: tiles kl, kl+NKL, ...) and run fully independent online
// softmaxes, merged in key-lane order at the end. The main loop has no workgroup barrier:
//   * K and V rows are streamed from HBM with 16-byte non-temporal loads, whole 512-byte head rows per half
//     wave (the KV cache is read once per call: non-temporal loads sustain a higher HBM rate and leave the
//     caches to the partials and Q),
//   * the K tile passes through the wave's private LDS slice into MFMA A fragments (lane = key),
//     S^T = K Q^T on 16x16x32 MFMA (Q fragments come from LDS, staged once),
//   * the V tile lands in the same slice and is read back with the gfx950 transpose read (ds_read_b64_tr_b16)
//     as the A fragments of O^T += V^T P^T on 16x16x16 MFMA; P^T comes straight from the softmax registers.
//
// Chunk boundaries and tile positions are absolute and the wave that owns a tile depends only on its position,
// so a row's result is identical whatever the batch, grid or maximum position (batch row == single row).
#include "attn_device.h"
#include "attn_internal.h"
#include <climits>
#include <cstdlib>


namespace dgx {

struct DecodeArgs {
    Problem p;
    Partials part;
    int C;
    float sl2;
};

template <int HD, int NKL_, int RW_>
struct DecodeCfg {
    static constexpr int NKL = NKL_, RW = RW_, NW = NKL_ * RW_, KT = 16;
    static constexpr int KS = HD / 32;                 // 32-dim blocks (QK k-steps, V fragment loads)
    static constexpr int DB = HD / 16;                 // 16-dim output blocks
    static constexpr int QSTR = HD + 16;               // Q row stride in LDS (16-bit elements; +16: no bank conflicts)
    static constexpr int BSTR = HD + 4;                // merge buffer row stride (floats)
    static constexpr int VSTR = HD + 16;               // V tile row stride in LDS (16-bit elements; +16: the K
                                                       // fragment and V transpose reads are free of bank conflicts)
    static constexpr int VCH = KT * HD / 8 / 64;       // 16-byte V chunks per lane per tile
    static constexpr size_t LDS_Q = (size_t)RW * 16 * QSTR * 2;
    static constexpr size_t LDS_V = (size_t)NW * KT * VSTR * 2;     // one private tile per wave (K, then V)
    static constexpr size_t LDS_MERGE = ((size_t)2 * NW * 16 + (size_t)RW * 16 * BSTR) * 4;
    static constexpr size_t LDS = LDS_Q + (LDS_V > LDS_MERGE ? LDS_V : LDS_MERGE);
};


// Work item blockIdx.x -> (sequence, chunk c, kv head blockIdx.x % NKV), enumerating only the chunks that hold keys
// of the sequence's tokens (kv head fastest): the workgroups with work come first in launch order and the dispatcher
// spreads them over all CUs; the tail of the upper-bound grid (false) exits at once. Two phases: first every chunk
// of each sequence but one, then that one: the shorter of its first and last chunk (both partial under a sliding
// window, only the last otherwise). The dispatcher hands workgroups out in
// index order and a CU that receives more workgroups than the others shares its bandwidth among them, so the short
// items go last, where they land on the CUs that get a third workgroup (measured: a CU with three full items runs
// 20% longer than one with two).
__device__ __forceinline__ bool find_item(const Problem &p, int C, int &seq, int &c, int &lo, int &hi) {
    const int lane_ = threadIdx.x & 63, cmax = p.max_pos / C;
    int rest = (int)blockIdx.x / p.NKV;
    seq = -1; c = 0;
    for (int phase = 0; phase < 2; phase++) {
        for (int s0 = 0; s0 < p.nseq; s0 += 64) {
            int n = 0, first = 0, lo_s = INT_MAX, hi_s = 0;   // key range of the sequence's tokens
            if (s0 + lane_ < p.nseq) {
                for (int t = 0; t < p.T; t++) {
                    const int ps = tok_pos(p, s0 + lane_, t);
                    lo_s = min(lo_s, win_lo(ps, p.window)); hi_s = max(hi_s, ps + 1);
                }
                first = lo_s / C;
                n = max(0, min((hi_s - 1) / C, cmax) - first + 1);
            }
            const int m = phase == 0 ? max(n - 1, 0) : min(n, 1);   // items of this sequence in this phase
            // The phase-1 chunk: the shorter of the first and the last chunk (a sliding window's first chunk is
            // partial too); phase 0 takes the others in order.
            int sh = 0;
            if (n >= 2) {
                const int kf = min(hi_s, (first + 1) * C) - lo_s, kl = hi_s - max(lo_s, (first + n - 1) * C);
                sh = kf < kl ? 0 : n - 1;
            }
            int incl = m;                                  // inclusive prefix sum over the 64 lanes
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o);
                if (lane_ >= o) incl += y;
            }
            const unsigned long long hit = __ballot(incl > rest);
            if (hit) {
                const int l = __builtin_ctzll(hit);
                seq = s0 + l;
                if (phase == 0) {
                    const int r = rest - (__shfl(incl, l) - __shfl(m, l));
                    c = __shfl(first, l) + (r < __shfl(sh, l) ? r : r + 1);
                } else {
                    c = __shfl(first, l) + __shfl(sh, l);
                }
                lo = __shfl(lo_s, l); hi = __shfl(hi_s, l);
                return true;
            }
            rest -= __shfl(incl, 63);
        }
    }
    return false;
}

template <int HD, int NKL_, int RW_, int KVT, int QT, bool EARLY>
__global__ void __launch_bounds__(NKL_ * RW_ * 64) decode_stream_kernel(const DecodeArgs a) {
    using Cf = DecodeCfg<HD, NKL_, RW_>;
    constexpr int NW = Cf::NW, NKL = Cf::NKL, RW = Cf::RW, KT = Cf::KT;
    constexpr bool F16 = OpIsF16<KVT>::value;
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];

    const Problem &p = a.p;
    const int C = a.C;
    int seq, c, lo, hi;
    if (!find_item(p, C, seq, c, lo, hi)) return;
    seq = __builtin_amdgcn_readfirstlane(seq); c = __builtin_amdgcn_readfirstlane(c);
    lo = __builtin_amdgcn_readfirstlane(lo); hi = __builtin_amdgcn_readfirstlane(hi);
    const int kvh = (int)blockIdx.x % p.NKV;
    const int GRP = p.NQ / p.NKV, nrows = p.T * GRP;          // rows rho = token-major (token, head)
    const int j_lo = max(c * C, lo), j_hi = min(c * C + C, hi);
    if (j_lo >= j_hi) return;

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, ln = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kl = wave % NKL, rw = wave / NKL;                 // key lane, 16-row block
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = kv_base<KE>(p, false, seq) + (size_t)kvh * HD;
    const KE *Vb = kv_base<KE>(p, true, seq) + (size_t)kvh * HD;
    uint16_t *qs = reinterpret_cast<uint16_t *>(smem);
    float *redm = reinterpret_cast<float *>(smem + Cf::LDS_Q), *redl = redm + NW * 16, *buf = redl + NW * 16;
    uint16_t *vs = reinterpret_cast<uint16_t *>(smem + Cf::LDS_Q) + (size_t)wave * KT * Cf::VSTR;   // reused by the merge
    uint16_t *kls = vs;                        // the K tile is consumed before the V tile lands in the same slice

    // Q rows of the workgroup (zero rows past the last), requested first: the LDS store below waits only for them.
    constexpr int QCH = RW * 16 * (HD / 8) / (NW * 64);
    static_assert(QCH >= 1 && (RW * 16 * (HD / 8)) % (NW * 64) == 0, "Q loads");
    auto qrow_of = [&](int u) { return (tid + NW * 64 * u) / (HD / 8); };
    auto qcol_of = [&](int u) { return ((tid + NW * 64 * u) % (HD / 8)) * 8; };
    u32x4 qv[QCH];
#pragma unroll
    for (int u = 0; u < QCH; u++) {
        qv[u] = u32x4{0u, 0u, 0u, 0u};
        const int rho = qrow_of(u);
        if (rho < nrows)
            qv[u] = load8_op<QT, F16>(reinterpret_cast<const QE *>(p.Q) +
                                      ((size_t)(seq * p.T + rho / GRP) * p.NQ + kvh * GRP + rho % GRP) * HD + qcol_of(u));
    }
    // This wave's rows and the wave-uniform bounds of its unmasked fast path.
    const int r_lo = rw * 16, r_hi = min(nrows, r_lo + 16);     // rows [r_lo, r_hi); none if r_lo >= nrows
    int lo_max = 0, pos_min = INT_MAX;
    for (int t = r_lo / GRP; r_lo < r_hi && t <= (r_hi - 1) / GRP; t++) {
        const int ps = tok_pos(p, seq, t);
        lo_max = max(lo_max, win_lo(ps, p.window)); pos_min = min(pos_min, ps);
    }
    if (p.anc) pos_min = min(pos_min, tok_pos(p, seq, 0) - 1);   // tree keys never take the fast path
    // This wave's tiles: k = k0 .. k1-1 with tile k at key c*C + KT*(kl + NKL*k), the ones meeting [j_lo, j_hi).
    const int tb0 = j_lo / KT - c * (C / KT), tb1 = (j_hi - 1) / KT - c * (C / KT);   // tile range in the chunk
    const int k0 = tb0 <= kl ? 0 : (tb0 - kl + NKL - 1) / NKL;
    const int k1 = r_lo >= r_hi ? k0 : (tb1 < kl ? 0 : (tb1 - kl) / NKL + 1);
    // Loads of tile k (K straight into A fragments; V rows coalesced for the private LDS transpose).
    // With RW > 1 the RW waves of a key lane read the same tiles: plain loads, so the L2 serves the repeats.
    // which: 1 = K, 2 = V, 3 = both.
    auto load_t = [&](int k, u32x4 (&kf)[Cf::VCH], u32x4 (&vr)[Cf::VCH], int which) {
        const int jt = c * C + KT * (kl + NKL * k), jrow = key_row(p, jt);
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {      // whole rows, 16 bytes per lane; the last tile clamps to the last key
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            const size_t off = (size_t)(jrow + min(key, hi - 1 - jt)) * krow + col;
            if constexpr (RW == 1) {
                if (which & 1) kf[u] = load8_op_stream<KVT, F16>(Kb + off);
                if (which & 2) vr[u] = load8_op_stream<KVT, F16>(Vb + off);
            } else {
                if (which & 1) kf[u] = load8_op<KVT, F16>(Kb + off);
                if (which & 2) vr[u] = load8_op<KVT, F16>(Vb + off);
            }
        }
    };
    auto load = [&](int k, u32x4 (&kf)[Cf::VCH], u32x4 (&vr)[Cf::VCH]) { load_t(k, kf, vr, 3); };
    // One register buffer per tensor. EARLY: tile k's K (V) registers are refilled with tile k+1's as soon as they
    // have gone to LDS, so the next tile's loads fly while tile k is computed, and tile k0 is requested before the
    // Q rows are staged (the sliding-window case, few waves per SIMD). Otherwise load, then compute (config 2: two
    // waves per SIMD already overlap one's loads with the other's math, and this measured 0.5% faster there).
    u32x4 kb[Cf::VCH], vb[Cf::VCH];
    if (EARLY && k0 < k1) load(k0, kb, vb);
#pragma unroll
    for (int u = 0; u < QCH; u++) *reinterpret_cast<u32x4 *>(qs + qrow_of(u) * Cf::QSTR + qcol_of(u)) = qv[u];
    RowMask rm;
    {
        const int rho = r_lo + ln;
        rm.valid = rho < nrows;
        const int t = rm.valid ? rho / GRP : 0;
        rm.pos = tok_pos(p, seq, t); rm.lo = win_lo(rm.pos, p.window); rm.tree = p.anc != nullptr;
        rm.anc = p.anc ? p.anc[seq * p.T + t] : 0u; rm.tb = tok_pos(p, seq, 0);
    }
    __syncthreads();

    float m = kNegInf, l = 0.f;
    f32x4 acc[Cf::DB];
#pragma unroll
    for (int db = 0; db < Cf::DB; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint16_t *qrow = qs + (r_lo + ln) * Cf::QSTR + 8 * g;
    auto compute = [&](int k, u32x4 (&kr)[Cf::VCH], u32x4 (&vr)[Cf::VCH]) {
        const int jt = c * C + KT * (kl + NKL * k);
        const bool more = EARLY && k + 1 < k1;
        // K rows through the wave's LDS slice into MFMA A fragments (lane = key ln, 16 bytes of dims 32 ks + 8 g).
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(kls + key * Cf::VSTR + col) = kr[u];
        }
        __builtin_amdgcn_wave_barrier();
        if (more) load_t(k + 1, kr, vr, 1);
        // S^T[key jt + 4g + i][row ln], two independent MFMA chains.
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int ks = 0; ks < Cf::KS; ks++) {
            const u32x4 qf = *reinterpret_cast<const u32x4 *>(qrow + 32 * ks);
            const u32x4 kf = *reinterpret_cast<const u32x4 *>(kls + ln * Cf::VSTR + 32 * ks + 8 * g);
            if (ks & 1) s1 = mfma16<F16>(kf, qf, s1);
            else s0 = mfma16<F16>(kf, qf, s0);
        }
        const f32x4 s = (s0 + s1) * a.sl2;
        // Online softmax (log2 domain), lazily moved reference max; l is this lane's share of the row sum.
        float tv[4];
        if (jt >= j_lo && jt + KT <= j_hi && jt >= lo_max && jt + KT - 1 <= pos_min) {
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
        const PFrag<F16> pop = p_frag<F16>(pv[0], pv[1], pv[2], pv[3]);
        // O^T += V^T P^T (16x16x16): stage the V tile in this wave's LDS slice, read it back transposed.
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(vs + key * Cf::VSTR + col) = vr[u];
        }
        __builtin_amdgcn_wave_barrier();
        if (more) load_t(k + 1, kr, vr, 2);
        const uint16_t *vt = vs + (4 * g + (ln >> 2)) * Cf::VSTR + 4 * (ln & 3);
#pragma unroll
        for (int db = 0; db < Cf::DB; db++) acc[db] = mfma_pv16<F16>(lds_read_tr16(vt + 16 * db), pop, acc[db]);
    };
    for (int k = k0; k < k1; k++) {
        if (!EARLY) load(k, kb, vb);
        compute(k, kb, vb);
    }
    l = sum_over_groups(l);

    // Merge the NKL key-lane states of each row block in key-lane order (LDS, over the tile slices), then write the
    // chunk partial of each row.
    __syncthreads();
    if (g == 0) { redm[wave * 16 + ln] = m; redl[wave * 16 + ln] = l; }
    __syncthreads();
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NKL; w++) M = fmaxf(M, redm[(rw * NKL + w) * 16 + ln]);
    const float f = (m == kNegInf) ? 0.f : fast_exp2(m - M);
    float *rbuf = buf + (size_t)rw * 16 * Cf::BSTR;
    for (int w = 0; w < NKL; w++) {
        if (kl == w && r_lo + ln < nrows) {
#pragma unroll
            for (int db = 0; db < Cf::DB; db++) {
                f32x4 *dst = reinterpret_cast<f32x4 *>(rbuf + ln * Cf::BSTR + 16 * db + 4 * g);
                f32x4 v = acc[db] * f;
                if (w > 0) v += *dst;
                *dst = v;
            }
        }
        __syncthreads();
    }
    const int ns = a.part.ns_cap;
    auto part_index = [&](int rho) {
        return ((size_t)(seq * p.T + rho / GRP) * p.NQ + kvh * GRP + rho % GRP) * ns + c;
    };
    for (int idx = tid; idx < nrows * (HD / 4); idx += NW * 64) {
        const int rho = idx / (HD / 4), d4 = idx % (HD / 4);
        *reinterpret_cast<f32x4 *>(a.part.acc + part_index(rho) * HD + 4 * d4) =
            *reinterpret_cast<const f32x4 *>(buf + (size_t)rho * Cf::BSTR + 4 * d4);
    }
    for (int rho = tid; rho < nrows; rho += NW * 64) {
        const int rb = rho / 16, rl = rho % 16;
        float Mr = kNegInf;
        for (int w = 0; w < NKL; w++) Mr = fmaxf(Mr, redm[(rb * NKL + w) * 16 + rl]);
        float L = 0.f;
        if (Mr != kNegInf)
            for (int w = 0; w < NKL; w++) {
                const float mw = redm[(rb * NKL + w) * 16 + rl];
                if (mw != kNegInf) L += redl[(rb * NKL + w) * 16 + rl] * fast_exp2(mw - Mr);
            }
        a.part.m[part_index(rho)] = Mr; a.part.l[part_index(rho)] = L;
    }
}

template <int HD, int RW, int KVT, int QT, bool EARLY>
static hipError_t launch_dec_e(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    constexpr int NKL = 2;
    using Cf = DecodeCfg<HD, NKL, RW>;
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&decode_stream_kernel<HD, NKL, RW, KVT, QT, EARLY>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL((decode_stream_kernel<HD, NKL, RW, KVT, QT, EARLY>), grid, dim3(Cf::NW * 64), Cf::LDS, st, a);
    return hipGetLastError();
}
template <int HD, int RW, int KVT, int QT>
static hipError_t launch_dec_rw(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    // (the choice depends on the layer only, so a row's bits do not depend on the batch)
    if (a.p.window > 0) return launch_dec_e<HD, RW, KVT, QT, true>(a, grid, st);
    return launch_dec_e<HD, RW, KVT, QT, false>(a, grid, st);
}

template <int HD, int KVT, int QT>
static hipError_t launch_dec_t(const DecodeArgs &a, dim3 grid, int rw, hipStream_t st) {
    switch (rw) {
    case 1: return launch_dec_rw<HD, 1, KVT, QT>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

template <int KVT, int QT>
static hipError_t dec_dispatch_hd(const DecodeArgs &a, dim3 grid, int rw, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return launch_dec_t<128, KVT, QT>(a, grid, rw, st);
    case 256: return launch_dec_t<256, KVT, QT>(a, grid, rw, st);
    default: return hipErrorNotSupported;
    }
}

// Upper bound of the work items (sequence, chunk, kv head) of a launch: every chunk up to max_pos, or, under a sliding
// window with consecutive token positions, the at most (window + T - 2) / chunk + 2 chunks a window of window + T - 1
// keys meets (a 32K-key cache with a 1K window then launches 6 items per sequence and head, not 128).
static long long decode_items_bound(const Problem &p, int chunk) {
    long long per = p.max_pos / chunk + 1;
    if (p.window > 0 && (p.T == 1 || p.pos_mode == 1)) {
        const long long w = ((long long)p.window + p.T - 2) / chunk + 2;
        if (w < per) per = w;
    }
    return per * p.NKV * p.nseq;
}

bool decode_stream_supported(const Problem &p) {
    // One 16-row block (RW = 1). The kernel also runs RW = 2..4 row blocks, one wave each per key lane, but then
    // the row waves re-read every tile, which measured slower than the cooperative split kernel on the B=16 x
    // 8-token tree workload (205 vs 193 us), so those shapes go to the split kernel.
    return p.T >= 1 && (p.HD == 128 || p.HD == 256) && p.NQ % p.NKV == 0 && p.T * (p.NQ / p.NKV) <= 16 &&
           p.kv_dtype != DT_FP32;
}

hipError_t launch_decode_stream(const Problem &p, int chunk, const Partials &part, hipStream_t st) {
    if (!decode_stream_supported(p)) return hipErrorNotSupported;
    if (chunk <= 0 || chunk % 16) return hipErrorInvalidValue;
    if (p.max_pos / chunk + 1 > part.ns_cap) return hipErrorInvalidValue;
    DecodeArgs a{p, part, chunk, p.scale * kLog2e};
    const long long items = decode_items_bound(p, chunk);
    if (items > INT_MAX) return hipErrorInvalidConfiguration;
    dim3 grid((unsigned)items);
    const int rw = (p.T * (p.NQ / p.NKV) + 15) / 16;   // 16-row blocks, one wave each per key lane
    const int kv = p.kv_dtype, q = p.q_dtype;
    if (kv == DT_F16 && q == DT_FP32) return dec_dispatch_hd<DT_F16, DT_FP32>(a, grid, rw, st);
    if (kv == DT_F16 && q == DT_F16) return dec_dispatch_hd<DT_F16, DT_F16>(a, grid, rw, st);
    if (kv == DT_BF16 && q == DT_FP32) return dec_dispatch_hd<DT_BF16, DT_FP32>(a, grid, rw, st);
    if (kv == DT_BF16 && q == DT_BF16) return dec_dispatch_hd<DT_BF16, DT_BF16>(a, grid, rw, st);
    return hipErrorNotSupported;
}

// ---------------------------------------------------------------- fp32 caches
// The same streaming decode in fp32 end to end (fp32 Q, K, V, P and accumulators) for fp32 caches, the
// reference's fp32 decode path (attention.cuh:120-198, attention_decode_split.cuh:228; its gate asks for a
// normalised error below 1e-5): S^T = K Q^T and O^T += V^T P^T on the fp32 MFMA v_mfma_f32_16x16x4_f32.
// Operands (16x16x4: A lane l holds A[l % 16][l / 16], B lane l holds B[l / 16][l % 16]):
//   * QK k-step ks (4 head dims): lane (key/row ln, group g) holds dim 16 (ks / 4) + 4 g + ks % 4, so one 16-byte
//     LDS read of K (and of Q) row ln at dims 16 kq + 4 g feeds four k-steps;
//   * PV k-step kb (4 keys): lane group g holds key 4 g + kb, which is element kb of the lane's own S^T fragment,
//     so P^T never moves; the V^T operand is V[4 g + kb][16 db + ln], one 4-byte LDS read.
template <int HD>
struct DecodeF32Cfg {
    static constexpr int NKL = 2, NW = 2, KT = 16;
    static constexpr int KQ = HD / 16;                 // 16-dim blocks (4 QK k-steps each; PV output blocks)
    static constexpr int STR = HD + 4;                 // LDS row stride (floats)
    static constexpr int VCH = KT * HD / 4 / 64;       // 16-byte chunks per lane per tile (K and V each)
    static constexpr int BSTR = HD + 4;
    static constexpr size_t LDS_Q = (size_t)16 * STR * 4;
    static constexpr size_t LDS_V = (size_t)NW * KT * STR * 4;
    static constexpr size_t LDS_MERGE = ((size_t)2 * NW * 16 + (size_t)16 * BSTR) * 4;
    static constexpr size_t LDS = LDS_Q + (LDS_V > LDS_MERGE ? LDS_V : LDS_MERGE);
};

__device__ __forceinline__ f32x4 mfma4f32(float a, float b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int HD>
__global__ void __launch_bounds__(128) decode_f32_kernel(const DecodeArgs a) {
    using Cf = DecodeF32Cfg<HD>;
    constexpr int NKL = Cf::NKL, NW = Cf::NW, KT = Cf::KT, KQ = Cf::KQ;
    extern __shared__ __align__(16) unsigned char smem[];
    const Problem &p = a.p;
    const int C = a.C;
    int seq, c, lo, hi;
    if (!find_item(p, C, seq, c, lo, hi)) return;
    seq = __builtin_amdgcn_readfirstlane(seq); c = __builtin_amdgcn_readfirstlane(c);
    lo = __builtin_amdgcn_readfirstlane(lo); hi = __builtin_amdgcn_readfirstlane(hi);
    const int kvh = (int)blockIdx.x % p.NKV;
    const int GRP = p.NQ / p.NKV, nrows = p.T * GRP;
    const int j_lo = max(c * C, lo), j_hi = min(c * C + C, hi);
    if (j_lo >= j_hi) return;

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, ln = lane & 15;
    const int kl = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t krow = (size_t)p.NKV * HD;
    const float *Kb = kv_base<float>(p, false, seq) + (size_t)kvh * HD;
    const float *Vb = kv_base<float>(p, true, seq) + (size_t)kvh * HD;
    float *qs = reinterpret_cast<float *>(smem);
    float *redm = reinterpret_cast<float *>(smem + Cf::LDS_Q), *redl = redm + NW * 16, *buf = redl + NW * 16;
    float *ts = reinterpret_cast<float *>(smem + Cf::LDS_Q) + (size_t)kl * KT * Cf::STR;   // K, then V, of a tile

    // Q rows (zero past the last row) -> LDS.
    const float *Qf = reinterpret_cast<const float *>(p.Q);
    for (int i = tid; i < 16 * (HD / 4); i += NW * 64) {
        const int rho = i / (HD / 4), col = (i % (HD / 4)) * 4;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (rho < nrows)
            v = *reinterpret_cast<const f32x4 *>(Qf + ((size_t)(seq * p.T + rho / GRP) * p.NQ + kvh * GRP + rho % GRP) * HD + col);
        *reinterpret_cast<f32x4 *>(qs + rho * Cf::STR + col) = v;
    }
    int lo_max = 0, pos_min = INT_MAX;
    for (int t = 0; t < p.T; t++) {
        const int ps = tok_pos(p, seq, t);
        lo_max = max(lo_max, win_lo(ps, p.window)); pos_min = min(pos_min, ps);
    }
    if (p.anc) pos_min = min(pos_min, tok_pos(p, seq, 0) - 1);
    RowMask rm;
    {
        rm.valid = ln < nrows;
        const int t = rm.valid ? ln / GRP : 0;
        rm.pos = tok_pos(p, seq, t); rm.lo = win_lo(rm.pos, p.window); rm.tree = p.anc != nullptr;
        rm.anc = p.anc ? p.anc[seq * p.T + t] : 0u; rm.tb = tok_pos(p, seq, 0);
    }
    __syncthreads();

    const int tb0 = j_lo / KT - c * (C / KT), tb1 = (j_hi - 1) / KT - c * (C / KT);
    const int k0 = tb0 <= kl ? 0 : (tb0 - kl + NKL - 1) / NKL;
    const int k1 = tb1 < kl ? 0 : (tb1 - kl) / NKL + 1;
    float m = kNegInf, l = 0.f;
    f32x4 acc[KQ];
#pragma unroll
    for (int db = 0; db < KQ; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = k0; k < k1; k++) {
        const int jt = c * C + KT * (kl + NKL * k), jrow = key_row(p, jt);
        f32x4 kr[Cf::VCH], vr[Cf::VCH];
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {    // whole rows, 16 bytes per lane; the last tile clamps to the last key
            const int q = lane + 64 * u, key = q / (HD / 4), col = (q % (HD / 4)) * 4;
            const size_t off = (size_t)(jrow + min(key, hi - 1 - jt)) * krow + col;
            kr[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(Kb + off));
            vr[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(Vb + off));
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 4), col = (q % (HD / 4)) * 4;
            *reinterpret_cast<f32x4 *>(ts + key * Cf::STR + col) = kr[u];
        }
        __builtin_amdgcn_wave_barrier();
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int kq = 0; kq < KQ; kq++) {
            const f32x4 kf = *reinterpret_cast<const f32x4 *>(ts + ln * Cf::STR + 16 * kq + 4 * g);
            const f32x4 qf = *reinterpret_cast<const f32x4 *>(qs + ln * Cf::STR + 16 * kq + 4 * g);
            s0 = mfma4f32(kf.x, qf.x, s0); s1 = mfma4f32(kf.y, qf.y, s1);
            s0 = mfma4f32(kf.z, qf.z, s0); s1 = mfma4f32(kf.w, qf.w, s1);
        }
        const f32x4 sc = (s0 + s1) * a.sl2;
        float tv[4];
        const bool full = jt >= j_lo && jt + KT <= j_hi && jt >= lo_max && jt + KT - 1 <= pos_min;
#pragma unroll
        for (int i = 0; i < 4; i++) tv[i] = sc[i];
        if (!full) {                                            // one wave-uniform test; per key only off the fast path
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = jt + 4 * g + i;
                if (!((key >= j_lo) & (key < j_hi) & rm.attends(key))) tv[i] = kNegInf;
            }
        }
        float mx = fmaxf(fmaxf(tv[0], tv[1]), fmaxf(tv[2], tv[3]));
        mx = max_over_groups(mx);
        const float mnew = (mx > m + kRescaleThreshold) ? mx : m;
        if (__any(mnew != m)) {
            const float alpha = (mnew == m) ? 1.f : fast_exp2(m - mnew);
            l *= alpha; m = mnew;
#pragma unroll
            for (int db = 0; db < KQ; db++) acc[db] *= alpha;
        }
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) pv[i] = fast_exp2(tv[i] - m);
        if (m == kNegInf) pv[0] = pv[1] = pv[2] = pv[3] = 0.f;
        l += (pv[0] + pv[1]) + (pv[2] + pv[3]);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int u = 0; u < Cf::VCH; u++) {
            const int q = lane + 64 * u, key = q / (HD / 4), col = (q % (HD / 4)) * 4;
            *reinterpret_cast<f32x4 *>(ts + key * Cf::STR + col) = vr[u];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int db = 0; db < KQ; db++)
#pragma unroll
            for (int kb = 0; kb < 4; kb++) acc[db] = mfma4f32(ts[(4 * g + kb) * Cf::STR + 16 * db + ln], pv[kb], acc[db]);
    }
    l = sum_over_groups(l);

    // Merge the two key-lane states in key-lane order, then write the chunk partial of each row.
    __syncthreads();
    if (g == 0) { redm[kl * 16 + ln] = m; redl[kl * 16 + ln] = l; }
    __syncthreads();
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NKL; w++) M = fmaxf(M, redm[w * 16 + ln]);
    const float f = (m == kNegInf) ? 0.f : fast_exp2(m - M);
    for (int w = 0; w < NKL; w++) {
        if (kl == w && ln < nrows) {
#pragma unroll
            for (int db = 0; db < KQ; db++) {
                f32x4 *dst = reinterpret_cast<f32x4 *>(buf + ln * Cf::BSTR + 16 * db + 4 * g);
                f32x4 v = acc[db] * f;
                if (w > 0) v += *dst;
                *dst = v;
            }
        }
        __syncthreads();
    }
    const int ns = a.part.ns_cap;
    auto part_index = [&](int rho) {
        return ((size_t)(seq * p.T + rho / GRP) * p.NQ + kvh * GRP + rho % GRP) * ns + c;
    };
    for (int idx = tid; idx < nrows * (HD / 4); idx += NW * 64) {
        const int rho = idx / (HD / 4), d4 = idx % (HD / 4);
        *reinterpret_cast<f32x4 *>(a.part.acc + part_index(rho) * HD + 4 * d4) =
            *reinterpret_cast<const f32x4 *>(buf + (size_t)rho * Cf::BSTR + 4 * d4);
    }
    for (int rho = tid; rho < nrows; rho += NW * 64) {
        float Mr = kNegInf;
        for (int w = 0; w < NKL; w++) Mr = fmaxf(Mr, redm[w * 16 + rho]);
        float L = 0.f;
        if (Mr != kNegInf)
            for (int w = 0; w < NKL; w++) {
                const float mw = redm[w * 16 + rho];
                if (mw != kNegInf) L += redl[w * 16 + rho] * fast_exp2(mw - Mr);
            }
        a.part.m[part_index(rho)] = Mr; a.part.l[part_index(rho)] = L;
    }
}

bool decode_f32_supported(const Problem &p) {
    return p.kv_dtype == DT_FP32 && p.q_dtype == DT_FP32 && (p.HD == 128 || p.HD == 256) && p.NQ % p.NKV == 0 &&
           p.T * (p.NQ / p.NKV) <= 16;
}

hipError_t launch_decode_f32(const Problem &p, int chunk, const Partials &part, hipStream_t st) {
    if (!decode_f32_supported(p)) return hipErrorNotSupported;
    if (chunk <= 0 || chunk % 16) return hipErrorInvalidValue;
    if (p.max_pos / chunk + 1 > part.ns_cap) return hipErrorInvalidValue;
    DecodeArgs a{p, part, chunk, p.scale * kLog2e};
    const long long items = decode_items_bound(p, chunk);
    if (items > INT_MAX) return hipErrorInvalidConfiguration;
    dim3 grid((unsigned)items);
    if (p.HD == 128) {
        static bool conf = false;
        if (!conf) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&decode_f32_kernel<128>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)DecodeF32Cfg<128>::LDS);
            if (e != hipSuccess) return e;
            conf = true;
        }
        hipLaunchKernelGGL(decode_f32_kernel<128>, grid, dim3(128), DecodeF32Cfg<128>::LDS, st, a);
    } else {
        static bool conf = false;
        if (!conf) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&decode_f32_kernel<256>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)DecodeF32Cfg<256>::LDS);
            if (e != hipSuccess) return e;
            conf = true;
        }
        hipLaunchKernelGGL(decode_f32_kernel<256>, grid, dim3(128), DecodeF32Cfg<256>::LDS, st, a);
    }
    return hipGetLastError();
}

}  // namespace dgx

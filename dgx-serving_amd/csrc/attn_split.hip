// Split-KV GQA attention for verify, speculative tree verify and the decode shapes the streaming decode kernel
// does not take (fp32 caches, HD 512, more than 16 query heads per KV head) on gfx950.
//
// Replaces the reference's attn_split_p1_kernel / attn_split_combine_kernel
// (kernels/attention_decode_split.cuh:43-165) and, for short query runs, flash_attn2bs_p1(_custom)_kernel /
// flash_attn2bs_p2_kernel (kernels/attention_flash.cuh:28-227).
//
// Grid: (kv head, chunk c, sequence x query-token tile). One workgroup = 4 wave64s. It owns the query rows
// (token, head) of one KV head (GQA group, rows token-major, RB blocks of 16) for a token tile and the keys
// [c*C, (c+1)*C) of its sequence, and writes one LSE partial per (row, chunk). The chunk's keys stream in
// 16-key tiles at absolute positions:
//   * the workgroup fetches each K and V tile cooperatively with 16-byte loads (whole head rows),
//     two tiles ahead in registers, and stages it in a double-buffered LDS tile (one barrier per tile),
//   * every wave computes S^T = K Q^T for all rows of the tile on 16x16x32 MFMA (Q fragments in registers when
//     they fit, else from LDS), applies the causal / sliding-window / tree mask and the online softmax on the
//     S^T fragment (a query row sits in 4 lanes; row max and row sum are two xor shuffles),
//   * wave w accumulates O^T += V^T P^T for head dims [w*HD/4, (w+1)*HD/4) on 16x16x16 MFMA, V^T fragments read
//     with the gfx950 transpose read (ds_read_b64_tr_b16), P^T straight from the softmax registers.
// Every K/V byte of a chunk is read once per workgroup and serves all GRP query heads of the KV head.
// With 2-4 row blocks (RB >= 2) wave w instead owns row block w with all head dims, so no S or PV work is repeated
// across waves. For 16-bit caches at HD 128/256 those shapes (verify and tree verify runs) go to verify_kernel,
// the same layout fed by a four-stage direct-to-LDS ring (global_load_lds, no staging registers) over a grid of
// resident workgroups that each stream an equal run of key tiles (see seg_scan).
//
// Invariants (kept from the reference, attention_decode_split.cuh:8-12) for split_kernel: chunk and tile
// boundaries are absolute key positions and the chunk combine runs in fixed order. A row's result therefore does
// not depend on the batch, the other rows of its tile, the grid size or the maximum position: a row is
// bit-identical alone or as a batch row. verify_kernel keeps this in its default mode (slot_runs: partials at
// absolute key chunks of each sequence); its other mode gives it up for equal runs (boundaries that follow the total
// key count), deterministic for given inputs.
#include "attn_device.h"
#include "attn_internal.h"
#include <algorithm>
#include <climits>
#include <cstdlib>

namespace dgx {

struct SplitArgs {
    Problem p;
    Partials part;
    int C;          // chunk (keys), multiple of 32
    int tpb;        // query tokens per workgroup
    int nchunks;    // token tiles per sequence
    float sl2;      // scale * log2(e)
    int slot_runs = 1;   // verify_kernel: 1 = runs are each pair's absolute key chunks (batch-invariant), 0 = equal runs
};

// Wave-wide reductions over all 64 lanes (fixed xor-butterfly order, identical result in every lane).
__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Work split of verify_kernel. Pair z is (sequence, token tile) with n_z key tiles per KV head. The key tiles of one
// KV head's list (pairs in order) are cut into G / NKV equal runs of q tiles, and every KV head takes the same cut:
// workgroup w streams run w / NKV of KV head w % NKV. So every workgroup streams the same number of bytes whatever
// the mix of sequence lengths (a grid of fixed key chunks leaves a partly filled last round of workgroups), and
// the NKV workgroups that read the head slices of the same key rows run side by side (HBM row locality). A run
// writes one partial per pair it meets, into slot (run index - index of the pair's first run); the last run of a
// pair marks the slot after its own for the combine. q depends on the total tile count, so verify results depend
// on the batch; they are deterministic for given inputs.
// With slot_runs (the default) each cut moves forward to the next absolute key-chunk boundary of its pair (C keys),
// and a run flushes its state into partial slot (key / C) at every chunk boundary it crosses: the float operations
// of a chunk then start from a fresh state at the chunk's first key whatever run holds it, so a row's result
// depends only on its own sequence (the combine reads slots lo / C .. pos / C as for split_kernel). The cost is the
// cut granularity: runs differ by up to C keys.
struct SegPair { int seq, tok0, tok1, lo, hi, jb, n; };

__device__ __forceinline__ SegPair seg_pair(const Problem &p, int tpb, int nchunks, int z) {
    SegPair s;
    s.seq = z / nchunks;
    s.tok0 = (z % nchunks) * tpb;
    s.tok1 = min(p.T, s.tok0 + tpb);
    s.lo = INT_MAX; s.hi = 0;
    for (int t = s.tok0; t < s.tok1; t++) {
        const int ps = tok_pos(p, s.seq, t);
        s.lo = min(s.lo, win_lo(ps, p.window)); s.hi = max(s.hi, ps + 1);
    }
    s.jb = (s.lo / 16) * 16;
    s.n = (s.hi - s.jb + 15) / 16;
    return s;
}

// The same for a z that is equal in every lane of the wave (seg_pair itself also serves one pair per lane).
__device__ __forceinline__ SegPair seg_pair_u(const Problem &p, int tpb, int nchunks, int z) {
    SegPair s = seg_pair(p, tpb, nchunks, __builtin_amdgcn_readfirstlane(z));
    s.lo = __builtin_amdgcn_readfirstlane(s.lo); s.hi = __builtin_amdgcn_readfirstlane(s.hi);
    s.jb = __builtin_amdgcn_readfirstlane(s.jb); s.n = __builtin_amdgcn_readfirstlane(s.n);
    return s;
}

// Over pairs z = 0 .. nseq * nchunks - 1 (pair z holds n_z tiles per KV head): the total N, the pair zx holding
// tile x of one KV head's list and the tiles before it px, and the tiles before pair zq (pq). Called by whole waves
// (wave-uniform).
__device__ __forceinline__ void seg_scan(const Problem &p, int tpb, int nchunks, int x, int zq, int &N, int &zx,
                                         int &px, int &pq) {
    const int lane = threadIdx.x & 63, nz = p.nseq * nchunks;
    N = 0; zx = -1; px = 0; pq = 0;
    for (int z0 = 0; z0 < nz; z0 += 64) {
        const int zl = z0 + lane;
        const int cnt = zl < nz ? seg_pair(p, tpb, nchunks, zl).n : 0;
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (zq >= z0 && zq < z0 + 64) pq = N + __shfl(incl, zq - z0) - __shfl(cnt, zq - z0);
        if (zx < 0) {
            const unsigned long long hit = __ballot(N + incl > x);
            if (hit) {
                const int l = __builtin_ctzll(hit);
                zx = z0 + l;
                px = N + __shfl(incl, l) - __shfl(cnt, l);
            }
        }
        N += __shfl(incl, 63);
    }
    // The results are the same in every lane: say so, so that they and what derives from them live in SGPRs.
    N = __builtin_amdgcn_readfirstlane(N); zx = __builtin_amdgcn_readfirstlane(zx);
    px = __builtin_amdgcn_readfirstlane(px); pq = __builtin_amdgcn_readfirstlane(pq);
}

// LSE combine of the chunk partials of one (row, head) by a row group of PH * HD / 4 threads: thread (phase ph,
// 4-dim group d4) sums the chunks c = ph, ph + PH, ... of the row, each weighted by 2^(m_c - max m), in increasing
// order; the PH phase sums are then added in phase order. NB chunks per thread are requested at once, so a row of
// up to PH * NB chunks costs one memory round trip. HD 512 rows (a 32K-key cache holds 64 chunks of 512 keys, at
// 2 KB of partial each) take eight phases; narrower rows take one wave each. The phase count depends
// only on the head dim: a row's result does not depend on the batch.
template <int HD> struct CombineCfg {
    static constexpr int PH = HD >= 512 ? 8 : 256 / HD;   // chunk phases per row (a row is at least one wave)
    static constexpr int D4 = HD / 4, RT = PH * D4;  // threads per row
    static constexpr int NR = RT >= 128 ? 1 : 128 / RT;   // rows per workgroup
    static constexpr int NT = NR * RT, NWR = (RT + 63) / 64;   // threads, waves per row
    static constexpr int NB = PH >= 8 ? 8 : 16;      // partial rows in flight per thread
    static_assert(RT % 64 == 0, "a row is whole waves");
};

template <int HD>
__global__ void __launch_bounds__(CombineCfg<HD>::NT) combine_kernel(const Problem p, const Partials part, int C) {
    using Cf = CombineCfg<HD>;
    constexpr int D4 = Cf::D4, NB = Cf::NB, NWR = Cf::NWR, PH = Cf::PH, NR = Cf::NR;
    __shared__ float red[NR][2 * NWR];
    __shared__ f32x4 sum[NR][PH > 1 ? PH - 1 : 1][D4];
    const int tid = threadIdx.x, lane = tid & 63, rg = tid / Cf::RT, rt = tid % Cf::RT;
    const int wave = rt >> 6, ph = rt / D4, d4 = rt % D4;
    const int rh = blockIdx.x * NR + rg;
    const bool live = rh < p.nseq * p.T * p.NQ;      // row-group uniform (whole waves)
    const int rr = live ? rh : 0, r = rr / p.NQ, h = rr % p.NQ, s = r / p.T, t = r % p.T;
    // Chunks [c_lo, c_lo + n) of the row. verify_kernel's partials sit in slots 0 .. n-1, and its last run of each
    // pair marks slot n (when there is one) with m = +inf: n is the first marked slot (every wave finds the same).
    int c_lo = 0, n = 0;
    if (!live) {
    } else if (part.seg_g == 0) {
        const int pos = tok_pos(p, s, t), lo = win_lo(pos, p.window);
        c_lo = lo / C; n = pos / C - c_lo + 1;
    } else {
        const size_t b0 = ((size_t)r * p.NQ + h) * part.ns_cap;
        n = part.ns_cap;
        for (int c0 = 0; c0 < part.ns_cap; c0 += 64) {
            const int c = c0 + lane;
            const float mv = c < part.ns_cap ? part.m[b0 + c] : kPosInf;
            const unsigned long long hit = __ballot(mv == kPosInf);
            if (hit) { n = c0 + __builtin_ctzll(hit); break; }
        }
    }
    const size_t base = ((size_t)r * p.NQ + h) * part.ns_cap + c_lo;
    const float *accb = part.acc + base * HD + 4 * d4;
    // Statistics of chunks rt, rt + RT, ... (the first are requested ahead of the accumulators).
    float m0 = kNegInf, l0 = 0.f;
    if (rt < n) { m0 = part.m[base + rt]; l0 = part.l[base + rt]; }
    f32x4 v[NB];
    float mc[NB];
    auto load_batch = [&](int c0) {                  // chunks c0 + ph + PH u
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int c = c0 + ph + PH * u;
            mc[u] = kNegInf;
            if (c < n) {
                v[u] = *reinterpret_cast<const f32x4 *>(accb + (size_t)c * HD);
                mc[u] = part.m[base + c];
            }
        }
    };
    load_batch(0);                                   // in flight while the statistics are reduced
    // Row statistics: max of m, then L = sum of l_c 2^(m_c - max) (thread-strided, then wave, then wave order).
    float mx = m0;
    for (int c = rt + Cf::RT; c < n; c += Cf::RT) mx = fmaxf(mx, part.m[base + c]);
    mx = wave_max(mx);
    float mg = mx;
    if constexpr (NWR > 1) {
        if (lane == 0) red[rg][wave] = mx;
        __syncthreads();
        mg = kNegInf;
#pragma unroll
        for (int w = 0; w < NWR; w++) mg = fmaxf(mg, red[rg][w]);
    }
    float x = 0.f;
    if (mg != kNegInf) {
        if (m0 != kNegInf) x = l0 * fast_exp2(m0 - mg);
        for (int c = rt + Cf::RT; c < n; c += Cf::RT) {
            const float m = part.m[base + c];
            if (m != kNegInf) x += part.l[base + c] * fast_exp2(m - mg);
        }
    }
    float L = wave_sum(x);
    if constexpr (NWR > 1) {
        if (lane == 0) red[rg][NWR + wave] = L;
        __syncthreads();
        L = 0.f;
#pragma unroll
        for (int w = 0; w < NWR; w++) L += red[rg][NWR + w];
    }
    // This thread's phase sum.
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < n; c0 += PH * NB) {
        if (c0 > 0) load_batch(c0);
#pragma unroll
        for (int u = 0; u < NB; u++) {
            if (mc[u] != kNegInf && mg != kNegInf) acc += v[u] * fast_exp2(mc[u] - mg);
        }
    }
    if constexpr (PH > 1) {
        if (ph > 0) sum[rg][ph - 1][d4] = acc;
        __syncthreads();
        if (ph > 0) return;
#pragma unroll
        for (int k = 0; k < PH - 1; k++) acc += sum[rg][k][d4];
    }
    if (!live) return;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    f32x4 o = acc * inv;
    const size_t oi = ((size_t)r * p.NQ + h) * HD + 4 * d4;
    if (p.gate) {                                    // output gate: o *= 1 / (1 + 2^(-g log2 e))
        float gv[4];
        if (p.gate_dtype == DT_FP32) {
            const f32x4 gg = *reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(p.gate) + oi);
            gv[0] = gg.x; gv[1] = gg.y; gv[2] = gg.z; gv[3] = gg.w;
        } else {
            const u32x2 gw = *reinterpret_cast<const u32x2 *>(reinterpret_cast<const uint16_t *>(p.gate) + oi);
            const bool f16 = p.gate_dtype == DT_F16;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint16_t b16 = (uint16_t)(gw[e / 2] >> (16 * (e & 1)));
                gv[e] = f16 ? f16_bits_to_f32(b16) : bf16_bits_to_f32(b16);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] *= 1.f / (1.f + fast_exp2(-gv[e] * kLog2e));
    }
    if (p.o_dtype == DT_FP32) *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.O) + oi) = o;
    else {
        const bool f16 = p.o_dtype == DT_F16;
        const u32x2 ow = u32x2{(uint32_t)f32_to_op(o.x, f16) | ((uint32_t)f32_to_op(o.y, f16) << 16),
                               (uint32_t)f32_to_op(o.z, f16) | ((uint32_t)f32_to_op(o.w, f16) << 16)};
        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(p.O) + oi) = ow;
    }
    if (p.lse && rt == 0) p.lse[(size_t)r * p.NQ + h] = (L > 0.f) ? (mg + log2f(L)) * kLn2 : kNegInf;
}

template <int HD, int RB>
struct SplitCfg {
    static constexpr int NW = 4;              // waves per workgroup; wave w owns head dims [w*HD/NW, (w+1)*HD/NW)
    static constexpr int KT = 16;             // keys per tile (KT/16 sub-tiles of 16 keys)
    static constexpr int NSUB = KT / 16;
    static constexpr int KS = HD / 32;        // QK k-steps (16x16x32)
    static constexpr int DBW = HD / 16 / NW;  // PV output dim blocks (16x16x16) per wave
    static constexpr int STR = HD + 16;       // LDS row stride of Q, K and V tiles (16-bit elements; +16: the
                                              // fragment and transpose reads are free of bank conflicts)
    static constexpr int RR = RB * 16;        // query rows per workgroup
    static constexpr int CPT = KT * HD / 8 / (NW * 64);   // 16-byte chunks per thread per tile (K and V each)
    static constexpr int NSTG = 2;                          // register stages of the K/V stream
    static constexpr size_t TILE = (size_t)KT * STR;      // elements of one K or V tile
    static constexpr bool QREG = RB * KS <= 16;           // Q fragments live in registers (straight from HBM)
    static constexpr size_t LDS = ((QREG ? 0 : (size_t)RR * STR) + 4 * TILE) * 2;   // [Q] + (K, V) x double buffer
    static_assert(CPT >= 1 && (KT * HD / 8) % (NW * 64) == 0, "tile chunks");
};


template <int HD, int RB, int KVT, int QT>
__global__ void __launch_bounds__(256) split_kernel(const SplitArgs a) {
    using Cf = SplitCfg<HD, RB>;
    constexpr int NW = Cf::NW;
    constexpr bool F16 = OpIsF16<KVT>::value;
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];

    const Problem &p = a.p;
    // blockIdx.x = kv head (fastest), so the NKV workgroups of one key chunk are dispatched together and read the
    // interleaved head slices of the same cache rows at the same time.
    const int kvh = blockIdx.x, c = blockIdx.y;
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

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, ln = lane & 15;
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = kv_base<KE>(p, false, seq) + (size_t)kvh * HD;
    const KE *Vb = kv_base<KE>(p, true, seq) + (size_t)kvh * HD;
    // Two wave layouts. RB == 1: every wave computes S for the 16 rows and owns HD/4 output dims of PV. RB >= 2: wave
    // w owns row block w (all dims), so S and PV are not repeated across waves; waves past the last row block only
    // fetch and stash.
    constexpr bool ROWS = RB >= 2;
    constexpr int RBW = ROWS ? 1 : RB;                          // row blocks held by a wave
    constexpr int DBN = ROWS ? HD / 16 : Cf::DBW;               // 16-dim PV blocks of a wave
    auto rbg = [&](int j) { return ROWS ? wave : j; };         // row block of a wave's j-th block
    const int dim0 = ROWS ? 0 : wave * (HD / NW);               // first output dim of the wave
    const bool active = !ROWS || wave < RB;
    constexpr bool QREG = ROWS ? RBW * Cf::KS <= 8 : Cf::QREG;
    uint16_t *qs = reinterpret_cast<uint16_t *>(smem);
    uint16_t *tiles = qs + (Cf::QREG ? 0 : (size_t)Cf::RR * Cf::STR);   // [buf][K | V][KT][STR]

    // Q rows of the workgroup (row rho = token-major (token, head)) in the MFMA operand format: straight into
    // registers when they fit (lane (row ln, group g) holds dims 32 ks + 8 g ..), else through LDS.
    u32x4 qreg[QREG ? RBW : 1][QREG ? Cf::KS : 1];
    if constexpr (QREG) {
#pragma unroll
        for (int j = 0; j < RBW; j++) {
            const int rho = rbg(j) * 16 + ln;
            const bool ok = rho < nrows;
            const int t = tok0 + (ok ? rho / GRP : 0), h = kvh * GRP + (ok ? rho % GRP : 0);
            const QE *qrow = reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + t) * p.NQ + h) * HD + 8 * g;
#pragma unroll
            for (int ks = 0; ks < Cf::KS; ks++) qreg[j][ks] = ok ? load8_op<QT, F16>(qrow + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
        }
    } else {
        for (int i = tid; i < Cf::RR * (HD / 8); i += NW * 64) {
            const int rho = i / (HD / 8), col = (i % (HD / 8)) * 8;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (rho < nrows) {
                const int t = tok0 + rho / GRP, h = kvh * GRP + rho % GRP;
                v = load8_op<QT, F16>(reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + t) * p.NQ + h) * HD + col);
            }
            *reinterpret_cast<u32x4 *>(qs + rho * Cf::STR + col) = v;
        }
    }
    RowMask rm[RBW];
#pragma unroll
    for (int j = 0; j < RBW; j++) {
        const int rho = rbg(j) * 16 + ln;
        const bool valid = rho < nrows;
        const int t = tok0 + (valid ? rho / GRP : 0);
        const int ps = tok_pos(p, seq, t);
        rm[j].pos = ps; rm[j].lo = win_lo(ps, p.window); rm[j].valid = valid;
        rm[j].tree = p.anc != nullptr;
        rm[j].anc = p.anc ? p.anc[seq * p.T + t] : 0u;
        rm[j].tb = p.anc ? tok_pos(p, seq, 0) : 0;
    }

    // Block-uniform bounds for the unmasked fast path: a tile is "full" when every valid row attends all its keys.
    int lo_max = 0, pos_min = INT_MAX;
    for (int t = tok0; t < tok1; t++) {
        const int ps = tok_pos(p, seq, t);
        lo_max = max(lo_max, win_lo(ps, p.window));
        pos_min = min(pos_min, ps);
    }
    if (p.anc) pos_min = min(pos_min, tok_pos(p, seq, 0) - 1);   // tree keys are never in the fast path

    // Cooperative tile fetch (global -> registers): chunk q = tid + 256*u -> key q / (HD/8), column (q % (HD/8))*8.
    // NSTG register stages keep the loads of the next NSTG tiles in flight while tile it is computed from LDS (HBM
    // bandwidth grows with the bytes in flight, and a decode tile's compute is short).
    constexpr int NSTG = Cf::NSTG;
    u32x4 kst[NSTG][Cf::CPT], vst[NSTG][Cf::CPT];
    auto fetch = [&](u32x4 (&kr)[Cf::CPT], u32x4 (&vr)[Cf::CPT], int jt) {
        // A tile past the last one re-reads the last (in a ring its row base is that of the last tile).
        const int jc = min(jt, ((hi_b - 1) / Cf::KT) * Cf::KT), jrow = key_row(p, jc);
#pragma unroll
        for (int u = 0; u < Cf::CPT; u++) {
            const int q = tid + NW * 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            const size_t off = (size_t)(jrow + min(key, hi_b - 1 - jc)) * krow + col;
            kr[u] = load8_op<KVT, F16>(Kb + off);
            vr[u] = load8_op<KVT, F16>(Vb + off);
        }
    };
    auto stash = [&](const u32x4 (&kr)[Cf::CPT], const u32x4 (&vr)[Cf::CPT], int buf) {
        uint16_t *kt = tiles + (size_t)buf * 2 * Cf::TILE, *vt = kt + Cf::TILE;
#pragma unroll
        for (int u = 0; u < Cf::CPT; u++) {
            const int q = tid + NW * 64 * u, key = q / (HD / 8), col = (q % (HD / 8)) * 8;
            *reinterpret_cast<u32x4 *>(kt + key * Cf::STR + col) = kr[u];
            *reinterpret_cast<u32x4 *>(vt + key * Cf::STR + col) = vr[u];
        }
    };

    float m[RBW], l[RBW], mnew[RBW];
    f32x4 acc[RBW][DBN];
#pragma unroll
    for (int rb = 0; rb < RBW; rb++) {
        m[rb] = kNegInf; l[rb] = 0.f;
#pragma unroll
        for (int db = 0; db < DBN; db++) acc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int jb = (j_lo / Cf::KT) * Cf::KT;
    const int ntile = (j_hi - jb + Cf::KT - 1) / Cf::KT;
#pragma unroll
    for (int k = 0; k < NSTG; k++) fetch(kst[k], vst[k], jb + Cf::KT * k);
    stash(kst[0], vst[0], 0);
    __syncthreads();                                           // tile 0 (and the Q rows without QREG) in LDS

    auto compute = [&](int it) {
        const int jt = jb + Cf::KT * it;
        const uint16_t *kt = tiles + (size_t)(it & 1) * 2 * Cf::TILE, *vt = kt + Cf::TILE;
        // S^T[key][row] = K Q^T (every wave computes the whole tile), two independent MFMA chains per sub-tile.
        constexpr int NSUB = Cf::NSUB;
        f32x4 s[NSUB][RBW], s2[NSUB][RBW];
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int rb = 0; rb < RBW; rb++) s[sub][rb] = s2[sub][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < Cf::KS; ks++) {
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
                const u32x4 kf = *reinterpret_cast<const u32x4 *>(kt + (16 * sub + ln) * Cf::STR + 32 * ks + 8 * g);
#pragma unroll
                for (int rb = 0; rb < RBW; rb++) {
                    u32x4 qf;
                    if constexpr (QREG) qf = qreg[rb][ks];
                    else qf = *reinterpret_cast<const u32x4 *>(qs + (rbg(rb) * 16 + ln) * Cf::STR + 32 * ks + 8 * g);
                    if (ks & 1) s2[sub][rb] = mfma16<F16>(kf, qf, s2[sub][rb]);
                    else s[sub][rb] = mfma16<F16>(kf, qf, s[sub][rb]);
                }
            }
        }
        // Online softmax (log2 domain) over the tile's keys with a lazily moved reference max m (see
        // kRescaleThreshold). l holds this lane's share of the row sum; the four lanes of a row are added once,
        // after the loop.
        const bool full = jt >= j_lo && jt + Cf::KT <= j_hi && jt >= lo_max && jt + Cf::KT - 1 <= pos_min;
        PFrag<F16> pop[NSUB][RBW];
        float tv[NSUB][RBW][4];
        bool need = false;
#pragma unroll
        for (int rb = 0; rb < RBW; rb++) {
            float mx = kNegInf;
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
                const f32x4 sc = s[sub][rb] + s2[sub][rb];
#pragma unroll
                for (int i = 0; i < 4; i++) tv[sub][rb][i] = sc[i] * a.sl2;
            }
            if (!full) {                                        // one wave-uniform test; per key only off the fast path
#pragma unroll
                for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = jt + 16 * sub + 4 * g + i;
                        if (!(key >= j_lo && key < j_hi && rm[rb].attends(key))) tv[sub][rb][i] = kNegInf;
                    }
            }
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
                for (int i = 0; i < 4; i++) mx = fmaxf(mx, tv[sub][rb][i]);
            mx = max_over_groups(mx);
            if (mx > m[rb] + kRescaleThreshold) { mnew[rb] = mx; need = true; } else mnew[rb] = m[rb];
        }
        if (__any(need)) {
#pragma unroll
            for (int rb = 0; rb < RBW; rb++) {
                const float alpha = (mnew[rb] == m[rb]) ? 1.f : fast_exp2(m[rb] - mnew[rb]);
                l[rb] *= alpha; m[rb] = mnew[rb];
#pragma unroll
                for (int db = 0; db < DBN; db++) acc[rb][db] *= alpha;
            }
        }
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int rb = 0; rb < RBW; rb++) {
                float pv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) { pv[i] = (tv[sub][rb][i] == kNegInf) ? 0.f : fast_exp2(tv[sub][rb][i] - m[rb]); l[rb] += pv[i]; }
                pop[sub][rb] = p_frag<F16>(pv[0], pv[1], pv[2], pv[3]);
            }
        // O^T[this wave's dims] += V^T P^T (16x16x16): the A fragment is a transposed LDS read of the V tile.
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++) {
            const uint16_t *vtr = vt + (16 * sub + 4 * g + (ln >> 2)) * Cf::STR + dim0 + 4 * (ln & 3);
#pragma unroll
            for (int db = 0; db < DBN; db++) {
                const u32x2 vop = lds_read_tr16(vtr + 16 * db);
#pragma unroll
                for (int rb = 0; rb < RBW; rb++) acc[rb][db] = mfma_pv16<F16>(vop, pop[sub][rb], acc[rb][db]);
            }
        }
    };
    // Step it (stage k = it % NSTG): refill stage k with tile it+NSTG, compute tile it from LDS, stash tile it+1
    // (stage (k+1) % NSTG) into the other LDS buffer, barrier. Fetches and stashes are unconditional (past the last
    // tile a fetch re-reads the last key row, an L2 hit, and a stash fills a buffer that is never read again) so
    // that every wait before a stash sees exactly the younger stages' loads in flight and the compiler never has
    // to drain the pipeline at a control-flow merge.
    int it = 0;
    for (; it + NSTG <= ntile; it += NSTG) {
#pragma unroll
        for (int k = 0; k < NSTG; k++) {
            fetch(kst[k], vst[k], jb + Cf::KT * (it + k + NSTG));
            if (active) compute(it + k);
            stash(kst[(k + 1) % NSTG], vst[(k + 1) % NSTG], (it + k + 1) & 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int k = 0; k < NSTG; k++) {                            // the last ntile % NSTG tiles
        if (it + k < ntile) {
            if (active) compute(it + k);
            stash(kst[(k + 1) % NSTG], vst[(k + 1) % NSTG], (it + k + 1) & 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int rb = 0; rb < RBW; rb++) l[rb] = sum_over_groups(l[rb]);
    if (!active) return;

    // Chunk partial: a wave writes its dims of its rows (and (m, l): wave 0 of the dims split, every wave of the
    // rows split). Lane (row ln, group g) holds O^T[dims dim0 + 16*db + 4g + i][row].
    const int NQ = p.NQ, ns = a.part.ns_cap;
#pragma unroll
    for (int rb = 0; rb < RBW; rb++) {
        const int row = rbg(rb) * 16 + ln;
        if (row >= nrows) continue;
        const int r = seq * p.T + tok0 + row / GRP, h = kvh * GRP + row % GRP;
        const size_t pi = ((size_t)r * NQ + h) * ns + c;
#pragma unroll
        for (int db = 0; db < DBN; db++) {
            float *dst = a.part.acc + pi * HD + dim0 + 16 * db + 4 * g;
            *reinterpret_cast<f32x4 *>(dst) = acc[rb][db];
        }
        if ((ROWS || wave == 0) && g == 0) {
            a.part.m[pi] = m[rb]; a.part.l[pi] = l[rb];
        }
    }
}

// ---------------------------------------------------------------- verify / tree kernel (16-bit caches, 2-4 row blocks)
// The rows-split layout of split_kernel with a deeper K/V stream: tiles go from HBM straight into an NS-stage LDS
// ring with gfx950 direct-to-LDS loads (no staging registers, so more tiles in flight per workgroup at the same
// occupancy), rows unpadded with their 16-byte slots XOR-swizzled by the key. Wave w owns row block w (all head
// dims); the wave past the last row block only loads.
// Swizzles (slot s of key row k holds head-dim column s ^ swz(k)): K rows are read 16 bytes per lane by key
// (lane = key ln, column 4 ks + g), so kswz(ln) = ln puts the 8 (16) keys of a lane group on distinct bank quads;
// V rows are read by the transpose read with lane bit 1 selecting the column, so vswz keeps bit 0 free for it.
__device__ __forceinline__ int kswz(int k) { return k & 15; }
__device__ __forceinline__ int vswz(int k) { return ((k & 7) << 1) | ((k >> 3) & 1); }
typedef __attribute__((address_space(3))) void vlds_void;
typedef __attribute__((address_space(1))) void vglb_void;

template <int HD>
struct VerifyCfg {
    static constexpr int NW = 4, KT = 16, NS = 4;   // 64 KB of LDS at HD 256: two workgroups per CU
    static constexpr int KS = HD / 32, DB = HD / 16, SLOTS = HD / 8, ROWB = HD * 2;
    static constexpr int TILE = KT * ROWB;               // bytes of one K (or V) tile
    static constexpr int STAGE = 2 * TILE;
    static constexpr int NLD = KT * SLOTS / (NW * 64);    // direct-to-LDS loads per thread per tile and tensor
    static constexpr size_t LDS = (size_t)NS * STAGE;
    static_assert(NLD >= 1 && (KT * SLOTS) % (NW * 64) == 0, "tile loads");
};

// Tiles [t0, t1) of pair sp, KV head kvh (keys sp.jb + 16 t ..), into partial slot `slot`; `last`: the run ends
// the pair, and marks the next slot (if any) as the end of the pair's slots for the combine. Called by all waves;
// returns with every load landed (the caller's barrier then frees the ring).
template <int HD, int RB, int KVT, int QT>
__device__ __forceinline__ void verify_segment(const SplitArgs &a, const SegPair &sp, int kvh, int t0, int t1, int slot,
                                               bool last, unsigned char *smem) {
    using Cf = VerifyCfg<HD>;
    constexpr int NS = Cf::NS, KT = Cf::KT, KS = Cf::KS, DB = Cf::DB, NLD = Cf::NLD, SLOTS = Cf::SLOTS;
    constexpr int ROWB = Cf::ROWB;
    constexpr bool F16 = OpIsF16<KVT>::value;
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    const Problem &p = a.p;
    const int GRP = p.NQ / p.NKV, seq = sp.seq, tok0 = sp.tok0, tok1 = sp.tok1;
    const int nrows = (tok1 - tok0) * GRP, lo_b = sp.lo, hi_b = sp.hi;
    (void)lo_b;
    const int jb = sp.jb + KT * t0, ntile = t1 - t0;
    const int j_lo = max(jb, sp.lo), j_hi = min(sp.jb + KT * t1, sp.hi);
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, ln = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool active = wave < RB;
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = kv_base<KE>(p, false, seq) + (size_t)kvh * HD;
    const KE *Vb = kv_base<KE>(p, true, seq) + (size_t)kvh * HD;

    // Tile k (keys jb + KT k ..) -> stage k % NS. Thread slot S of a tensor's tile holds the 16-byte column
    // (S % SLOTS) ^ swz(key) of key row S / SLOTS (per-thread offsets below; the tile's first row is a scalar);
    // keys past the end re-read the last key (they are masked). Nothing is issued past the segment's last tile
    // (the loads are non-temporal: a re-read would go to HBM).
    unsigned koff[NLD], voff[NLD];
#pragma unroll
    for (int u = 0; u < NLD; u++) {
        const int S = (wave * NLD + u) * 64 + lane, key = S / SLOTS;
        koff[u] = (unsigned)(key * krow) + (unsigned)(((S % SLOTS) ^ kswz(key)) * 8);
        voff[u] = (unsigned)(key * krow) + (unsigned)(((S % SLOTS) ^ vswz(key)) * 8);
    }
    auto issue = [&](int k) {
        if (k >= ntile) return;
        const int jt = jb + KT * k;
        const KE *kt = Kb + (size_t)key_row(p, jt) * krow, *vt = Vb + (size_t)key_row(p, jt) * krow;
        unsigned char *kd = smem + (size_t)(k % NS) * Cf::STAGE, *vd = kd + Cf::TILE;
        const bool whole = jt + KT <= hi_b;              // wave-uniform: only a pair's last tile clamps
#pragma unroll
        for (int u = 0; u < NLD; u++) {
            const int i = wave * NLD + u;
            unsigned ko = koff[u], vo = voff[u];
            if (!whole) {
                const int key = (i * 64 + lane) / SLOTS, kc = min(key, hi_b - 1 - jt);
                ko += (unsigned)((kc - key) * (int)krow); vo += (unsigned)((kc - key) * (int)krow);
            }
            __builtin_amdgcn_global_load_lds((vglb_void *)(kt + ko), (vlds_void *)(kd + (size_t)i * 1024), 16, 0, 2);
            __builtin_amdgcn_global_load_lds((vglb_void *)(vt + vo), (vlds_void *)(vd + (size_t)i * 1024), 16, 0, 2);
        }
    };
#pragma unroll
    for (int k = 0; k < NS - 1; k++) issue(k);
    // This wave's rows (row block `wave`): Q fragments in registers, the row mask (requested after the first tiles,
    // which therefore leave at once).
    const int rho = wave * 16 + ln;
    const bool valid = active && rho < nrows;
    const int tq = tok0 + (valid ? rho / GRP : 0);
    u32x4 qf[KS];
    {
        const QE *qrow = reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + tq) * p.NQ + kvh * GRP + (valid ? rho % GRP : 0)) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qf[ks] = valid ? load8_op<QT, F16>(qrow + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
    }
    RowMask rm;
    rm.pos = tok_pos(p, seq, tq); rm.lo = win_lo(rm.pos, p.window); rm.valid = valid;
    rm.tree = p.anc != nullptr; rm.anc = p.anc ? p.anc[seq * p.T + tq] : 0u; rm.tb = p.anc ? tok_pos(p, seq, 0) : 0;
    int lo_max = 0, pos_min = INT_MAX;
    for (int t = tok0; t < tok1; t++) {
        const int ps = tok_pos(p, seq, t);
        lo_max = max(lo_max, win_lo(ps, p.window)); pos_min = min(pos_min, ps);
    }
    if (p.anc) pos_min = min(pos_min, tok_pos(p, seq, 0) - 1);

    // Tile it landed (the min(NS - 2, ntile - 1 - it) younger tiles may still fly).
    static_assert(NS >= 3 && NS <= 6, "tail waits");
    auto wait_tile = [&](int it) {
        const int younger = min(NS - 2, ntile - 1 - it);
        if (younger >= NS - 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NLD * (NS - 2)) : "memory");
        else if (younger == 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NLD * 3) : "memory");
        else if (younger == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NLD * 2) : "memory");
        else if (younger == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NLD) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    if (!active) {                // a wave past the last row block only streams its share of the ring
        for (int it = 0; it < ntile; it++) {
            wait_tile(it);
            __syncthreads();
            issue(it + NS - 1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    float m = kNegInf, l = 0.f;
    f32x4 acc[DB];
#pragma unroll
    for (int db = 0; db < DB; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    const unsigned lds0 = (unsigned)(uintptr_t)smem;
    const int vr = 4 * g + (ln >> 2);
    const unsigned kaddr = lds0 + ln * ROWB + ((g ^ kswz(ln)) << 4);
    const unsigned vaddr = lds0 + Cf::TILE + vr * ROWB + 8 * (ln & 1) + ((((ln & 3) >> 1) ^ vswz(vr)) << 4);

    // The rows' partial (slot `sl`); `mark`: the slot after it ends the pair's slots for the combine.
    const int r_out = seq * p.T + tq, h_out = kvh * GRP + rho % GRP;
    auto write = [&](int sl, bool mark) {
        const float ls = sum_over_groups(l);
        if (!valid) return;
        const size_t pi = ((size_t)r_out * p.NQ + h_out) * a.part.ns_cap + sl;
#pragma unroll
        for (int db = 0; db < DB; db++) *reinterpret_cast<f32x4 *>(a.part.acc + pi * HD + 16 * db + 4 * g) = acc[db];
        if (g == 0) {
            a.part.m[pi] = m; a.part.l[pi] = ls;
            if (mark && sl + 1 < a.part.ns_cap) a.part.m[pi + 1] = kPosInf;
        }
    };

    for (int it = 0; it < ntile; it++) {
        // The barrier makes every wave's loads of tile it visible and frees the stage of tile it-1 for tile it+NS-1.
        wait_tile(it);
        __syncthreads();
        issue(it + NS - 1);
        const int jt = jb + KT * it;
        const unsigned stage = (it % NS) * Cf::STAGE;
        unsigned kb = kaddr + stage, vb = vaddr + stage;
        asm volatile("" : "+v"(kb), "+v"(vb));
        u32x4 kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) asm volatile("ds_read_b128 %0, %1" : "=v"(kf[ks]) : "v"(kb ^ (64u * ks)) : "memory");
        if constexpr (KS == 8)
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3]), "+v"(kf[4]), "+v"(kf[5]), "+v"(kf[6]), "+v"(kf[7])::"memory");
        else
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kf[0]), "+v"(kf[1]), "+v"(kf[2]), "+v"(kf[3])::"memory");
        f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (ks & 1) s1 = mfma16<F16>(kf[ks], qf[ks], s1);
            else s0 = mfma16<F16>(kf[ks], qf[ks], s0);
        }
        const f32x4 sc = (s0 + s1) * a.sl2;
        // Masks: one wave-uniform test for a tile whose keys every row attends; else per key.
        float tv[4];
        if (jt >= j_lo && jt + KT <= j_hi && jt >= lo_max && jt + KT - 1 <= pos_min) {
#pragma unroll
            for (int i = 0; i < 4; i++) tv[i] = sc[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = jt + 4 * g + i;
                tv[i] = (key >= j_lo && key < j_hi && rm.attends(key)) ? sc[i] : kNegInf;
            }
        }
        float mx = fmaxf(fmaxf(tv[0], tv[1]), fmaxf(tv[2], tv[3]));
        mx = max_over_groups(mx);
        const float mnew = (mx > m + kRescaleThreshold) ? mx : m;
        if (__any(mnew != m)) {
            const float alpha = (mnew == m) ? 1.f : fast_exp2(m - mnew);
            l *= alpha; m = mnew;
#pragma unroll
            for (int db = 0; db < DB; db++) acc[db] *= alpha;
        }
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) { pv[i] = (tv[i] == kNegInf) ? 0.f : fast_exp2(tv[i] - m); l += pv[i]; }
        const PFrag<F16> pop = p_frag<F16>(pv[0], pv[1], pv[2], pv[3]);
#pragma unroll
        for (int d8 = 0; d8 < DB; d8 += 8) {
            u32x2 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v[j]) : "v"(vb ^ (32u * (d8 + j))) : "memory");
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]),
                         "+v"(v[5]), "+v"(v[6]), "+v"(v[7])::"memory");
#pragma unroll
            for (int j = 0; j < 8; j++) acc[d8 + j] = mfma_pv16<F16>(v[j], pop, acc[d8 + j]);
        }
        if (a.slot_runs && it + 1 < ntile && (jt + KT) % a.C == 0) {
            // The tile ends an absolute key chunk: its partial goes to slot (chunk index), the next chunk starts
            // from a fresh state (the same float operations as a run that starts at that chunk).
            write(jt / a.C, false);
            m = kNegInf; l = 0.f;
#pragma unroll
            for (int db = 0; db < DB; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");        // no load may land after the workgroup ends
    write(a.slot_runs ? (jb + KT * (ntile - 1)) / a.C : slot, last && !a.slot_runs);
}

template <int HD, int RB, int KVT, int QT>
__global__ void __launch_bounds__(256) verify_kernel(const SplitArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const Problem &p = a.p;
    const int G1 = gridDim.x / p.NKV, run = blockIdx.x / p.NKV, kvh = blockIdx.x % p.NKV;
    if (run >= G1) return;
    const int lane = threadIdx.x & 63, nz = p.nseq * a.nchunks;
    // Up to 64 pairs: lane z holds pair z, so one round of position loads gives the totals, the run's first pair and
    // every later pair (by lane exchange). More pairs: scans over the positions.
    const bool small = nz <= 64;
    const SegPair mine = (small && lane < nz) ? seg_pair(p, a.tpb, a.nchunks, lane) : SegPair{0, 0, 0, 0, 0, 0, 0};
    auto pair_at = [&](int z) {
        if (!small) return seg_pair_u(p, a.tpb, a.nchunks, z);
        SegPair sp;
        sp.seq = __builtin_amdgcn_readfirstlane(__shfl(mine.seq, z));
        sp.tok0 = __builtin_amdgcn_readfirstlane(__shfl(mine.tok0, z));
        sp.tok1 = __builtin_amdgcn_readfirstlane(__shfl(mine.tok1, z));
        sp.lo = __builtin_amdgcn_readfirstlane(__shfl(mine.lo, z));
        sp.hi = __builtin_amdgcn_readfirstlane(__shfl(mine.hi, z));
        sp.jb = __builtin_amdgcn_readfirstlane(__shfl(mine.jb, z));
        sp.n = __builtin_amdgcn_readfirstlane(__shfl(mine.n, z));
        return sp;
    };
    int incl = mine.n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    int N, z, P, pz;
    if (small) N = __builtin_amdgcn_readfirstlane(__shfl(incl, 63));
    else seg_scan(p, a.tpb, a.nchunks, INT_MAX, 0, N, z, P, pz);
    // Pair z holding tile x of the list, and the tiles before it (P).
    auto locate = [&](int x) {
        if (small) {
            z = __builtin_amdgcn_readfirstlane(__builtin_ctzll(__ballot(incl > x)));
            P = __builtin_amdgcn_readfirstlane(__shfl(incl, z) - __shfl(mine.n, z));
        } else {
            int n_;
            seg_scan(p, a.tpb, a.nchunks, x, 0, n_, z, P, pz);
        }
    };
    int x, x1;
    if (a.slot_runs) {
        // Equal runs, each end moved forward to the next absolute key-chunk boundary of its pair (or the pair's
        // end): every chunk of a pair falls in one run, which writes it to partial slot (first key / C).
        const int q = (N + G1 - 1) / G1, C = a.C;
        auto snap = [&](long long xl) -> int {
            if (xl >= N) return N;
            const int xx = (int)xl;
            locate(xx);
            const int t = xx - P;
            if (t == 0) return xx;
            const SegPair s = pair_at(z);
            const int kb = (s.jb + 16 * t + C - 1) / C * C;
            return P + min((kb - s.jb) / 16, s.n);
        };
        x1 = snap((long long)(run + 1) * q);
        x = snap((long long)run * q);
        if (x >= x1) return;
        locate(x);                                        // the snap may have moved x to the next pair
    } else {
        const int q = max((N + G1 - 1) / G1, a.part.seg_qmin);
        const long long xs = (long long)run * q;
        if (xs >= N) return;
        x = (int)xs;
        x1 = (int)min((long long)N, xs + q);
        locate(x);
    }
    const int q = max((N + G1 - 1) / G1, a.part.seg_qmin);
    SegPair sp = pair_at(z);
    for (;;) {
        const int t0 = x - P, t1 = min(sp.n, t0 + (x1 - x)), slot = a.slot_runs ? 0 : run - P / q;
        if (slot < 0 || slot >= a.part.ns_cap) break;     // unreachable while the counts agree
        if (t0 >= t1) break;                              // unreachable: x lies inside pair z
        verify_segment<HD, RB, KVT, QT>(a, sp, kvh, t0, t1, slot, t1 == sp.n, smem);
        x += t1 - t0;
        if (x >= x1) break;
        P += sp.n;                                        // next pair (every pair holds at least one tile)
        sp = pair_at(++z);
        __syncthreads();                                  // every wave is done with the ring
    }
}


// ---------------------------------------------------------------- host side
// verify_kernel's grid: the workgroups that are resident at once on the current device (per device, cached).
template <int HD, int RB, int KVT, int QT>
static hipError_t verify_grid(int &G) {
    using Cf = VerifyCfg<HD>;
    static int per_cu = 0;
    static int ncu[64] = {0};
    if (per_cu == 0) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&verify_kernel<HD, RB, KVT, QT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::LDS);
        if (e != hipSuccess) return e;
        int nb = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(&verify_kernel<HD, RB, KVT, QT>),
                                                         256, Cf::LDS);
        if (e != hipSuccess) return e;
        per_cu = nb > 0 ? nb : 1;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (ncu[dev] == 0) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        ncu[dev] = n > 0 ? n : 1;
    }
    G = per_cu * ncu[dev];
    return hipSuccess;
}

template <int HD, int RB, int KVT, int QT>
static hipError_t launch_split_t(SplitArgs &a, dim3 grid, hipStream_t st) {
    if constexpr (RB >= 2 && HD <= 256 && KVT != DT_FP32) {
        if (a.part.ns_cap >= 2) {
            int G = 0;
            hipError_t e = verify_grid<HD, RB, KVT, QT>(G);
            if (e != hipSuccess) return e;
            // q >= qmin keeps a pair within ns_cap slots: a pair of n <= max_pos/16 + 1 tiles meets at most
            // floor((n - 1) / q) + 2 runs (with fewer than ns_cap, the slot after the last holds the end mark).
            const int nmax = a.p.max_pos / 16 + 1;
            G = std::max(a.p.NKV, G - G % a.p.NKV);          // the same G / NKV runs for every KV head
            if (!a.slot_runs) {
                a.part.seg_g = G;
                a.part.seg_qmin = std::max(8, (nmax - 1) / (a.part.ns_cap - 1) + 1);
            }
            hipLaunchKernelGGL((verify_kernel<HD, RB, KVT, QT>), dim3(G), dim3(256), VerifyCfg<HD>::LDS, st, a);
            return hipGetLastError();
        }
    }
    using Cf = SplitCfg<HD, RB>;
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&split_kernel<HD, RB, KVT, QT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL((split_kernel<HD, RB, KVT, QT>), grid, dim3(Cf::NW * 64), Cf::LDS, st, a);
    return hipGetLastError();
}

template <int HD, int KVT, int QT>
static hipError_t dispatch_rb(SplitArgs &a, int RB, dim3 grid, hipStream_t st) {
    switch (RB) {
    case 1: return launch_split_t<HD, 1, KVT, QT>(a, grid, st);
    case 2: return launch_split_t<HD, 2, KVT, QT>(a, grid, st);
    case 3: return launch_split_t<HD, 3, KVT, QT>(a, grid, st);
    case 4: return launch_split_t<HD, 4, KVT, QT>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

template <int KVT, int QT>
static hipError_t dispatch_hd(SplitArgs &a, int RB, dim3 grid, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return dispatch_rb<128, KVT, QT>(a, RB, grid, st);
    case 512: return dispatch_rb<512, KVT, QT>(a, RB, grid, st);
    case 256: return dispatch_rb<256, KVT, QT>(a, RB, grid, st);
    default: return hipErrorInvalidValue;
    }
}

static void split_tiling(const Problem &p, int &RB, int &tpb, int &nchunks) {
    const int GRP = p.NQ / p.NKV;
    const int maxrb = 4;
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

hipError_t launch_split(const Problem &p, int chunk, Partials &part, hipStream_t st, bool slot_runs) {
    part.seg_g = 0;
    if (chunk <= 0 || chunk % 16) return hipErrorInvalidValue;
    // Up to 16 rows per KV head (one query token at GRP <= 16): the streaming decode kernel.
    if (decode_stream_supported(p))
        return launch_decode_stream(p, chunk, part, st);
    if (p.NQ % p.NKV) return hipErrorInvalidValue;
    const int GRP = p.NQ / p.NKV;
    int RB, tpb, nchunks;
    split_tiling(p, RB, tpb, nchunks);
    if (RB * 16 < GRP || RB > 4) return hipErrorInvalidValue;
    if (p.max_pos / chunk + 1 > part.ns_cap) return hipErrorInvalidValue;
    SplitArgs a{p, part, chunk, tpb, nchunks, p.scale * kLog2e, slot_runs ? 1 : 0};
    dim3 grid(p.NKV, p.max_pos / chunk + 1, p.nseq * nchunks);
    if (grid.z > 65535u || grid.y > 65535u) return hipErrorInvalidConfiguration;
    if ((long long)p.nseq * p.NKV * (p.max_pos / 16 + 2) > INT_MAX) return hipErrorInvalidConfiguration;
    const int kv = p.kv_dtype, q = p.q_dtype;
    hipError_t e = hipErrorInvalidValue;
    if (kv == DT_F16 && q == DT_FP32) e = dispatch_hd<DT_F16, DT_FP32>(a, RB, grid, st);
    else if (kv == DT_F16 && q == DT_F16) e = dispatch_hd<DT_F16, DT_F16>(a, RB, grid, st);
    else if (kv == DT_BF16 && q == DT_FP32) e = dispatch_hd<DT_BF16, DT_FP32>(a, RB, grid, st);
    else if (kv == DT_BF16 && q == DT_BF16) e = dispatch_hd<DT_BF16, DT_BF16>(a, RB, grid, st);
    else if (kv == DT_FP32 && q == DT_FP32) e = dispatch_hd<DT_FP32, DT_FP32>(a, RB, grid, st);
    part = a.part;                                     // the combine reads how the partials were laid out
    return e;
}

size_t split_lds_bytes(int HD) {
    switch (HD) {
    case 128: return SplitCfg<128, 1>::LDS;
    case 256: return SplitCfg<256, 1>::LDS;
    case 512: return SplitCfg<512, 1>::LDS;
    default: return 0;
    }
}

hipError_t launch_combine(const Problem &p, int chunk, const Partials &part, hipStream_t st) {
    const int rows = p.nseq * p.T * p.NQ;
    if (rows <= 0) return hipSuccess;
    auto grid = [&](int nr) { return dim3((unsigned)((rows + nr - 1) / nr)); };
    switch (p.HD) {
    case 128: hipLaunchKernelGGL(combine_kernel<128>, grid(CombineCfg<128>::NR), dim3(CombineCfg<128>::NT), 0, st, p, part, chunk); break;
    case 256: hipLaunchKernelGGL(combine_kernel<256>, grid(CombineCfg<256>::NR), dim3(CombineCfg<256>::NT), 0, st, p, part, chunk); break;
    case 512: hipLaunchKernelGGL(combine_kernel<512>, grid(CombineCfg<512>::NR), dim3(CombineCfg<512>::NT), 0, st, p, part, chunk); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dgx

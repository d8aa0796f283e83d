// Flash prefill / chunked prefill attention on gfx950 (causal and sliding window).
//
// Replaces the reference's fav2::flash_v2_kernel (kernels/attention_flash_v2.cuh:104-259) and, for long query
// runs, flash_attn2bs_p1(_custom)_kernel (kernels/attention_flash.cuh:28-217).
//
// Work decomposition. A half tile is 32 rows (16 at HD 512): tqh tokens x the GRP q-heads of one KV head
// (token-major), so every K/V byte a workgroup fetches serves the whole GQA group. A workgroup (8 wave64s; 4 at
// HD 512) takes two half tiles at once and walks the union of their key ranges: for causal prompts the pair
// (i, n-1-i), so the keys of the short half are fetched once for both and every workgroup carries the same work
// (a T=1024 prompt at 8 KV heads is 256 equal workgroups); otherwise two neighbouring half tiles. Work items of
// one (sequence, KV head) get consecutive indices and are mapped onto one XCD (workgroups are dispatched
// round-robin over the 8 XCDs), so that head's K/V stays in one L2.
//
// Keys are walked in steps of SK keys at absolute positions; each wave takes the NSUB 16-key sub-tiles of its key
// group in a step (one wave per key group and row group). K and V of a step go from HBM/L2 straight into LDS
// with gfx950 direct-to-LDS loads (global_load_lds_dwordx4: no staging registers), NS-stage ring, one barrier
// per step. The LDS rows are unpadded and their 16-byte slots are XOR-swizzled by the key (swz). Each wave then
//   * computes S^T = K Q^T for its rows on 16x16x32 MFMA (K fragments from LDS, Q fragments in registers),
//   * masks (causal / window; a wave-uniform test picks the unmasked fast path) and runs the online softmax in
//     registers over all its keys of the step (a row lives in 4 lanes; the running max moves lazily, so the
//     accumulator is rescaled on few steps),
//   * computes O^T += V^T P^T on 16x16x16 MFMA with V^T read transposed from LDS (ds_read_b64_tr_b16) and P^T
//     straight from the softmax registers.
// At the end the two key-group states of each row are merged through LDS.
//
// Determinism and chunk invariance: step boundaries are absolute, the key group of a sub-tile depends only on
// its position, a sub-tile a row does not attend leaves the row's state exactly unchanged, and the merge order is
// fixed. A row's bits therefore depend only on its query, position and keys - not on the other rows of its tile,
// the tile pairing or how the prompt is chunked (attention_flash_v2.cuh:13-18).
//
// Key splits (kv_split > 0) restrict each work item to the keys of one absolute split and write LSE partials for
// launch_combine. Tree masks are not served here: the reference's ancestor mask covers at most 32 draft nodes
// (attention_flash.cuh:177), and such short query runs go to the split kernel.
#include "attn_device.h"
#include "attn_internal.h"
#include <climits>
#include <type_traits>

namespace dgx {

struct PrefArgs {
    Problem p;
    Partials part;
    int kv_split;      // 0: none
    int nht;           // half tiles per sequence
    int nsplit;        // key splits per sequence
    int tqh;           // tokens per half tile
    int pair;          // 1: a work item is the half-tile pair (i, nht-1-i); 0: the half tiles (2i, 2i+1)
    int nitems;        // work items per (sequence, kv head)
    int nwg;           // total work items
    float sl2;         // scale * log2(e)
};

// A workgroup is RG x KG waves. RB: 16-row blocks per wave; RG: row groups (waves splitting the tile's rows, the
// first half of them on the first half tile); KG: key groups (waves splitting each step's keys); NS: LDS stages;
// NSUB: 16-key sub-tiles per wave and step.
template <int HD, int RB, int RG, int KG_, int NS_, int NSUB_>
struct PrefCfg {
    static constexpr int KG = KG_, NS = NS_, NW = RG * KG_, NT = NW * 64, NSUB = NSUB_;
    static constexpr int KT = 16 * NSUB;                 // keys per wave per step (NSUB 16-key sub-tiles)
    static constexpr int SK = KG * KT;                   // keys per step
    static constexpr int RR = RG * RB * 16;              // rows per workgroup tile
    static constexpr int HR = RR / 2;                    // rows per half tile
    static constexpr int KS = HD / 32;                   // QK k-steps (16x16x32)
    static constexpr int DB = HD / 16;                   // PV output dim blocks (16x16x16)
    static constexpr int SLOTS = HD / 8;                 // 16-byte slots per key row
    static constexpr int ROWB = HD * 2;                  // bytes per key row (16-bit operands)
    static constexpr int HALF = SK * ROWB;               // bytes of one K (or V) step tile
    static constexpr int STAGE = 2 * HALF;               // K and V of one step
    static constexpr int NLD = SK * SLOTS / NT;          // 16-byte loads per thread per step (K and V each)
    static constexpr size_t LDS_TILES = (size_t)NS * STAGE;
    static constexpr int XSTR = HD / 2 + 4;              // merge exchange row stride (floats)
    static constexpr size_t LDS_MERGE = (size_t)RG * 2 * RB * 16 * XSTR * 4;
    static constexpr size_t LDS_STATS = (size_t)2 * NW * RB * 16 * 4;
    static constexpr size_t LDS_MAIN = LDS_TILES > LDS_MERGE ? LDS_TILES : LDS_MERGE;
    static constexpr size_t LDS = LDS_MAIN + LDS_STATS;
    static_assert(NLD >= 1 && (SK * SLOTS) % NT == 0, "step loads");
    static_assert(RG % 2 == 0 && HR % (RB * 16) == 0, "each wave's rows lie in one half tile");
    static_assert(NS >= 2 && NS <= 4, "stages");
    static_assert(KG == 2, "the merge pairs two key groups");
};

// Slot swizzle of key row k: 16-byte column c of key k sits in slot c ^ swz(k), a permutation of the low 4 key
// bits (keys 0-7 to the even slots, 8-15 to the odd ones). It spreads the 16 keys of a K fragment read over the
// 16 slots of a 256-byte bank row, and the 8 keys x 2 columns that the 32 lanes of a half V transpose read
// (keys 4g..4g+3 for g = 0, 1 or g = 2, 3) over all 16 slots as well.
__device__ __forceinline__ int swz(int k) { return ((k & 7) << 1) | ((k >> 3) & 1); }

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// Wait until at most `pending` later steps (PER memory operations each) are still in flight.
template <int PER>
__device__ __forceinline__ void wait_steps(int pending) {
    if (pending >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PER) : "memory");
    else if (pending == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int HD, int RB, int RG, int KG_, int NS_, int NSUB, int KVT, int QT, int OT>
__global__ void __launch_bounds__(RG * KG_ * 64) prefill_kernel(const PrefArgs a) {
    using Cf = PrefCfg<HD, RB, RG, KG_, NS_, NSUB>;
    constexpr int KG = Cf::KG, NS = Cf::NS, SK = Cf::SK, KS = Cf::KS, DB = Cf::DB, NLD = Cf::NLD;
    constexpr int SLOTS = Cf::SLOTS, ROWB = Cf::ROWB, HR = Cf::HR;
    constexpr bool F16 = OpIsF16<KVT>::value;
    constexpr bool DMA = KVT != DT_FP32;                 // 16-bit caches go straight to LDS
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];
    float *stm = reinterpret_cast<float *>(smem + Cf::LDS_MAIN), *stl = stm + Cf::NW * RB * 16;

    const Problem &p = a.p;
    // XCD-aware work index: dispatch slot b runs on XCD b % 8; consecutive work items share an XCD.
    const int per = (int)gridDim.x / 8;
    const int w_item = ((int)blockIdx.x % 8) * per + (int)blockIdx.x / 8;
    if (w_item >= a.nwg) return;
    const int seq = w_item / (p.NKV * a.nitems);
    const int kvh = (w_item / a.nitems) % p.NKV;
    const int item = w_item % a.nitems;
    const int sp = item % a.nsplit, qi = item / a.nsplit;
    const int GRP = p.NQ / p.NKV;

    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, ln = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave / KG, kg = wave % KG;
    const size_t krow = (size_t)p.NKV * HD;
    const KE *Kb = kv_base<KE>(p, false, seq) + (size_t)kvh * HD;
    const KE *Vb = kv_base<KE>(p, true, seq) + (size_t)kvh * HD;
    // Prefill tokens are consecutive: token t of this sequence sits at position pbase + t.
    const int pbase = __builtin_amdgcn_readfirstlane(p.pos_arr ? p.pos_arr[seq] : p.base);

    // The two half tiles of this work item (longest first) and their tokens; an empty half has tok1 == tok0.
    const int nhalf_items = a.nitems / a.nsplit;
    int ht0, ht1;
    if (a.pair) { ht0 = a.nht - 1 - qi; ht1 = qi < ht0 ? qi : -1; }
    else { const int i2 = nhalf_items - 1 - qi; ht0 = 2 * i2 + 1 < a.nht ? 2 * i2 + 1 : 2 * i2; ht1 = 2 * i2 + 1 < a.nht ? 2 * i2 : -1; }
    int tok0[2], tok1[2];
    tok0[0] = ht0 * a.tqh; tok1[0] = min(p.T, tok0[0] + a.tqh);
    tok0[1] = ht1 < 0 ? 0 : ht1 * a.tqh; tok1[1] = ht1 < 0 ? 0 : min(p.T, tok0[1] + a.tqh);
    // Keys of the workgroup: the union of both halves' ranges (the first half holds the latest tokens).
    int j_lo = win_lo(pbase + tok0[0], p.window);
    if (tok1[1] > tok0[1]) j_lo = min(j_lo, win_lo(pbase + tok0[1], p.window));
    const int hi_b = pbase + tok1[0];                                   // one past the last key (clamp bound)
    int j_hi = hi_b;
    if (a.kv_split > 0) { j_lo = max(j_lo, sp * a.kv_split); j_hi = min(j_hi, (sp + 1) * a.kv_split); }
    const int s0 = j_lo / SK, nsteps = j_lo < j_hi ? (j_hi - 1) / SK - s0 + 1 : 0;

    // Step loads: thread slot S = (wave*NLD + u)*64 + lane of the K (V) half of a stage holds the 16-byte column
    // (S % SLOTS) ^ swz(key) of key row key = S / SLOTS; its byte offset from the step's first key row is fixed.
    const unsigned krow_b = (unsigned)(krow * sizeof(KE));
    unsigned ld_off[NLD];
#pragma unroll
    for (int u = 0; u < NLD; u++) {
        const int S = (wave * NLD + u) * 64 + lane, key = S / SLOTS;
        ld_off[u] = (unsigned)key * krow_b + (unsigned)(((S % SLOTS) ^ swz(key)) * 8 * sizeof(KE));
    }
    // Step k of the walk into stage k % NS. Keys past the last position re-read that position (they are masked), so
    // every load is in bounds; only a step that crosses the end needs the clamped addresses.
    auto issue = [&](int k) {
        const int s = s0 + k;
        unsigned char *kd = smem + (size_t)(k % NS) * Cf::STAGE, *vd = kd + Cf::HALF;
        const char *ks = reinterpret_cast<const char *>(Kb) + (size_t)key_row(p, s * SK) * krow_b;
        const char *vs = reinterpret_cast<const char *>(Vb) + (size_t)key_row(p, s * SK) * krow_b;
        const bool inside = s * SK + SK <= hi_b;
#pragma unroll
        for (int u = 0; u < NLD; u++) {
            const int i = wave * NLD + u;
            unsigned off = ld_off[u];
            if (!inside) {
                const unsigned key = off / krow_b, lim = (unsigned)(hi_b - 1 - s * SK);
                if (key > lim) off -= (key - lim) * krow_b;
            }
            if constexpr (!DMA) {
                const int S = i * 64 + lane;
                *reinterpret_cast<u32x4 *>(kd + (size_t)S * 16) = load8_op<KVT, F16>(reinterpret_cast<const KE *>(ks + off));
                *reinterpret_cast<u32x4 *>(vd + (size_t)S * 16) = load8_op<KVT, F16>(reinterpret_cast<const KE *>(vs + off));
            } else {
                __builtin_amdgcn_global_load_lds((glb_void *)(ks + off), (lds_void *)(kd + (size_t)i * 1024), 16, 0, 0);
                __builtin_amdgcn_global_load_lds((glb_void *)(vs + off), (lds_void *)(vd + (size_t)i * 1024), 16, 0, 0);
            }
        }
    };
    if (nsteps > 0) issue(0);

    // This wave's rows (all in one half tile): Q fragments and positions (an invalid row has pos = -1 and attends
    // nothing), and the wave-uniform key span of its rows (positions grow with the row's token).
    const int half = (rg * RB * 16) / HR, lr0 = rg * RB * 16 - half * HR;
    const int htok0 = half ? tok0[1] : tok0[0], hnrows = (half ? tok1[1] - tok0[1] : tok1[0] - tok0[0]) * GRP;
    int rpos[RB], rlo[RB];
    u32x4 qop[RB][KS];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int rho = lr0 + rb * 16 + ln;
        const bool valid = rho < hnrows;
        const int t = htok0 + (valid ? rho / GRP : 0), h = kvh * GRP + (valid ? rho % GRP : 0);
        const int ps = pbase + t;
        rpos[rb] = valid ? ps : -1;
        rlo[rb] = win_lo(ps, p.window);
        const QE *qrow = reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + t) * p.NQ + h) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
            qop[rb][ks] = valid ? load8_op<QT, F16>(qrow + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
    }
    // Steps 1..NS-2 go out after the Q loads, so that waiting for step it never waits for younger steps.
#pragma unroll
    for (int k = 1; k < NS - 1; k++)
        if (k < nsteps) issue(k);
    const int rho1 = min(hnrows, lr0 + RB * 16);
    int wlo = INT_MAX, whi = -1, lo_max = 0, pos_min = INT_MAX;
    if (lr0 < rho1) {
        const int pf = pbase + htok0 + lr0 / GRP, pl = pbase + htok0 + (rho1 - 1) / GRP;
        wlo = max(win_lo(pf, p.window), j_lo); whi = min(pl, j_hi - 1);
        lo_max = win_lo(pl, p.window); pos_min = pf;
    }

    float m[RB], l[RB];
    f32x4 acc[RB][DB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        m[rb] = kNegInf; l[rb] = 0.f;
#pragma unroll
        for (int db = 0; db < DB; db++) acc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Per-lane LDS byte addresses inside a step stage (the key group's rows start at kg*KT). A slot index
    // occupies address bits 4.., and the row base has those bits clear, so "slot s ^ x" is an XOR on the
    // address: K fragment (ks, g) of row ln is at kaddr ^ (64 ks); V transpose-read block db of row
    // 4g + ln/4 is at vaddr ^ (32 db).
    const unsigned lds0 = (unsigned)(uintptr_t)smem;
    const int vr = 4 * g + (ln >> 2);
    const unsigned kaddr = lds0 + (kg * Cf::KT + ln) * ROWB + ((g ^ swz(ln)) << 4);
    const unsigned vaddr = lds0 + Cf::HALF + (kg * Cf::KT + vr) * ROWB + 8 * (ln & 1) + ((((ln & 3) >> 1) ^ swz(vr)) << 4);
    for (int it = 0; it < nsteps; it++) {
        // Step it is the oldest load batch in flight; up to NS-2 younger steps may stay in flight.
        wait_steps<DMA ? 2 * NLD : 0>(min(NS - 2, nsteps - 1 - it));
        __syncthreads();                                                // everyone's step it, and step it-1 is consumed
        if (it + NS - 1 < nsteps) issue(it + NS - 1);
        // This wave's keys of the step: NSUB 16-key sub-tiles from jw. QK for all of them first (independent MFMA
        // chains), one softmax update over all of them, then PV.
        const int jw = (s0 + it) * SK + kg * Cf::KT;
        if (jw > whi || jw + Cf::KT - 1 < wlo) continue;                // no row of the wave attends them
        const unsigned stage = (it % NS) * Cf::STAGE;
        f32x4 s[NSUB][RB], s2[NSUB][RB];
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) s[sub][rb] = s2[sub][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
                const u32x4 kf = *reinterpret_cast<const u32x4 *>(smem + ((kaddr + stage + sub * 16 * ROWB) ^ (64u * ks)) - lds0);
#pragma unroll
                for (int rb = 0; rb < RB; rb++) {
                    if (ks & 1) s2[sub][rb] = mfma16<F16>(kf, qop[rb][ks], s2[sub][rb]);
                    else s[sub][rb] = mfma16<F16>(kf, qop[rb][ks], s[sub][rb]);
                }
            }
        }
        const bool full = jw >= j_lo && jw + Cf::KT <= j_hi && jw >= lo_max && jw + Cf::KT - 1 <= pos_min;
        float tv[NSUB][RB][4], mnew[RB];
        bool need = false;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            float mx = kNegInf;
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
                const f32x4 sc = (s[sub][rb] + s2[sub][rb]) * a.sl2;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = jw + 16 * sub + 4 * g + i;
                    const bool in = full || (key >= j_lo && key < j_hi && key >= rlo[rb] && key <= rpos[rb]);
                    tv[sub][rb][i] = in ? sc[i] : kNegInf;
                    mx = fmaxf(mx, tv[sub][rb][i]);
                }
            }
            mx = max_over_groups(mx);
            if (mx > m[rb] + kRescaleThreshold) { mnew[rb] = mx; need = true; } else mnew[rb] = m[rb];
        }
        if (__any(need)) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                const float alpha = (mnew[rb] == m[rb]) ? 1.f : fast_exp2(m[rb] - mnew[rb]);
                l[rb] *= alpha; m[rb] = mnew[rb];
#pragma unroll
                for (int db = 0; db < DB; db++) acc[rb][db] *= alpha;
            }
        }
        u32x2 pop[NSUB][RB];
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                float pv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) pv[i] = (tv[sub][rb][i] == kNegInf) ? 0.f : fast_exp2(tv[sub][rb][i] - m[rb]);
                l[rb] += (pv[0] + pv[1]) + (pv[2] + pv[3]);
                pop[sub][rb] = u32x2{pack2<F16>(pv[0], pv[1]), pack2<F16>(pv[2], pv[3])};
            }
        // V^T fragments in batches of 8 transpose reads, then one wait: the reads are issued as inline asm so
        // that the compiler does not order them behind the direct-to-LDS loads of later steps.
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int d8 = 0; d8 < DB; d8 += 8) {
                u32x2 v[8];
                const unsigned va = vaddr + stage + sub * 16 * ROWB;
#pragma unroll
                for (int j = 0; j < 8; j++)
                    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v[j]) : "v"(va ^ (32u * (d8 + j))) : "memory");
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]),
                             "+v"(v[5]), "+v"(v[6]), "+v"(v[7])::"memory");
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int rb = 0; rb < RB; rb++) acc[rb][d8 + j] = mfma16k16<F16>(v[j], pop[sub][rb], acc[rb][d8 + j]);
            }
    }
#pragma unroll
    for (int rb = 0; rb < RB; rb++) l[rb] = sum_over_groups(l[rb]);
    __syncthreads();                                                 // every wave is done with the K/V tiles

    // Merge the two key-group states of each row (waves kg = 0 and 1 of a row group hold the same rows). Every
    // lane derives the row's M = max m and L = sum l 2^(m - M) from the published (m, l) and scales its
    // accumulator by 2^(m - M) / L (2^(m - M) for a split partial). Wave kg then owns output dims
    // [kg*HD/2, (kg+1)*HD/2): it parks the other half of its scaled accumulator in LDS for its partner, reads
    // the partner's half for its own dims, adds (a + b == b + a, so both orders give the same bits) and stores.
    const int NQ = p.NQ;
    if (g == 0) {
#pragma unroll
        for (int rb = 0; rb < RB; rb++) { stm[wave * RB * 16 + rb * 16 + ln] = m[rb]; stl[wave * RB * 16 + rb * 16 + ln] = l[rb]; }
    }
    __syncthreads();
    constexpr int DH = DB / 2;                                          // dim blocks per owner
    float *xb = reinterpret_cast<float *>(smem);                        // [rg][owner kg][row][XSTR] (reuses tiles)
    float fsc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int srow = rb * 16 + ln;
        const float m0 = stm[(rg * 2) * RB * 16 + srow], m1 = stm[(rg * 2 + 1) * RB * 16 + srow];
        const float M = fmaxf(m0, m1);
        float L = 0.f;
        if (m0 != kNegInf) L += stl[(rg * 2) * RB * 16 + srow] * fast_exp2(m0 - M);
        if (m1 != kNegInf) L += stl[(rg * 2 + 1) * RB * 16 + srow] * fast_exp2(m1 - M);
        float f = (m[rb] == kNegInf) ? 0.f : fast_exp2(m[rb] - M);
        if (a.kv_split <= 0) f *= (L > 0.f ? 1.f / L : 0.f);
        fsc[rb] = f;
        float *dst = xb + (((size_t)rg * 2 + (kg ^ 1)) * RB * 16 + srow) * Cf::XSTR + 4 * g;
        // (constant indices in both branches keep acc in registers)
        if (kg == 0) {
#pragma unroll
            for (int j = 0; j < DH; j++) *reinterpret_cast<f32x4 *>(dst + 16 * j) = acc[rb][DH + j] * f;
        } else {
#pragma unroll
            for (int j = 0; j < DH; j++) *reinterpret_cast<f32x4 *>(dst + 16 * j) = acc[rb][j] * f;
        }
        const int rho = lr0 + srow;
        if (kg == 0 && g == 0 && rho < hnrows) {
            const int r = seq * p.T + htok0 + rho / GRP, h = kvh * GRP + rho % GRP;
            if (a.kv_split > 0) {
                const size_t pi = ((size_t)r * NQ + h) * a.part.ns_cap + sp;
                a.part.m[pi] = M; a.part.l[pi] = L;
            } else if (p.lse) {
                p.lse[(size_t)r * NQ + h] = (L > 0.f) ? (M + log2f(L)) * kLn2 : kNegInf;
            }
        }
    }
    __syncthreads();
    // Output dims of this wave: blocks [OWN*DH, (OWN+1)*DH) of its accumulator (OWN a constant, so acc stays in
    // registers).
    auto finish = [&](auto own_c) {
        constexpr int OWN = decltype(own_c)::value;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const int srow = rb * 16 + ln, rho = lr0 + srow;
            if (rho >= hnrows) continue;
            const int r = seq * p.T + htok0 + rho / GRP, h = kvh * GRP + rho % GRP;
            const float *src = xb + (((size_t)rg * 2 + OWN) * RB * 16 + srow) * Cf::XSTR + 4 * g;
#pragma unroll
            for (int j = 0; j < DH; j++) {
                const int d = 16 * (OWN * DH + j) + 4 * g;
                const f32x4 o = acc[rb][OWN * DH + j] * fsc[rb] + *reinterpret_cast<const f32x4 *>(src + 16 * j);
                if (a.kv_split > 0) {
                    const size_t pi = ((size_t)r * NQ + h) * a.part.ns_cap + sp;
                    *reinterpret_cast<f32x4 *>(a.part.acc + pi * HD + d) = o;
                    continue;
                }
                const size_t ob = ((size_t)r * NQ + h) * HD + d;
                if constexpr (OT == DT_FP32) *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p.O) + ob) = o;
                else {
                    const u32x2 wv = u32x2{pack2<OT == DT_F16>(o.x, o.y), pack2<OT == DT_F16>(o.z, o.w)};
                    *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(p.O) + ob) = wv;
                }
            }
        }
    };
    if (kg == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 1>{});
}

// ---------------------------------------------------------------- host side
// Tile shapes. HD 128/256: 8 waves (two per SIMD, so one wave's MFMAs overlap the other's softmax and LDS
// traffic) as 4 row groups x 2 key groups, 16 rows and HD accumulator columns per wave, a 64-row workgroup tile
// (two 32-row half tiles), 64-key steps (two 16-key sub-tiles per wave) in two LDS stages. HD 512: 4 waves, a
// 32-row tile, 32-key steps (a 32-key stage of HD 512 is 64 KB).
template <int HD> struct PrefTile;
template <> struct PrefTile<128> { static constexpr int RB = 1, RG = 4, KG = 2, NS = 2, NSUB = 2; };
template <> struct PrefTile<256> { static constexpr int RB = 1, RG = 4, KG = 2, NS = 2, NSUB = 2; };
template <> struct PrefTile<512> { static constexpr int RB = 1, RG = 2, KG = 2, NS = 2, NSUB = 1; };
template <int HD>
using PrefTileCfg = PrefCfg<HD, PrefTile<HD>::RB, PrefTile<HD>::RG, PrefTile<HD>::KG, PrefTile<HD>::NS, PrefTile<HD>::NSUB>;

template <int HD, int KVT, int QT, int OT>
static hipError_t launch_pref_t(const PrefArgs &a, dim3 grid, hipStream_t st) {
    using T = PrefTile<HD>;
    using Cf = PrefTileCfg<HD>;
    static bool configured = false;
    auto kern = prefill_kernel<HD, T::RB, T::RG, T::KG, T::NS, T::NSUB, KVT, QT, OT>;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cf::LDS);
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(kern, grid, dim3(Cf::NT), Cf::LDS, st, a);
    return hipGetLastError();
}

template <int KVT, int QT, int OT>
static hipError_t pref_dispatch_hd(const PrefArgs &a, dim3 grid, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return launch_pref_t<128, KVT, QT, OT>(a, grid, st);
    case 256: return launch_pref_t<256, KVT, QT, OT>(a, grid, st);
    case 512: return launch_pref_t<512, KVT, QT, OT>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

static int pref_half_rows(int HD) {
    switch (HD) {
    case 128: return PrefTileCfg<128>::HR;
    case 256: return PrefTileCfg<256>::HR;
    case 512: return PrefTileCfg<512>::HR;
    default: return 0;
    }
}

// Key split for kv_split = -1: when the unsplit grid would fill at most half of the CUs (a short run of queries
// over a long cached prefix), cut the keys into as many absolute splits as whole grids fit on the CUs.
int prefill_auto_split(const Problem &p) {
    if (p.NQ % p.NKV) return 0;
    const int GRP = p.NQ / p.NKV, HR = pref_half_rows(p.HD);
    if (HR == 0 || GRP > HR) return 0;
    const int tqh = HR / GRP, nht = (p.T + tqh - 1) / tqh;
    const long nwg = (long)p.nseq * p.NKV * ((nht + 1) / 2);
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (nwg <= 0 || 2 * nwg > ncu) return 0;
    const int nsplit = (int)(ncu / nwg);
    const int keys = p.max_pos + 1;
    int ks = (keys + nsplit - 1) / nsplit;
    ks = ((ks + 63) / 64) * 64;
    return ks >= keys ? 0 : ks;
}

hipError_t launch_prefill(const Problem &p, int kv_split, const Partials &part, hipStream_t st) {
    if (p.NQ % p.NKV || p.anc || p.pos_mode != 1) return hipErrorInvalidValue;
    const int GRP = p.NQ / p.NKV, HR = pref_half_rows(p.HD);
    if (HR == 0 || GRP > HR) return hipErrorInvalidValue;
    if (kv_split < 0 || (kv_split > 0 && kv_split % 64)) return hipErrorInvalidValue;
    const int tqh = HR / GRP;
    const int nht = (p.T + tqh - 1) / tqh;
    const int nsplit = kv_split > 0 ? p.max_pos / kv_split + 1 : 1;
    if (kv_split > 0 && nsplit > part.ns_cap) return hipErrorInvalidValue;
    // Pair half tiles (i, n-1-i) when causal work varies across the prompt (no window, prefix shorter than the
    // chunk); otherwise a workgroup takes two neighbouring half tiles.
    const int pair = (kv_split == 0 && p.window == 0 && nht >= 2 && p.max_pos < 2 * p.T) ? 1 : 0;
    const int nitems = ((nht + 1) / 2) * nsplit;
    const long nwg = (long)p.nseq * p.NKV * nitems;
    if (nwg <= 0 || nwg > (1L << 30)) return hipErrorInvalidConfiguration;
    PrefArgs a{p, part, kv_split, nht, nsplit, tqh, pair, nitems, (int)nwg, p.scale * kLog2e};
    dim3 grid((unsigned)(8 * ((nwg + 7) / 8)));
    hipError_t e = hipErrorInvalidValue;
    const int kv = p.kv_dtype, q = p.q_dtype, o = p.o_dtype;
    if (kv == DT_F16 && q == DT_FP32 && o == DT_FP32) e = pref_dispatch_hd<DT_F16, DT_FP32, DT_FP32>(a, grid, st);
    else if (kv == DT_BF16 && q == DT_FP32 && o == DT_FP32) e = pref_dispatch_hd<DT_BF16, DT_FP32, DT_FP32>(a, grid, st);
    else if (kv == DT_FP32 && q == DT_FP32 && o == DT_FP32) e = pref_dispatch_hd<DT_FP32, DT_FP32, DT_FP32>(a, grid, st);
    else if (kv == DT_F16 && q == DT_F16 && o == DT_F16) e = pref_dispatch_hd<DT_F16, DT_F16, DT_F16>(a, grid, st);
    else if (kv == DT_BF16 && q == DT_BF16 && o == DT_BF16) e = pref_dispatch_hd<DT_BF16, DT_BF16, DT_BF16>(a, grid, st);
    else return hipErrorInvalidValue;
    if (e != hipSuccess || kv_split <= 0) return e;
    return launch_combine(p, kv_split, part, st);
}

}  // namespace dgx

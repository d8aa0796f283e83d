// Flash prefill / chunked prefill attention on gfx950 (causal and sliding window).
//
// Replaces the reference's fav2::flash_v2_kernel (kernels/attention_flash_v2.cuh:104-259) and, for long query
// runs, flash_attn2bs_p1(_custom)_kernel (kernels/attention_flash.cuh:28-217).
//
// Work decomposition. A half tile is 32 rows: tqh tokens x the GRP q-heads of one KV head (token-major), so every
// K/V byte a workgroup fetches serves the whole GQA group. A workgroup (8 wave64s) takes two half tiles at once
// and walks the union of their key ranges: for causal prompts the pair (i, n-1-i), so the keys of the short half
// are fetched once for both and every workgroup carries the same work (a T=1024 prompt at 8 KV heads is 256 equal
// workgroups); otherwise two neighbouring half tiles. Work items of
// one (sequence, KV head) get consecutive indices and are mapped onto one XCD (workgroups are dispatched
// round-robin over the 8 XCDs), so that head's K/V stays in one L2.
//
// Keys are walked in steps of SK keys at absolute positions; each wave takes the NSUB 16-key sub-tiles of its key
// group in a step (one wave per key group and row group). K and V of a step go from HBM/L2 straight into LDS
// with gfx950 direct-to-LDS buffer loads (no staging registers; the buffer range makes rows past the last key
// read as zeros), NS-stage ring, one barrier per step. The LDS rows are unpadded and their 16-byte slots are
// XOR-swizzled by the key (kswz, vswz). Each wave then
//   * computes S^T = K Q^T for its rows on 16x16x32 MFMA (K fragments from LDS, Q fragments in registers),
//   * masks (causal / window; a wave-uniform test picks the unmasked fast path) and runs the online softmax in
//     registers over all its keys of the step (a row lives in 4 lanes; the running max moves lazily, so the
//     accumulator is rescaled on few steps),
//   * computes O^T += V^T P^T on 16x16x32 MFMA over its two sub-tiles at once (16x16x16 at HD 512) with V^T
//     read transposed from LDS (ds_read_b64_tr_b16) and P^T straight from the softmax registers.
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
#include <algorithm>
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
    int fold;          // 1: fold each XCD's slots (two co-resident workgroups per CU take a long and a short item)
};

// A workgroup is RG x KG waves. RB: 16-row blocks per wave; RG: row groups (waves splitting the tile's rows); KG:
// key groups (waves splitting each step's keys); NS: LDS stages; NSUB: 16-key sub-tiles per wave and step.
// RB = 1: the row groups split the tile's rows (the first half of them on the first half tile).
template <int HD, int RB, int RG, int KG_, int NS_, int NSUB_>
struct PrefCfg {
    static constexpr int KG = KG_, NS = NS_, NW = RG * KG_, NT = NW * 64, NSUB = NSUB_;
    static constexpr int KT = 16 * NSUB;                 // keys per wave per step (NSUB 16-key sub-tiles)
    static constexpr int SK = KG * KT;                   // keys per step
    static constexpr int RR = RG * RB * 16;              // rows per workgroup tile
    static constexpr int HR = RR / 2;                    // rows per half tile
    static constexpr int KS = HD / 32;                   // QK k-steps (16x16x32)
    static constexpr int DB = HD / 16;                   // PV output dim blocks (16x16x16)
    static constexpr int DO = DB / KG;                   // output dim blocks each key group finishes
    static constexpr int SLOTS = HD / 8;                 // 16-byte slots per key row
    static constexpr int ROWB = HD * 2;                  // bytes per key row (16-bit operands)
    static constexpr int HALF = SK * ROWB;               // bytes of one K (or V) step tile
    static constexpr int STAGE = 2 * HALF;               // K and V of one step
    static constexpr int NLR = SK * SLOTS / 64;          // 64-slot rows of a step tile (one per wave load)
    static constexpr int NLD = (NLR + NW - 1) / NW;      // 16-byte loads per thread per step (K and V each)
    static constexpr size_t LDS_TILES = (size_t)NS * STAGE;
    static constexpr int XSTR = HD / KG + 4;             // merge exchange row stride (floats)
    // merge exchange of one row block: [row group][owner key group][sender slot (KG-1)][16 rows][XSTR]
    static constexpr size_t LDS_MERGE = (size_t)RG * KG * (KG - 1) * 16 * XSTR * 4;
    static constexpr size_t LDS_STATS = (size_t)2 * NW * RB * 16 * 4;
    static constexpr size_t LDS_MAIN = LDS_TILES > LDS_MERGE ? LDS_TILES : LDS_MERGE;
    static constexpr size_t STATS_OFF = LDS_MAIN;        // merge statistics past the tiles
    static constexpr size_t LDS = LDS_MAIN + LDS_STATS;
    // Waves past the last 64-slot row issue fewer loads; the step wait is then exact only without younger steps in
    // flight (NS = 2 waits for vmcnt 0).
    static_assert((SK * SLOTS) % 64 == 0 && (NLR % NW == 0 || NS == 2), "step loads");
    static_assert(RB == 1 && RG % 2 == 0, "row block layout");
    static_assert(NS >= 2 && NS <= 4, "stages");
    static_assert((KG == 2 || KG == 4) && DB % KG == 0, "key groups");
};

// Slot swizzles of key row k: 16-byte column c of key k sits in slot c ^ swz(k). V rows use vswz, a permutation of
// the low 4 key bits (keys 0-7 to the even slots, 8-15 to the odd ones), which spreads the 8 keys x 2 columns that
// the 32 lanes of a half V transpose read (keys 4g..4g+3 for g = 0, 1 or g = 2, 3) over all 16 slots of a 256-byte
// bank row. K rows are read 16 bytes per lane by key (lane = key, column 4 ks + g): kswz(k) = k puts the 8 (16)
// keys of a lane group on distinct bank quads (vswz, with its even slots for keys 0-7, measured 4 conflict cycles
// per read there).
__device__ __forceinline__ int vswz(int k) { return ((k & 7) << 1) | ((k >> 3) & 1); }
__device__ __forceinline__ int kswz(int k) { return k & 15; }

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// Wait until at most `pending` later steps (PER memory operations each) are still in flight.
template <int PER>
__device__ __forceinline__ void wait_steps(int pending) {
    if (pending >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PER) : "memory");
    else if (pending == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int HD, int RB, int RG, int KG_, int NS_, int NSUB, int WPE, int KVT, int QT, int OT>
__global__ void __launch_bounds__(RG * KG_ * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
prefill_kernel(const PrefArgs a) {
    using Cf = PrefCfg<HD, RB, RG, KG_, NS_, NSUB>;
    constexpr int KG = Cf::KG, NS = Cf::NS, SK = Cf::SK, KS = Cf::KS, DB = Cf::DB, NLD = Cf::NLD, DO = Cf::DO;
    constexpr int SLOTS = Cf::SLOTS, ROWB = Cf::ROWB, HR = Cf::HR;
    constexpr bool F16 = OpIsF16<KVT>::value;
    constexpr bool DMA = KVT != DT_FP32;                 // 16-bit caches go straight to LDS
    using KE = typename Elem<KVT>::T;
    using QE = typename Elem<QT>::T;
    extern __shared__ __align__(16) unsigned char smem[];
    float *stm = reinterpret_cast<float *>(smem + Cf::STATS_OFF), *stl = stm + Cf::NW * RB * 16;

    const Problem &p = a.p;
    // XCD-aware work index: dispatch slot b runs on XCD b % 8, and consecutive work items (one KV head's tiles,
    // longest first) share an XCD, so that head's K/V stays in one L2. With a.fold the local slot k is folded:
    // slots k and k + per/2 - which the dispatcher places on the same CU when two workgroups fit a CU and the grid
    // is one round - take the k-th longest and the k-th shortest item.
    const int per = (int)gridDim.x / 8, k_loc = (int)blockIdx.x / 8, h_loc = (per + 1) / 2;
    const int w_item = ((int)blockIdx.x % 8) * per + (!a.fold || k_loc < h_loc ? k_loc : per - 1 - (k_loc - h_loc));
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
    // (S % SLOTS) ^ kswz(key) (vswz(key)) of key row key = S / SLOTS; its byte offset from the step's first key row
    // is fixed.
    const unsigned krow_b = (unsigned)(krow * sizeof(KE));
    unsigned ld_koff[NLD], ld_voff[NLD];
#pragma unroll
    for (int u = 0; u < NLD; u++) {
        const int S = (wave * NLD + u) * 64 + lane, key = S / SLOTS;
        ld_koff[u] = (unsigned)key * krow_b + (unsigned)(((S % SLOTS) ^ kswz(key)) * 8 * sizeof(KE));
        ld_voff[u] = (unsigned)key * krow_b + (unsigned)(((S % SLOTS) ^ vswz(key)) * 8 * sizeof(KE));
    }
    // Step k of the walk into stage k % NS. Keys past the last position re-read that position (they are masked), so
    // every load is in bounds; only a step that crosses the end needs the clamped addresses.
    // Loads [u0, u1) of the thread's NLD slots (K and V each).
    // 16-bit caches: buffer loads straight into LDS over the byte range the workgroup may read (the ring, or the
    // keys below hi_b), so the rows past the last key of a step read as zeros (they are masked) without clamping.
    const uint32_t kv_bytes = p.kv_cap > 0 ? (uint32_t)p.kv_cap * krow_b
                                           : (uint32_t)(max(hi_b, 1) - 1) * krow_b + (uint32_t)(HD * sizeof(KE));
    int it_cur = 0;                                                     // the step being computed
    // Step k < 0 is a no-op step: every lane is out of range, so its loads write zeros into the stage of the step
    // before (already consumed by every wave) and touch no memory; this keeps the issue points branch-free.
    // prep(k) forms a step's buffer descriptors and stage once; issue_part(st, u0, u1) issues slots [u0, u1).
    struct StepLd { __amdgpu_buffer_rsrc_t krs, vrs; unsigned char *kd; int s, soff; };
    auto prep = [&](int k) {
        StepLd st;
        st.s = s0 + (k < 0 ? 0 : k);
        st.kd = smem + (size_t)((k < 0 ? it_cur + 1 : k) % NS) * Cf::STAGE;
        st.soff = __builtin_amdgcn_readfirstlane(key_row(p, st.s * SK) * (int)krow_b);
        // the step's rows as the buffer (the range check covers the vector offset only)
        const uint32_t left = k < 0 || (uint32_t)st.soff >= kv_bytes ? 0u : kv_bytes - (uint32_t)st.soff;
        st.krs = make_rsrc(reinterpret_cast<const char *>(Kb) + st.soff, left);
        st.vrs = make_rsrc(reinterpret_cast<const char *>(Vb) + st.soff, left);
        return st;
    };
    auto issue_part = [&](const StepLd &st, int u0, int u1) {
        const int s = st.s, soff = st.soff;
        unsigned char *kd = st.kd, *vd = kd + Cf::HALF;
#pragma unroll
        for (int u = 0; u < NLD; u++) {
            if (u < u0 || u >= u1) continue;
            const int i = wave * NLD + u;
            if (Cf::NLR % Cf::NW != 0 && i >= Cf::NLR) continue;       // wave-uniform: past the tile
            if constexpr (!DMA) {
                const char *ks = reinterpret_cast<const char *>(Kb) + soff;
                const char *vs = reinterpret_cast<const char *>(Vb) + soff;
                unsigned koff = ld_koff[u], voff = ld_voff[u];
                const int S = i * 64 + lane;
                if (s * SK + SK > hi_b) {
                    const unsigned key = (unsigned)(S / SLOTS), lim = (unsigned)(hi_b - 1 - s * SK);
                    if (key > lim) { koff -= (key - lim) * krow_b; voff -= (key - lim) * krow_b; }
                }
                *reinterpret_cast<u32x4 *>(kd + (size_t)S * 16) = load8_op<KVT, F16>(reinterpret_cast<const KE *>(ks + koff));
                *reinterpret_cast<u32x4 *>(vd + (size_t)S * 16) = load8_op<KVT, F16>(reinterpret_cast<const KE *>(vs + voff));
            } else {
                buffer_load_lds16(st.krs, kd + (size_t)i * 1024, (int)ld_koff[u]);
                buffer_load_lds16(st.vrs, vd + (size_t)i * 1024, (int)ld_voff[u]);
            }
        }
    };
    auto issue = [&](int k) { issue_part(prep(k), 0, NLD); };
    // The next step's loads go out in four parts spread over the current step (between the QK batches, after
    // the softmax, between the PV batches): a workgroup's 8 waves issuing all of them at once stalled every wave
    // on the vector memory pipe for about a thousand cycles per step.
    constexpr int NPART = 4, PPART = (NLD + NPART - 1) / NPART;
    auto issue_pt = [&](const StepLd &st, int pt) { issue_part(st, pt * PPART, min(NLD, (pt + 1) * PPART)); };
    if (nsteps > 0) issue(0);

    // This wave's row blocks: block rb covers rows [lrow[rb], lrow[rb] + 16) of half tile hb[rb]. Q fragments and
    // positions per row (an invalid row has pos = -1 and attends nothing), and the wave-uniform key span of each
    // block (positions grow with the row's token).
    int htok[RB], hrows[RB], lrow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int hb = (rg * 16) / HR;
        lrow[rb] = rg * 16 - hb * HR;
        htok[rb] = hb ? tok0[1] : tok0[0];
        hrows[rb] = (hb ? tok1[1] - tok0[1] : tok1[0] - tok0[0]) * GRP;
    }
    int rpos[RB], rlo[RB];
    u32x4 qop[RB][KS];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int rho = lrow[rb] + ln;
        const bool valid = rho < hrows[rb];
        const int t = htok[rb] + (valid ? rho / GRP : 0), h = kvh * GRP + (valid ? rho % GRP : 0);
        const int ps = pbase + t;
        rpos[rb] = valid ? ps : -1;
        rlo[rb] = win_lo(ps, p.window);
        const QE *qrow = reinterpret_cast<const QE *>(p.Q) + ((size_t)(seq * p.T + t) * p.NQ + h) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qop[rb][ks] = valid ? load8_op<QT, F16>(qrow + 32 * ks) : u32x4{0u, 0u, 0u, 0u};
    }
    // Steps 1..NS-2 go out after the Q loads, so that waiting for step it never waits for younger steps.
#pragma unroll
    for (int k = 1; k < NS - 1; k++)
        if (k < nsteps) issue(k);
    int wlo[RB], whi[RB], lo_max[RB], pos_min[RB];
    int wlo_all = INT_MAX, whi_all = -1;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int rho1 = min(hrows[rb], lrow[rb] + 16);
        wlo[rb] = INT_MAX; whi[rb] = -1; lo_max[rb] = 0; pos_min[rb] = INT_MAX;
        if (lrow[rb] < rho1) {
            const int pf = pbase + htok[rb] + lrow[rb] / GRP, pl = pbase + htok[rb] + (rho1 - 1) / GRP;
            wlo[rb] = max(win_lo(pf, p.window), j_lo); whi[rb] = min(pl, j_hi - 1);
            lo_max[rb] = win_lo(pl, p.window); pos_min[rb] = pf;
        }
        wlo_all = min(wlo_all, wlo[rb]); whi_all = max(whi_all, whi[rb]);
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
    const unsigned kaddr = lds0 + (kg * Cf::KT + ln) * ROWB + ((g ^ kswz(ln)) << 4);
    const unsigned vaddr = lds0 + Cf::HALF + (kg * Cf::KT + vr) * ROWB + 8 * (ln & 1) + ((((ln & 3) >> 1) ^ vswz(vr)) << 4);

    // One step's work for the row blocks in ACT (a wave-uniform bit mask). QK: the K fragments of a sub-tile are
    // read in batches of 4 k-steps (inline asm, one wait per batch, so the reads are not serialised behind the
    // MFMAs) and each active row block runs its MFMA chain on them. Then one softmax update, then PV with V^T
    // fragments in batches of 8 transpose reads. A block left out keeps its state exactly (it attends no key).
    auto step = [&](const int ACT, int jw, unsigned stage, const StepLd &nxt) {
        int pt = 0;
        // Per-lane LDS bases, made opaque so that the XOR-swizzled fragment addresses are formed next to their
        // reads instead of being hoisted out of the step loop (which held ~30 address registers live and spilled).
        unsigned kbase = kaddr + stage, vbase = vaddr + stage;
        asm volatile("" : "+v"(kbase), "+v"(vbase));
        f32x4 s[NSUB][RB], s2[NSUB][RB];
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) s[sub][rb] = s2[sub][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
        {
            // Software-pipelined: batch b = k-steps 2b, 2b+1 of every sub-tile (4 reads at NSUB = 2); batch b+1 is
            // read before batch b's MFMAs, so the LDS latency hides under them (4 independent MFMA chains).
            constexpr int KPB = 2, NB = KS / KPB, RPB = KPB * NSUB;
            static_assert(RPB == 4 || RPB == 2, "batch size");
            u32x4 kb[2][RPB];
            auto rd = [&](int b, u32x4 (&dst)[RPB]) {
#pragma unroll
                for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
                    for (int kk = 0; kk < KPB; kk++)
                        asm volatile("ds_read_b128 %0, %1" : "=v"(dst[sub * KPB + kk])
                                     : "v"((kbase + sub * 16 * ROWB) ^ (64u * (b * KPB + kk))) : "memory");
            };
            rd(0, kb[0]);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                u32x4 (&cur)[RPB] = kb[b & 1];
                if (b + 1 < NB) {
                    rd(b + 1, kb[(b + 1) & 1]);
                    if constexpr (RPB == 4)
                        asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3])::"memory");
                    else
                        asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(cur[0]), "+v"(cur[RPB - 1])::"memory");
                } else {
                    if constexpr (RPB == 4)
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3])::"memory");
                    else
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(cur[0]), "+v"(cur[RPB - 1])::"memory");
                }
                if (b == 0 || b == NB / 2) issue_pt(nxt, pt++);
#pragma unroll
                for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
                    for (int kk = 0; kk < KPB; kk++) {
                        if (kk & 1) s2[sub][0] = mfma16<F16>(cur[sub * KPB + kk], qop[0][b * KPB + kk], s2[sub][0]);
                        else s[sub][0] = mfma16<F16>(cur[sub * KPB + kk], qop[0][b * KPB + kk], s[sub][0]);
                    }
            }
        }
        float tv[NSUB][RB][4], mnew[RB];
        bool need = false;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            mnew[rb] = m[rb];
            if (!((ACT >> rb) & 1)) continue;
            const bool full = jw >= j_lo && jw + Cf::KT <= j_hi && jw >= lo_max[rb] && jw + Cf::KT - 1 <= pos_min[rb];
            float mx = kNegInf;
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++) {
                const f32x4 sc = (s[sub][rb] + s2[sub][rb]) * a.sl2;
#pragma unroll
                for (int i = 0; i < 4; i++) tv[sub][rb][i] = sc[i];
            }
            if (!full) {                                        // one wave-uniform test; per key only off the fast path
#pragma unroll
                for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = jw + 16 * sub + 4 * g + i;
                        if (!(key >= j_lo && key < j_hi && key >= rlo[rb] && key <= rpos[rb])) tv[sub][rb][i] = kNegInf;
                    }
            }
#pragma unroll
            for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
                for (int i = 0; i < 4; i++) mx = fmaxf(mx, tv[sub][rb][i]);
            mx = max_over_groups(mx);
            if (mx > m[rb] + kRescaleThreshold) { mnew[rb] = mx; need = true; }
        }
        if (__any(need)) {
            // every block (an inactive one has mnew == m, alpha = 1): a per-block condition here made the compiler
            // keep two copies of the accumulator
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                const float alpha = (mnew[rb] == m[rb]) ? 1.f : fast_exp2(m[rb] - mnew[rb]);
                l[rb] *= alpha; m[rb] = mnew[rb];
#pragma unroll
                for (int db = 0; db < DB; db++) acc[rb][db] *= alpha;
            }
        }
        while (pt < 3) issue_pt(nxt, pt++);
        PFrag<F16> pop[NSUB][RB];
#pragma unroll
        for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                if (!((ACT >> rb) & 1)) { pop[sub][rb] = PFrag<F16>{u32x2{0u, 0u}, u32x2{0u, 0u}}; continue; }
                float pv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) pv[i] = (tv[sub][rb][i] == kNegInf) ? 0.f : fast_exp2(tv[sub][rb][i] - m[rb]);
                l[rb] += (pv[0] + pv[1]) + (pv[2] + pv[3]);
                pop[sub][rb] = p_frag<F16>(pv[0], pv[1], pv[2], pv[3]);
            }
        if constexpr (NSUB == 2) {
            // PV on 16x16x32 over both sub-tiles at once (the order of keys inside an MFMA's reduction is free):
            // k-group g of the MFMA holds keys 4g..4g+3 of sub-tile 0 and then of sub-tile 1, which is what the
            // lane's two S^T fragments hold (B operand = the two P^T halves) and what two transpose reads of V give
            // (A operand). Software-pipelined: batch b = 4 dim blocks (8 reads); batch b+1 is read before batch b's
            // MFMAs.
            constexpr int PB = 4, NPB = DB / PB;
            u32x2 vb2[2][2 * PB];
            auto rdv = [&](int b, u32x2 (&dst)[2 * PB]) {
#pragma unroll
                for (int j = 0; j < PB; j++)
#pragma unroll
                    for (int sub = 0; sub < 2; sub++)
                        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(dst[2 * j + sub])
                                     : "v"((vbase + sub * 16 * ROWB) ^ (32u * (b * PB + j))) : "memory");
            };
            rdv(0, vb2[0]);
#pragma unroll
            for (int b = 0; b < NPB; b++) {
                u32x2 (&cur)[2 * PB] = vb2[b & 1];
                if (b + 1 < NPB) {
                    rdv(b + 1, vb2[(b + 1) & 1]);
                    asm volatile("s_waitcnt lgkmcnt(8)" : "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3]), "+v"(cur[4]),
                                 "+v"(cur[5]), "+v"(cur[6]), "+v"(cur[7])::"memory");
                } else {
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3]), "+v"(cur[4]),
                                 "+v"(cur[5]), "+v"(cur[6]), "+v"(cur[7])::"memory");
                }
#pragma unroll
                for (int j = 0; j < PB; j++)
                    acc[0][b * PB + j] = mfma_pv32_hi<F16>(u32x4{cur[2 * j][0], cur[2 * j][1], cur[2 * j + 1][0], cur[2 * j + 1][1]},
                                                           pop[0][0], pop[1][0], acc[0][b * PB + j]);
#pragma unroll
                for (int j = 0; j < PB; j++)
                    acc[0][b * PB + j] = mfma_pv32_lo<F16>(u32x4{cur[2 * j][0], cur[2 * j][1], cur[2 * j + 1][0], cur[2 * j + 1][1]},
                                                           pop[0][0], pop[1][0], acc[0][b * PB + j]);
                if (pt < NPART && b % 2 == 1) issue_pt(nxt, pt++);
            }
        }
        if constexpr (NSUB != 2) {
            // Software-pipelined PV: batch b = 4 dim blocks of one sub-tile; batch b+1 is read before batch b's MFMAs.
            constexpr int PB = 4, NPB = NSUB * DB / PB;
            u32x2 vb2[2][PB];
            auto rdv = [&](int b, u32x2 (&dst)[PB]) {
                const int sub = b / (DB / PB), d0 = (b % (DB / PB)) * PB;
#pragma unroll
                for (int j = 0; j < PB; j++)
                    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(dst[j]) : "v"((vbase + sub * 16 * ROWB) ^ (32u * (d0 + j))) : "memory");
            };
            rdv(0, vb2[0]);
#pragma unroll
            for (int b = 0; b < NPB; b++) {
                u32x2 (&cur)[PB] = vb2[b & 1];
                if (b + 1 < NPB) {
                    rdv(b + 1, vb2[(b + 1) & 1]);
                    asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3])::"memory");
                } else {
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(cur[0]), "+v"(cur[1]), "+v"(cur[2]), "+v"(cur[3])::"memory");
                }
                const int sub = b / (DB / PB), d0 = (b % (DB / PB)) * PB;
#pragma unroll
                for (int j = 0; j < PB; j++) acc[0][d0 + j] = mfma_pv16<F16, KVT != DT_FP32>(cur[j], pop[sub][0], acc[0][d0 + j]);
                if (pt < NPART && b % 4 == 3) issue_pt(nxt, pt++);
            }
        }
        while (pt < NPART) issue_pt(nxt, pt++);
    };

    // The wave's keys of step it start at jw(it) = (s0 + it) * SK + kg * KT. It attends steps [it0, it1]: before
    // and after them it only keeps the barriers and the loads going. Three loops instead of a skip branch keep the
    // step loop a single path (a skip path made the register allocator copy the accumulator on every step).
    auto fdiv = [](int x, int y) { return x >= 0 ? x / y : -((-x + y - 1) / y); };
    const int jb = s0 * SK + kg * Cf::KT;
    const int it0 = __builtin_amdgcn_readfirstlane(max(0, -fdiv(-(wlo_all - Cf::KT + 1 - jb), SK)));
    const int it1 = __builtin_amdgcn_readfirstlane(whi_all < 0 ? -1 : min(nsteps - 1, fdiv(whi_all - jb, SK)));
    auto sync_step = [&](int it) {
        // Step it is the oldest load batch in flight; up to NS-2 younger steps may stay in flight.
        wait_steps<DMA ? 2 * NLD : 0>(min(NS - 2, nsteps - 1 - it));
        __syncthreads();                                                // everyone's step it, and step it-1 is consumed
        it_cur = it;
        return it + NS - 1 < nsteps ? it + NS - 1 : -1;
    };
    int it = 0;
    for (; it < min(it0, nsteps); it++) issue(sync_step(it));
    for (; it <= it1; it++) {
        const int nxt = sync_step(it);
        const int jw = (s0 + it) * SK + kg * Cf::KT;
        const unsigned stage = (it % NS) * Cf::STAGE;
        int act = 0;                                                    // wave-uniform mask of active row blocks
#pragma unroll
        for (int rb = 0; rb < RB; rb++) act |= (jw > whi[rb] || jw + Cf::KT - 1 < wlo[rb]) ? 0 : 1 << rb;
        step(RB == 1 ? 1 : __builtin_amdgcn_readfirstlane(act), jw, stage, prep(nxt));
    }
    for (; it < nsteps; it++) issue(sync_step(it));
    // The no-op loads of the last steps still write (zeros) into a stage: drain them before the merge reuses the
    // tile region for its exchange and statistics.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int rb = 0; rb < RB; rb++) l[rb] = sum_over_groups(l[rb]);
    __syncthreads();                                                 // every wave is done with the K/V tiles

    // Merge the KG key-group states of each row (waves kg = 0..KG-1 of a row group hold the same rows). Every
    // lane derives the row's M = max m and L = sum l 2^(m - M) (key groups in order) from the published (m, l)
    // and scales its accumulator by 2^(m - M) / L (2^(m - M) for a split partial). Key group kg then owns output
    // dim blocks [kg*DO, (kg+1)*DO): it parks the other groups' blocks of its scaled accumulator in LDS, and sums
    // its own blocks over the key groups in order 0..KG-1 (the same order for every row and tiling).
    const int NQ = p.NQ;
    if (g == 0) {
#pragma unroll
        for (int rb = 0; rb < RB; rb++) { stm[wave * RB * 16 + rb * 16 + ln] = m[rb]; stl[wave * RB * 16 + rb * 16 + ln] = l[rb]; }
    }
    __syncthreads();
    float *xb = reinterpret_cast<float *>(smem);                        // exchange (reuses the tiles)
    auto slot = [](int sender, int owner) { return sender < owner ? sender : sender - 1; };
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int srow = rb * 16 + ln;
        float M = kNegInf;
#pragma unroll
        for (int k = 0; k < KG; k++) M = fmaxf(M, stm[(rg * KG + k) * RB * 16 + srow]);
        float L = 0.f;
#pragma unroll
        for (int k = 0; k < KG; k++) {
            const float mk = stm[(rg * KG + k) * RB * 16 + srow];
            if (mk != kNegInf) L += stl[(rg * KG + k) * RB * 16 + srow] * fast_exp2(mk - M);
        }
        float f = (m[rb] == kNegInf) ? 0.f : fast_exp2(m[rb] - M);
        if (a.kv_split <= 0) f *= (L > 0.f ? 1.f / L : 0.f);
        const int rho = lrow[rb] + ln;
        const bool rvalid = rho < hrows[rb];
        const int r = seq * p.T + htok[rb] + (rvalid ? rho / GRP : 0), h = kvh * GRP + (rvalid ? rho % GRP : 0);
        if (kg == 0 && g == 0 && rvalid) {
            if (a.kv_split > 0) {
                const size_t pi = ((size_t)r * NQ + h) * a.part.ns_cap + sp;
                a.part.m[pi] = M; a.part.l[pi] = L;
            } else if (p.lse) {
                p.lse[(size_t)r * NQ + h] = (L > 0.f) ? (M + log2f(L)) * kLn2 : kNegInf;
            }
        }
        // park the blocks of the other owners (constant indices keep acc in registers)
        static_for<KG>([&](auto o_c) {
            constexpr int O = decltype(o_c)::value;
            if (O == kg) return;
            float *dst = xb + ((((size_t)rg * KG + O) * (KG - 1) + slot(kg, O)) * 16 + ln) * Cf::XSTR + 4 * g;
#pragma unroll
            for (int j = 0; j < DO; j++) *reinterpret_cast<f32x4 *>(dst + 16 * j) = acc[rb][O * DO + j] * f;
        });
        __syncthreads();
        static_for<KG>([&](auto o_c) {
            constexpr int O = decltype(o_c)::value;
            if (O != kg || !rvalid) return;
#pragma unroll
            for (int j = 0; j < DO; j++) {
                f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < KG; k++) {
                    if (k == O) o = (k == 0) ? acc[rb][O * DO + j] * f : o + acc[rb][O * DO + j] * f;
                    else {
                        const f32x4 x = *reinterpret_cast<const f32x4 *>(
                            xb + ((((size_t)rg * KG + O) * (KG - 1) + slot(k, O)) * 16 + ln) * Cf::XSTR + 4 * g + 16 * j);
                        o = (k == 0) ? x : o + x;
                    }
                }
                const int d = 16 * (O * DO + j) + 4 * g;
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
        });
        if (rb + 1 < RB) __syncthreads();                               // the next block reuses the exchange
    }
}

// ---------------------------------------------------------------- host side
// Tile shapes. HD 128/256: 8 waves (two per SIMD, so one wave's MFMAs overlap the other's softmax and LDS
// traffic) as 4 row groups x 2 key groups, 16 rows and HD accumulator columns per wave, a 64-row workgroup tile
// (two 32-row half tiles), 64-key steps (two 16-key sub-tiles per wave) in two LDS stages. HD 512: the same 8 waves
// and 64-row tile with 32-key steps (a 32-key stage of HD 512 is 64 KB) and 252 VGPRs (a 16 x 512 accumulator per
// wave); the 4-wave 32-row tile it replaces ran the Gemma4 global prompt (T = 1024, one KV head, 16 q-heads) in
// two rounds of 256 workgroups: 92 vs 55 us.
// Measured alternatives at HD 256 (config 3, T = 1024): 4 waves over a 32-row tile, two workgroups per CU, 38.8
// vs 30.0 us; 16-key steps per wave, 33.1 us; two 16-row blocks per wave (one wave per SIMD), 36.9 us.
// HD 256, wide tile (W = 1): 12 waves (6 row groups, three per SIMD, 168 VGPRs) over a 96-row tile. Its half tile
// of 48 rows holds 8 tokens of a 6-head GQA group where the 32-row one holds 5 (30 rows), so the Qwen3.5 prompt
// (T = 1024, 24 q-heads over 4 KV heads) is 256 workgroups, one round, instead of 412 in two: 53.4 vs 37.2 us. It
// runs a prompt only when it needs fewer rounds of resident workgroups than the 64-row tile (config 3 is one
// round either way, and 31.0 vs 35.5 us there). The two tiles share the step (64 keys), the key groups and the
// merge order, so a row's bits do not depend on which one ran it.
// WPE: waves per SIMD the register allocation must allow. PAIR: whether a workgroup may take the causal
// half-tile pair (i, n-1-i) (one workgroup per CU) instead of neighbours.
template <int HD, int W> struct PrefTile;
template <> struct PrefTile<128, 0> { static constexpr int RB = 1, RG = 4, KG = 2, NS = 2, NSUB = 2, WPE = 2; static constexpr bool PAIR = true; };
template <> struct PrefTile<256, 0> { static constexpr int RB = 1, RG = 4, KG = 2, NS = 2, NSUB = 2, WPE = 2; static constexpr bool PAIR = true; };
template <> struct PrefTile<256, 1> { static constexpr int RB = 1, RG = 6, KG = 2, NS = 2, NSUB = 2, WPE = 3; static constexpr bool PAIR = true; };
template <> struct PrefTile<512, 0> { static constexpr int RB = 1, RG = 4, KG = 2, NS = 2, NSUB = 1, WPE = 2; static constexpr bool PAIR = true; };
template <int HD, int W>
using PrefTileCfg = PrefCfg<HD, PrefTile<HD, W>::RB, PrefTile<HD, W>::RG, PrefTile<HD, W>::KG, PrefTile<HD, W>::NS,
                            PrefTile<HD, W>::NSUB>;

template <int HD, int W, int KVT, int QT, int OT>
static hipError_t launch_pref_t(const PrefArgs &a, dim3 grid, hipStream_t st) {
    using T = PrefTile<HD, W>;
    using Cf = PrefTileCfg<HD, W>;
    static bool configured = false;
    auto kern = prefill_kernel<HD, T::RB, T::RG, T::KG, T::NS, T::NSUB, T::WPE, KVT, QT, OT>;
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
static hipError_t pref_dispatch_hd(const PrefArgs &a, int wide, dim3 grid, hipStream_t st) {
    switch (a.p.HD) {
    case 128: return launch_pref_t<128, 0, KVT, QT, OT>(a, grid, st);
    case 256: return wide ? launch_pref_t<256, 1, KVT, QT, OT>(a, grid, st) : launch_pref_t<256, 0, KVT, QT, OT>(a, grid, st);
    case 512: return launch_pref_t<512, 0, KVT, QT, OT>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

// Per tile shape (head dim, W): rows of a half tile, workgroups resident per CU, and whether it takes causal
// half-tile pairs. HD 128 and 512 have the one shape.
struct PrefShape { int hr, per_cu; bool pair; };
template <int HD, int W> static PrefShape pref_shape_t() {
    return PrefShape{PrefTileCfg<HD, W>::HR, (int)std::max<size_t>(1, (160u << 10) / PrefTileCfg<HD, W>::LDS),
                     PrefTile<HD, W>::PAIR};
}
static PrefShape pref_shape(int HD, int wide) {
    switch (HD) {
    case 128: return pref_shape_t<128, 0>();
    case 256: return wide ? pref_shape_t<256, 1>() : pref_shape_t<256, 0>();
    case 512: return pref_shape_t<512, 0>();
    default: return PrefShape{0, 1, false};
    }
}
static int pref_half_rows(int HD) { return pref_shape(HD, 0).hr; }
static int pref_per_cu(int HD) { return pref_shape(HD, 0).per_cu; }

// Key split for kv_split = -1: when the unsplit grid would fill at most half of the workgroup slots (a short run
// of queries over a long cached prefix), cut the keys into as many absolute splits as whole grids fit on them.
size_t prefill_lds_bytes(int HD) {
    switch (HD) {
    case 128: return PrefTileCfg<128, 0>::LDS;
    case 256: return PrefTileCfg<256, 0>::LDS;
    case 512: return PrefTileCfg<512, 0>::LDS;
    default: return 0;
    }
}

int prefill_auto_split(const Problem &p) {
    if (p.NQ % p.NKV) return 0;
    const int GRP = p.NQ / p.NKV, HR = pref_half_rows(p.HD);
    if (HR == 0 || GRP > HR) return 0;
    const int tqh = HR / GRP, nht = (p.T + tqh - 1) / tqh;
    const long nwg = (long)p.nseq * p.NKV * ((nht + 1) / 2);
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    const long slots = (long)ncu * pref_per_cu(p.HD);
    if (nwg <= 0 || 2 * nwg > slots) return 0;
    const int nsplit = (int)(slots / nwg);
    const int keys = p.max_pos + 1;
    int ks = (keys + nsplit - 1) / nsplit;
    ks = ((ks + 63) / 64) * 64;
    return ks >= keys ? 0 : ks;
}

hipError_t launch_prefill(const Problem &p, int kv_split, const Partials &part, hipStream_t st) {
    if (p.NQ % p.NKV || p.anc || p.pos_mode != 1) return hipErrorInvalidValue;
    const int GRP = p.NQ / p.NKV;
    if (pref_half_rows(p.HD) == 0 || GRP > pref_half_rows(p.HD)) return hipErrorInvalidValue;
    if (kv_split < 0 || (kv_split > 0 && kv_split % 64)) return hipErrorInvalidValue;
    const int nsplit = kv_split > 0 ? p.max_pos / kv_split + 1 : 1;
    if (kv_split > 0 && nsplit > part.ns_cap) return hipErrorInvalidValue;
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        ncu = 0;
    // Workgroups of a tile shape: half tiles of tqh tokens, two per workgroup.
    auto wgs = [&](const PrefShape &sh) { return (long)p.nseq * p.NKV * (((p.T + sh.hr / GRP - 1) / (sh.hr / GRP) + 1) / 2); };
    auto rounds = [&](const PrefShape &sh) { const long slots = (long)std::max(ncu, 1) * sh.per_cu; return (wgs(sh) + slots - 1) / slots; };
    // The wide HD 256 tile, when it takes fewer rounds of resident workgroups (unsplit prompts, 16-bit caches: the
    // fp32 cache's register staging spills in it).
    int wide = 0;
    if (p.HD == 256 && kv_split == 0 && p.kv_dtype != DT_FP32 && ncu > 0 && GRP <= pref_shape(256, 1).hr &&
        rounds(pref_shape(256, 1)) < rounds(pref_shape(256, 0)))
        wide = 1;
    const PrefShape sh = pref_shape(p.HD, wide);
    const int tqh = sh.hr / GRP;
    const int nht = (p.T + tqh - 1) / tqh;
    // Pair half tiles (i, n-1-i) when causal work varies across the prompt (no window, prefix shorter than the
    // chunk); otherwise a workgroup takes two neighbouring half tiles.
    const int pair = (sh.pair && kv_split == 0 && p.window == 0 && nht >= 2 && p.max_pos < 2 * p.T) ? 1 : 0;
    const int nitems = ((nht + 1) / 2) * nsplit;
    const long nwg = (long)p.nseq * p.NKV * nitems;
    if (nwg <= 0 || nwg > (1L << 30)) return hipErrorInvalidConfiguration;
    const int fold = (sh.per_cu >= 2 && nwg <= (long)sh.per_cu * ncu) ? 1 : 0;
    PrefArgs a{p, part, kv_split, nht, nsplit, tqh, pair, nitems, (int)nwg, p.scale * kLog2e, fold};
    dim3 grid((unsigned)(8 * ((nwg + 7) / 8)));
    hipError_t e = hipErrorInvalidValue;
    const int kv = p.kv_dtype, q = p.q_dtype, o = p.o_dtype;
    if (kv == DT_F16 && q == DT_FP32 && o == DT_FP32) e = pref_dispatch_hd<DT_F16, DT_FP32, DT_FP32>(a, wide, grid, st);
    else if (kv == DT_BF16 && q == DT_FP32 && o == DT_FP32) e = pref_dispatch_hd<DT_BF16, DT_FP32, DT_FP32>(a, wide, grid, st);
    else if (kv == DT_FP32 && q == DT_FP32 && o == DT_FP32) e = pref_dispatch_hd<DT_FP32, DT_FP32, DT_FP32>(a, wide, grid, st);
    else if (kv == DT_F16 && q == DT_F16 && o == DT_F16) e = pref_dispatch_hd<DT_F16, DT_F16, DT_F16>(a, wide, grid, st);
    else if (kv == DT_BF16 && q == DT_BF16 && o == DT_BF16) e = pref_dispatch_hd<DT_BF16, DT_BF16, DT_BF16>(a, wide, grid, st);
    else return hipErrorInvalidValue;
    if (e != hipSuccess || kv_split <= 0) return e;
    return launch_combine(p, kv_split, part, st);
}

}  // namespace dgx

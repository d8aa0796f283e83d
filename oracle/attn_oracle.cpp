// TEST INFRASTRUCTURE ONLY. CPU oracle for the attention hot path of hyunlord/dgx-serving.
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, and only as the
// checker / the timed CPU baseline. The product path (dgx-serving_amd/) never links, loads or calls it.
//
// What it restates (all citations are into the reference tree):
//   * fp64 attention over a KV cache, one (token, q-head) row at a time: dot products in double, softmax
//     in double, P.V in double, normalised at the end.
//       tests/test_attn_decode_split.cu:59-90   (decode / window, fp64 reference, error normalised by sum p|V|)
//       tests/test_flash_gemma.cu:128-161       (scale / window variants, threaded over rows)
//       tests/test_flash_v2.cu:281-297          (prefill / chunked prefill over a cached prefix)
//   * the "host-side C++/fp32" reference: dot in double, score rounded to float, expf softmax in float,
//     P.V accumulated in double of (p/sum)*V, written as float.
//       tests/test_kernels.cu:94-108
//   * key-attendance predicate (causal + sliding window + speculative tree mask):
//       kernels/attention_decode_split.cuh:51-52   lo = max(0, pos-window+1), keys [lo, pos]
//       kernels/attention_flash.cuh:177-178        tree: key < base always; key >= base iff bit (key-base) of
//                                                  anc[q] (key-base < 32); plus causal/window
//   * log-sum-exp of each row, LSE = m + ln(sum exp(s-m)) with s = scale * q.k. The reference keeps m and l in
//     private scratch (kernels/attention_decode_split.cuh:116, attention_flash.cuh:216); this exposes it.
//   * the split-KV LSE combine over absolute chunks of C keys, in ascending chunk order
//       kernels/attention_decode_split.cuh:147-165
//   * RN-even fp32 -> f16 / bf16 storage rounding (kv_store.cuh:85,102-103 __float2half_rn/__float2bfloat16_rn).
//   * the reference tests' input generators (LCG, xorshift*, the tree draft builder).
//       tests/test_flash_v2.cu:29, tests/test_flash_gemma.cu:39-42 (LCG (s>>8)/2^23-1)
//       tests/test_attn_decode_split.cu:21-22 (xorshift64*)
//       tests/test_fa2bs.cu:12 (LCG ((s>>8)&0xFFFFFF)/2^23-1), tests/test_treeattn.cu:10 (LCG 16-bit - 0.5)
//       tools/bench_serve_spec.cu:186-200 (draft tree: root, W children, chain of K-1; anc = OR of ancestors)
// Build: oracle/Makefile (g++ -O2 -shared -fPIC -pthread).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

extern "C" {

// ---------------------------------------------------------------- storage rounding (RN-even)
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x7fffffu;
    int exp = (int)((x >> 23) & 0xff);
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));     // inf / nan
    int e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);                              // overflow -> inf
    if (e <= 0) {                                                                  // subnormal / zero
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const int shift = 14 - e;                                                  // 24-bit mantissa -> (10+e)
        uint32_t h = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;                        // may carry into exponent
    return (uint16_t)(sign | h);
}
float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ffu, x;
    if (exp == 0x1f) x = sign | 0x7f800000u | (mant << 13);
    else if (exp == 0) {
        if (!mant) x = sign;
        else { int e = -1; do { e++; mant <<= 1; } while (!(mant & 0x400u)); x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13); }
    } else x = sign | ((uint32_t)(exp - 15 + 127) << 23) | (mant << 13);
    float f; memcpy(&f, &x, 4); return f;
}
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu)) return (uint16_t)((x >> 16) | 0x40u);   // quiet nan
    const uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}
float oracle_bf16_to_f32(uint16_t b) { uint32_t x = (uint32_t)b << 16; float f; memcpy(&f, &x, 4); return f; }

void oracle_round_f16(const float *src, float *dst, uint16_t *bits, size_t n) {
    for (size_t i = 0; i < n; i++) { const uint16_t h = oracle_f32_to_f16(src[i]); if (bits) bits[i] = h; if (dst) dst[i] = oracle_f16_to_f32(h); }
}
void oracle_round_bf16(const float *src, float *dst, uint16_t *bits, size_t n) {
    for (size_t i = 0; i < n; i++) { const uint16_t b = oracle_f32_to_bf16(src[i]); if (bits) bits[i] = b; if (dst) dst[i] = oracle_bf16_to_f32(b); }
}

// ---------------------------------------------------------------- generators of the reference tests
// tests/test_flash_v2.cu:29 and tests/test_flash_gemma.cu:39-42: s = s*1664525+1013904223, (s>>8)/2^23 - 1.
void oracle_gen_lcg(uint32_t *state, float *out, size_t n) {
    uint32_t s = *state;
    for (size_t i = 0; i < n; i++) { s = s * 1664525u + 1013904223u; out[i] = (float)(s >> 8) / 8388608.0f - 1.0f; }
    *state = s;
}
// tests/test_fa2bs.cu:12: ((s>>8)&0xFFFFFF)/2^23 - 1.
void oracle_gen_lcg24(uint32_t *state, float *out, size_t n) {
    uint32_t s = *state;
    for (size_t i = 0; i < n; i++) { s = s * 1664525u + 1013904223u; out[i] = (float)((s >> 8) & 0xFFFFFFu) / 8388608.0f - 1.0f; }
    *state = s;
}
// tests/test_treeattn.cu:10 and tests/test_kernels.cu frand: ((s>>8)&0xFFFF)/65536 - 0.5.
void oracle_gen_lcg16(uint32_t *state, float *out, size_t n) {
    uint32_t s = *state;
    for (size_t i = 0; i < n; i++) { s = s * 1664525u + 1013904223u; out[i] = (float)((s >> 8) & 0xFFFFu) / 65536.0f - 0.5f; }
    *state = s;
}
// tests/test_attn_decode_split.cu:21-22: xorshift64* -> [-1, 1).
void oracle_gen_xorshift(uint64_t *state, float *out, size_t n) {
    uint64_t s = *state;
    for (size_t i = 0; i < n; i++) {
        s ^= s >> 12; s ^= s << 25; s ^= s >> 27;
        out[i] = ((float)(uint32_t)((s * 2685821657736338717ull) >> 40) / 16777216.0f) * 2.f - 1.f;
    }
    *state = s;
}
// Seeded N(mean, sd^2) by Box-Muller over a splitmix64 counter stream (element i depends only on seed and i,
// so any slice can be regenerated independently). Used for the BASELINE.json configs (Q~N(0,1), K,V~N(0,0.5^2)).
static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull; z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull; return z ^ (z >> 31);
}
void oracle_gen_normal(uint64_t seed, uint64_t offset, float mean, float sd, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const uint64_t idx = offset + i, pair = idx >> 1;
        const uint64_t a = splitmix64(seed ^ (pair * 2 + 0) * 0xd1342543de82ef95ull);
        const uint64_t b = splitmix64(seed ^ (pair * 2 + 1) * 0xd1342543de82ef95ull);
        const double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740993.0);   // (0, 1]
        const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);           // [0, 1)
        const double r = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586476925 * u2;
        out[i] = (float)(mean + sd * ((idx & 1) ? r * std::sin(th) : r * std::cos(th)));
    }
}
// Seeded uniform integers in [lo, hi] (inclusive), one splitmix64 draw per value.
void oracle_gen_uniform_int(uint64_t seed, int lo, int hi, int *out, int n) {
    const uint64_t span = (uint64_t)(hi - lo) + 1;
    for (int i = 0; i < n; i++) out[i] = lo + (int)(splitmix64(seed * 0x9e3779b97f4a7c15ull + (uint64_t)i) % span);
}

// Ancestor-or-self bitmask of each node from parent indices (parent < child, root parent = -1).
// tools/bench_serve_spec.cu:199: anc[j] = OR over x = j, par[j], par[par[j]], ... of (1 << x).
int oracle_tree_anc(const int *parent, int n, uint32_t *anc) {
    if (n > 32) return -1;
    for (int j = 0; j < n; j++) {
        if (j > 0 && (parent[j] < 0 || parent[j] >= j)) return -2;
        uint32_t m = 0; for (int x = j; x >= 0; x = parent[x]) m |= 1u << x;
        anc[j] = m;
    }
    return 0;
}
// The reference's K/W draft tree shape (tools/bench_serve_spec.cu:186-196): node 0 root; nodes 1..W children of
// the root; then a chain of K-1 nodes hanging off node 1 (node W+i's parent is node W+i-1, first is node 1).
int oracle_tree_kw(int K, int W, int *parent, int *depth) {
    const int n = K + W;
    if (n > 32 || K < 1 || W < 1) return -1;
    parent[0] = -1; depth[0] = 0;
    for (int j = 0; j < W; j++) { parent[1 + j] = 0; depth[1 + j] = 1; }
    int prev = 1;
    for (int i = 1; i < K; i++) { const int idx = W + i; parent[idx] = prev; depth[idx] = depth[prev] + 1; prev = idx; }
    return n;
}
// Seeded random tree in BFS order: every node has at most `width` children and depth <= max_depth.
int oracle_tree_random(uint64_t seed, int n, int width, int max_depth, int *parent, int *depth) {
    if (n < 1 || n > 32) return -1;
    parent[0] = -1; depth[0] = 0;
    std::vector<int> kids(n, 0);
    for (int j = 1; j < n; j++) {
        std::vector<int> cand;
        for (int p = 0; p < j; p++) if (kids[p] < width && depth[p] < max_depth) cand.push_back(p);
        if (cand.empty()) return -2;
        // BFS order: prefer the shallowest candidates, pick among them at random.
        int dmin = 1 << 30; for (int p : cand) dmin = std::min(dmin, depth[p]);
        std::vector<int> best; for (int p : cand) if (depth[p] <= dmin + 1) best.push_back(p);
        const int p = best[splitmix64(seed * 0x2545f4914f6cdd1dull + (uint64_t)j) % best.size()];
        parent[j] = p; depth[j] = depth[p] + 1; kids[p]++;
    }
    return n;
}

// ---------------------------------------------------------------- attention
// One problem = T query tokens over per-sequence KV caches.
//   q     : [T, NQ, HD] fp32 values (the caller applies any operand rounding first)
//   k, v  : fp32 values; token t reads its sequence's cache at element offset kv_off[t] (layout [len, NKV, HD])
//   pos   : [T] absolute position of token t; the token attends keys j in [lo, pos] with lo = max(0, pos-window+1)
//   anc   : [T] tree bitmask or NULL; with anc, key j >= tree_base[t] is attended iff (j - tree_base[t]) < 32 and
//           bit (j - tree_base[t]) of anc[t] is set (keys below tree_base[t] follow the causal/window rule)
//   scale : softmax scale (0 -> 1/sqrt(HD))
//   mode  : 0 = fp64 throughout (the parity oracle), 1 = fp32 host reference of tests/test_kernels.cu:94-108
//   out   : [T, NQ, HD] double, lse: [T, NQ] double (natural log), either may be NULL
//   nthreads: worker threads over (token, head) rows (0 -> hardware concurrency)
// Returns 0, or -1 on bad arguments. A row that attends no key gets out = 0 and lse = -inf.
static inline bool attends(int j, int lo, int pos, const uint32_t *anc, const int *tree_base, int t) {
    if (j < lo || j > pos) return false;
    if (!anc) return true;
    const int tb = tree_base[t];
    if (j < tb) return true;
    const int d = j - tb;
    return d < 32 && ((anc[t] >> d) & 1u);
}

int oracle_attention(const float *q, const float *k, const float *v, const long *kv_off, const int *pos,
                     const uint32_t *anc, const int *tree_base, int T, int NQ, int NKV, int HD, float scale,
                     int window, int mode, double *out, double *lse, int nthreads) {
    if (T < 0 || NQ <= 0 || NKV <= 0 || HD <= 0 || NQ % NKV) return -1;
    if (anc && !tree_base) return -1;
    const int GRP = NQ / NKV;
    const double sc = scale > 0.f ? (double)scale : 1.0 / std::sqrt((double)HD);
    const float scf = scale > 0.f ? scale : 1.0f / std::sqrt((float)HD);
    if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
    std::atomic<long> next{0};
    const long rows = (long)T * NQ;
    auto worker = [&]() {
        std::vector<double> s64; std::vector<float> s32; std::vector<double> acc(HD);
        for (long row = next.fetch_add(1); row < rows; row = next.fetch_add(1)) {
            const int t = (int)(row / NQ), h = (int)(row % NQ), kvh = h / GRP, p = pos[t];
            const int lo = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
            const float *qq = q + (size_t)row * HD;
            const float *kb = k + kv_off[t], *vb = v + kv_off[t];
            const int n = p - lo + 1 > 0 ? p - lo + 1 : 0;
            std::fill(acc.begin(), acc.end(), 0.0);
            double rlse = -std::numeric_limits<double>::infinity();
            if (mode == 0) {
                s64.assign(n, 0.0);
                double m = -std::numeric_limits<double>::infinity();
                for (int j = lo; j <= p; j++) {
                    if (!attends(j, lo, p, anc, tree_base, t)) { s64[j - lo] = -std::numeric_limits<double>::infinity(); continue; }
                    const float *kk = kb + ((size_t)j * NKV + kvh) * HD;
                    double d = 0; for (int c = 0; c < HD; c++) d += (double)qq[c] * kk[c];
                    s64[j - lo] = d * sc; m = std::max(m, s64[j - lo]);
                }
                if (m > -std::numeric_limits<double>::infinity()) {
                    double z = 0; for (auto &x : s64) { x = std::exp(x - m); z += x; }
                    for (int j = lo; j <= p; j++) {
                        const double w = s64[j - lo]; if (w == 0.0) continue;
                        const float *vv = vb + ((size_t)j * NKV + kvh) * HD;
                        for (int c = 0; c < HD; c++) acc[c] += w * vv[c];
                    }
                    for (int c = 0; c < HD; c++) acc[c] /= z;
                    rlse = m + std::log(z);
                }
            } else {
                // tests/test_kernels.cu:94-108: double dot, float score, float max/expf/sum, double P.V of (p/sum)*V.
                s32.assign(n, 0.f);
                float m = -std::numeric_limits<float>::max(); bool any = false;
                for (int j = lo; j <= p; j++) {
                    if (!attends(j, lo, p, anc, tree_base, t)) { s32[j - lo] = -std::numeric_limits<float>::infinity(); continue; }
                    const float *kk = kb + ((size_t)j * NKV + kvh) * HD;
                    double d = 0; for (int c = 0; c < HD; c++) d += (double)qq[c] * kk[c];
                    s32[j - lo] = (float)(d * sc); (void)scf; m = std::max(m, s32[j - lo]); any = true;
                }
                if (any) {
                    float z = 0.f; for (auto &x : s32) { x = expf(x - m); z += x; }
                    for (int j = lo; j <= p; j++) {
                        const float w = s32[j - lo] / z; if (w == 0.f) continue;
                        const float *vv = vb + ((size_t)j * NKV + kvh) * HD;
                        for (int c = 0; c < HD; c++) acc[c] += (double)w * vv[c];
                    }
                    for (int c = 0; c < HD; c++) acc[c] = (double)(float)acc[c];
                    rlse = (double)m + std::log((double)z);
                }
            }
            if (out) for (int c = 0; c < HD; c++) out[(size_t)row * HD + c] = acc[c];
            if (lse) lse[row] = rlse;
        }
    };
    std::vector<std::thread> pool;
    for (int i = 0; i < nthreads - 1; i++) pool.emplace_back(worker);
    worker();
    for (auto &th : pool) th.join();
    return 0;
}

// Split-KV LSE combine restated (kernels/attention_decode_split.cuh:147-165): partial (m_c, l_c, acc_c) of
// absolute chunks c in [c_lo, c_hi], combined in ascending order: mg = max m_c, w_c = exp(m_c - mg),
// O = sum w_c acc_c / sum w_c l_c, LSE = mg + ln(sum w_c l_c). Partials are computed here in fp64 from the
// same inputs, chunk by chunk, so the result can be compared with the unsplit oracle (associativity check).
int oracle_attention_split(const float *q, const float *k, const float *v, const long *kv_off, const int *pos,
                           int T, int NQ, int NKV, int HD, float scale, int window, int C,
                           double *out, double *lse) {
    if (C <= 0 || NQ % NKV) return -1;
    const int GRP = NQ / NKV;
    const double sc = scale > 0.f ? (double)scale : 1.0 / std::sqrt((double)HD);
    std::vector<double> acc(HD), tot(HD);
    for (long row = 0; row < (long)T * NQ; row++) {
        const int t = (int)(row / NQ), h = (int)(row % NQ), kvh = h / GRP, p = pos[t];
        const int lo = (window > 0 && p - window + 1 > 0) ? p - window + 1 : 0;
        const float *qq = q + (size_t)row * HD;
        const float *kb = k + kv_off[t], *vb = v + kv_off[t];
        std::vector<double> cm, cl; std::vector<std::vector<double>> cacc;
        for (int c = lo / C; c <= p / C; c++) {
            const int j0 = std::max(lo, c * C), j1 = std::min(p + 1, (c + 1) * C);
            double m = -INFINITY; std::vector<double> s(j1 - j0);
            for (int j = j0; j < j1; j++) {
                const float *kk = kb + ((size_t)j * NKV + kvh) * HD;
                double d = 0; for (int x = 0; x < HD; x++) d += (double)qq[x] * kk[x];
                s[j - j0] = d * sc; m = std::max(m, s[j - j0]);
            }
            double l = 0; std::fill(acc.begin(), acc.end(), 0.0);
            for (int j = j0; j < j1; j++) {
                const double w = std::exp(s[j - j0] - m); l += w;
                const float *vv = vb + ((size_t)j * NKV + kvh) * HD;
                for (int x = 0; x < HD; x++) acc[x] += w * vv[x];
            }
            cm.push_back(m); cl.push_back(l); cacc.push_back(acc);
        }
        double mg = -INFINITY; for (double m : cm) mg = std::max(mg, m);
        double lg = 0; std::fill(tot.begin(), tot.end(), 0.0);
        for (size_t c = 0; c < cm.size(); c++) {
            const double w = std::exp(cm[c] - mg); lg += cl[c] * w;
            for (int x = 0; x < HD; x++) tot[x] += cacc[c][x] * w;
        }
        if (out) for (int x = 0; x < HD; x++) out[(size_t)row * HD + x] = cm.empty() ? 0.0 : tot[x] / lg;
        if (lse) lse[row] = cm.empty() ? -INFINITY : mg + std::log(lg);
    }
    return 0;
}

// Per-head RMSNorm (+ rotate-half RoPE) of rows x [rows, hd] in fp64, restating norm_rope_store_kernel
// (kernels/norm_fused.cuh:84-126): y = x / sqrt(sum(x^2) / hd + eps) * W (W null: no scale; :34-52), then with
// c = cosT[p * hd + e], s = sinT[p * hd + e] for e < hd / 2 and p = pos[r] (:111-118):
// o_e = y_e c - y_{e+hd/2} s, o_{e+hd/2} = y_{e+hd/2} c + y_e s. rope = 0: o = y.
int oracle_norm_rope(const float *x, const float *W, int rows, int hd, float eps, const float *cosT,
                     const float *sinT, const int *pos, int rope, double *out) {
    if (rows < 0 || hd <= 0 || (rope && (hd % 2 || !cosT || !sinT || !pos))) return -1;
    std::vector<double> y(hd);
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * hd;
        double ss = 0;
        for (int e = 0; e < hd; e++) ss += (double)xr[e] * xr[e];
        const double inv = 1.0 / std::sqrt(ss / hd + (double)eps);
        for (int e = 0; e < hd; e++) y[e] = (double)xr[e] * inv * (W ? (double)W[e] : 1.0);
        double *o = out + (size_t)r * hd;
        if (!rope) { for (int e = 0; e < hd; e++) o[e] = y[e]; continue; }
        const int h = hd / 2;
        const float *cr = cosT + (size_t)pos[r] * hd, *sr = sinT + (size_t)pos[r] * hd;
        for (int e = 0; e < h; e++) {
            const double c = cr[e], sn = sr[e];
            o[e] = y[e] * c - y[e + h] * sn;
            o[e + h] = y[e + h] * c + y[e] * sn;
        }
    }
    return 0;
}

}  // extern "C"

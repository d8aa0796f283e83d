// Reference-style C++ gates run through include/dgx_attn.hpp: the reference's own launcher names, argument order
// and defaults, called from a plain C++ main as the reference's tests/test_*.cu mains call them.
//
//   gate1   tests/test_attn_decode_split.cu:58-90   launch_attn_decode_split over KV lengths 1..32768, both Gemma
//                                                   layer shapes (sliding HD256 16q/8kv w1024, full HD512 16q/1kv),
//                                                   scale 1.0, xorshift inputs; K/V in the G4_KV_DTYPE storage
//   gate2v  tests/test_attn_decode_split.cu:92-105  verify rows: bases {1000,1017,1023,2040,8190} x S=2..16 on a
//                                                   shared cache, each row bitwise equal to its S=1 launch
//   gate2b  tests/test_attn_decode_split.cu:107-125 batch rows W=1..12 with own KV and ragged positions, bitwise
//                                                   equal to the S=1 launch on that slot
//   tree40  attention_flash.cuh:177                 launch_flash_attn<bf16> with a 40-node ancestor mask: nodes at
//                                                   bit 32 and beyond are never attended
//   v2      tests/test_flash_v2.cu                  launch_flash_attn_v2<bf16> chunked prefill with a window
//   fp32    tests/test_decode_kernels.cu:24-35      launch_attn_decode (Sq > 1, base > 0) at HD 128/256/512
//   norm    tests/test_norm_fused.cu                launch_norm_rope_store<float / __half / __hip_bfloat16>: the
//                                                   norm alone at the gate's 1e-6 relative bar, a row's bits
//                                                   independent of the row count (S = 1..16), and K rows stored
//                                                   into a 16-bit cache slice within one unit in the last place
//
// Expected values come from the CPU oracle (oracle/liboracle.so), which is test infrastructure. Bars: the
// reference's fp32 bar (error / sum_j p_j |V_j,d| < 1e-5) for fp32 caches and fp32 launchers
// (max-abs <= 1e-2, mean-abs <= 1e-3) where MFMA operands are 16-bit. Prints one line per case and exits 1 on
// any failure.
#include "dgx_attn.hpp"
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <type_traits>
#include <vector>

extern "C" {
void oracle_gen_xorshift(uint64_t *state, float *out, size_t n);
void oracle_round_f16(const float *src, float *dst, uint16_t *bits, size_t n);
void oracle_round_bf16(const float *src, float *dst, uint16_t *bits, size_t n);
int oracle_attention(const float *q, const float *k, const float *v, const long *kv_off, const int *pos,
                     const uint32_t *anc, const int *tree_base, int T, int NQ, int NKV, int HD, float scale,
                     int window, int mode, double *out, double *lse, int nthreads);
int oracle_norm_rope(const float *x, const float *W, int rows, int hd, float eps, const float *cosT,
                     const float *sinT, const int *pos, int rope, double *out);
float oracle_f16_to_f32(uint16_t h);
float oracle_bf16_to_f32(uint16_t h);
}

static void ck(hipError_t e) { if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e)); }
static int g_fails = 0;

struct Layer { const char *name; int HD, NQ, NKV, window; };
static const Layer LAYERS[2] = {{"sliding", 256, 16, 8, 1024}, {"full", 512, 16, 1, 0}};

static std::vector<float> xs(uint64_t &st, size_t n, float mul = 1.f) {
    std::vector<float> v(n);
    oracle_gen_xorshift(&st, v.data(), n);
    if (mul != 1.f) for (auto &x : v) x *= mul;
    return v;
}
template <class T> static T *dev(const std::vector<T> &h) {
    T *p; ck(hipMalloc(&p, h.size() * sizeof(T) + 16));
    ck(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return p;
}
// Round host values to storage dtype dt in place and upload them in that dtype.
static void *dev_store(std::vector<float> &h, int dt) {
    if (dt == KV_FP32) return dev(h);
    std::vector<uint16_t> bits(h.size());
    if (dt == KV_F16) oracle_round_f16(h.data(), h.data(), bits.data(), h.size());
    else oracle_round_bf16(h.data(), h.data(), bits.data(), h.size());
    return dev(bits);
}
static std::vector<float> down(const float *d, size_t n) {
    std::vector<float> h(n);
    ck(hipMemcpy(h.data(), d, n * sizeof(float), hipMemcpyDeviceToHost));
    return h;
}
static uint32_t bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }

// Oracle rows: token t at position pos[t] over the cache at kv_off[t].
static std::vector<double> oracle(const std::vector<float> &q, const std::vector<float> &k, const std::vector<float> &v,
                                  const std::vector<long> &kv_off, const std::vector<int> &pos, int NQ, int NKV, int HD,
                                  float scale, int window, int mode, const uint32_t *anc = nullptr, int tree_base = 0) {
    const int T = (int)pos.size();
    std::vector<double> out((size_t)T * NQ * HD);
    std::vector<int> tb(T, tree_base);
    if (oracle_attention(q.data(), k.data(), v.data(), kv_off.data(), pos.data(), anc, anc ? tb.data() : nullptr, T,
                         NQ, NKV, HD, scale, window, mode, out.data(), nullptr, 0))
        throw std::runtime_error("oracle_attention: bad arguments");
    return out;
}

// Error of out against the oracle: max |e| / sum_j p_j |V_j,d| (the reference's fp32 gate) and plain max / mean.
struct Err { double norm = 0, max = 0, mean = 0; };
static Err compare(const std::vector<float> &o, const std::vector<double> &ref, const std::vector<float> &q,
                   const std::vector<float> &k, const std::vector<float> &v, const std::vector<long> &kv_off,
                   const std::vector<int> &pos, int NQ, int NKV, int HD, float scale, int window,
                   const uint32_t *anc = nullptr, int tree_base = 0) {
    Err e;
    // sum_j p_j |V_j,d|: the oracle over |V|.
    std::vector<float> va(v.size());
    for (size_t i = 0; i < v.size(); i++) va[i] = std::fabs(v[i]);
    const std::vector<double> den = oracle(q, k, va, kv_off, pos, NQ, NKV, HD, scale, window, 0, anc, tree_base);
    double sum = 0;
    for (size_t i = 0; i < o.size(); i++) {
        const double d = std::fabs((double)o[i] - ref[i]);
        if (!std::isfinite(o[i])) { e.norm = e.max = INFINITY; return e; }
        e.max = std::max(e.max, d); sum += d;
        if (den[i] > 0) e.norm = std::max(e.norm, d / den[i]);
    }
    e.mean = sum / (double)o.size();
    return e;
}
static void report(const char *gate, const char *what, bool ok, const Err &e) {
    printf("%s %s %s norm=%.3e max_abs=%.3e mean_abs=%.3e\n", gate, ok ? "PASS" : "FAIL", what, e.norm, e.max, e.mean);
    g_fails += !ok;
}

static std::vector<float> run_split(const Layer &L, const float *dq, const float *dk, const float *dv, int rows,
                                    int base, int pos_step, const int *dpos, int max_pos, long kv_stride, int max_len) {
    float *dout; ck(hipMalloc(&dout, (size_t)rows * L.NQ * L.HD * 4));
    attn_split_reserve(rows, L.NQ, max_len, L.HD);
    launch_attn_decode_split(dq, dk, dv, dout, rows, L.NQ, L.NKV, L.HD, base, pos_step, dpos, max_pos, kv_stride,
                             attn_split_ns_cap(max_len), 0, 1.0f, L.window);
    ck(hipDeviceSynchronize());
    std::vector<float> o = down(dout, (size_t)rows * L.NQ * L.HD);
    ck(hipFree(dout));
    return o;
}

static void gates_split() {
    const int dt = g4_kv_dtype();
    for (const Layer &L : LAYERS) {
        const int maxd = 32768;
        uint64_t st = 0x5eed1500ull + (uint64_t)L.HD;
        std::vector<float> k = xs(st, (size_t)maxd * L.NKV * L.HD), v = xs(st, k.size());
        std::vector<float> q = xs(st, (size_t)L.NQ * L.HD, 0.25f);
        float *dk = (float *)dev_store(k, dt), *dv = (float *)dev_store(v, dt), *dq = dev(q);
        for (int d : {1, 31, 32, 33, 1023, 1024, 1025, 2048, 8192, 32768}) {
            const int pos = d - 1;
            const std::vector<float> o = run_split(L, dq, dk, dv, 1, pos, 1, nullptr, pos, 0, d);
            const std::vector<double> ref = oracle(q, k, v, {0}, {pos}, L.NQ, L.NKV, L.HD, 1.0f, L.window, 0);
            const Err e = compare(o, ref, q, k, v, {0}, {pos}, L.NQ, L.NKV, L.HD, 1.0f, L.window);
            const bool ok = dt == KV_FP32 ? e.norm < 1e-5 : (e.max <= 1e-2 && e.mean <= 1e-3);
            char what[64]; snprintf(what, sizeof what, "%s d=%d", L.name, d);
            report("GATE1", what, ok, e);
        }
        int vfail = 0, vcases = 0;
        for (int base : {1000, 1017, 1023, 2040, 8190})
            for (int S = 2; S <= 16; S++) {
                std::vector<float> qs = xs(st, (size_t)S * L.NQ * L.HD, 0.25f);
                float *dqs = dev(qs);
                const int max_len = base + 16 + 1;
                const std::vector<float> multi = run_split(L, dqs, dk, dv, S, base, 1, nullptr, base + S - 1, 0, max_len);
                for (int r = 0; r < S; r++) {
                    const std::vector<float> single = run_split(L, dqs + (size_t)r * L.NQ * L.HD, dk, dv, 1, base + r, 1,
                                                                nullptr, base + r, 0, max_len);
                    for (size_t i = 0; i < single.size(); i++)
                        if (bits(single[i]) != bits(multi[(size_t)r * L.NQ * L.HD + i])) {
                            printf("GATE2 FAIL verify %s base=%d S=%d row=%d elem=%zu\n", L.name, base, S, r, i);
                            vfail++;
                            break;
                        }
                }
                vcases++;
                ck(hipFree(dqs));
            }
        printf("GATE2 %s verify %s: %d (base, S) cases\n", vfail ? "FAIL" : "PASS", L.name, vcases);
        g_fails += vfail;
        ck(hipFree(dk)); ck(hipFree(dv)); ck(hipFree(dq));

        const int cap = 4096; const long stride = (long)cap * L.NKV * L.HD;
        std::vector<float> bk = xs(st, (size_t)12 * stride), bv = xs(st, bk.size());
        float *dbk = (float *)dev_store(bk, dt), *dbv = (float *)dev_store(bv, dt);
        int bfail = 0;
        for (int W = 1; W <= 12; W++) {
            std::vector<int> pos(W); int mx = 0;
            for (int b = 0; b < W; b++) { pos[b] = (b * 977 + W * 131 + 63) % (cap - 1); mx = std::max(mx, pos[b]); }
            std::vector<float> qs = xs(st, (size_t)W * L.NQ * L.HD, 0.25f);
            float *dqs = dev(qs); int *dpos = dev(pos);
            const std::vector<float> multi = run_split(L, dqs, dbk, dbv, W, 0, 0, dpos, mx, stride, cap);
            for (int b = 0; b < W; b++) {
                const std::vector<float> single = run_split(L, dqs + (size_t)b * L.NQ * L.HD, kv_at(dbk, (size_t)b * stride),
                                                            kv_at(dbv, (size_t)b * stride), 1, pos[b], 1, nullptr, pos[b], 0, cap);
                for (size_t i = 0; i < single.size(); i++)
                    if (bits(single[i]) != bits(multi[(size_t)b * L.NQ * L.HD + i])) {
                        printf("GATE2 FAIL batch %s W=%d slot=%d pos=%d elem=%zu\n", L.name, W, b, pos[b], i);
                        bfail++;
                        break;
                    }
            }
            if (W == 12) {                                   // the whole batch against the oracle as well
                std::vector<long> off(W); for (int b = 0; b < W; b++) off[b] = (long)b * stride;
                const std::vector<double> ref = oracle(qs, bk, bv, off, pos, L.NQ, L.NKV, L.HD, 1.0f, L.window, 0);
                const Err e = compare(multi, ref, qs, bk, bv, off, pos, L.NQ, L.NKV, L.HD, 1.0f, L.window);
                const bool ok = dt == KV_FP32 ? e.norm < 1e-5 : (e.max <= 1e-2 && e.mean <= 1e-3);
                char what[64]; snprintf(what, sizeof what, "%s batch W=12 vs oracle", L.name);
                report("GATE2", what, ok, e);
            }
            ck(hipFree(dqs)); ck(hipFree(dpos));
        }
        printf("GATE2 %s batch %s\n", bfail ? "FAIL" : "PASS", L.name);
        g_fails += bfail;
        ck(hipFree(dbk)); ck(hipFree(dbv));
    }
}

// Tree verify of Sq nodes over a committed prefix through launch_flash_attn<bf16>; nodes >= 32 carry no bits.
static void gate_tree(int Sq, int base, uint64_t seed) {
    const int NQ = 24, NKV = 4, HD = 256, len = base + Sq;
    uint64_t st = seed;
    std::vector<float> k = xs(st, (size_t)len * NKV * HD), v = xs(st, k.size()), q = xs(st, (size_t)Sq * NQ * HD);
    std::vector<int> parent(Sq);
    std::vector<uint32_t> anc(Sq);
    for (int j = 0; j < Sq; j++) {
        parent[j] = j == 0 ? -1 : (int)((j * 2654435761u + seed) % (unsigned)j);
        uint32_t m = 0;
        for (int x = j; x >= 0; x = parent[x]) if (x < 32) m |= 1u << x;
        anc[j] = m;
    }
    std::vector<uint16_t> kb(k.size()), vb(v.size());
    oracle_round_bf16(k.data(), k.data(), kb.data(), k.size());
    oracle_round_bf16(v.data(), v.data(), vb.data(), v.size());
    __hip_bfloat16 *dk = (__hip_bfloat16 *)dev(kb), *dv = (__hip_bfloat16 *)dev(vb);
    float *dq = dev(q), *dout; unsigned *danc = dev(std::vector<unsigned>(anc.begin(), anc.end()));
    ck(hipMalloc(&dout, q.size() * 4));
    launch_flash_attn(dq, dk, dv, dout, Sq, NQ, NKV, HD, base, 0, danc);
    ck(hipDeviceSynchronize());
    const std::vector<float> o = down(dout, q.size());
    std::vector<int> pos(Sq); std::vector<long> off(Sq, 0);
    for (int j = 0; j < Sq; j++) pos[j] = base + j;
    const std::vector<double> ref = oracle(q, k, v, off, pos, NQ, NKV, HD, 0.f, 0, 0, anc.data(), base);
    const Err e = compare(o, ref, q, k, v, off, pos, NQ, NKV, HD, 0.f, 0, anc.data(), base);
    char what[64]; snprintf(what, sizeof what, "flash_attn<bf16> Sq=%d base=%d", Sq, base);
    report("TREE", what, e.max <= 1e-2 && e.mean <= 1e-3, e);
    ck(hipFree(dk)); ck(hipFree(dv)); ck(hipFree(dq)); ck(hipFree(dout)); ck(hipFree(danc));
}

// Chunked prefill of Sq tokens over a base-token prefix through launch_flash_attn_v2<bf16> (and the long-run
// branch of launch_flash_attn).
static void gate_v2(int Sq, int base, int window, bool via_flash) {
    const int NQ = 16, NKV = 8, HD = 256, len = base + Sq;
    uint64_t st = 909 + Sq + base;
    std::vector<float> k = xs(st, (size_t)len * NKV * HD), v = xs(st, k.size()), q = xs(st, (size_t)Sq * NQ * HD);
    std::vector<uint16_t> kb(k.size()), vb(v.size()), qb(q.size());
    oracle_round_bf16(k.data(), k.data(), kb.data(), k.size());
    oracle_round_bf16(v.data(), v.data(), vb.data(), v.size());
    oracle_round_bf16(q.data(), q.data(), qb.data(), q.size());   // operands are bf16 on the MFMA path
    __hip_bfloat16 *dk = (__hip_bfloat16 *)dev(kb), *dv = (__hip_bfloat16 *)dev(vb);
    float *dq = dev(q), *dout; ck(hipMalloc(&dout, q.size() * 4));
    if (via_flash) launch_flash_attn(dq, dk, dv, dout, Sq, NQ, NKV, HD, base, 0, nullptr, 0.f, window);
    else launch_flash_attn_v2(dq, dk, dv, dout, Sq, NQ, NKV, HD, base, 0, 0.f, window);
    ck(hipDeviceSynchronize());
    const std::vector<float> o = down(dout, q.size());
    std::vector<int> pos(Sq); std::vector<long> off(Sq, 0);
    for (int j = 0; j < Sq; j++) pos[j] = base + j;
    const std::vector<double> ref = oracle(q, k, v, off, pos, NQ, NKV, HD, 0.f, window, 0);
    const Err e = compare(o, ref, q, k, v, off, pos, NQ, NKV, HD, 0.f, window);
    char what[96];
    snprintf(what, sizeof what, "%s Sq=%d base=%d window=%d", via_flash ? "flash_attn<bf16>" : "flash_attn_v2<bf16>", Sq,
             base, window);
    report("PREFILL", what, e.max <= 1e-2 && e.mean <= 1e-3, e);
    ck(hipFree(dk)); ck(hipFree(dv)); ck(hipFree(dq)); ck(hipFree(dout));
}

// launch_attn_decode over an fp32 cache: Sq tokens at base .. base+Sq-1 (tests/test_decode_kernels.cu:24-35 form),
// against the fp32 host reference (oracle mode 1) at the reference's fp32 bar.
static void gate_fp32_decode(int HD, int Sq, int base) {
    const int NQ = 4, NKV = 2, len = base + Sq;
    uint64_t st = 2024 + HD;
    std::vector<float> q = xs(st, (size_t)Sq * NQ * HD, 0.2f), k = xs(st, (size_t)len * NKV * HD, 0.2f),
                       v = xs(st, (size_t)len * NKV * HD);
    float *dq = dev(q), *dk = dev(k), *dv = dev(v), *dout; ck(hipMalloc(&dout, q.size() * 4));
    launch_attn_decode(dq, dk, dv, dout, Sq, NQ, NKV, HD, base);
    ck(hipDeviceSynchronize());
    const std::vector<float> o = down(dout, q.size());
    std::vector<int> pos(Sq); std::vector<long> off(Sq, 0);
    for (int j = 0; j < Sq; j++) pos[j] = base + j;
    const std::vector<double> ref = oracle(q, k, v, off, pos, NQ, NKV, HD, 0.f, 0, 1);
    const Err e = compare(o, ref, q, k, v, off, pos, NQ, NKV, HD, 0.f, 0);
    char what[64]; snprintf(what, sizeof what, "attn_decode HD=%d Sq=%d base=%d", HD, Sq, base);
    report("FP32", what, e.norm < 1e-5 && e.max <= 1e-4, e);
    ck(hipFree(dq)); ck(hipFree(dk)); ck(hipFree(dv)); ck(hipFree(dout));
}

// RoPE tables [maxpos, hd] as the reference's gate builds them (tests/test_norm_fused.cu:90-95): angle
// p * 10000^(-2i/hd) in fp32, cos / sin written to entries i and hd/2 + i.
static void rope_tables(int maxpos, int hd, std::vector<float> &c, std::vector<float> &s) {
    c.assign((size_t)maxpos * hd, 0.f); s.assign((size_t)maxpos * hd, 0.f);
    for (int p = 0; p < maxpos; p++)
        for (int i = 0; i < hd / 2; i++) {
            const float a = (float)p * powf(10000.f, -2.f * (float)i / (float)hd);
            c[(size_t)p * hd + i] = c[(size_t)p * hd + hd / 2 + i] = cosf(a);
            s[(size_t)p * hd + i] = s[(size_t)p * hd + hd / 2 + i] = sinf(a);
        }
}

// launch_norm_rope_store gates (tests/test_norm_fused.cu): q rows of S tokens at base .. base+S-1 into scratch
// (slot stride NQ*hd, row stride 0), k rows of the same tokens into a 16-bit cache slice (slot stride 0, row
// stride NKV*hd), the norm alone into fp32.
template <class TO> static bool store_k16(int hd, int NKV, int S, int base, int L, const float *dx, const float *dw,
                                          const float *dc, const float *ds, const std::vector<double> &ref) {
    const size_t n = (size_t)L * NKV * hd;
    std::vector<uint16_t> init(n, 0x7fffu);                           // sentinel: a NaN pattern in both formats
    uint16_t *dcache = dev(init);
    launch_norm_rope_store<TO>(dx, dw, reinterpret_cast<TO *>(dcache), S * NKV, NKV, hd, 1e-6f, dc, ds, base, 1,
                               nullptr, 0, (long)NKV * hd, true);
    ck(hipDeviceSynchronize());
    std::vector<uint16_t> h(n);
    ck(hipMemcpy(h.data(), dcache, n * 2, hipMemcpyDeviceToHost));
    ck(hipFree(dcache));
    const bool f16 = std::is_same<TO, __half>::value;
    const double ulp = f16 ? 1.0 / 1024 : 1.0 / 128, tiny = f16 ? 6.103515625e-05 : 1.1754943508222875e-38;
    bool ok = true;
    for (size_t i = 0; i < n; i++) {
        const size_t row = i / ((size_t)NKV * hd);
        if (row < (size_t)base || row >= (size_t)(base + S)) { ok &= h[i] == 0x7fffu; continue; }
        const double r = ref[i - (size_t)base * NKV * hd];
        const double v = f16 ? oracle_f16_to_f32(h[i]) : oracle_bf16_to_f32(h[i]);
        ok &= std::fabs(v - r) <= ulp * std::max(std::fabs(r), tiny) + 1e-6;
    }
    return ok;
}

static void gate_norm(int hd) {
    const int NQ = 16, NKV = hd >= 512 ? 1 : 8, S = 16, base = 4100, L = 4200;
    const float eps = 1e-6f;
    uint64_t st = 4242 + hd;
    std::vector<float> x = xs(st, (size_t)S * NQ * hd, 2.f), w = xs(st, hd), c, s;
    rope_tables(L, hd, c, s);
    float *dx = dev(x), *dw = dev(w), *dc = dev(c), *ds = dev(s), *dy;
    ck(hipMalloc(&dy, x.size() * 4));
    char what[96];
    // 1. the norm alone (fp32), relative error < 1e-6 where |ref| >= 1e-3 (tests/test_norm_fused.cu:32-56)
    launch_norm_rope_store<float>(dx, dw, dy, S * NQ, NQ, hd, eps, nullptr, nullptr, 0, 0, nullptr, (long)NQ * hd, 0,
                                  false);
    ck(hipDeviceSynchronize());
    std::vector<float> y = down(dy, x.size());
    std::vector<double> ref(x.size());
    oracle_norm_rope(x.data(), w.data(), S * NQ, hd, eps, nullptr, nullptr, nullptr, 0, ref.data());
    double worst = 0;
    for (size_t i = 0; i < y.size(); i++)
        if (std::fabs(ref[i]) >= 1e-3) worst = std::max(worst, std::fabs(y[i] - ref[i]) / std::fabs(ref[i]));
    Err e; e.max = worst;
    snprintf(what, sizeof what, "norm alone hd=%d rel < 1e-6", hd);
    report("NORM", what, worst < 1e-6, e);
    // 2. q rows with RoPE for S = 1..16 tokens ending at the same token: that token's rows bit-identical in every
    //    launch, and the full launch against the oracle
    std::vector<int> pos(S * NQ);
    for (int r = 0; r < S * NQ; r++) pos[r] = base + r / NQ;
    std::vector<double> qref(x.size());
    oracle_norm_rope(x.data(), w.data(), S * NQ, hd, eps, c.data(), s.data(), pos.data(), 1, qref.data());
    std::vector<uint32_t> last;
    bool ident = true;
    double qmax = 0;
    for (int n = 1; n <= S; n++) {
        const int s0 = S - n;
        launch_norm_rope_store<float>(dx + (size_t)s0 * NQ * hd, dw, dy, n * NQ, NQ, hd, eps, dc, ds, base + s0, 1,
                                      nullptr, (long)NQ * hd, 0, true);
        ck(hipDeviceSynchronize());
        const std::vector<float> o = down(dy, (size_t)n * NQ * hd);
        std::vector<uint32_t> b(NQ * hd);
        for (int i = 0; i < NQ * hd; i++) b[i] = bits(o[(size_t)(n - 1) * NQ * hd + i]);
        if (n == 1) last = b; else ident &= b == last;
        if (n == S) {
            double scale = 0;
            for (double v : qref) scale = std::max(scale, std::fabs(v));
            for (size_t i = 0; i < o.size(); i++) qmax = std::max(qmax, std::fabs(o[i] - qref[i]) / scale);
        }
    }
    e.max = qmax;
    snprintf(what, sizeof what, "q norm+RoPE hd=%d S=1..16 row identity, normalised err < 1e-5", hd);
    report("NORM", what, ident && qmax < 1e-5, e);
    // 3. k rows (NKV heads) into f16 and bf16 cache slices at rows base .. base+S-1, nothing else written
    std::vector<int> kpos(S * NKV);
    for (int r = 0; r < S * NKV; r++) kpos[r] = base + r / NKV;
    std::vector<double> kref((size_t)S * NKV * hd);
    oracle_norm_rope(x.data(), w.data(), S * NKV, hd, eps, c.data(), s.data(), kpos.data(), 1, kref.data());
    const bool k16 = store_k16<__half>(hd, NKV, S, base, L, dx, dw, dc, ds, kref);
    const bool kb16 = store_k16<__hip_bfloat16>(hd, NKV, S, base, L, dx, dw, dc, ds, kref);
    e.max = 0;
    snprintf(what, sizeof what, "k norm+RoPE+store hd=%d f16 / bf16 within 1 ulp, other rows untouched", hd);
    report("NORM", what, k16 && kb16, e);
    ck(hipFree(dx)); ck(hipFree(dw)); ck(hipFree(dc)); ck(hipFree(ds)); ck(hipFree(dy));
}

int main(int argc, char **argv) try {
    setvbuf(stdout, nullptr, _IOLBF, 0);
    const char *only = argc > 1 ? argv[1] : "all";
    const bool all = !strcmp(only, "all");
    printf("REF_GATES %s chunk=%d kv_dtype=%d\n", dgx_attn_version(), attn_split_chunk(), g4_kv_dtype());
    if (all || !strcmp(only, "split")) gates_split();
    if (all || !strcmp(only, "tree")) {
        gate_tree(40, 3000, 77);
        gate_tree(8, 2048, 78);
        gate_tree(33, 517, 79);
    }
    if (all || !strcmp(only, "prefill")) {
        gate_v2(300, 200, 0, false);
        gate_v2(512, 1500, 1024, false);
        gate_v2(100, 0, 0, true);
    }
    if (all || !strcmp(only, "fp32")) {
        for (int hd : {128, 256, 512}) gate_fp32_decode(hd, 6, 37);
        reserve_flash_attn_scratch(4096, 512);          // the fp32 MFMA kernel once its partials are reserved
        for (int hd : {128, 256}) gate_fp32_decode(hd, 6, 1200);
    }
    if (all || !strcmp(only, "norm"))
        for (int hd : {128, 256, 512}) gate_norm(hd);
    printf("[ref_gates] %s\n", g_fails ? "FAIL" : "PASS");
    return g_fails ? 1 : 0;
} catch (const std::exception &e) {
    fprintf(stderr, "[ref_gates] FAIL: %s\n", e.what());
    return 1;
}

// extern "C" layer of the MI355X attention library: knobs, per-device scratch and the entry points declared in
// include/dgx_attn.h. Host code only; every call returns a hipError_t and never aborts or exits.
#include "attn_device.h"
#include "attn_internal.h"
#include "../../include/dgx_attn.h"
#include <climits>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unistd.h>
#include <fstream>
#include <map>
#include <mutex>
#include <string>
#include <vector>
#include <algorithm>

using namespace dgx;

namespace {

// ---------------------------------------------------------------- knobs
// The attention subsystem's slice of the reference registry (runtime/knobs.h:49-69, 130-131): these names, their
// value sets and the resolution order env > DGX_KNOBS_FILE recipe > default (runtime/knobs.h:9-13, 297-303). The
// recipe format and checks follow runtime/knobs.h:241-275: '#' comments, NAME=VALUE lines, a line without '=' or
// with an empty name is an error, a name under this subsystem's prefixes (G4_ATTN_, G4_KV_, G4_FLASH_) that is not
// registered is an error, and every set value (env or recipe) must be in its set; an unregistered environment
// name under those prefixes only warns (runtime/knobs.h:273-283). Names under other prefixes belong to other
// subsystems and are skipped. Where the reference exits with status 2, the C ABI reports the
// first error once on stderr and the knob queries return -1 (dgx_knobs_status; the C++ wrapper exits 2).
struct KnobDef { const char *name, *allowed; bool int_min1; };
const KnobDef kKnobs[] = {
    {"G4_ATTN_SPLIT", "0|1", false},          {"G4_ATTN_CHUNK", "32|64|128|256", false},
    {"G4_KV_DTYPE", "fp32|f16|bf16", false},  {"G4_FLASH_PREFILL", "0|1", false},
    {"G4_FLASH_MIN_S", "1..", true},          {"G4_FLASH_V2", "0|1", false},
    {"G4_FLASH_F16_MMA", "0|1", false},       {"G4_KV_STATS", "0|1", false},
    {"G4_ATTN_DIAG_REVERSE", "0|1", false},
};
const char *const kKnobPrefixes[] = {"G4_ATTN_", "G4_KV_", "G4_FLASH_"};

const KnobDef *knob_find(const std::string &n) {
    for (const KnobDef &k : kKnobs) if (n == k.name) return &k;
    return nullptr;
}
bool knob_valid(const KnobDef &k, const char *v) {
    if (k.int_min1) {
        char *end = nullptr;
        errno = 0;
        const long x = strtol(v, &end, 10);
        return errno == 0 && end != v && *end == '\0' && x >= 1;
    }
    const std::string set = std::string("|") + k.allowed + "|", item = std::string("|") + v + "|";
    return *v && set.find(item) != std::string::npos;
}

// Levenshtein distance (insert, delete, substitute: cost 1 each), two rolling rows.
size_t edit_distance(const std::string &a, const std::string &b) {
    std::vector<size_t> prev(b.size() + 1), cur(b.size() + 1);
    for (size_t j = 0; j <= b.size(); j++) prev[j] = j;
    for (size_t i = 1; i <= a.size(); i++) {
        cur[0] = i;
        for (size_t j = 1; j <= b.size(); j++)
            cur[j] = std::min({prev[j] + 1, cur[j - 1] + 1, prev[j - 1] + (a[i - 1] == b[j - 1] ? 0 : 1)});
        std::swap(prev, cur);
    }
    return prev[b.size()];
}

struct KnobState {
    bool ok = true;
    std::string err;
    std::map<std::string, std::string> recipe;
};
KnobState knob_load() {
    KnobState s;
    auto fail = [&](const std::string &m) { if (s.ok) { s.ok = false; s.err = m; } };
    if (const char *path = getenv("DGX_KNOBS_FILE")) {
        std::ifstream in(path);
        if (!in) fail(std::string("cannot read DGX_KNOBS_FILE=") + path);
        std::string line;
        int n = 0;
        auto trim = [](const std::string &t) {
            const size_t a = t.find_first_not_of(" \t\r"), b = t.find_last_not_of(" \t\r");
            return a == std::string::npos ? std::string() : t.substr(a, b - a + 1);
        };
        while (in && std::getline(in, line)) {
            n++;
            const size_t h = line.find('#');
            if (h != std::string::npos) line.resize(h);
            line = trim(line);
            if (line.empty()) continue;
            const size_t eq = line.find('=');
            if (eq == std::string::npos || eq == 0) { fail(std::string(path) + ":" + std::to_string(n) + ": expected NAME=VALUE"); continue; }
            const std::string key = trim(line.substr(0, eq)), val = trim(line.substr(eq + 1));
            bool ours = false;
            for (const char *pre : kKnobPrefixes) if (key.compare(0, strlen(pre), pre) == 0) ours = true;
            if (ours && !knob_find(key)) { fail(std::string(path) + ": unknown knob " + key); continue; }
            s.recipe[key] = val;
        }
    }
    // Environment names under this subsystem's prefixes that are not registered only warn (a likely typo: the
    // closest registered name within 3 edits is suggested), as in the reference.
    for (char **e = environ; e && *e; e++) {
        const char *eqp = strchr(*e, '=');
        if (!eqp) continue;
        const std::string name(*e, eqp - *e);
        bool ours = false;
        for (const char *pre : kKnobPrefixes) if (name.compare(0, strlen(pre), pre) == 0) ours = true;
        if (!ours || knob_find(name)) continue;
        const KnobDef *best = nullptr;
        size_t bd = 4;
        for (const KnobDef &k : kKnobs) {
            const size_t d = edit_distance(name, k.name);
            if (d < bd) { bd = d; best = &k; }
        }
        if (best) fprintf(stderr, "knobs: warning: unknown knob env %s (did you mean %s?)\n", name.c_str(), best->name);
        else fprintf(stderr, "knobs: warning: unknown knob env %s\n", name.c_str());
    }
    for (const KnobDef &k : kKnobs) {
        const char *v = getenv(k.name), *src = "env";
        auto it = s.recipe.find(k.name);
        if (!v && it != s.recipe.end()) { v = it->second.c_str(); src = "recipe"; }
        if (v && !knob_valid(k, v))
            fail(std::string("invalid ") + k.name + "=" + v + " (" + src + "); allowed: " + k.allowed);
    }
    if (!s.ok) fprintf(stderr, "knobs: %s\n", s.err.c_str());
    return s;
}
const KnobState &knob_state() {
    static const KnobState s = knob_load();
    return s;
}

// Value of a registered knob as set by env or the recipe file, nullptr when unset or when the knob configuration
// is invalid (callers then fail; see dgx_knobs_status).
const char *knob_raw(const char *name) {
    const KnobState &s = knob_state();
    if (!s.ok) return nullptr;
    if (const char *v = getenv(name)) return v;
    auto it = s.recipe.find(name);
    return it == s.recipe.end() ? nullptr : it->second.c_str();
}

int g_kv_override = -1;

int parse_kv_dtype() {
    if (!knob_state().ok) return -1;
    const char *v = knob_raw("G4_KV_DTYPE");
    if (!v || !*v) {
        const char *split = knob_raw("G4_ATTN_SPLIT");
        return (split && !strcmp(split, "0")) ? DT_FP32 : DT_F16;
    }
    if (!strcmp(v, "fp32")) return DT_FP32;
    if (!strcmp(v, "f16")) return DT_F16;
    if (!strcmp(v, "bf16")) return DT_BF16;
    fprintf(stderr, "Invalid G4_KV_DTYPE=%s (fp32, f16 or bf16)\n", v);
    return -1;
}

int parse_chunk() {
    if (!knob_state().ok) return -1;
    int c = 256;                                  // MI355X default (the GB10 reference defaults to 64)
    if (const char *v = knob_raw("G4_ATTN_CHUNK")) {
        c = atoi(v);
        if (c != 32 && c != 64 && c != 128 && c != 256) {             // the reference's value set
            fprintf(stderr, "Invalid G4_ATTN_CHUNK=%s (32, 64, 128 or 256)\n", v);
            return -1;
        }
    }
    return c;
}

bool knob_on(const char *name) { const char *v = knob_raw(name); return v && v[0] == '1'; }

// ---------------------------------------------------------------- scratch pools (per device, grow only)
constexpr int kMaxDev = 64;
struct Pool {
    float *m = nullptr, *l = nullptr, *acc = nullptr;
    size_t cap = 0, acc_cap = 0;
};
Pool g_split[kMaxDev], g_flash[kMaxDev];
std::mutex g_pool_mu;

hipError_t pool_grow(Pool &p, size_t need, size_t hd) {
    if (hd && need > (SIZE_MAX / sizeof(float)) / hd) return hipErrorInvalidValue;
    if (p.cap < need) {
        if (p.m) { hipError_t e = hipFree(p.m); if (e != hipSuccess) return e; p.m = nullptr; }
        if (p.l) { hipError_t e = hipFree(p.l); if (e != hipSuccess) return e; p.l = nullptr; }
        p.cap = 0;
        hipError_t e = hipMalloc(&p.m, need * sizeof(float)); if (e != hipSuccess) return e;
        e = hipMalloc(&p.l, need * sizeof(float)); if (e != hipSuccess) return e;
        p.cap = need;
    }
    if (p.acc_cap < need * hd) {
        if (p.acc) { hipError_t e = hipFree(p.acc); if (e != hipSuccess) return e; p.acc = nullptr; }
        p.acc_cap = 0;
        hipError_t e = hipMalloc(&p.acc, need * hd * sizeof(float)); if (e != hipSuccess) return e;
        p.acc_cap = need * hd;
    }
    return hipSuccess;
}

hipError_t pool_for(Pool *pools, Pool *&out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDev) return hipErrorInvalidDevice;
    out = &pools[dev];
    return hipSuccess;
}

// ---------------------------------------------------------------- fixed scratch (allocation-free entry point)
// dgx_attn_batch_noalloc keeps its split partials in this file-scope device array instead of a pool. Every GPU the
// library runs on holds its own copy (kScratchBytes) until the process ends. Host code never passes the array's
// name to a kernel: it is a host-side stand-in there. The device address comes from hipGetSymbolAddress, once per
// device with that device current, and is kept in g_scratch_dev.
constexpr size_t kScratchBytes = 64ull << 20;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
float *g_scratch_dev[kMaxDev];
std::mutex g_scratch_mu;

hipError_t scratch_ptr(float *&out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDev) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!ptr) return hipErrorInvalidSymbol;
        g_scratch_dev[dev] = static_cast<float *>(ptr);
    }
    out = g_scratch_dev[dev];
    return hipSuccess;
}

// A ring-buffer cache of kv_cap rows holds the sliding window of every row of a launch: the keys a launch reads
// span at most window + T - 1 positions, and whole 64-key steps map to consecutive rows.
bool ring_ok(int kv_cap, int window, int T) {
    if (kv_cap == 0) return true;
    return kv_cap > 0 && kv_cap % 64 == 0 && window > 0 && (long)window + T - 1 <= kv_cap;
}

float resolve_scale(float scale, int HD) { return scale > 0.f ? scale : 1.0f / sqrtf((float)HD); }

bool valid_hd(int HD) { return HD == 128 || HD == 256 || HD == 512; }
bool valid_dtype(int d) { return d == DT_FP32 || d == DT_F16 || d == DT_BF16; }

// Flash-path split size for short query runs (the reference's FD_SPLIT_KV, attention_flash.cuh:11).
constexpr int kFlashChunk = 512;
// Query tokens up to which dgx_flash_attn runs the split kernel (decode, verify, trees of <= 32 nodes).
constexpr int kFlashShortSq = 32;

Problem make_problem(const void *Q, int qt, const void *K, const void *V, int kvt, void *O, int ot, float *lse,
                     int nseq, int T, int NQ, int NKV, int HD, long kv_stride, int pos_mode, int base, int pos_step,
                     const int *pos_arr, const unsigned *anc, int max_pos, float scale, int window) {
    Problem p;
    p.Q = Q; p.q_dtype = qt; p.K = K; p.V = V; p.kv_dtype = kvt; p.O = O; p.o_dtype = ot; p.lse = lse;
    p.nseq = nseq; p.T = T; p.NQ = NQ; p.NKV = NKV; p.HD = HD; p.kv_stride = kv_stride;
    p.pos_mode = pos_mode; p.base = base; p.pos_step = pos_step; p.pos_arr = pos_arr;
    p.anc = reinterpret_cast<const uint32_t *>(anc); p.max_pos = max_pos;
    p.scale = resolve_scale(scale, HD); p.window = window < 0 ? 0 : window;
    p.Kp = nullptr; p.Vp = nullptr; p.gate = nullptr; p.gate_dtype = DT_FP32; p.kv_cap = 0;
    return p;
}

// ---------------------------------------------------------------- kernel timing (measurement hook)
// With timing on, the main kernel of every split/decode and prefill launch is bracketed by a HIP event pair on
// its launch stream (up to kTimed launches between reads).
constexpr int kTimed = 4096;
struct Timing {
    bool on = false;
    int n = 0;
    hipEvent_t a[kTimed], b[kTimed];
    bool made = false;
};
Timing g_timing;
std::mutex g_timing_mu;
std::atomic<bool> g_timing_on{false};

template <class F>
hipError_t timed_launch(hipStream_t st, F &&launch) {
    int slot = -1;
    if (g_timing_on.load(std::memory_order_acquire)) {            // atomic flag; the slots under the mutex
        std::lock_guard<std::mutex> lk(g_timing_mu);
        if (g_timing.on && g_timing.n < kTimed) slot = g_timing.n++;
    }
    if (slot >= 0) { hipError_t e = hipEventRecord(g_timing.a[slot], st); if (e != hipSuccess) return e; }
    hipError_t e = launch();
    if (slot >= 0 && e == hipSuccess) e = hipEventRecord(g_timing.b[slot], st);
    return e;
}

// How verify_kernel cuts its runs (dgx_attn_verify_runs): 0 = each sequence's absolute key chunks, 1 = equal runs
// over the whole batch.
std::atomic<int> g_verify_runs{0};

hipError_t run_split(const Problem &p, int chunk, Pool &pool, int ns_cap, hipStream_t st) {
    Partials part{pool.m, pool.l, pool.acc, ns_cap};
    const bool slot_runs = g_verify_runs.load(std::memory_order_relaxed) == 0;
    hipError_t e = timed_launch(st, [&] { return launch_split(p, chunk, part, st, slot_runs); });
    if (e != hipSuccess) return e;
    return launch_combine(p, chunk, part, st);
}

// fp32 caches, up to 16 rows per KV head, no reverse-order diagnostic: the fp32 MFMA streaming kernel + combine on
// the given pool. Never allocates: the caller checks f32_reserved first (the reference's fp32 launchers use only
// shared memory, attention.cuh:137-198, so these calls must stay capture-safe and allocation-free).
constexpr int kF32Chunk = 512;
bool f32_fast(const Problem &p) { return decode_f32_supported(p) && !knob_on("G4_ATTN_DIAG_REVERSE"); }
size_t f32_need(const Problem &p) { return (size_t)p.nseq * p.T * p.NQ * (size_t)(p.max_pos / kF32Chunk + 1); }
bool f32_reserved(const Problem &p, const Pool &pool) {
    const size_t need = f32_need(p);
    return need <= pool.cap && need * (size_t)p.HD <= pool.acc_cap;
}
hipError_t run_f32(const Problem &p, const Pool &pool, hipStream_t st) {
    Partials part{pool.m, pool.l, pool.acc, p.max_pos / kF32Chunk + 1};
    hipError_t e = timed_launch(st, [&] { return launch_decode_f32(p, kF32Chunk, part, st); });
    if (e != hipSuccess) return e;
    return launch_combine(p, kF32Chunk, part, st);
}
// The fp32 drop-in launchers take the MFMA kernel when the flash pool already holds its partials (reserved with
// dgx_flash_attn_reserve_partials or grown by an earlier flash call), else the scalar kernels.
bool f32_take_fast(const Problem &p, const Pool *&pool) {
    if (!f32_fast(p)) return false;
    Pool *pl; if (pool_for(g_flash, pl) != hipSuccess) return false;
    pool = pl;
    return f32_reserved(p, *pl);
}

}  // namespace

extern "C" {

int dgx_knobs_status(void) { return knob_state().ok ? 0 : -1; }

int dgx_attn_verify_runs(int mode) {
    if (mode == 0 || mode == 1) return g_verify_runs.exchange(mode);
    return mode == -1 ? g_verify_runs.load() : -1;
}

size_t dgx_flash_attn_hd512_lds(void) {
    const size_t a = split_lds_bytes(512), b = prefill_lds_bytes(512);
    return a > b ? a : b;
}
int dgx_kv_stats_enabled(void) { return knob_on("G4_KV_STATS") ? 1 : 0; }
int dgx_kv_dtype(void) {
    if (g_kv_override >= 0) return g_kv_override;
    static const int dt = parse_kv_dtype();
    return dt;
}
void dgx_kv_force_fp32(const char *why) {
    if (g_kv_override == DT_FP32) return;
    const char *v = knob_raw("G4_KV_DTYPE");
    if (v && strcmp(v, "fp32")) fprintf(stderr, "G4_KV_DTYPE ignored (%s): fp32 KV\n", why ? why : "");
    g_kv_override = DT_FP32;
}
size_t dgx_kv_elem(void) { return dgx_kv_dtype() == DT_FP32 ? 4 : 2; }

int dgx_attn_split_chunk(void) {
    static const int c = parse_chunk();
    return c;
}
int dgx_attn_split_ns_cap(int max_len) {
    const int C = dgx_attn_split_chunk();
    if (C <= 0 || max_len < 0) return -1;
    return (max_len + C - 1) / C;
}

hipError_t dgx_attn_split_reserve(int rows, int NQ, int max_len, int hd_max) {
    if (rows < 0 || NQ <= 0 || max_len < 0 || hd_max <= 0) return hipErrorInvalidValue;
    const int ns = dgx_attn_split_ns_cap(max_len);
    if (ns < 0) return hipErrorInvalidValue;
    Pool *pool; hipError_t e = pool_for(g_split, pool); if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_pool_mu);
    return pool_grow(*pool, (size_t)rows * NQ * ns, (size_t)hd_max);
}

hipError_t dgx_attn_decode_split(const float *Q, const void *Kc, const void *Vc, int kv_dtype, float *O, float *lse,
                                 int rows, int NQ, int NKV, int HD, int base, int pos_step, const int *pos_arr,
                                 int max_pos, long kv_stride, int ns_cap, hipStream_t st, float scale, int window) {
    if (rows == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || rows < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) || max_pos < 0 ||
        !valid_dtype(kv_dtype))
        return hipErrorInvalidValue;
    const int C = dgx_attn_split_chunk();
    if (C <= 0) return hipErrorInvalidValue;
    Pool *pool; hipError_t e = pool_for(g_split, pool); if (e != hipSuccess) return e;
    if (max_pos / C + 1 > ns_cap || (size_t)rows * NQ * ns_cap > pool->cap || (size_t)rows * NQ * ns_cap * HD > pool->acc_cap) {
        fprintf(stderr, "[attn_split] scratch not reserved: rows=%d NQ=%d ns_cap=%d max_pos=%d\n", rows, NQ, ns_cap, max_pos);
        return hipErrorInvalidValue;
    }
    if (kv_dtype == DT_FP32) {
        const Problem pf = make_problem(Q, DT_FP32, Kc, Vc, DT_FP32, O, DT_FP32, lse, rows, 1, NQ, NKV, HD, kv_stride, 0,
                                        base, pos_step, pos_arr, nullptr, max_pos, scale, window);
        // (the reservation, made for the library chunk <= 512, always covers the streaming kernel's 512-key chunks)
        if (f32_fast(pf) && f32_reserved(pf, *pool)) return run_f32(pf, *pool, st);
        if (lse) return hipErrorInvalidValue;   // the fp32 path keeps the reference's outputs (O only)
        return launch_scalar_rows(Q, (const float *)Kc, (const float *)Vc, O, rows, NQ, NKV, HD, base, pos_step, pos_arr,
                                  kv_stride, resolve_scale(scale, HD), window, knob_on("G4_ATTN_DIAG_REVERSE") ? 1 : 0, st);
    }
    // Every row is its own one-token problem (KV at r * kv_stride; kv_stride = 0 re-reads one cache, mostly from
    // L2), so a verify row runs exactly the arithmetic of the same position launched alone.
    const Problem p = make_problem(Q, DT_FP32, Kc, Vc, kv_dtype, O, DT_FP32, lse, rows, 1, NQ, NKV, HD, kv_stride, 0,
                                   base, pos_step, pos_arr, nullptr, max_pos, scale, window);
    return run_split(p, C, *pool, ns_cap, st);
}

hipError_t dgx_flash_attn_reserve(int Sq, int NQ, int base, int HD) {
    if (Sq < 0 || NQ <= 0 || base < 0 || !valid_hd(HD)) return hipErrorInvalidValue;
    // Long query runs use the prefill kernel without key splits and need no scratch.
    if (Sq > kFlashShortSq) return hipSuccess;
    Pool *pool; hipError_t e = pool_for(g_flash, pool); if (e != hipSuccess) return e;
    const size_t ns = (size_t)(base + Sq) / kFlashChunk + 1;
    std::lock_guard<std::mutex> lock(g_pool_mu);
    return pool_grow(*pool, (size_t)Sq * NQ * ns, (size_t)HD);
}

hipError_t dgx_flash_attn_reserve_partials(size_t partials, int hd_max) {
    if (hd_max <= 0 || hd_max > 512) return hipErrorInvalidValue;
    Pool *pool; hipError_t e = pool_for(g_flash, pool); if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_pool_mu);
    return pool_grow(*pool, partials, (size_t)hd_max);
}

hipError_t dgx_flash_attn(const float *Q, const void *Kc, const void *Vc, int kv_dtype, float *O, float *lse,
                          int Sq, int NQ, int NKV, int HD, int base, hipStream_t st, const unsigned *anc,
                          float scale, int window) {
    if (Sq == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || Sq < 0 || base < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) ||
        !valid_dtype(kv_dtype))
        return hipErrorInvalidValue;
    // The reference's flash path takes a caller scale of exactly 0 as "default" and any other value as given.
    const float sc = scale == 0.f ? 1.0f / sqrtf((float)HD) : scale;
    hipError_t e = dgx_flash_attn_reserve(Sq, NQ, base, HD);
    if (e != hipSuccess) return e;
    Pool *pool; e = pool_for(g_flash, pool); if (e != hipSuccess) return e;
    Problem p = make_problem(Q, DT_FP32, Kc, Vc, kv_dtype, O, DT_FP32, lse, 1, Sq, NQ, NKV, HD, 0, 1, base, 1, nullptr,
                             anc, base + Sq - 1, 1.f, window);
    p.scale = sc;
    if (Sq <= kFlashShortSq || anc) {
        // Short runs and every tree-masked run take the split kernel. A tree run longer than 32 tokens keeps the
        // reference's rule: nodes at bit 32 and beyond are never attended (attention_flash.cuh:177), and its
        // partials grow the pool here as the reference's flash launch does.
        const int ns = (base + Sq - 1) / kFlashChunk + 1;
        if (Sq > kFlashShortSq) {
            std::lock_guard<std::mutex> lock(g_pool_mu);
            e = pool_grow(*pool, (size_t)Sq * NQ * ns, (size_t)HD);
            if (e != hipSuccess) return e;
        }
        return run_split(p, kFlashChunk, *pool, ns, st);
    }
    // No key split: the prefill kernel balances causal work by pairing query tiles, and a row's result does not
    // depend on how the prompt is chunked.
    return timed_launch(st, [&] { return launch_prefill(p, 0, Partials{nullptr, nullptr, nullptr, 0}, st); });
}

hipError_t dgx_flash_attn_v2(const float *Q, const void *Kc, const void *Vc, int kv_dtype, float *O, float *lse,
                             int Sq, int NQ, int NKV, int HD, int base, hipStream_t st, float scale, int window,
                             int f16_mma) {
    (void)f16_mma;
    if (Sq == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || Sq < 0 || base < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) ||
        !valid_dtype(kv_dtype))
        return hipErrorInvalidValue;
    const Problem p = make_problem(Q, DT_FP32, Kc, Vc, kv_dtype, O, DT_FP32, lse, 1, Sq, NQ, NKV, HD, 0, 1, base, 1,
                                   nullptr, nullptr, base + Sq - 1, scale, window);
    return timed_launch(st, [&] { return launch_prefill(p, 0, Partials{nullptr, nullptr, nullptr, 0}, st); });
}

hipError_t dgx_attn(const float *Q, const float *K, const float *V, float *O, int S, int NQ, int NKV, int HD,
                    hipStream_t st, float scale, int window) {
    if (S == 0) return hipSuccess;
    if (!Q || !K || !V || !O || S < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || HD <= 0 || HD > 512) return hipErrorInvalidValue;
    if (valid_hd(HD)) {                                   // short prompts: query i attends keys 0..i
        const Problem p = make_problem(Q, DT_FP32, K, V, DT_FP32, O, DT_FP32, nullptr, 1, S, NQ, NKV, HD, 0, 1, 0, 1,
                                       nullptr, nullptr, S - 1, scale, window);
        const Pool *pool = nullptr;
        if (f32_take_fast(p, pool)) return run_f32(p, *pool, st);
    }
    return launch_scalar_prefill(Q, K, V, O, S, NQ, NKV, HD, resolve_scale(scale, HD), window < 0 ? 0 : window, st);
}

hipError_t dgx_attn_decode(const float *Q, const float *Kc, const float *Vc, float *O, int Sq, int NQ, int NKV, int HD,
                           int base, hipStream_t st, float scale, int window) {
    if (Sq == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || Sq < 0 || base < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || HD <= 0 || HD > 512)
        return hipErrorInvalidValue;
    if (valid_hd(HD)) {
        const Problem p = make_problem(Q, DT_FP32, Kc, Vc, DT_FP32, O, DT_FP32, nullptr, 1, Sq, NQ, NKV, HD, 0, 1,
                                       base, 1, nullptr, nullptr, base + Sq - 1, scale, window);
        const Pool *pool = nullptr;
        if (f32_take_fast(p, pool)) return run_f32(p, *pool, st);
    }
    return launch_scalar_decode(Q, Kc, Vc, O, 1, Sq, NQ, NKV, HD, base, 0, nullptr, resolve_scale(scale, HD),
                                window < 0 ? 0 : window, knob_on("G4_ATTN_DIAG_REVERSE") ? 1 : 0, st);
}

hipError_t dgx_attn_decode_batch(const float *Q, const float *Kc, const float *Vc, float *O, int B, int NQ, int NKV,
                                 int HD, int base, long kv_stride, hipStream_t st, float scale, int window,
                                 const int *base_b) {
    if (B == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || B < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || HD <= 0 || HD > 512)
        return hipErrorInvalidValue;
    // The streaming kernel needs a host bound of the positions: `base` without base_b, else the cache capacity
    // kv_stride / (NKV*HD) rows.
    const long row = (long)NKV * HD;
    const long cap_rows = kv_stride > 0 ? kv_stride / row : 0;
    if (valid_hd(HD) && (!base_b || (cap_rows > 0 && cap_rows <= INT_MAX))) {
        const int max_pos = base_b ? (int)cap_rows - 1 : base;
        const Problem p = make_problem(Q, DT_FP32, Kc, Vc, DT_FP32, O, DT_FP32, nullptr, B, 1, NQ, NKV, HD, kv_stride, 1,
                                       base, 1, base_b, nullptr, max_pos, scale, window);
        const Pool *pool = nullptr;
        if (f32_take_fast(p, pool)) return run_f32(p, *pool, st);
    }
    return launch_scalar_decode(Q, Kc, Vc, O, B, 1, NQ, NKV, HD, base, kv_stride, base_b, resolve_scale(scale, HD),
                                window < 0 ? 0 : window, knob_on("G4_ATTN_DIAG_REVERSE") ? 1 : 0, st);
}

hipError_t dgx_kv_store(const float *src, void *dst, size_t n, int kv_dtype, int which, hipStream_t st) {
    if (n && (!src || !dst)) return hipErrorInvalidValue;
    if (!valid_dtype(kv_dtype)) return hipErrorInvalidValue;
    return launch_kv_store(src, dst, n, kv_dtype, which, knob_on("G4_KV_STATS") ? 1 : 0, st);
}
hipError_t dgx_gate_sigmoid(float *y, const float *gate, int n, hipStream_t st) {
    if (n < 0 || (n && (!y || !gate))) return hipErrorInvalidValue;
    return launch_gate_sigmoid(y, gate, (size_t)n, st);
}
hipError_t dgx_f32_to_bf16(const float *in, void *out, size_t n, hipStream_t st) {
    if (n && (!in || !out)) return hipErrorInvalidValue;
    return launch_kv_store(in, out, n, DT_BF16, 0, 0, st);        // the store's RN-even conversion, no statistics
}
hipError_t dgx_kv_stats(unsigned out[4]) { return read_kv_stats(out); }

hipError_t dgx_norm_rope_store(const float *X, const float *W, void *Y, int y_dtype, int rows, int NH, int hd, float eps,
                               const float *cosT, const float *sinT, int base, int pos_step, const int *pos_arr,
                               long slot_stride, long row_stride, int rope, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    if (!valid_dtype(y_dtype)) return hipErrorInvalidValue;
    return launch_norm_rope_store(X, W, Y, y_dtype, rows, NH, hd, eps, cosT, sinT, base, pos_step, pos_arr, slot_stride,
                                  row_stride, rope != 0, st);
}

hipError_t dgx_kv_append(const float *k_src, const float *v_src, void *Kc, void *Vc, int kv_dtype, int nseq, int T,
                         long kv_stride, int row_elems, const int *pos_b, int base, hipStream_t st) {
    if (nseq == 0 || T == 0) return hipSuccess;
    if (!k_src || !v_src || !Kc || !Vc || !valid_dtype(kv_dtype)) return hipErrorInvalidValue;
    return launch_kv_append(k_src, v_src, Kc, Vc, kv_dtype, nseq, T, kv_stride, row_elems, pos_b, base,
                            knob_on("G4_KV_STATS") ? 1 : 0, st);
}

hipError_t dgx_attn_batch(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                          int o_dtype, float *lse, int B, int Tq, int NQ, int NKV, int HD, const int *base_b, int base,
                          long kv_stride, const unsigned *anc, int max_pos, int chunk, hipStream_t st, float scale,
                          int window) {
    if (B == 0 || Tq == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || B < 0 || Tq < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) || max_pos < 0 ||
        !valid_dtype(q_dtype) || !valid_dtype(o_dtype) || kv_dtype == DT_FP32 || !valid_dtype(kv_dtype))
        return hipErrorInvalidValue;
    if (B > 1 && kv_stride == 0 && !base_b) return hipErrorInvalidValue;
    const int C = chunk > 0 ? chunk : dgx_attn_split_chunk();
    if (C <= 0 || C % 32) return hipErrorInvalidValue;
    Pool *pool; hipError_t e = pool_for(g_split, pool); if (e != hipSuccess) return e;
    const int ns = max_pos / C + 1;
    if ((size_t)B * Tq * NQ * ns > pool->cap || (size_t)B * Tq * NQ * ns * HD > pool->acc_cap) return hipErrorInvalidValue;
    const Problem p = make_problem(Q, q_dtype, Kc, Vc, kv_dtype, O, o_dtype, lse, B, Tq, NQ, NKV, HD, kv_stride, 1, base,
                                   1, base_b, anc, max_pos, scale, window);
    return run_split(p, C, *pool, ns, st);
}

hipError_t dgx_attn_batch_noalloc(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                                  int o_dtype, float *lse, int B, int Tq, int NQ, int NKV, int HD, const int *base_b,
                                  int base, long kv_stride, const unsigned *anc, int max_pos, int chunk,
                                  hipStream_t st, float scale, int window) {
    if (B == 0 || Tq == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || B < 0 || Tq < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) || max_pos < 0 ||
        !valid_dtype(q_dtype) || !valid_dtype(o_dtype) || kv_dtype == DT_FP32 || !valid_dtype(kv_dtype))
        return hipErrorInvalidValue;
    if (B > 1 && kv_stride == 0 && !base_b) return hipErrorInvalidValue;
    const int C = chunk > 0 ? chunk : dgx_attn_split_chunk();
    if (C <= 0 || C % 32) return hipErrorInvalidValue;
    // Partials m [P], l [P] (each rounded up to 64 floats = 256 bytes) and acc [P * HD] in the fixed array.
    const int ns = max_pos / C + 1;
    const size_t P = (size_t)B * Tq * NQ * ns, Pa = (P + 63) / 64 * 64;
    if (P > kScratchBytes / sizeof(float) || (2 * Pa + P * (size_t)HD) * sizeof(float) > kScratchBytes) {
        fprintf(stderr, "[attn_batch_noalloc] %zu partials x (HD %d + 2) floats exceed the fixed %zu-byte scratch\n",
                P, HD, kScratchBytes);
        return hipErrorInvalidValue;
    }
    float *base_ptr = nullptr;
    hipError_t e = scratch_ptr(base_ptr);
    if (e != hipSuccess) return e;
    Pool fixed;
    fixed.m = base_ptr; fixed.l = base_ptr + Pa; fixed.acc = base_ptr + 2 * Pa;
    fixed.cap = P; fixed.acc_cap = P * (size_t)HD;
    const Problem p = make_problem(Q, q_dtype, Kc, Vc, kv_dtype, O, o_dtype, lse, B, Tq, NQ, NKV, HD, kv_stride, 1, base,
                                   1, base_b, anc, max_pos, scale, window);
    return run_split(p, C, fixed, ns, st);
}

hipError_t dgx_attn_batch_ex(const void *Q, int q_dtype, const void *Kc, const void *Vc, const void *const *Kp,
                             const void *const *Vp, int kv_dtype, void *O, int o_dtype, float *lse, const void *gate,
                             int gate_dtype, int B, int Tq, int NQ, int NKV, int HD, const int *base_b, int base,
                             long kv_stride, const unsigned *anc, int max_pos, int chunk, hipStream_t st, float scale,
                             int window, int kv_cap) {
    if (B == 0 || Tq == 0) return hipSuccess;
    if ((!Kp) != (!Vp) || (!Kp && (!Kc || !Vc)) || (gate && !valid_dtype(gate_dtype))) return hipErrorInvalidValue;
    if (!ring_ok(kv_cap, window, Tq)) return hipErrorInvalidValue;
    if (!Q || !O || B < 0 || Tq < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) || max_pos < 0 ||
        !valid_dtype(q_dtype) || !valid_dtype(o_dtype) || kv_dtype == DT_FP32 || !valid_dtype(kv_dtype))
        return hipErrorInvalidValue;
    if (!Kp && B > 1 && kv_stride == 0 && !base_b) return hipErrorInvalidValue;
    const int C = chunk > 0 ? chunk : dgx_attn_split_chunk();
    if (C <= 0 || C % 32) return hipErrorInvalidValue;
    Pool *pool; hipError_t e = pool_for(g_split, pool); if (e != hipSuccess) return e;
    const int ns = max_pos / C + 1;
    if ((size_t)B * Tq * NQ * ns > pool->cap || (size_t)B * Tq * NQ * ns * HD > pool->acc_cap) return hipErrorInvalidValue;
    Problem p = make_problem(Q, q_dtype, Kc, Vc, kv_dtype, O, o_dtype, lse, B, Tq, NQ, NKV, HD, kv_stride, 1, base,
                             1, base_b, anc, max_pos, scale, window);
    p.Kp = Kp; p.Vp = Vp; p.gate = gate; p.gate_dtype = gate_dtype; p.kv_cap = kv_cap;
    return run_split(p, C, *pool, ns, st);
}

hipError_t dgx_attn_prefill_ex(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                               int o_dtype, float *lse, int nseq, int Sq, int NQ, int NKV, int HD, const int *base_b,
                               int base, long kv_stride, int max_pos, int kv_split, hipStream_t st, float scale,
                               int window, int kv_cap) {
    if (nseq == 0 || Sq == 0) return hipSuccess;
    if (!Q || !Kc || !Vc || !O || nseq < 0 || Sq < 0 || NQ <= 0 || NKV <= 0 || NQ % NKV || !valid_hd(HD) ||
        max_pos < 0 || !valid_dtype(q_dtype) || !valid_dtype(o_dtype) || !valid_dtype(kv_dtype) || kv_split < -1 ||
        (kv_split > 0 && kv_split % 64) || !ring_ok(kv_cap, window, Sq))
        return hipErrorInvalidValue;
    Pool *pool; hipError_t e = pool_for(g_flash, pool); if (e != hipSuccess) return e;
    Problem p = make_problem(Q, q_dtype, Kc, Vc, kv_dtype, O, o_dtype, lse, nseq, Sq, NQ, NKV, HD, kv_stride, 1,
                             base, 1, base_b, nullptr, max_pos, scale, window);
    p.kv_cap = kv_cap;
    if (kv_split < 0) kv_split = prefill_auto_split(p);
    const int ns = kv_split > 0 ? max_pos / kv_split + 1 : 1;
    if (kv_split > 0) {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        e = pool_grow(*pool, (size_t)nseq * Sq * NQ * ns, (size_t)HD);
        if (e != hipSuccess) return e;
    }
    Partials part{pool->m, pool->l, pool->acc, ns};
    return timed_launch(st, [&] { return launch_prefill(p, kv_split, part, st); });
}

hipError_t dgx_attn_prefill(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                            int o_dtype, float *lse, int nseq, int Sq, int NQ, int NKV, int HD, const int *base_b,
                            int base, long kv_stride, int max_pos, int kv_split, hipStream_t st, float scale,
                            int window) {
    return dgx_attn_prefill_ex(Q, q_dtype, Kc, Vc, kv_dtype, O, o_dtype, lse, nseq, Sq, NQ, NKV, HD, base_b, base,
                               kv_stride, max_pos, kv_split, st, scale, window, 0);
}

hipError_t dgx_attn_timing(int on) {
    std::lock_guard<std::mutex> lk(g_timing_mu);
    if (on && !g_timing.made) {
        for (int i = 0; i < kTimed; i++) {
            hipError_t e = hipEventCreateWithFlags(&g_timing.a[i], hipEventDisableSystemFence);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&g_timing.b[i], hipEventDisableSystemFence);
            if (e != hipSuccess) return e;
        }
        g_timing.made = true;
    }
    g_timing.on = on != 0;
    g_timing.n = 0;
    g_timing_on.store(on != 0, std::memory_order_release);
    return hipSuccess;
}

hipError_t dgx_attn_timing_read(float *avg_ms, int *count) {
    std::lock_guard<std::mutex> lk(g_timing_mu);
    double sum = 0.0;
    for (int i = 0; i < g_timing.n; i++) {
        hipError_t e = hipEventSynchronize(g_timing.b[i]);
        if (e != hipSuccess) return e;
        float ms = 0.f;
        e = hipEventElapsedTime(&ms, g_timing.a[i], g_timing.b[i]);
        if (e != hipSuccess) return e;
        sum += ms;
    }
    if (count) *count = g_timing.n;
    if (avg_ms) *avg_ms = g_timing.n ? (float)(sum / g_timing.n) : 0.f;
    g_timing.n = 0;
    return hipSuccess;
}

const char *dgx_attn_version(void) { return "dgx-attn-mi355x 0.1 (gfx950)"; }

}  // extern "C"

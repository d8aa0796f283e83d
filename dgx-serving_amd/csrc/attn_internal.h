// Internal launch descriptors shared by the kernels and the C-ABI layer (not part of the public interface).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dgx {

// A batch of `nseq` sequences, each with `T` query tokens over its own KV cache (K/V at seq * kv_stride elements).
// Token (s, t) has global row index r = s * T + t (Q/O/LSE are [r][NQ][HD] / [r][NQ]).
// Its position is
//   pos_mode 0: pos_arr ? pos_arr[r] : base + r * pos_step              (launch_attn_decode_split rows)
//   pos_mode 1: (pos_arr ? pos_arr[s] : base) + t                        (a sequence of consecutive tokens)
// With anc, the tree of sequence s starts at tb = position of token (s, 0) and anc[r] masks keys >= tb.
struct Problem {
    const void *Q; int q_dtype;
    const void *K; const void *V; int kv_dtype;
    void *O; int o_dtype;
    float *lse;                       // optional [rows, NQ], natural log
    int nseq, T, NQ, NKV, HD;
    long kv_stride;
    int pos_mode, base, pos_step;
    const int *pos_arr;
    const uint32_t *anc;
    int max_pos;                      // host-side upper bound of every position (sizes the split grid)
    float scale;                      // resolved (> 0)
    int window;
    const void *const *Kp;            // optional device arrays of per-sequence K / V bases (override K, V + s*kv_stride)
    const void *const *Vp;
    const void *gate;                 // optional output gate [rows, NQ, HD]: O *= sigmoid(gate) (split path only)
    int gate_dtype;
    int kv_cap;                       // 0: key j in cache row j; > 0 (multiple of 64): ring buffer, row j % kv_cap
};

// Cache row of key j0, a multiple of 16: tiles of 16 (64 in prefill steps) keys never wrap inside a ring.
__device__ __forceinline__ int key_row(const Problem &p, int j0) {
    return p.kv_cap > 0 ? (int)((unsigned)j0 % (unsigned)p.kv_cap) : j0;
}

// K (v = false) or V cache base of sequence s.
template <class KE>
__device__ __forceinline__ const KE *kv_base(const Problem &p, bool v, int s) {
    const void *const *tab = v ? p.Vp : p.Kp;
    if (tab) return reinterpret_cast<const KE *>(tab[s]);
    return reinterpret_cast<const KE *>(v ? p.V : p.K) + (size_t)s * p.kv_stride;
}

// Split-KV partials in scratch: index (r * NQ + h) * ns_cap + c; m and l in the log2 domain (m = max of
// scale*log2(e)*q.k, l = sum of 2^(t - m)), acc = sum 2^(t - m) v, unnormalised.
struct Partials {
    float *m, *l, *acc;
    int ns_cap;
    // Set by launch_split when verify_kernel wrote the partials (seg_g > 0: its grid size and minimum run length;
    // the slots of a pair end at the first slot whose m is +inf); 0 for partials indexed by absolute key chunk.
    int seg_g = 0, seg_qmin = 0;
};

// Position of token t of sequence s, and the first key of its sliding window.
__device__ __forceinline__ int tok_pos(const Problem &p, int s, int t) {
    if (p.pos_mode == 0) {
        const int r = s * p.T + t;
        return p.pos_arr ? p.pos_arr[r] : p.base + r * p.pos_step;
    }
    return (p.pos_arr ? p.pos_arr[s] : p.base) + t;
}
__device__ __forceinline__ int win_lo(int pos, int window) {
    return (window > 0 && pos - window + 1 > 0) ? pos - window + 1 : 0;
}

// Split-KV decode / verify / tree kernel (waves split the keys of a chunk, small query-row tiles). Verify and tree
// rows on 16-bit caches at HD <= 256 run verify_kernel: slot_runs cuts its runs at absolute key chunks of each
// sequence (batch-invariant), otherwise into equal runs over the whole batch (faster, depends on the batch).
hipError_t launch_split(const Problem &p, int chunk, Partials &part, hipStream_t st, bool slot_runs = true);
// Streaming decode kernel (T x GRP <= 16 rows per KV head, HD 128/256, 16-bit cache);
// hipErrorNotSupported for other shapes. Writes chunk partials for launch_combine.
bool decode_stream_supported(const Problem &p);
hipError_t launch_decode_stream(const Problem &p, int chunk, const Partials &part, hipStream_t st);
// The same in fp32 end to end (fp32 Q and cache, fp32 MFMA) for fp32 caches, HD 128/256, T x GRP <= 16.
bool decode_f32_supported(const Problem &p);
hipError_t launch_decode_f32(const Problem &p, int chunk, const Partials &part, hipStream_t st);
// Flash prefill kernel (waves split query rows, K/V tiles shared through LDS). kv_split = 0: one pass per row
// tile writing O directly; kv_split > 0: keys cut at absolute multiples of kv_split, partials + combine.
hipError_t launch_prefill(const Problem &p, int kv_split, const Partials &part, hipStream_t st);
// The key split chosen for kv_split = -1 (0: none).
int prefill_auto_split(const Problem &p);
size_t prefill_lds_bytes(int HD);   // dynamic LDS of the HD-wide prefill tile (W = 0)
size_t split_lds_bytes(int HD);     // dynamic LDS of split_kernel at one row block
// LSE combine of split partials for every (row, head).
hipError_t launch_combine(const Problem &p, int chunk, const Partials &part, hipStream_t st);
// Scratch requirement (rows*NQ*ns_cap) of a problem at a given chunk.
size_t partial_rows(const Problem &p, int chunk);

// fp32 scalar kernels of the reference's attention.cuh (small-shape prefill and smem-free decode).
hipError_t launch_scalar_prefill(const float *Q, const float *K, const float *V, float *O, int S, int NQ, int NKV,
                                 int HD, float scale, int window, hipStream_t st);
hipError_t launch_scalar_decode(const float *Q, const float *Kc, const float *Vc, float *O, int nseq, int Sq,
                                int NQ, int NKV, int HD, int base, long kv_stride, const int *base_b, float scale,
                                int window, int reverse, hipStream_t st);
hipError_t launch_scalar_rows(const float *Q, const float *Kc, const float *Vc, float *O, int rows, int NQ, int NKV,
                              int HD, int base, int pos_step, const int *pos_arr, long kv_stride, float scale,
                              int window, int reverse, hipStream_t st);
hipError_t launch_gate_sigmoid(float *y, const float *gate, size_t n, hipStream_t st);
hipError_t launch_kv_store(const float *src, void *dst, size_t n, int kv_dtype, int which, int stats,
                           hipStream_t st);
hipError_t launch_kv_append(const float *ks, const float *vs, void *Kc, void *Vc, int kv_dtype, int nseq, int T,
                            long kv_stride, int row, const int *pos_b, int base, int stats, hipStream_t st);
hipError_t read_kv_stats(unsigned out[4]);
bool norm_rope_shape_ok(int hd, bool rope);
hipError_t launch_norm_rope_store(const float *X, const float *W, void *Y, int y_dtype, int rows, int NH, int hd,
                                  float eps, const float *cosT, const float *sinT, int base, int pos_step,
                                  const int *pos_arr, long slot_stride, long row_stride, bool rope, hipStream_t st);

}  // namespace dgx

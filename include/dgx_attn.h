/* dgx_attn.h - C ABI of the MI355X (gfx950) attention library for hyunlord/dgx-serving.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t, returns a hipError_t
 * (hipSuccess = 0) and never aborts. The C++ header dgx_attn.hpp wraps these under the reference's own
 * launcher names and turns a failure into the reference's fprintf + abort().
 *
 * Layouts (unchanged from the reference, kernels/attention_decode_split.cuh:13-15):
 *   Q, O      [rows, NQ, HD]              (fp32 at the drop-in entry points)
 *   K/V cache [len, NKV, HD] per sequence; a batch is [B, max_len, NKV, HD] with
 *             kv_stride = max_len * NKV * HD elements between sequences
 *   lse       optional [rows, NQ] fp32, natural-log log-sum-exp of scale * q.k over the attended keys
 *             (the reference keeps it private; pass NULL to skip)
 * KV dtype codes are the reference's enum (kernels/kv_store.cuh:20): 0 = fp32, 1 = f16, 2 = bf16.
 * Q/O dtype codes of the native entry points use the same codes.
 * scale = 0 selects 1/sqrt(HD); window = 0 is plain causal, window = w keeps keys [pos - w + 1, pos].
 *
 * Threading: calls on one device are stream-ordered; library scratch is per device and shared by calls, so
 * calls that run concurrently on different streams of one device must not share a scratch pool (the decode
 * split pool and the flash pool are separate, as in the reference).
 */
#ifndef DGX_ATTN_H
#define DGX_ATTN_H
#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DGX_DT_FP32 0
#define DGX_DT_F16 1
#define DGX_DT_BF16 2

/* ---- knobs (runtime/knobs.h registry semantics: env > DGX_KNOBS_FILE recipe > default) ---- */

/* 0 when the attention knobs are valid, -1 otherwise (the first error is printed once, "knobs: ..."): a recipe line
 * that is not NAME=VALUE, an unregistered name under G4_ATTN_ / G4_KV_ / G4_FLASH_, an unreadable DGX_KNOBS_FILE,
 * or a value outside its set (G4_ATTN_SPLIT, G4_ATTN_CHUNK, G4_KV_DTYPE, G4_FLASH_PREFILL, G4_FLASH_MIN_S,
 * G4_FLASH_V2, G4_FLASH_F16_MMA, G4_KV_STATS, G4_ATTN_DIAG_REVERSE). With an invalid configuration the knob queries
 * below return -1. Replaces the registry load and its exit(2), runtime/knobs.h:241-275 (the C++ wrapper exits 2). */
int dgx_knobs_status(void);

/* How the batched verify / tree kernel (16-bit caches, HD <= 256, more than one query token) divides the keys
 * among its workgroups, process-wide. mode 0 (the default): each sequence's keys in absolute chunks of the split
 * chunk, so a row's result depends only on its own sequence, bit-identical to the same slot launched alone (the
 * reference verifies each slot with its own launch, models/qwen35_batch.cu:333-335). mode 1: equal runs over the
 * whole batch's key tiles (every workgroup streams the same bytes; results are deterministic but depend on the other
 * sequences' lengths). mode -1 queries. Returns the previous mode, or -1 for another value. No reference
 * counterpart: the reference has only the per-slot behaviour of mode 0. */
int dgx_attn_verify_runs(int mode);

/* Process-wide KV storage dtype from G4_KV_DTYPE (fp32 | f16 | bf16; unset -> f16, or fp32 when
 * G4_ATTN_SPLIT=0). Returns -1 for an invalid value or knob configuration (the C++ wrapper exits 2 like the
 * reference registry).
 * Replaces g4_kv_dtype(), kernels/kv_store.cuh:23-35. */
int dgx_kv_dtype(void);
/* Dynamic LDS bytes of the head-dim 512 flash path (the larger of its short-query split and prefill tiles; each
 * kernel sets its own limit at its first launch, within the 160 KB of a gfx950 CU). Replaces the value that
 * configure_flash_attn_hd512() returns, kernels/attention_flash.cuh:254-270. */
size_t dgx_flash_attn_hd512_lds(void);
/* 1 when G4_KV_STATS=1 (the stores count non-finite values and max |x|), else 0. Replaces the knob test of
 * g4_kv_stats_enabled(), kernels/kv_store.cuh:87-90. */
int dgx_kv_stats_enabled(void);
/* Force fp32 KV for this process (MoE models). Replaces g4_kv_force_fp32(), kernels/kv_store.cuh:37-41. */
void dgx_kv_force_fp32(const char *why);
/* Bytes per stored KV element (4 or 2). Replaces g4_kv_elem(), kernels/kv_store.cuh:42. */
size_t dgx_kv_elem(void);

/* Split-KV chunk from G4_ATTN_CHUNK (32, 64, 128 or 256, the reference's set; unset -> 256 on MI355X, where the
 * reference defaults to 64). -1 if invalid (value or knob configuration).
 * Replaces attn_split_chunk(), kernels/attention_decode_split.cuh:26-37. */
int dgx_attn_split_chunk(void);
/* ceil(max_len / chunk). Replaces attn_split_ns_cap(), kernels/attention_decode_split.cuh:173. */
int dgx_attn_split_ns_cap(int max_len);
/* Reserve the decode-split scratch (never shrinks) on the current device; call before graph capture.
 * Replaces attn_split_reserve(), kernels/attention_decode_split.cuh:174-188. */
hipError_t dgx_attn_split_reserve(int rows, int NQ, int max_len, int hd_max);

/* ---- drop-in launchers ---- */

/* Split-KV decode/verify/batch rows. Row r has position pos_arr ? pos_arr[r] : base + r * pos_step and KV at
 * Kc + r * kv_stride (kv_stride = 0: rows share one sequence's KV, e.g. verify). max_pos bounds every row
 * position (host), ns_cap = dgx_attn_split_ns_cap(max_len) of the reservation. Chunk = dgx_attn_split_chunk().
 * Returns hipErrorInvalidValue when the scratch is not reserved (the reference aborts, :210-213) or the shape
 * is unsupported. HD in {128, 256, 512}, NQ / NKV <= 64.
 * Replaces launch_attn_decode_split(), kernels/attention_decode_split.cuh:205-231. */
hipError_t dgx_attn_decode_split(const float *Q, const void *Kc, const void *Vc, int kv_dtype, float *O, float *lse,
                                 int rows, int NQ, int NKV, int HD, int base, int pos_step, const int *pos_arr,
                                 int max_pos, long kv_stride, int ns_cap, hipStream_t st, float scale, int window);

/* Flash attention over a KV cache: Sq query tokens at positions base .. base+Sq-1, causal, optional sliding
 * window, optional tree mask anc[Sq] (key j >= base attended iff bit j-base of anc[q], j-base < 32).
 * Runs of up to 32 tokens and every tree-masked run take the split kernel; a tree run of more than 32 tokens
 * never attends nodes at bit 32 and beyond, as in the reference. Its scratch grows inside the call when needed
 * (as the reference's does); pre-size it with dgx_flash_attn_reserve / _reserve_partials before graph capture.
 * Replaces launch_flash_attn<KV>() / launch_flash_attn2bs<HD,BC,NW,KV>(), kernels/attention_flash.cuh:273-306. */
hipError_t dgx_flash_attn(const float *Q, const void *Kc, const void *Vc, int kv_dtype, float *O, float *lse,
                          int Sq, int NQ, int NKV, int HD, int base, hipStream_t st, const unsigned *anc,
                          float scale, int window);
/* Pre-size the flash scratch for Sq tokens at base (runs of up to 32 tokens; longer runs without a tree mask take
 * the prefill kernel and need none). A tree-masked run of more than 32 tokens needs
 * dgx_flash_attn_reserve_partials(Sq * NQ * ((base + Sq - 1) / 512 + 1), HD) before graph capture.
 * Replaces reserve_flash_attn_scratch(), attention_flash.cuh:236. */
hipError_t dgx_flash_attn_reserve(int Sq, int NQ, int base, int HD);
/* Pre-size the flash scratch to `partials` (row, head, split) partials of hd_max floats, the reference's own
 * unit. Replaces reserve_flash_attn_scratch(need, hd), attention_flash.cuh:236-252. */
hipError_t dgx_flash_attn_reserve_partials(size_t partials, int hd_max);

/* Prefill / chunked prefill (base > 0 = chunk over a cached prefix). f16_mma: operand precision request of the
 * reference; here the MFMA operand format always follows the cache (f16 cache: f16, bf16/fp32 cache: bf16).
 * Replaces launch_flash_attn_v2<KV>(), kernels/attention_flash_v2.cuh:284-292. */
hipError_t dgx_flash_attn_v2(const float *Q, const void *Kc, const void *Vc, int kv_dtype, float *O, float *lse,
                             int Sq, int NQ, int NKV, int HD, int base, hipStream_t st, float scale, int window,
                             int f16_mma);

/* fp32 launchers below never allocate. They run the fp32 MFMA kernel (HD 128/256, up to 16 rows per KV head)
 * when the flash scratch already holds its partials - rows * NQ * (max_pos / 512 + 1) of them, reserved with
 * dgx_flash_attn_reserve_partials (or grown by an earlier flash call) - and the scalar fp32 kernels otherwise. */
/* fp32 causal prefill over fp32 K/V [S, NKV, HD] (no S <= HD limit). Replaces launch_attn(), attention.cuh:72-79. */
hipError_t dgx_attn(const float *Q, const float *K, const float *V, float *O, int S, int NQ, int NKV, int HD,
                    hipStream_t st, float scale, int window);
/* fp32 decode/verify over an fp32 cache (no shared-memory context limit). Honors G4_ATTN_DIAG_REVERSE.
 * Replaces launch_attn_decode(), attention.cuh:137-146. */
hipError_t dgx_attn_decode(const float *Q, const float *Kc, const float *Vc, float *O, int Sq, int NQ, int NKV, int HD,
                           int base, hipStream_t st, float scale, int window);
/* fp32 batch decode: B sequences, one token each at base_b ? base_b[b] : base, KV at b * kv_stride.
 * Replaces launch_attn_decode_batch(), attention.cuh:189-198. */
hipError_t dgx_attn_decode_batch(const float *Q, const float *Kc, const float *Vc, float *O, int B, int NQ, int NKV,
                                 int HD, int base, long kv_stride, hipStream_t st, float scale, int window,
                                 const int *base_b);

/* fp32 -> cache dtype store (RN-even), which = 0 for K, 1 for V; counts non-finite / max |x| with G4_KV_STATS=1.
 * dst already offset by the caller (kv_at). Replaces kv_store() / kv_store_kernel, kernels/kv_store.cuh:76-113. */
hipError_t dgx_kv_store(const float *src, void *dst, size_t n, int kv_dtype, int which, hipStream_t st);
/* y[i] *= sigmoid(gate[i]) for n fp32 elements in place, the Qwen3.5 full-attention output gate applied after the
 * attention call, with the same float operations as the gate fused into dgx_attn_batch_ex. Replaces
 * launch_gate_sigmoid() / gate_sigmoid_kernel, kernels/elementwise.cuh:50-60 (models/qwen35.cu:96,
 * models/qwen35_decode.cu:166, models/qwen35_batch.cu:168,336). */
hipError_t dgx_gate_sigmoid(float *y, const float *gate, int n, hipStream_t st);
/* fp32 -> bf16 (RN-even) of n elements, the Qwen KV-cache hand-off: replaces launch_f32_to_bf16() /
 * f32_to_bf16_kernel, kernels/elementwise.cuh:85-95 (used per slot at models/qwen35_batch.cu:159-162). */
hipError_t dgx_f32_to_bf16(const float *in, void *out, size_t n, hipStream_t st);
/* Read the G4_KV_STATS counters {nonfinite K, nonfinite V, max|K| bits, max|V| bits} (kv_store.cuh:86-98). */
hipError_t dgx_kv_stats(unsigned out[4]);
/* Ragged KV append in one launch: token t of sequence b (rows b*T + t of k_src / v_src, fp32 [nseq*T][row_elems])
 * is stored at cache row (pos_b ? pos_b[b] : base) + t of sequence b (element b*kv_stride + pos*row_elems), converted
 * to kv_dtype exactly as dgx_kv_store does (same G4_KV_STATS counters). pos_b is a device array or null;
 * row_elems (= NKV*HD) and kv_stride must be multiples of 4. Replaces the per-slot kv_store / launch_f32_to_bf16 /
 * cudaMemcpy loops of the batch decoders, models/gemma4_batch.cu:160-171 and models/qwen35_batch.cu:159-162. */
hipError_t dgx_kv_append(const float *k_src, const float *v_src, void *Kc, void *Vc, int kv_dtype, int nseq, int T,
                         long kv_stride, int row_elems, const int *pos_b, int base, hipStream_t st);

/* Per-head RMSNorm (+ RoPE) (+ store): row r = (token s = r / NH, head h = r % NH) of hd fp32 values in X;
 * y = x * rsqrt(mean(x^2) + eps) * W (W == NULL: no scale); with rope != 0 the rotate-half RoPE of position
 * p = pos_arr ? pos_arr[s] : base + s * pos_step from the tables cosT / sinT (row p: entries [p*hd, p*hd + hd/2));
 * stored at Y + s*slot_stride + p*row_stride + h*hd elements of y_dtype (0 fp32, 1 f16, 2 bf16; nearest-even).
 * hd % 4 == 0, hd <= 1024, with or without rope. pos_arr is a device array or null.
 * Replaces launch_norm_rope_store<TO>() / norm_rope_store_kernel, kernels/norm_fused.cuh:84-133 (the Gemma4 q, k
 * and v appends of models/gemma4_decode.cu:340,353-354 and models/gemma4_batch.cu:142,153,477,486). */
hipError_t dgx_norm_rope_store(const float *X, const float *W, void *Y, int y_dtype, int rows, int NH, int hd, float eps,
                               const float *cosT, const float *sinT, int base, int pos_step, const int *pos_arr,
                               long slot_stride, long row_stride, int rope, hipStream_t st);

/* ---- native entry points (16-bit Q/O, one ragged launch, explicit chunking) ---- */

/* One launch over B sequences x Tq query tokens (decode: Tq = 1; tree verify: Tq nodes). Token i of sequence b
 * is at position (base_b ? base_b[b] : base) + i, its KV at Kc + b * kv_stride; anc[B * Tq] optional tree masks
 * relative to the sequence's first token. max_pos bounds every position (host). chunk = split size (multiple of
 * 32; 0 -> dgx_attn_split_chunk()). Uses the decode-split scratch, which must hold B*Tq*NQ*(max_pos/chunk+1)
 * partials (dgx_attn_split_reserve(B*Tq, NQ, max_pos+1, HD) with the same chunk).
 * No reference counterpart in one call: it replaces the per-slot loops of launch_flash_attn at
 * models/qwen35_batch.cu:165-167 (decode) and :333-335 (tree verify). */
hipError_t dgx_attn_batch(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                          int o_dtype, float *lse, int B, int Tq, int NQ, int NKV, int HD, const int *base_b, int base,
                          long kv_stride, const unsigned *anc, int max_pos, int chunk, hipStream_t st, float scale,
                          int window);
/* dgx_attn_batch that allocates nothing, for callers that cannot call hipMalloc (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation). No counterpart in the reference. Same arguments, rows
 * and results as dgx_attn_batch (bit-identical: the same kernels), but the split partials live in a fixed 64 MiB
 * device array inside the library (one per GPU, held until the process ends) instead of the reserved pool, so no
 * dgx_attn_split_reserve is needed. Limit: B * Tq * NQ * (max_pos / chunk + 1) partials of (HD + 2) floats must
 * fit in 64 MiB (e.g. BASELINE config 2 at chunk 512 needs 6.3 MB); larger calls return hipErrorInvalidValue.
 * Calls that overlap on one GPU (different streams or host threads) share the array and race; serialize them. */
hipError_t dgx_attn_batch_noalloc(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                                  int o_dtype, float *lse, int B, int Tq, int NQ, int NKV, int HD, const int *base_b,
                                  int base, long kv_stride, const unsigned *anc, int max_pos, int chunk,
                                  hipStream_t st, float scale, int window);
/* dgx_attn_batch with two caller-side fusions for the Qwen callers (models/qwen35_batch.cu:165-167,333-335 and
 * models/qwen35_decode.cu:165-166):
 *   - Kp / Vp: device arrays of B per-slot K / V base pointers (each [max_len, NKV, HD]); when given they replace
 *     Kc / Vc + b*kv_stride (Kc, Vc, kv_stride are then ignored), so slots need not share one allocation;
 *   - gate: optional [B*Tq, NQ, HD] tensor of dtype gate_dtype; the output is multiplied by sigmoid(gate) in the
 *     LSE combine (the reference's separate launch_gate_sigmoid(attn, gate) after attention).
 *   - kv_cap > 0: the caches are ring buffers of kv_cap rows (a multiple of 64) for a sliding window: key j lives in
 *     row j % kv_cap (the sliding-window ring layout of runtime/decode_state_gemma4.h:9-16, kv_cap). Needs
 *     window > 0 and window + Tq - 1 <= kv_cap, so the keys a launch reads never alias.
 * Same rows, positions and masks as dgx_attn_batch; a row's result is bit-identical to dgx_attn_batch's when Kp,
 * Vp point at the same caches, gate is null and kv_cap is 0 (or the ring holds the same keys). */
hipError_t dgx_attn_batch_ex(const void *Q, int q_dtype, const void *Kc, const void *Vc, const void *const *Kp,
                             const void *const *Vp, int kv_dtype, void *O, int o_dtype, float *lse, const void *gate,
                             int gate_dtype, int B, int Tq, int NQ, int NKV, int HD, const int *base_b, int base,
                             long kv_stride, const unsigned *anc, int max_pos, int chunk, hipStream_t st, float scale,
                             int window, int kv_cap);
/* Prefill with explicit key split (kv_split = 0: none; else a multiple of 64, partials + combine for rows that
 * span splits; -1: chosen by the library, a split only when the unsplit grid fills at most half the CUs, e.g. a
 * short chunk over a long prefix; the choice depends on the launch's own shape, so a row's bits then depend on how
 * the prompt is chunked) over nseq sequences of Sq tokens at (base_b ? base_b[s] : base) + i. Uses the flash
 * scratch (grown in the call when needed). Native form of launch_flash_attn_v2 (attention_flash_v2.cuh:284-292). */
hipError_t dgx_attn_prefill(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                            int o_dtype, float *lse, int nseq, int Sq, int NQ, int NKV, int HD, const int *base_b,
                            int base, long kv_stride, int max_pos, int kv_split, hipStream_t st, float scale,
                            int window);

/* dgx_attn_prefill over ring-buffer caches (kv_cap as in dgx_attn_batch_ex; window + Sq - 1 <= kv_cap). */
hipError_t dgx_attn_prefill_ex(const void *Q, int q_dtype, const void *Kc, const void *Vc, int kv_dtype, void *O,
                               int o_dtype, float *lse, int nseq, int Sq, int NQ, int NKV, int HD, const int *base_b,
                               int base, long kv_stride, int max_pos, int kv_split, hipStream_t st, float scale,
                               int window, int kv_cap);

/* Measurement hook (no counterpart in the reference; for benchmarks and profilers). With timing on, the main
 * kernel of every decode/verify (split or streaming kernel, without the LSE combine) and every prefill launch is
 * bracketed by a HIP event pair on its launch stream, for up to 4096 launches. dgx_attn_timing_read waits for the
 * recorded launches and returns their average duration in ms and their count, then starts a new record.
 * dgx_attn_timing(0) switches it off. Not for concurrent use from several threads. */
hipError_t dgx_attn_timing(int on);
hipError_t dgx_attn_timing_read(float *avg_ms, int *count);

/* Library version string. */
const char *dgx_attn_version(void);

#ifdef __cplusplus
}
#endif
#endif /* DGX_ATTN_H */

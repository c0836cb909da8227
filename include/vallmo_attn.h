/*
 * vallmo_attn.h — C ABI of libvallmo_attn.so, the MI355X (gfx950) gated
 * full-attention path of Vallmo.jl: per-head QK-RMSNorm, partial RoPE, GQA
 * causal attention for prefill and KV-cache decode, and the sigmoid output gate.
 *
 * Conventions (every entry point):
 *   - Returns int status: 0 = ok, > 0 = a passed-through hipError_t,
 *     < 0 = an argument/shape error (VM_E_*). vm_last_error() returns the
 *     message of the last failure on the calling thread.
 *   - Every data pointer is a DEVICE pointer. bf16 tensors are passed as
 *     vm_bf16* (the raw 16-bit pattern). Lengths/positions are device int32.
 *   - Strides are in ELEMENTS; the innermost (head_dim) stride is always 1.
 *   - Tensor layouts are named in the reference's column-major order, e.g.
 *     K_cache (D, Ctx, Hk, B), which is row-major [B][Hk][Ctx][D] here.
 *   - Compute entry points are asynchronous on `stream` (NULL = default
 *     stream), allocate no device memory, never synchronise, and are legal
 *     under hipStreamBeginCapture (hipGraph replay), as the reference requires
 *     of its decode step (src/llm/generate.jl:17-27). The one exception is
 *     vm_linear_tune, a load-time call, marked where it is declared.
 *   - Compiled for head_dim D = 256 and HALF_ROT = 32 (rotary dim 64), the
 *     Qwen3.5 attention facts (src/llm/qwen35.jl:15-23). Other D/HALF_ROT are
 *     rejected with VM_E_UNSUPPORTED. GQA group H/Hk <= 8 for decode.
 */
#ifndef VALLMO_ATTN_H
#define VALLMO_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t vm_bf16;   /* bfloat16 bit pattern                         */
typedef void*    vm_stream; /* hipStream_t; NULL selects the default stream */

enum {
  VM_OK             = 0,
  VM_E_ARG          = -1, /* null pointer / negative size / bad stride      */
  VM_E_DIM          = -2, /* shape mismatch (the reference's DimensionMismatch) */
  VM_E_UNSUPPORTED  = -3, /* shape outside what the kernels are built for   */
  VM_E_SCRATCH      = -4  /* scratch buffer too small                       */
};

/* ---- errors / version ------------------------------------------------- */
const char* vm_last_error(void);
int vm_abi_version(void);

/* ---- kernel timing (benchmarks; not a reference op) ----------------------
 * While enabled on the calling thread, every kernel a compute entry point
 * launches outside graph capture is bracketed by hipEvents on its stream.
 * vm_profile_enable(1) also clears earlier records. vm_profile_read waits for
 * the recorded events and returns the launch count and summed duration of one
 * kernel class.                                                              */
enum {
  VM_K_ROWS = 0,          /* norm+RoPE / append row kernels (the gated
                             prefill's append + V^T staging kernel too)      */
  VM_K_DECODE_SPLIT = 1,  /* split-KV decode attention                       */
  VM_K_DECODE_COMBINE = 2,/* LSE merge (+ gate)                              */
  VM_K_PREFILL = 3,       /* flash attention (prefill)                       */
  VM_K_ADVANCE = 4,       /* device clock                                    */
  VM_K_LM_HEAD = 5,       /* lm-head GEMV + argmax (split and combine)       */
  VM_K_DELTANET = 6,      /* delta-rule recurrence (decode step, sequence)   */
  VM_K_CONV = 7,          /* causal conv1d (decode step, sequence)           */
  VM_K_COUNT = 8
};
int vm_profile_enable(int on);
int vm_profile_read(int kernel, int* count, double* total_ms);
/* Restricts the bracketing to the kernel classes whose bit (1 << VM_K_*) is
 * set in kernel_mask (default: all), so a benchmark can time one kernel
 * without events around the others.                                          */
int vm_profile_select(unsigned kernel_mask);

/* ---- runtime (thin HIP wrappers so FFI hosts need no HIP headers) ------ */
int vm_malloc(void** ptr, size_t bytes);
int vm_free(void* ptr);
int vm_memcpy_h2d(void* dst, const void* src, size_t bytes, vm_stream stream);
int vm_memcpy_d2h(void* dst, const void* src, size_t bytes, vm_stream stream);
int vm_memcpy_d2d(void* dst, const void* src, size_t bytes, vm_stream stream);
int vm_memset(void* dst, int value, size_t bytes, vm_stream stream);
int vm_stream_create(vm_stream* stream);
int vm_stream_destroy(vm_stream stream);
int vm_stream_sync(vm_stream stream);
int vm_device_sync(void);
int vm_event_create(void** event);
int vm_event_destroy(void* event);
int vm_event_record(void* event, vm_stream stream);
int vm_event_elapsed_ms(float* ms, void* start, void* stop);
/* Graph capture of everything launched on `stream` between begin and end
 * (src/llm/generate.jl:185-191: capture → instantiate → launch). */
int vm_graph_begin_capture(vm_stream stream);
int vm_graph_end_capture(vm_stream stream, void** graph_exec);
int vm_graph_launch(void* graph_exec, vm_stream stream);
int vm_graph_destroy(void* graph_exec);

/* ---- a1: RoPE tables (src/llm/qwen35.jl:115-119) -----------------------
 * cos/sin :: (HALF_ROT, Ctx) fp32 = row-major [Ctx][half_rot].
 * inv_freq_i = f32(theta^(-i/half_rot)) (power in f64); angle = inv_freq_i *
 * f32(t) in f32; table = f32 of the f64 cos/sin of that f32 angle. */
int vm_rope_tables(float* cos_tab, float* sin_tab, int half_rot, int64_t ctx,
                   double theta, vm_stream stream);

/* ---- a3: qnorm_rope! (src/kernels/qknorm_rope_append.jl:100-117) -------
 * In place on Q :: (D, Hq, B) bf16 with head stride q_sh, batch stride q_sb.
 * q = q / sqrt(mean(q^2) + eps) * (qw + w_offset), then rotate-half RoPE on
 * dims [0, 2*half_rot) at 0-based position positions[b]-1. D is a power of
 * two from 16 to 512 (qknorm_rope_append.jl:108), 1 <= half_rot <= D/2; D =
 * 256 with half_rot = 32 runs the tuned row kernel, other shapes a generic one. */
int vm_qnorm_rope(vm_bf16* q, int64_t q_sh, int64_t q_sb,
                  const vm_bf16* qw, const float* cos_tab, const float* sin_tab,
                  int64_t ctx, const int32_t* positions,
                  int B, int Hq, int D, int half_rot, float eps, float w_offset,
                  vm_stream stream);

/* ---- a4: knorm_rope_append! (src/kernels/qknorm_rope_append.jl:119-141)
 * K_cache :: (Dk, Ctx, Hk, B) strides (kc_st, kc_sh, kc_sb), V_cache :: (Dv,
 * Ctx, Hk, B) strides (vc_st, vc_sh, vc_sb); K_raw :: (Dk, Hk, B) strides
 * (kr_sh, kr_sb), V_raw :: (Dv, Hk, B) strides (vr_sh, vr_sb). Writes
 * norm+RoPE(k) and v into cache column positions[b] (1-based). Dk, Dv powers
 * of two from 16 to 512 (:132), 1 <= half_rot <= Dk/2; Dk = Dv = 256, half_rot
 * = 32 with K and V sharing strides runs the tuned kernel.                   */
int vm_knorm_rope_append(vm_bf16* k_cache, int64_t kc_st, int64_t kc_sh, int64_t kc_sb,
                         vm_bf16* v_cache, int64_t vc_st, int64_t vc_sh, int64_t vc_sb,
                         int64_t ctx,
                         const vm_bf16* k_raw, int64_t kr_sh, int64_t kr_sb,
                         const vm_bf16* v_raw, int64_t vr_sh, int64_t vr_sb,
                         const vm_bf16* kw, const float* cos_tab, const float* sin_tab,
                         const int32_t* positions,
                         int B, int Hk, int Dk, int Dv, int half_rot, float eps, float w_offset,
                         vm_stream stream);

/* ---- a5: decode_attention! (src/kernels/attention_decode.jl:134-200) ----
 * Split-KV flash-decoding: Q :: (Dk, H, B) (normalised + rotated), K cache ::
 * (Dk, Ctx, Hk, B) strides (k_st, k_sh, k_sb), V cache :: (Dv, Ctx, Hk, B)
 * strides (v_st, v_sh, v_sb), lengths[b] = attended keys (cache columns
 * 1..len). O :: (Dv, H, B). Dk, Dv powers of two from 16 to 512, any H / Hk.
 *
 * Dk = Dv = 256, H / Hk <= 8, K and V sharing strides and B*Ctx*Hk < 2^31
 * run the tuned stream kernel. Its work is split as a stream over all
 * token-heads sum_b lengths[b] * Hk: NW
 * waves each take one contiguous equal chunk (>= 64 keys, a multiple of 16),
 * so every CU streams the same bytes whatever the length mix. n_splits > 0
 * gives NW = n_splits * B * Hk (the reference's n_splits per (b, hk) on
 * average); n_splits = 0 gives NW = 4 waves per CU of the device. The result
 * does not depend on NW beyond fp32 rounding of the merge.
 * scratch holds one fp32 partial (G*D values + G (max, sum) pairs) per wave
 * and per (b, hk) segment, then a snapshot of the partition (1 + 2B int32
 * in whole 256-byte blocks) that the merge reads instead of lengths.
 *
 * Other shapes run a generic kernel with the reference's split: n_splits
 * tile-aligned key ranges per (b, hk) (n_splits = 0: about four workgroups
 * per CU, at least 128 keys each), partials (Dv values, max, sum) per split,
 * sequence and head, merged in split order.
 *
 * Size scratch with vm_decode_scratch_bytes(B, H, Hk, Dv, ctx, n_splits)
 * (D = Dv; 0 for an invalid shape).                                         */
size_t vm_decode_scratch_bytes(int B, int H, int Hk, int D, int64_t ctx, int n_splits);
int vm_decode_attention(vm_bf16* o, int64_t o_sh, int64_t o_sb,
                        const vm_bf16* q, int64_t q_sh, int64_t q_sb,
                        const vm_bf16* k_cache, int64_t k_st, int64_t k_sh, int64_t k_sb,
                        const vm_bf16* v_cache, int64_t v_st, int64_t v_sh, int64_t v_sb,
                        int64_t ctx, const int32_t* lengths, int B, int H, int Hk, int Dk,
                        int Dv, int n_splits, void* scratch, size_t scratch_bytes,
                        vm_stream stream);

/* ---- a6: decode gate O .*= sigmoid.(q_gate) (src/llm/qwen35.jl:205) ---- */
int vm_sigmoid_gate(vm_bf16* o, int64_t o_sh, int64_t o_sb,
                    const vm_bf16* g, int64_t g_sh, int64_t g_sb,
                    int B, int H, int D, vm_stream stream);

/* ---- a7: decode!(h, ::AttnLayer, …) attention part (src/llm/qwen35.jl:187-208)
 * qkv :: packed projection (D, 2Hq+2Hk, B), slots [q1 g1 … qHq gHq | k1…kHk |
 * v1…vHk], batch stride qkv_sb. Runs a3 (fused into the split kernel), a4,
 * a5 and a6 (fused into the merge) and writes out :: (D, Hq, B) = the Wo
 * input, batch stride out_sb. positions[b] = 1-based column of the new token
 * = attended length. If advance != 0, positions[b] += 1 on the device after
 * the step (src/llm/generate.jl:82-88), so a captured graph self-advances.  */
int vm_gated_attn_decode(vm_bf16* out, int64_t out_sb,
                         const vm_bf16* qkv, int64_t qkv_sb,
                         vm_bf16* k_cache, vm_bf16* v_cache,
                         int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                         const vm_bf16* qw, const vm_bf16* kw,
                         const float* cos_tab, const float* sin_tab,
                         int32_t* positions, int advance,
                         int B, int Hq, int Hk, int D, int half_rot,
                         float eps, float w_offset, int n_splits,
                         void* scratch, size_t scratch_bytes, vm_stream stream);

/* ---- a7 with no allocation of any kind. No counterpart in the reference: it
 * is for callers that cannot allocate or hand over a workspace (code under
 * graph capture that must not call hipMalloc, tight serving loops, harnesses
 * that forbid allocation). Same step and arguments as vm_gated_attn_decode,
 * but the workspace is a static array inside the library, one per GPU, of
 * VM_DECODE_STATIC_SCRATCH_BYTES (16 MiB, held until the process ends). A step
 * whose vm_decode_scratch_bytes(B, Hq, Hk, D, ctx, n_splits) exceeds it fails
 * with VM_E_SCRATCH. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams or threads) race; calls ordered on one
 * stream are safe. Nothing in the array has to start at zero.              */
#define VM_DECODE_STATIC_SCRATCH_BYTES ((size_t)16 << 20)
int vm_gated_attn_decode_noalloc(vm_bf16* out, int64_t out_sb,
                                 const vm_bf16* qkv, int64_t qkv_sb,
                                 vm_bf16* k_cache, vm_bf16* v_cache,
                                 int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                                 const vm_bf16* qw, const vm_bf16* kw,
                                 const float* cos_tab, const float* sin_tab,
                                 int32_t* positions, int advance,
                                 int B, int Hq, int Hk, int D, int half_rot,
                                 float eps, float w_offset, int n_splits, vm_stream stream);

/* ---- a12: advance! (src/llm/generate.jl:82-88): positions[b] += 1 ------ */
int vm_advance_positions(int32_t* positions, int B, vm_stream stream);

/* ---- a8: attention! (src/kernels/attention.jl:93-129) ------------------
 * Flash attention. Q :: (Dk, L, H, B) strides (q_st, q_sh, q_sb); K :: (Dk,
 * Lk, Hk, B) strides (k_st, k_sh, k_sb), V :: (Dv, Lk, Hk, B) strides (v_st,
 * v_sh, v_sb) (typically cache prefixes); O :: (Dv, L, H, B); scores scaled
 * by 1/sqrt(Dk). k_lengths/q_lengths (device, nullable) give ragged lengths;
 * queries are the suffix of keys, causal offset = k_len - q_len. Rows t >=
 * q_len[b] are not written. Dk, Dv powers of two from 16 to 512; Dk = Dv = 256,
 * 128 or 64 with K and V sharing strides runs the tuned MFMA kernel, other
 * shapes a generic one.                                                     */
int vm_attention_fwd(vm_bf16* o, int64_t o_st, int64_t o_sh, int64_t o_sb,
                     const vm_bf16* q, int64_t q_st, int64_t q_sh, int64_t q_sb,
                     const vm_bf16* k, int64_t k_st, int64_t k_sh, int64_t k_sb,
                     const vm_bf16* v, int64_t v_st, int64_t v_sh, int64_t v_sb,
                     const int32_t* k_lengths, const int32_t* q_lengths,
                     int B, int H, int Hk, int Dk, int Dv, int L, int Lk, int causal,
                     vm_stream stream);

/* ---- a9: prefill prologue (src/llm/qwen35.jl:293-307) ------------------
 * From the packed projection qkv :: (D, 2Hq+2Hk, T, B) (token stride qkv_st,
 * batch stride qkv_sb): norm+RoPE(k) and v of chunk token t (0-based
 * position prior[b]+t) into cache column prior[b]+t+1. prior (device,
 * nullable = all 0) is the prefix already in the cache; q_lengths (device,
 * nullable = all T) the ragged chunk lengths.                                */
int vm_prefill_kv_append(vm_bf16* k_cache, vm_bf16* v_cache,
                         int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                         const vm_bf16* qkv, int64_t qkv_st, int64_t qkv_sb,
                         const vm_bf16* kw, const float* cos_tab, const float* sin_tab,
                         const int32_t* prior, const int32_t* q_lengths,
                         int B, int T, int Hq, int Hk, int D, int half_rot,
                         float eps, float w_offset, vm_stream stream);
/* norm+RoPE(q) of the packed projection into Q :: (D, T, Hq, B) bf16 with
 * strides (q_st, q_sh, q_sb) — the unfused prologue, for attention!.         */
int vm_prefill_q_norm_rope(vm_bf16* q_out, int64_t q_st, int64_t q_sh, int64_t q_sb,
                           const vm_bf16* qkv, int64_t qkv_st, int64_t qkv_sb,
                           const vm_bf16* qw, const float* cos_tab, const float* sin_tab,
                           const int32_t* prior, const int32_t* q_lengths,
                           int B, int T, int Hq, int Hk, int D, int half_rot,
                           float eps, float w_offset, vm_stream stream);

/* ---- a11: forward(::AttnLayer, …; offset) attention part
 * (src/llm/qwen35.jl:292-318): one kernel appends the chunk's K/V to the
 * cache (a9) and stages the attended V transposed in scratch, then one flash-
 * attention kernel whose prologue norms+rotates q from qkv and whose
 * epilogue applies the sigmoid gate (a10) and writes out :: (D*Hq, T, B) —
 * the Wo input layout, token stride out_st, batch stride out_sb.
 * Attends cache columns 1..prior[b]+q_len[b] of each sequence (prior NULL:
 * no prior tokens). Contract: prior[b] + q_len[b] <= ctx (the reference's
 * cache view throws a BoundsError past it, src/llm/qwen35.jl:306); device-side
 * values are not read on the host, so keys past ctx are masked instead. scratch (device, 256-byte aligned) is a workspace of at
 * least vm_prefill_scratch_bytes(B, Hk, D, ctx) bytes: the attended V is staged
 * there transposed for the attention kernel. Its contents are not preserved
 * (the role of the reference's arena scratch, attention_decode.jl:183-200).  */
size_t vm_prefill_scratch_bytes(int B, int Hk, int D, int64_t ctx);
int vm_gated_attn_prefill(vm_bf16* out, int64_t out_st, int64_t out_sb,
                          const vm_bf16* qkv, int64_t qkv_st, int64_t qkv_sb,
                          vm_bf16* k_cache, vm_bf16* v_cache,
                          int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                          const vm_bf16* qw, const vm_bf16* kw,
                          const float* cos_tab, const float* sin_tab,
                          const int32_t* prior, const int32_t* q_lengths,
                          int B, int T, int Hq, int Hk, int D, int half_rot,
                          float eps, float w_offset, void* scratch, size_t scratch_bytes,
                          vm_stream stream);
/* vm_gated_attn_prefill for a prefill run as successive chunks (the same
 * forward(::AttnLayer, …; offset) of src/llm/qwen35.jl:292-318, called chunk
 * after chunk): `vt` (device, 256-byte aligned, at least
 * vm_prefill_scratch_bytes(B, Hk, D, ctx) bytes) persists between the calls of
 * one layer and holds the V^T tiles of the rows staged so far; vt_rows (device
 * int32[2B], zeroed before the first call) holds in [b] how many leading cache
 * rows of sequence b those are, and in [B + b] a counter the library uses
 * during a call and leaves zero. A call
 * stages only rows min(vt_rows[b], prior[b]) .. prior[b]+q_len[b]-1 (the chunk,
 * and any rows written since, such as decode steps' appends), so its cost
 * scales with the chunk, not with the prior; it then sets vt_rows[b] =
 * min(prior[b] + q_len[b], ctx). The caller zeroes vt_rows[b] (or lowers it
 * to the rows it knows unchanged) for a new sequence in slot b and
 * whenever it writes V cache rows below vt_rows[b] by other means (a copied
 * prefix, for example). Outputs equal vm_gated_attn_prefill's bit for bit.
 * No counterpart in the reference, which keeps no transposed V.              */
int vm_gated_attn_prefill_staged(vm_bf16* out, int64_t out_st, int64_t out_sb,
                                 const vm_bf16* qkv, int64_t qkv_st, int64_t qkv_sb,
                                 vm_bf16* k_cache, vm_bf16* v_cache,
                                 int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                                 const vm_bf16* qw, const vm_bf16* kw,
                                 const float* cos_tab, const float* sin_tab,
                                 const int32_t* prior, const int32_t* q_lengths,
                                 int B, int T, int Hq, int Hk, int D, int half_rot,
                                 float eps, float w_offset, int32_t* vt_rows,
                                 void* vt, size_t vt_bytes, vm_stream stream);

/* ---- f1: linear!((; y), x, W) (src/linear.jl:40-57): y = W^T x ------------
 * The qkv projection in front of the block and the Wo projection after it
 * (src/llm/qwen35.jl:194, :206, :296, :316-317). Column-major, as the
 * reference: x :: (K, N) with column stride ldx >= K, W :: (K, M) (K-major,
 * the checkpoint's orientation) with column stride ldw >= K, y :: (M, N) with
 * column stride ldy >= M; all bf16, fp32 accumulation (linear.jl:29). Narrow
 * problems (N <= 16, or N <= 32 with M <= 4096; K % 64 == 0, M % 4 == 0,
 * 16-byte aligned W and x columns)
 * run on the library's split-K MFMA GEMV, whose K slices add in a fixed order
 * (bitwise reproducible); the rest on hipBLASLt. A plan per
 * problem (hipBLASLt) is built on the first call and cached (linear.jl:17-38)
 * with the heuristic's first algorithm, as the reference takes it: building it
 * is host work only, so the first call of a shape may run inside a capture;
 * vm_linear_workspace_bytes builds it and returns the workspace it needs (at
 * most 64 MiB), which the caller passes to vm_linear (the reference takes it
 * from the ambient arena, linear.jl:62-66). Returns (size_t)-1 on failure.
 * The role of the reference's mul! fallback (linear.jl:59-61, :67) is the
 * library's general bf16 MFMA GEMM (any shape, 2-byte alignment, no
 * workspace): it takes a problem hipBLASLt has no algorithm for, views whose
 * column strides are not multiples of 8 (outside the GEMV's reach) or whose
 * pointers are not 16-byte aligned, and calls hipBLASLt refuses.          */
size_t vm_linear_workspace_bytes(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy);
/* vm_linear_tune: no counterpart in the reference (its plan keeps the
 * heuristic's first). For callers that load a model and then run it: times up
 * to 48 of the heuristic's candidates for the problem's plan and keeps the
 * fastest (on MI355X the first can be a third slower). The exception to the
 * conventions above: it allocates scratch buffers (up to ~800 MB for the
 * timing of a narrow problem's weights), runs the timing on a private stream
 * and waits for it, so it must not be called while the device is captured.
 * Call it at load, before vm_linear_workspace_bytes (a tuned plan may need a
 * larger workspace); once per problem (later calls return at once).
 * VM_LINEAR_TUNE=0 in the environment keeps the first. Narrow problems that
 * run the GEMV have nothing to tune.
 * vm_linear_plan_state: -2 no plan, -1 the heuristic's first, k >= 0 tuned
 * (candidate k kept, 0 = the heuristic's first).                              */
int vm_linear_tune(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy);
int vm_linear_plan_state(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy);
int vm_linear(vm_bf16* y, int64_t ldy, const vm_bf16* x, int64_t ldx, const vm_bf16* w,
              int64_t ldw, int M, int N, int K, void* workspace, size_t workspace_bytes,
              vm_stream stream);

/* ---- linear! + fused_add_rms_norm! in one call ---------------------------
 * No counterpart in the reference: its decode step runs linear! into a bf16 h
 * and then fused_add_rms_norm! on it, after every out projection and MLP
 * (src/llm/qwen35.jl:206 + :265, :241 + :268). This does exactly that in one
 * call, for callers that want the launches saved:
 *   h = bf16(W^T a)          (linear!, a :: (K, N), W :: (K, M) K-major)
 *   x = bf16(x + h)          in place (X' = X, residual_norm.jl:39-60)
 *   y = x rstd (w + offset)  rstd over the fp32 x + h, y from the stored x
 * bit-identical to the two calls. A narrow problem whose GEMV splits K hands
 * its fp32 slices straight to the norm, which adds them in slice order (no
 * reduce launch, no h in HBM). M a multiple of 8, at most 16384; workspace
 * (256-byte aligned) of vm_linear_add_rms_norm_workspace_bytes bytes
 * ((size_t)-1 on a bad shape).                                              */
size_t vm_linear_add_rms_norm_workspace_bytes(int M, int N, int K, int64_t ldw, int64_t lda);
int vm_linear_add_rms_norm(vm_bf16* y, int64_t y_st, vm_bf16* x, int64_t x_st, const vm_bf16* a,
                           int64_t lda, const vm_bf16* w, int64_t ldw, const vm_bf16* norm_w,
                           int M, int N, int K, float eps, float offset, void* workspace,
                           size_t workspace_bytes, vm_stream stream);

/* ---- linear! + silu .* mul in one call --------------------------------
 * No counterpart in the reference as one op: its MLP runs linear! into the
 * packed bf16 gate-up projection gu and then silu .* mul on it
 * (src/llm/qwen35.jl:234-243, :249-250 in step!). This does both:
 *   gu  = W^T x               (W :: (K, 2I) K-major, gate rows 0 .. I-1, up
 *                              rows I .. 2I-1; x :: (K, N)), rounded to bf16
 *   mid = silu(gate) .* up    fp32 from the bf16 gate and up, one rounding
 * for callers that want the bf16 gu never written. At N <= 32 (a decode
 * batch; K a multiple of 64, aligned columns) the projection runs a stream-K
 * GEMV whose fp32 partials the silu kernel adds in a fixed order (bitwise
 * repeatable; the same rounding points as the two calls, the sums in another
 * order). Otherwise it is linear! + silu .* mul. I a multiple of 8; mid a
 * 16-byte aligned (I, N) with an element column stride (a multiple of 8);
 * workspace (256-byte aligned) of vm_linear_silu_mul_workspace_bytes bytes
 * ((size_t)-1 on a bad shape).                                              */
size_t vm_linear_silu_mul_workspace_bytes(int I, int N, int K, int64_t ldw, int64_t ldx);
int vm_linear_silu_mul(vm_bf16* mid, int64_t mid_st, const vm_bf16* x, int64_t ldx,
                       const vm_bf16* w, int64_t ldw, int I, int N, int K, void* workspace,
                       size_t workspace_bytes, vm_stream stream);

/* ---- linear! + causal_conv1d! in one call -------------------------------
 * No counterpart in the reference as one op: the DeltaNet layer's decode step
 * runs linear! into its packed projection [q k v | z | alpha beta] and then
 * causal_conv1d! on the first D channels (src/llm/qwen35.jl:212-223). This does
 * both:
 *   y = bf16(W^T x)   W :: (K, M) K-major, x :: (K, N), y :: (M, N) (every
 *                     channel written, as linear! leaves it)
 *   causal_conv1d!((; Y, S'), y[1:D, :], S, Weight, Bias; sigma) as
 *                     vm_causal_conv1d (yc = Y, s_in/s_out = S/S', the ring
 *                     strides, conv_w = Weight, conv_b = Bias or NULL, Kc its
 *                     kernel size, act = 1 for silu)
 * At N <= 32 (a decode batch; K a multiple of 64, aligned columns) the
 * projection runs a stream-K GEMV whose fp32 partials the conv kernel adds in a
 * fixed order (bitwise repeatable; the same rounding points as the two calls,
 * the sums in another order); otherwise it is linear! + causal_conv1d!. M and
 * D multiples of 8, D <= M; workspace (256-byte aligned) of
 * vm_linear_causal_conv1d_workspace_bytes bytes ((size_t)-1 on a bad shape). */
size_t vm_linear_causal_conv1d_workspace_bytes(int M, int N, int K, int64_t ldw, int64_t ldx,
                                               int64_t ldy);
int vm_linear_causal_conv1d(vm_bf16* y, int64_t ldy, const vm_bf16* x, int64_t ldx,
                            const vm_bf16* w, int64_t ldw, int M, int N, int K, vm_bf16* yc,
                            int64_t yc_sb, const vm_bf16* s_in, vm_bf16* s_out, int64_t s_cs,
                            int64_t s_sb, const vm_bf16* conv_w, int64_t conv_w_cs,
                            const vm_bf16* conv_b, int D, int Kc, int act, void* workspace,
                            size_t workspace_bytes, vm_stream stream);

/* decode!(h, ::DeltaNetLayer, ...) through its recurrence in one call
 * (src/llm/qwen35.jl:212-232 without the out projection): linear! of the
 * projection W (K, M) K-major over x (K, B) into [q | k | v | z | alpha |
 * beta] (M = 2 Hk Dk + 2 Hv Dv + 2 Hv rows), causal_conv1d! of its q | k | v
 * channels on the ring (sigma = silu) and fused_deltanet_decode! into O
 * (Dv, Hv, B) (sequence stride o_sb) and the state: the results of
 * vm_linear_causal_conv1d (act = 1) followed by vm_fused_deltanet_decode on
 * its outputs, bit for bit. At B <= 32 with 16-byte aligned x and W and Hv /
 * Hk in {1, 2, 4} the projection's stream-K partials go straight to one
 * kernel per (qk head, sequence) and y (ldy) and yc (the conv output,
 * yc_sb) are not written; otherwise the two calls run, through y and yc.
 * workspace: vm_linear_causal_conv1d_workspace_bytes(M, B, K, ldw, ldx, ldy). */
int vm_linear_deltanet_decode(vm_bf16* o, int64_t o_sb, vm_bf16* y, int64_t ldy, vm_bf16* yc,
                              int64_t yc_sb, const vm_bf16* x, int64_t ldx, const vm_bf16* w,
                              int64_t ldw, int M, int K, const vm_bf16* ring_in, vm_bf16* ring_out,
                              int64_t s_cs, int64_t s_sb, const vm_bf16* conv_w,
                              int64_t conv_w_cs, const vm_bf16* conv_b, int Kc, const float* a_log,
                              const float* dt_bias, const vm_bf16* norm_w, const float* s_in,
                              float* s_out, int Dk, int Dv, int Hk, int Hv, int B, float eps,
                              void* workspace, size_t workspace_bytes, vm_stream stream);

/* ---- f2: the rest of the decode step (src/llm/qwen35.jl:247-273) --------
 * Matrices are column-major bf16 with an element column stride (a multiple of
 * 8, pointers 16-byte aligned); M, I, D, K multiples of 8.
 *
 * rms_norm! (src/kernels/rms_norm.jl:38-50): Y[:, n] = X[:, n] * rstd_n *
 * (w + offset), rstd_n = 1 / sqrt(sum(X[:, n]^2) / M + eps), fp32, one bf16
 * rounding. M <= 16384 rows, N columns.                                      */
int vm_rms_norm(vm_bf16* y, int64_t y_st, const vm_bf16* x, int64_t x_st, const vm_bf16* w,
                int M, int N, float eps, float offset, vm_stream stream);
/* fused_add_rms_norm! (src/kernels/residual_norm.jl:43-60): X' = bf16(X + dX)
 * (xo may be x: the reference's in-place (; X' = x) use, qwen35.jl:265), Y =
 * rms_norm of X' -- rstd from the fp32 sum, applied to the rounded X', as the
 * reference's second pass reloads it.                                         */
int vm_fused_add_rms_norm(vm_bf16* y, int64_t y_st, vm_bf16* xo, int64_t xo_st, const vm_bf16* x,
                          int64_t x_st, const vm_bf16* dx, int64_t dx_st, const vm_bf16* w, int M,
                          int N, float eps, float offset, vm_stream stream);
/* The MLP's mid = silu(gate) .* up (src/llm/qwen35.jl:234-243): gate and up are
 * rows 0..I-1 and I..2I-1 of each column of gu (the packed gate-up projection);
 * mid (I, N). fp32, one rounding.                                            */
int vm_silu_mul(vm_bf16* mid, int64_t mid_st, const vm_bf16* gu, int64_t gu_st, int I, int N,
                vm_stream stream);
/* x[:, b] = E[:, ids[b]] (src/llm/qwen35.jl:251), ids 1-based (an id outside
 * 1..vocab reads the nearest valid column). E (D, vocab), column stride e_st. */
int vm_embed(vm_bf16* x, int64_t x_st, const vm_bf16* e, int64_t e_st, const int32_t* ids, int D,
             int B, int vocab, vm_stream stream);
/* advance!(gen) (src/llm/generate.jl:82-88), the engine's clock on the device:
 * tokens_out[step, b] = result[b] (column-major (max_new, B), column b at
 * col_offsets[b]; nothing harvested when step is outside 1..max_new), then
 * step += 1 and positions[b] += 1. One kernel: capturable.                   */
int vm_generation_advance(int32_t* tokens_out, const int32_t* col_offsets, int32_t* step,
                          int32_t* positions, const int32_t* result, int B, int max_new,
                          vm_stream stream);

/* ---- f3: lm_head_argmax! (src/kernels/lm_head_topk.jl:109-147) ----------
 * Result[b] = argmax_v W[:, v] . X[:, b], 1-based, ties to the smallest v;
 * bf16 products, fp32 sums; the logits are never written. X (K, B), W (K, N)
 * K-major (the embedding's own orientation, so a tied head needs no copy).
 * K a multiple of 64. scratch: vm_lm_head_argmax_scratch_bytes(K, N, B) bytes
 * of device memory (per-wave partials; the reference's LocalMax / LocalIdx),
 * 16-byte aligned.                                                           */
size_t vm_lm_head_argmax_scratch_bytes(int K, int N, int B);
int vm_lm_head_argmax(int32_t* result, const vm_bf16* x, int64_t x_st, const vm_bf16* w,
                      int64_t w_st, int K, int N, int B, void* scratch, size_t scratch_bytes,
                      vm_stream stream);

/* ---- f4: the linear-attention layer parts (3 of every 4 Qwen3.5 layers,
 * src/llm/gguf_llamacpp.jl:47) -------------------------------------------
 * Column-major as the reference; element strides. All kernels run Dk = Dv =
 * 128 (Qwen3.5, src/llm/qwen35.jl:19); other head sizes are VM_E_UNSUPPORTED.
 * Hv % Hk != 0 is VM_E_DIM (deltanet_fused.jl:128-129). States may be updated
 * in place (S_out == S, the reference's output_override at qwen35.jl:223,
 * :229, :358) or written to a disjoint buffer; a partial overlap is VM_E_ARG. */

/* causal_conv1d!((; Y, S'), X, S, Weight, Bias; sigma) — one decode step
 * (src/kernels/causal_conv1d.jl:43-61, kernel :7-41): the ring S (D, K, B)
 * (column stride s_cs, sequence stride s_sb) shifts one column left, X (D, B)
 * enters as column K, Y (D, B) = sum_i S'[:, i] .* Weight[:, i] (+ Bias)
 * (silu when act != 0, the call site's sigma = silu, qwen35.jl:222-223).
 * Weight (D, K) column stride w_cs; Bias (D,) or NULL. bf16; D % 8 == 0,
 * 16-byte aligned rows, 1 <= K <= 8. */
int vm_causal_conv1d(vm_bf16* y, int64_t y_sb, const vm_bf16* x, int64_t x_sb,
                     const vm_bf16* s_in, vm_bf16* s_out, int64_t s_cs, int64_t s_sb,
                     const vm_bf16* w, int64_t w_cs, const vm_bf16* bias, int D, int K, int B,
                     int act, vm_stream stream);

/* causal_conv1d_sequence!((; Y), X, Weight, Bias; sigma, S') (causal_conv1d.jl:
 * 130-149, kernel :73-128): X, Y (D, T, B) with token / sequence strides;
 * Y[:, t] = sum_k Weight[:, k] X[:, t - K + k] with the left context zeros
 * (s_in NULL) or the ring's columns 2..K (s_in: a prefix's ring, the suffix
 * prefill of qwen35.jl:333-344, done here without the copy). s_out (NULL:
 * none) receives the ring a decode step continues from: the last K inputs of
 * the context-extended sequence, zeros where it is shorter. */
int vm_causal_conv1d_sequence(vm_bf16* y, int64_t y_st, int64_t y_sb, const vm_bf16* x,
                              int64_t x_st, int64_t x_sb, const vm_bf16* w, int64_t w_cs,
                              const vm_bf16* bias, const vm_bf16* s_in, vm_bf16* s_out,
                              int64_t s_cs, int64_t s_sb, int D, int K, int T, int B, int act,
                              vm_stream stream);

/* fused_deltanet_decode!((; O, S'), Q_raw, K_raw, V, Alpha, BetaRaw, Z, A_log,
 * DtBias, NormWeight, S; eps) (src/kernels/deltanet_fused.jl:109-141, kernel
 * :27-107): l2-normed q (also / sqrt(Dk)) and k of the shared qk head
 * h_v / (Hv / Hk), decay = exp(-exp(A_log) softplus(Alpha + DtBias)), beta =
 * sigmoid(BetaRaw), the delta-rule step on S (Dk, Dv, Hv, B) fp32, then
 * O = o rstd NormWeight silu(Z). Q_raw, K_raw (Dk, Hk, B), V, Z, O (Dv, Hv, B),
 * Alpha, BetaRaw (Hv, B): bf16, heads contiguous, per-sequence strides *_sb
 * (Q_raw, K_raw 8-byte aligned); A_log, DtBias (Hv,) fp32; NormWeight (Dv,)
 * bf16; S, S_out 16-byte aligned. */
int vm_fused_deltanet_decode(vm_bf16* o, int64_t o_sb, const vm_bf16* q, int64_t q_sb,
                             const vm_bf16* k, int64_t k_sb, const vm_bf16* v, int64_t v_sb,
                             const vm_bf16* alpha, int64_t a_sb, const vm_bf16* beta_raw,
                             int64_t b_sb, const vm_bf16* z, int64_t z_sb, const float* a_log,
                             const float* dt_bias, const vm_bf16* norm_w, const float* s_in,
                             float* s_out, int Dk, int Dv, int Hk, int Hv, int B, float eps,
                             vm_stream stream);

/* deltanet_recurrent_decode!((; O, S'), Q, K, V, Beta, Gate, S)
 * (src/kernels/deltanet_recurrent.jl:72-95, kernel :15-70), fp32 throughout:
 * Q, K (Dk, Hk, B), V, O (Dv, Hv, B), Beta, Gate (Hv, B) (decay = exp(Gate)),
 * S (Dk, Dv, Hv, B); contiguous, 16-byte aligned. */
int vm_deltanet_recurrent_decode(float* o, const float* q, const float* k, const float* v,
                                 const float* beta, const float* gate, const float* s_in,
                                 float* s_out, int Dk, int Dv, int Hk, int Hv, int B,
                                 vm_stream stream);

/* deltanet_sequence!((; O, S'), Q, K, V, Beta, Gate, S) (deltanet_recurrent.jl:
 * 174-198, kernel :109-172): T steps in order, fp32. Q, K (Dk, T, Hk, B),
 * V, O (Dv, T, Hv, B), Beta, Gate (Hv, T, B), S (Dk, Dv, Hv, B). T = 0 copies
 * the state through. */
int vm_deltanet_sequence(float* o, const float* q, const float* k, const float* v,
                         const float* beta, const float* gate, const float* s_in, float* s_out,
                         int Dk, int Dv, int T, int Hk, int Hv, int B, vm_stream stream);

/* deltanet_sequence! in its chunked form: the same arguments and results
 * (within 5e-4 of the sequential fp32 result, the tests' bar), computed per
 * 64-token chunk as a lower-triangular solve and matrix products (delta = U -
 * W S_0, O = gamma Q S_0 + M delta, S_C = gamma_C S_0 + K~^T delta: the
 * sequential recurrence's exact algebra) on the bf16 MFMA in split precision
 * (each fp32 operand as bf16 hi + lo, products hi hi + hi lo + lo hi, fp32
 * accumulation and state), the chunks' state carried by one sequential scan. No separate reference
 * function: the reference runs the sequential loop (deltanet_recurrent.jl:
 * 109-172); this is the same operator, parallel over each chunk: a chunk
 * kernel, one sequential scan over the chunks' states, and a chunk-parallel
 * output kernel. workspace: vm_deltanet_sequence_workspace_bytes(T, Hv, B)
 * bytes, 256-byte aligned (about 197 KB per 64-token chunk per value head
 * and sequence). */
size_t vm_deltanet_sequence_workspace_bytes(int T, int Hv, int B);
int vm_deltanet_sequence_chunked(float* o, const float* q, const float* k, const float* v,
                                 const float* beta, const float* gate, const float* s_in,
                                 float* s_out, int Dk, int Dv, int T, int Hk, int Hv, int B,
                                 void* workspace, size_t workspace_bytes, vm_stream stream);

/* forward(::DeltaNetLayer)'s recurrence and gated norm in one call
 * (src/llm/qwen35.jl:357-364: deltanet_sequence! into O, then y = O rstd
 * NormWeight silu(z), the out projection's input): the chunked recurrence of
 * vm_deltanet_sequence_chunked with the norm applied in its output kernel,
 * so O never reaches memory. y, z :: (Dv, Hv, T, B) bf16 rows at token
 * stride *_st and sequence stride *_sb (heads contiguous), as
 * vm_gated_rms_norm; the state and workspace as vm_deltanet_sequence_chunked. */
int vm_deltanet_sequence_chunked_gated_norm(vm_bf16* y, int64_t y_st, int64_t y_sb,
                                            const vm_bf16* z, int64_t z_st, int64_t z_sb,
                                            const vm_bf16* norm_w, float eps, const float* q,
                                            const float* k, const float* v, const float* beta,
                                            const float* gate, const float* s_in, float* s_out,
                                            int Dk, int Dv, int T, int Hk, int Hv, int B,
                                            void* workspace, size_t workspace_bytes,
                                            vm_stream stream);

/* The prefill's inputs to deltanet_sequence! (forward(::DeltaNetLayer),
 * src/llm/qwen35.jl:347-356): from the conv output cv (the q | k | v channels,
 * n = 2 Hk Dk + Hv Dv rows per token, token stride cv_st, sequence stride
 * cv_sb) and the alpha | beta projection ab (2 Hv rows, ab_st, ab_sb), bf16:
 * qe, ke (Dk, T, Hk, B) = l2n(q) / sqrt(Dk), l2n(k); ve (Dv, T, Hv, B);
 * beta = sigmoid(b), gate = -exp(A_log) softplus(a + DtBias) (Hv, T, B). fp32
 * outputs, contiguous. */
int vm_deltanet_prefill_prep(float* qe, float* ke, float* ve, float* beta, float* gate,
                             const vm_bf16* cv, int64_t cv_st, int64_t cv_sb, const vm_bf16* ab,
                             int64_t ab_st, int64_t ab_sb, const float* a_log,
                             const float* dt_bias, int Dk, int Dv, int Hk, int Hv, int T, int B,
                             vm_stream stream);

/* forward(::DeltaNetLayer)'s sequence conv and prep in one pass
 * (src/llm/qwen35.jl:333-356: causal_conv1d_sequence! with sigma = silu, then
 * the l2 norms and gates): x the projection's q | k | v channels (n = 2 Hk Dk
 * + Hv Dv rows per token, x_st, x_sb), the conv weight, bias and ring as
 * vm_causal_conv1d_sequence (s_in NULL: zero left context; s_out NULL: no
 * ring written), ab and the outputs as vm_deltanet_prefill_prep. The results
 * are bit for bit those of vm_causal_conv1d_sequence (act = 1) followed by
 * vm_deltanet_prefill_prep: the conv output is rounded to bf16 in registers
 * and never written. 16-byte aligned rows (x, weight, bias, ring, the fp32
 * outputs) with strides of whole 8-element chunks. */
int vm_deltanet_conv_prep(float* qe, float* ke, float* ve, float* beta, float* gate,
                          const vm_bf16* x, int64_t x_st, int64_t x_sb, const vm_bf16* w,
                          int64_t w_cs, const vm_bf16* bias, const vm_bf16* s_in, vm_bf16* s_out,
                          int64_t s_cs, int64_t s_sb, int K, const vm_bf16* ab, int64_t ab_st,
                          int64_t ab_sb, const float* a_log, const float* dt_bias, int Dk, int Dv,
                          int Hk, int Hv, int T, int B, vm_stream stream);

/* The prefill's gated RMSNorm + z gate (qwen35.jl:360-364): o (Dv, T, Hv, B)
 * fp32 and z (Dv, Hv) rows of each token (token stride z_st, sequence stride
 * z_sb, bf16) -> y = o rstd NormWeight silu(z), bf16, (Dv, Hv) rows at y_st /
 * y_sb: the out projection's input (Dv Hv, T B) (qwen35.jl:365). */
int vm_gated_rms_norm(vm_bf16* y, int64_t y_st, int64_t y_sb, const float* o, const vm_bf16* z,
                      int64_t z_st, int64_t z_sb, const vm_bf16* norm_w, int Dv, int Hv, int T,
                      int B, float eps, vm_stream stream);

/* ---- synthetic inputs for tests and benchmarks (not a reference op) ----
 * Fills n bf16 values with the seeded N(0,1) stream used by the CPU oracle
 * (SplitMix64 -> Box-Muller in f64 -> f32 -> bf16 RNE), element i of stream
 * `seed` scaled by `scale` and shifted by `shift` before rounding.           */
int vm_fill_normal_bf16(vm_bf16* dst, int64_t n, uint64_t seed,
                        float scale, float shift, vm_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* VALLMO_ATTN_H */

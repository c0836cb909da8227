// kernels.h — argument blocks and launchers shared between the kernel sources
// and the C-ABI layer (vallmo_attn.cpp). Strides are in elements.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vallmo_attn.h"

namespace vm {

constexpr int HEAD_DIM_ABI = 256;     // compiled head_dim
constexpr int HALF_ROT_ABI = 32;      // compiled rotary half-width
constexpr int PREFILL_ROWS_ABI = 128; // query rows per prefill workgroup

struct RowArgs {
  const uint16_t* in;   // first tensor: normed + rotated
  const uint16_t* in2;  // optional second tensor (V): copied verbatim
  int64_t in_st, in_sh, in_sb;
  uint16_t* out;
  uint16_t* out2;
  int64_t out_st, out_sh, out_sb;
  const uint16_t* w;    // per-head norm weight (D,), applied as (w + w_offset)
  const float* cos_tab;
  const float* sin_tab;
  int64_t ctx;          // columns of the tables (and of the cache when appending)
  const int32_t* positions;  // decode: 1-based column per sequence (T must be 1)
  const int32_t* prior;      // prefill: tokens already in the cache (nullable)
  const int32_t* q_lengths;  // prefill: ragged chunk lengths (nullable)
  int B, H, T;
  int out_at_pos;       // 1: token index of the output row = position
  float eps, w_offset;
};

// ---- generic.hip: the operators at head shapes outside the tuned kernels
// (power-of-two head dims 16..512, Dk != Dv, any rotary half-width, any group)
struct RowAnyArgs {
  const uint16_t* in;  // rows normed + rotated (Q in place, or raw K)
  int64_t in_sh, in_sb;
  uint16_t* out;
  int64_t out_st, out_sh, out_sb;  // out_st: the cache's token stride (append)
  const uint16_t* in2;             // optional V rows, copied (D2 wide)
  int64_t in2_sh, in2_sb;
  uint16_t* out2;
  int64_t out2_st, out2_sh, out2_sb;
  const uint16_t* w;  // norm weight (D,), applied as (w + w_offset)
  const float* cos_tab;
  const float* sin_tab;
  int64_t ctx;
  const int32_t* positions;  // 1-based column per sequence
  int B, H, D, D2, half;
  int out_at_pos;  // 1: the output row is the cache column positions[b] - 1
  float eps, w_offset;
};
hipError_t launch_norm_rope_any(const RowAnyArgs& a, hipStream_t st);
struct AttnAnyArgs {
  const uint16_t* q;
  int64_t q_st, q_sh, q_sb;
  const uint16_t* k;
  int64_t k_st, k_sh, k_sb;
  const uint16_t* v;
  int64_t v_st, v_sh, v_sb;
  uint16_t* o;
  int64_t o_st, o_sh, o_sb;
  const int32_t* k_lengths;  // nullable
  const int32_t* q_lengths;  // nullable
  float* part;  // decode: n_split x B x H partial rows of Dv + 2 floats, merged; NULL: O direct
  int B, H, Hk, Dk, Dv, L, Lk, causal, n_split, split_keys;
  float scale;
};
int attn_any_splits(int B, int H, int Hk, int64_t ctx, int n_splits);
int attn_any_split_keys(int64_t ctx, int n_split);
hipError_t launch_attn_any(const AttnAnyArgs& a, hipStream_t st);

struct DecodeArgs {
  const uint16_t* q;    // raw q (fused) or normalised q
  int64_t q_sh, q_sb;
  const uint16_t* qw;   // fused prologue only
  const uint16_t* kw;   // fused: bounds |k| for the static softmax shift
  const float* cos_tab;
  const float* sin_tab;
  float eps, w_offset;
  uint16_t* kc;          // written only at the appended row (fused, k_new set)
  uint16_t* vc;
  int64_t c_st, c_sh, c_sb, ctx;
  const int32_t* lengths;
  // fused only (nullable): raw k / v of the new token, (D, Hk, B) with strides
  // (new_sh, new_sb); normed + rotated k and v go to cache row lengths[b]-1
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t new_sh, new_sb;
  float* part_o;        // [slots][G][256], slots = NW + B*Hk
  float* part_ml;       // [slots][G][2]  (shift m in log2 units, sum l)
  int B, Hk, G;
  int NW;               // waves of the stream partition (multiple of 4)
  int min_chunk;        // smallest per-wave chunk (token-heads, multiple of 16)
  int32_t* geom;        // partition snapshot for the merge: [chunk | len_b (B) | start_b (B)]
};

struct CombineArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* geom;   // written by the stream kernel (the merge never reads lengths)
  uint16_t* out;
  int64_t o_sh, o_sb;
  const uint16_t* gate;  // nullable: sigmoid gate logits
  int64_t g_sh, g_sb;
  int B, Hk, G;
  int NW;                // waves of the stream partition (chooses the merge shape)
  int32_t* advance;      // nullable: positions[b] += 1 (no other merge thread reads them)
};

struct PrefillArgs {
  // q: normalised (attention! operator) or the raw packed projection (fused path)
  const uint16_t* q;
  int64_t q_st, q_sh, q_sb;
  const uint16_t* qw;   // fused path: q norm weight
  const uint16_t* kw;   // fused path: bounds |k| for the static softmax shift
  const float* cos_tab;
  const float* sin_tab;
  float eps, w_offset;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_st, kv_sh, kv_sb;
  uint16_t* o;
  int64_t o_st, o_sh, o_sb;
  const uint16_t* gate;   // fused path: sigmoid gate logits
  int64_t g_st, g_sh, g_sb;
  const int32_t* k_lengths;  // nullable -> Lk
  const int32_t* q_lengths;  // nullable -> L
  const int32_t* prior;      // fused path: k_len = prior + q_len (nullable -> 0)
  int B, H, Hk, L, Lk, n_qt, causal;
  int D;                     // attention! operator: head dim 64, 128 or 256 (0: 256)
  const uint16_t* vt;        // fused path: V^T tiles of the attended keys (workspace)
  int vt_tiles;              // tiles per (b, hk) in the workspace: ceil(Lk / 32)
  int pairs;                 // fused path, set by the launcher: one heavy + one light item per workgroup
};

// V cache -> V^T tiles for the fused prefill (one 16-KB tile per 32 keys)
struct VtArgs {
  uint16_t* v;               // V cache (read; written for the chunk's keys when fused)
  int64_t v_st, v_sh, v_sb;  // cache strides (the K cache shares them)
  uint16_t* vt;
  int vt_tiles;
  const int32_t* prior;      // nullable -> 0
  const int32_t* q_lengths;  // nullable -> L
  // nullable, int32[2B]: [b] = leading V rows of sequence b that vt already
  // holds from earlier calls (rows below min(vt_rows[b], prior[b]) are not
  // staged again; set to k_len at the end), [B + b] = an arrival counter that
  // is zero between calls
  int32_t* vt_rows;
  int B, Hk, L;
  int64_t ctx;
  // fused cache append (k_raw != nullptr): the chunk's K rows are normed,
  // rotated and written to kc, its V rows copied to the V cache, and the V^T
  // tiles of the chunk's keys are built from those same rows
  uint16_t* kc;
  const uint16_t* k_raw;
  const uint16_t* v_raw;
  int64_t raw_st, raw_sh, raw_sb;
  const uint16_t* kw;
  const float* cos_tab;
  const float* sin_tab;
  float eps, w_offset;
};
constexpr int PREFILL_VT_TILE_KEYS = 32;
constexpr int64_t PREFILL_VT_TILE_BYTES = 32 * 256 * 2;

hipError_t launch_rope_tables(float* c, float* s, int half, int64_t ctx, double theta,
                              hipStream_t st);
hipError_t launch_norm_rope_rows(const RowArgs& a, hipStream_t st);
hipError_t launch_sigmoid_gate(uint16_t* o, int64_t o_sh, int64_t o_sb, const uint16_t* g,
                               int64_t g_sh, int64_t g_sb, int B, int H, hipStream_t st);
hipError_t launch_advance(int32_t* positions, int B, hipStream_t st);
hipError_t launch_fill_normal(uint16_t* dst, int64_t n, uint64_t seed, float scale, float shift,
                              hipStream_t st);
hipError_t launch_decode(const DecodeArgs& a, bool fused_q, hipStream_t st);
hipError_t launch_combine(const CombineArgs& a, hipStream_t st);
hipError_t launch_prefill(const PrefillArgs& a, hipStream_t st);
// fused gated prefill (q norm+RoPE prologue, sigmoid-gate epilogue), persistent
// t0 / t1 (nullable): events stamped by the dispatch itself at the kernel's
// start and end (hipExtLaunchKernelGGL), for timing without extra packets
hipError_t launch_prefill_fused(const PrefillArgs& a, hipStream_t st, hipEvent_t t0 = nullptr,
                                hipEvent_t t1 = nullptr);
hipError_t launch_vt_transpose(const VtArgs& a, hipStream_t st);

// Static per-GPU workspace of the no-allocation decode entry point: the largest
// decode scratch it serves (vm_decode_scratch_bytes), and its device address on
// the current GPU (looked up once per GPU, then cached).
constexpr size_t DECODE_STATIC_SCRATCH_BYTES = VM_DECODE_STATIC_SCRATCH_BYTES;
hipError_t decode_static_scratch(void** ptr);

// Projections y = W^T x on hipBLASLt (linear.cpp): plan workspace size, and the
// product on `st`. Return VM_OK, a VM_E_* code or a hipError_t, with the message
// in err.
constexpr size_t LINEAR_MAX_WORKSPACE_BYTES = (size_t)64 << 20;
// the one linear call that allocates (scratch) and synchronises: times the
// heuristic's candidates for a problem's plan and keeps the fastest
int linear_tune(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy, char* err, size_t errn);
// -2: no plan; -1: the heuristic's first, untuned; k >= 0: tuned, candidate k kept
int linear_plan_state(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy);
int linear_workspace(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy, size_t* bytes,
                     char* err, size_t errn);
// y = W^T a, then x = bf16(x + bf16(y)) in place and yn = rms_norm(x): linear!
// and fused_add_rms_norm! back to back; a split narrow GEMV hands its fp32
// slices straight to the norm (no reduce launch, no bf16 y in HBM)
int linear_add_norm_workspace(int M, int N, int K, int64_t ldw, int64_t lda, size_t* bytes,
                              char* err, size_t errn);
int linear_add_norm_run(uint16_t* yn, int64_t yn_st, uint16_t* x, int64_t x_st, const uint16_t* a,
                        int64_t lda, const uint16_t* w, int64_t ldw, const uint16_t* nw, int M,
                        int N, int K, float eps, float offset, void* workspace,
                        size_t workspace_bytes, hipStream_t st, char* err, size_t errn);
int linear_run(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
               int64_t ldw, int M, int N, int K, void* workspace, size_t workspace_bytes,
               hipStream_t st, char* err, size_t errn);

// ---- the rest of the decode step (step.hip) ----
// RMSNorm of each column of x (M rows), optionally fused with the residual add:
// dx != nullptr -> xo = bf16(x + dx) (xo may be x), y = norm of that.
struct NormArgs {
  uint16_t* y;
  int64_t y_st;
  uint16_t* xo;
  int64_t xo_st;
  const uint16_t* x;
  int64_t x_st;
  const uint16_t* dx;   // nullable
  int64_t dx_st;
  const uint16_t* w;
  int M, N;             // M a multiple of 8, at most 16384
  float offset, eps;
  // instead of dx: dx = bf16(sum of S2 fp32 slices in slice order), slice k of
  // column n at dpart + k * dpart_ss + n * dpart_cs (a split GEMV's partials)
  const float* dpart;
  int64_t dpart_ss, dpart_cs;
  int S2;
};
struct SiluMulArgs {
  uint16_t* mid;        // (I, N), column stride mid_st
  int64_t mid_st;
  const uint16_t* gu;   // (2I, N): gate rows 0 .. I-1, up rows I .. 2I-1
  int64_t gu_st;
  int I, N;             // I a multiple of 8
};
struct EmbedArgs {
  uint16_t* x;          // (D, B)
  int64_t x_st;
  const uint16_t* e;    // (D, vocab), column v at e + v * e_st
  int64_t e_st;
  const int32_t* ids;   // (B,) 1-based
  int D, B, vocab;
};
struct AdvanceArgs {
  int32_t* tokens_out;  // (max_new, B) column-major
  const int32_t* col_offsets;
  int32_t* step;        // (1,) 1-based row of tokens_out to write
  int32_t* positions;   // (B,)
  const int32_t* result;
  int B, max_new;
};
struct LmHeadArgs {
  const uint16_t* x;    // (K, B), column b at x + b * x_st
  int64_t x_st;
  const uint16_t* w;    // (K, N) K-major, column v at w + v * w_st
  int64_t w_st;
  int K, N, B;          // K a multiple of 64
  int cols;             // vocab columns per wave (set by the launcher)
  int NW;               // waves of the split pass (lm_head_waves())
  float* pmax;          // partials [NW][B]
  int32_t* pidx;
  int32_t* result;      // (B,) 1-based
};
// y = W^T x for N <= 32 columns (the decode projections): W (K, M) K-major, x
// (K, N), y (M, N), column strides w_st, x_st, y_st. K a multiple of 64, M of 4.
struct GemvArgs {
  const uint16_t* w;
  int64_t w_st;
  const uint16_t* x;
  int64_t x_st;
  uint16_t* y;
  int64_t y_st;
  int M, N, K;
  int T, S2, gps, G;    // set by the launcher (gemv_plan)
  float* part;          // S2 > 1: fp32 partials [S2][32][M] (gemv_workspace_bytes)
};
struct GemvPlan {
  int T, S2, gps, ntg;
};
GemvPlan gemv_plan(int M, int K, int waves);
size_t gemv_workspace_bytes(int M, int K);

// Stream-K GEMV for wide weights at N <= 32 (step.hip): y = W^T x as fp32
// partials, one 16 KB slot per (workgroup, 128-row group) it touches; the
// consumer adds a row's slots in workgroup order (gemv_sk_sum4).
struct GemvSkPlan {
  int G;      // 64-k groups of K
  int RG;     // 128-row groups of M
  int U;      // units = RG * G
  int chunk;  // units per workgroup
  int nwg;    // workgroups
};
struct GemvSkArgs {
  const uint16_t* w;    // (K, M) K-major: row m of W^T at w + m * w_st
  int64_t w_st;
  const uint16_t* x;    // (K, N): column n at x + n * x_st
  int64_t x_st;
  float* part;          // slots [nwg + RG - 1][4 tiles][32 columns][32 rows]
  int M, N, K;
  GemvSkPlan p;
};
GemvSkPlan gemv_sk_plan(int M, int K);
size_t gemv_sk_workspace_bytes(int M, int K);
hipError_t launch_gemv_sk(const GemvSkArgs& a, hipStream_t st);
// mid = silu(bf16(g)) .* bf16(u) from the stream-K partials of the packed
// gate-up projection (gate rows 0 .. I-1, up rows I .. 2I-1)
struct SiluMulSkArgs {
  uint16_t* mid;
  int64_t mid_st;
  const float* part;
  int I, N;
  GemvSkPlan p;
};
hipError_t launch_silu_mul_sk(const SiluMulSkArgs& a, hipStream_t st);
// linear! + silu .* mul (linear.cpp): mid (I, N) from x (K, N) and the packed
// gate-up W (K, 2I); the stream-K GEMV + silu_mul_sk_kernel at N <= 32, else
// linear! into a bf16 gu in the workspace and silu_mul_kernel
int linear_silu_mul_workspace(int I, int N, int K, int64_t ldw, int64_t ldx, size_t* bytes,
                              char* err, size_t errn);
int linear_silu_mul_run(uint16_t* mid, int64_t mid_st, const uint16_t* x, int64_t ldx,
                        const uint16_t* w, int64_t ldw, int I, int N, int K, void* workspace,
                        size_t workspace_bytes, hipStream_t st, char* err, size_t errn);
hipError_t launch_gemv(GemvArgs a, hipStream_t st);

// y = W^T x for a problem the GEMM library has no algorithm for (gemm.hip):
// column-major x (K, N) / W (K, M) / y (M, N) with column strides, any shape,
// any stride, 2-byte alignment; no workspace
struct GemmAnyArgs {
  const uint16_t* w;
  const uint16_t* x;
  uint16_t* y;
  int64_t ldw, ldx, ldy;
  int64_t M, N, K;
};
hipError_t launch_gemm_any(const GemmAnyArgs& a, hipStream_t st);
// the split GEMV without its reduce: leaves the slices' fp32 partials in
// a.part (layout [S2][32][M]); returns the plan through *plan
hipError_t launch_gemv_partials(GemvArgs a, GemvPlan* plan, hipStream_t st);
hipError_t launch_rms_norm(const NormArgs& a, hipStream_t st);

// ---- linear-attention layer parts (deltanet.hip). Dk = Dv = 128; element
// strides; state S (Dk, Dv, Hv, B) fp32 contiguous.
// fused_deltanet_decode!: q, k (Dk, Hk, B), v, z (Dv, Hv, B), alpha, beta
// (Hv, B) with per-sequence strides *_sb, heads contiguous; o (Dv, Hv, B) bf16.
struct DeltaFusedArgs {
  uint16_t* o;
  int64_t o_sb;
  const uint16_t *q, *k, *v, *z, *alpha, *beta;
  int64_t q_sb, k_sb, v_sb, z_sb, a_sb, b_sb;
  const float *a_log, *dt_bias;
  const uint16_t* norm_w;
  const float* s_in;
  float* s_out;
  int Hk, Hv, B;
  float eps;
};
// deltanet_sequence! / deltanet_recurrent_decode! (T = 1): q, k (Dk, T, Hk, B),
// v, o (Dv, T, Hv, B), beta, gate (Hv, T, B), all fp32 contiguous.
struct DeltaSeqArgs {
  float* o;
  const float *q, *k, *v, *beta, *gate;
  const float* s_in;
  float* s_out;
  int T, Hk, Hv, B;
};
// the generic forms (generic.hip): Dk, Dv multiples of 16 up to 256; one of
// seq (deltanet_sequence! / recurrent decode) or fused (fused_deltanet_decode!)
hipError_t launch_deltanet_any(const DeltaSeqArgs* seq, const DeltaFusedArgs* fused, int Dk,
                               int Dv, hipStream_t st);
// the prefill's prep: conv output cv (2 Hk Dk + Hv Dv channels, token stride
// cv_st, sequence stride cv_sb), ab (alpha | beta, 2 Hv rows, ab_st, ab_sb) ->
// qe, ke (Dk, T, Hk, B), ve (Dv, T, Hv, B), beta, gate (Hv, T, B) fp32.
struct DeltaPrepArgs {
  const uint16_t* cv;
  int64_t cv_st, cv_sb;
  const uint16_t* ab;
  int64_t ab_st, ab_sb;
  const float *a_log, *dt_bias;
  float *qe, *ke, *ve, *beta, *gate;
  int T, Hk, Hv, B;
};
// the prefill's gated RMSNorm: o (Dv, T, Hv, B) fp32, z (Dv, Hv) rows at token
// stride z_st / sequence stride z_sb -> y (Dv, Hv) rows at y_st / y_sb, bf16.
struct GatedNormArgs {
  const float* o;
  const uint16_t* z;
  int64_t z_st, z_sb;
  const uint16_t* norm_w;
  uint16_t* y;
  int64_t y_st, y_sb;
  int T, Hv, B;
  float eps;
};
// causal conv1d over D channels (D % 8 == 0, 16-byte aligned rows): x, y rows
// at token stride *_st / sequence stride *_sb; ring (D, K, B) with column
// stride s_cs and sequence stride s_sb; w (D, K) with column stride w_cs;
// bias (D) or NULL; act: silu. Decode reads s_in and writes s_out (may alias);
// the sequence form reads s_in (NULL: zero context) and seeds s_out (NULL: no).
constexpr int CONV_TC = 16;  // tokens per thread in the sequence form
struct Conv1dArgs {
  uint16_t* y;
  int64_t y_st, y_sb;
  const uint16_t* x;
  int64_t x_st, x_sb;
  const uint16_t* s_in;
  uint16_t* s_out;
  int64_t s_cs, s_sb;
  const uint16_t* w;
  int64_t w_cs;
  const uint16_t* bias;
  int D, K, T, B, act;
};
// the prefill's conv (c: x the projection's q | k | v channels, D = (2 Hk + Hv)
// Dk, c.y unused) and prep (p: p.cv unused; outputs and gates as DeltaPrepArgs)
// in one pass; the launcher's caller checks 16-byte alignment of every row
struct ConvPrepArgs {
  Conv1dArgs c;
  DeltaPrepArgs p;
};
// causal_conv1d! on the first D channels of a projection given as stream-K
// partials (gemv_sk_kernel): the projection's M channels are written rounded to
// bf16 at yp (column stride yp_sb), c.x is unused
struct Conv1dSkArgs {
  Conv1dArgs c;
  uint16_t* yp;
  int64_t yp_sb;
  const float* part;
  int G, chunk, M;
};
hipError_t launch_conv1d_update_sk(const Conv1dSkArgs& a, hipStream_t st);
// linear! + causal_conv1d! (linear.cpp): y (M, N) = W^T x, then the conv step
// on y's first conv.D channels; the stream-K GEMV + conv1d_update_sk_kernel at
// N <= 32, else linear! + conv1d_update_kernel
int linear_conv_workspace(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy,
                          size_t* bytes, char* err, size_t errn);
int linear_conv_run(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
                    int64_t ldw, int M, int N, int K, Conv1dArgs conv, void* workspace,
                    size_t workspace_bytes, hipStream_t st, char* err, size_t errn);
// the DeltaNet layer's decode step through its recurrence: linear! of the
// projection, causal_conv1d! of its first conv.D channels and
// fused_deltanet_decode! (f: q .. beta point into y and conv.y, used by the
// two-call form only); at N <= 32 with aligned views the projection's
// stream-K partials go straight to deltanet_decode_sk_kernel
int linear_dn_decode_run(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx,
                         const uint16_t* w, int64_t ldw, int M, int N, int K, Conv1dArgs conv,
                         const DeltaFusedArgs& f, void* workspace, size_t workspace_bytes,
                         hipStream_t st, char* err, size_t errn);
// the chunked form of deltanet_sequence!: same arguments, plus a workspace of
// deltanet_chunk_workspace_bytes(T, Hv, B) bytes (256-byte aligned)
struct DeltaChunkArgs {
  DeltaSeqArgs s;
  float* ws;
  // g.y set: the gated RMSNorm with z (qwen35.jl:360-364) is fused into the
  // output phase, which writes y (bf16) instead of s.o; g.o is unused
  GatedNormArgs g;
};
size_t deltanet_chunk_workspace_bytes(int T, int Hv, int B);
hipError_t launch_deltanet_sequence_chunked(const DeltaChunkArgs& a, hipStream_t st);
hipError_t launch_deltanet_fused_decode(const DeltaFusedArgs& a, hipStream_t st);
// The DeltaNet layer's decode step after its stream-K projection: f's state,
// gates, norm and output (f.q .. f.beta unused: they come from the partials),
// c's ring, weight and bias (c.x, c.y unused; c.D = 2 Hk Dk + Hv Dv conv
// channels, c.B = f.B), the projection's partials (GemvSkArgs::part, its G
// and chunk); Hv / Hk in {1, 2, 4}
struct DeltaDecodeSkArgs {
  DeltaFusedArgs f;
  Conv1dArgs c;
  const float* part;
  int G, chunk;
};
hipError_t launch_deltanet_decode_sk(const DeltaDecodeSkArgs& a, hipStream_t st);
hipError_t launch_deltanet_sequence(const DeltaSeqArgs& a, hipStream_t st);
hipError_t launch_deltanet_prep(const DeltaPrepArgs& a, hipStream_t st);
hipError_t launch_gated_rms_norm(const GatedNormArgs& a, hipStream_t st);
hipError_t launch_conv1d_update(const Conv1dArgs& a, hipStream_t st);
hipError_t launch_conv1d_sequence(const Conv1dArgs& a, hipStream_t st);
hipError_t launch_deltanet_conv_prep(const ConvPrepArgs& a, hipStream_t st);
hipError_t launch_silu_mul(const SiluMulArgs& a, hipStream_t st);
hipError_t launch_embed(const EmbedArgs& a, hipStream_t st);
hipError_t launch_gen_advance(const AdvanceArgs& a, hipStream_t st);
int lm_head_waves();
hipError_t launch_lm_head_argmax(LmHeadArgs a, hipStream_t st);

// Decode stream partition shared by the scratch-size query and the launchers:
// NW waves cover the token-heads sum_b len_b * Hk in equal contiguous chunks.
constexpr int DECODE_MIN_CHUNK = 64;
int decode_stream_waves(int B, int Hk, int n_splits);

}  // namespace vm

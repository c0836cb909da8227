// vallmo_attn.cpp — the C ABI of libvallmo_attn.so (declared in
// include/vallmo_attn.h). Host code only: argument and shape validation with
// the reference's error semantics, then kernel launches on the caller's stream.
//
// Error convention: < 0 = argument/shape error (message in vm_last_error()),
// > 0 = hipError_t passed through. Shape errors mirror @sizes
// (src/sizes.jl:3-22) and the H % Hk check (src/kernels/attention.jl:110-111).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>
#include "../../include/vallmo_attn.h"
#include "kernels.h"

namespace {

// ---- optional per-kernel timing (vm_profile_*): hipEvents around each launch
struct ProfRec {
  int id;
  hipEvent_t a, b;
};
struct Prof {
  bool on = false;
  unsigned mask = ~0u;  // kernel classes bracketed while on
  std::vector<ProfRec> recs;
  std::vector<hipEvent_t> pool;
};
thread_local Prof g_prof;

hipEvent_t prof_event() {
  if (!g_prof.pool.empty()) {
    hipEvent_t e = g_prof.pool.back();
    g_prof.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Launch through `f`, bracketed by events on `st` when profiling is on and the
// stream is not being captured into a graph.
template <class F>
hipError_t timed(int id, hipStream_t st, F&& f) {
  if (!g_prof.on || !((g_prof.mask >> id) & 1u)) return f();
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return f();
  hipEvent_t a = prof_event(), b = prof_event();
  if (!a || !b) return f();
  (void)hipEventRecord(a, st);
  hipError_t e = f();
  (void)hipEventRecord(b, st);
  g_prof.recs.push_back({id, a, b});
  return e;
}

// As timed(), for a launcher that takes (start, stop) events and has the
// dispatch stamp them (hipExtLaunchKernelGGL): the kernel's own span, with no
// event packets between launches.
template <class F>
hipError_t timed_ext(int id, hipStream_t st, F&& f) {
  if (!g_prof.on || !((g_prof.mask >> id) & 1u)) return f(nullptr, nullptr);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
    return f(nullptr, nullptr);
  hipEvent_t a = prof_event(), b = prof_event();
  if (!a || !b) return f(nullptr, nullptr);
  hipError_t e = f(a, b);
  g_prof.recs.push_back({id, a, b});
  return e;
}

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}
int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return VM_OK;
  snprintf(g_err, sizeof g_err, "%s: %s", where, hipGetErrorString(e));
  return (int)e;
}
inline hipStream_t S(vm_stream s) { return reinterpret_cast<hipStream_t>(s); }

#define REQUIRE(cond, code, ...) \
  do {                           \
    if (!(cond)) return fail(code, __VA_ARGS__); \
  } while (0)

int check_head(int D, int half_rot) {
  REQUIRE(D == vm::HEAD_DIM_ABI, VM_E_UNSUPPORTED,
          "head_dim D = %d is not supported (this build is compiled for D = 256)", D);
  REQUIRE(half_rot == vm::HALF_ROT_ABI, VM_E_UNSUPPORTED,
          "HALF_ROT = %d is not supported (this build is compiled for HALF_ROT = 32)", half_rot);
  return VM_OK;
}
// the generic operators' head shapes: power-of-two dims 16..512
int check_head_any(int D, const char* what, const char* name) {
  REQUIRE(D >= 16 && D <= 512 && (D & (D - 1)) == 0, VM_E_UNSUPPORTED,
          "%s: %s = %d (head dims are powers of two from 16 to 512)", what, name, D);
  return VM_OK;
}
int check_rot(int D, int half_rot, const char* what) {
  REQUIRE(half_rot >= 1 && 2 * half_rot <= D, VM_E_ARG,
          "%s: HALF_ROT = %d (the rotary part 2 HALF_ROT must fit in D = %d)", what, half_rot, D);
  return VM_OK;
}
int check_gqa(int H, int Hk) {
  REQUIRE(H > 0 && Hk > 0, VM_E_ARG, "head counts must be positive (H = %d, Hk = %d)", H, Hk);
  REQUIRE(H % Hk == 0, VM_E_DIM,
          "Attention heads (%d) is not a multiple of key-value heads (%d)", H, Hk);
  return VM_OK;
}
int check_aligned(const void* p, const char* name) {
  REQUIRE(p != nullptr, VM_E_ARG, "%s is NULL", name);
  REQUIRE((reinterpret_cast<uintptr_t>(p) & 15u) == 0, VM_E_ARG,
          "%s must be 16-byte aligned", name);
  return VM_OK;
}
int check_stride(int64_t s, const char* name) {
  REQUIRE(s >= 0 && (s % 8) == 0, VM_E_ARG,
          "stride %s = %lld must be a non-negative multiple of 8 elements", name, (long long)s);
  return VM_OK;
}
#define TRY(x)                 \
  do {                         \
    int _rc = (x);             \
    if (_rc != VM_OK) return _rc; \
  } while (0)

size_t decode_slots(int B, int Hk, int NW) { return (size_t)NW + (size_t)B * Hk; }
size_t decode_part_o_bytes(int B, int Hk, int NW, int G) {
  return decode_slots(B, Hk, NW) * G * vm::HEAD_DIM_ABI * sizeof(float);
}
size_t decode_part_ml_bytes(int B, int Hk, int NW, int G) {
  return decode_slots(B, Hk, NW) * G * 2 * sizeof(float);
}
// partition snapshot for the merge: chunk, then len_b and start_b per sequence
size_t decode_geom_bytes(int B) { return ((size_t)(1 + 2 * B) * sizeof(int32_t) + 255) / 256 * 256; }

}  // namespace

extern "C" {

const char* vm_last_error(void) { return g_err; }
int vm_abi_version(void) { return 1; }

// ---- kernel timing ----------------------------------------------------------
int vm_profile_enable(int on) {
  for (auto& r : g_prof.recs) {
    g_prof.pool.push_back(r.a);
    g_prof.pool.push_back(r.b);
  }
  g_prof.recs.clear();
  g_prof.on = on != 0;
  return VM_OK;
}
int vm_profile_select(unsigned kernel_mask) {
  g_prof.mask = kernel_mask;
  return VM_OK;
}
int vm_profile_read(int kernel, int* count, double* total_ms) {
  REQUIRE(count && total_ms, VM_E_ARG, "vm_profile_read: NULL output");
  REQUIRE(kernel >= 0 && kernel < VM_K_COUNT, VM_E_ARG, "vm_profile_read: kernel id %d", kernel);
  int n = 0;
  double t = 0.0;
  for (auto& r : g_prof.recs) {
    if (r.id != kernel) continue;
    int rc = hip_status(hipEventSynchronize(r.b), "hipEventSynchronize");
    if (rc) return rc;
    float ms = 0.f;
    rc = hip_status(hipEventElapsedTime(&ms, r.a, r.b), "hipEventElapsedTime");
    if (rc) return rc;
    ++n;
    t += ms;
  }
  *count = n;
  *total_ms = t;
  return VM_OK;
}

// ---- runtime --------------------------------------------------------------
int vm_malloc(void** ptr, size_t bytes) {
  REQUIRE(ptr, VM_E_ARG, "vm_malloc: ptr is NULL");
  return hip_status(hipMalloc(ptr, bytes), "hipMalloc");
}
int vm_free(void* ptr) { return hip_status(hipFree(ptr), "hipFree"); }
int vm_memcpy_h2d(void* dst, const void* src, size_t n, vm_stream s) {
  return hip_status(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, S(s)), "hipMemcpyAsync");
}
int vm_memcpy_d2h(void* dst, const void* src, size_t n, vm_stream s) {
  return hip_status(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, S(s)), "hipMemcpyAsync");
}
int vm_memcpy_d2d(void* dst, const void* src, size_t n, vm_stream s) {
  return hip_status(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, S(s)), "hipMemcpyAsync");
}
int vm_memset(void* dst, int v, size_t n, vm_stream s) {
  return hip_status(hipMemsetAsync(dst, v, n, S(s)), "hipMemsetAsync");
}
int vm_stream_create(vm_stream* s) {
  REQUIRE(s, VM_E_ARG, "vm_stream_create: out pointer is NULL");
  hipStream_t st;
  int rc = hip_status(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
  *s = rc == VM_OK ? (vm_stream)st : nullptr;
  return rc;
}
int vm_stream_destroy(vm_stream s) { return hip_status(hipStreamDestroy(S(s)), "hipStreamDestroy"); }
int vm_stream_sync(vm_stream s) { return hip_status(hipStreamSynchronize(S(s)), "hipStreamSynchronize"); }
int vm_device_sync(void) { return hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
int vm_event_create(void** e) {
  REQUIRE(e, VM_E_ARG, "vm_event_create: out pointer is NULL");
  hipEvent_t ev;
  int rc = hip_status(hipEventCreate(&ev), "hipEventCreate");
  *e = rc == VM_OK ? (void*)ev : nullptr;
  return rc;
}
int vm_event_destroy(void* e) { return hip_status(hipEventDestroy((hipEvent_t)e), "hipEventDestroy"); }
int vm_event_record(void* e, vm_stream s) {
  return hip_status(hipEventRecord((hipEvent_t)e, S(s)), "hipEventRecord");
}
int vm_event_elapsed_ms(float* ms, void* a, void* b) {
  REQUIRE(ms, VM_E_ARG, "vm_event_elapsed_ms: out pointer is NULL");
  return hip_status(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b), "hipEventElapsedTime");
}
int vm_graph_begin_capture(vm_stream s) {
  REQUIRE(s, VM_E_ARG, "graph capture needs a non-default stream");
  return hip_status(hipStreamBeginCapture(S(s), hipStreamCaptureModeThreadLocal),
                    "hipStreamBeginCapture");
}
int vm_graph_end_capture(vm_stream s, void** exec) {
  REQUIRE(exec, VM_E_ARG, "vm_graph_end_capture: out pointer is NULL");
  hipGraph_t g = nullptr;
  int rc = hip_status(hipStreamEndCapture(S(s), &g), "hipStreamEndCapture");
  if (rc != VM_OK) return rc;
  hipGraphExec_t ge = nullptr;
  rc = hip_status(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  (void)hipGraphDestroy(g);
  *exec = rc == VM_OK ? (void*)ge : nullptr;
  return rc;
}
int vm_graph_launch(void* exec, vm_stream s) {
  REQUIRE(exec, VM_E_ARG, "vm_graph_launch: graph is NULL");
  return hip_status(hipGraphLaunch((hipGraphExec_t)exec, S(s)), "hipGraphLaunch");
}
int vm_graph_destroy(void* exec) {
  return hip_status(hipGraphExecDestroy((hipGraphExec_t)exec), "hipGraphExecDestroy");
}

// ---- a1 -------------------------------------------------------------------
int vm_rope_tables(float* c, float* s, int half_rot, int64_t ctx, double theta, vm_stream st) {
  REQUIRE(c && s, VM_E_ARG, "rope_tables: NULL table pointer");
  REQUIRE(half_rot > 0 && ctx >= 0, VM_E_ARG, "rope_tables: half_rot = %d, Ctx = %lld", half_rot,
          (long long)ctx);
  REQUIRE(theta > 0, VM_E_ARG, "rope_tables: theta must be positive");
  return hip_status(vm::launch_rope_tables(c, s, half_rot, ctx, theta, S(st)), "rope_tables");
}

// ---- a3 -------------------------------------------------------------------
int vm_qnorm_rope(vm_bf16* q, int64_t q_sh, int64_t q_sb, const vm_bf16* qw, const float* cs,
                  const float* sn, int64_t ctx, const int32_t* positions, int B, int Hq, int D,
                  int half_rot, float eps, float w_offset, vm_stream st) {
  TRY(check_head_any(D, "qnorm_rope", "D"));
  TRY(check_rot(D, half_rot, "qnorm_rope"));
  REQUIRE(B >= 0 && Hq > 0 && ctx > 0, VM_E_ARG, "qnorm_rope: B = %d, Hq = %d, Ctx = %lld", B, Hq,
          (long long)ctx);
  REQUIRE(q && qw && cs && sn && positions, VM_E_ARG, "qnorm_rope: NULL pointer argument");
  TRY(check_stride(q_sh, "q_sh"));
  TRY(check_stride(q_sb, "q_sb"));
  if (D != vm::HEAD_DIM_ABI || half_rot != vm::HALF_ROT_ABI) {  // the generic row kernel
    vm::RowAnyArgs g{};
    g.in = q; g.in_sh = q_sh; g.in_sb = q_sb;
    g.out = q; g.out_sh = q_sh; g.out_sb = q_sb;
    g.w = qw; g.cos_tab = cs; g.sin_tab = sn; g.ctx = ctx; g.positions = positions;
    g.B = B; g.H = Hq; g.D = D; g.half = half_rot; g.eps = eps; g.w_offset = w_offset;
    return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_norm_rope_any(g, S(st)); }),
                      "qnorm_rope");
  }
  vm::RowArgs a{};
  a.in = q; a.out = q; a.in_sh = a.out_sh = q_sh; a.in_sb = a.out_sb = q_sb;
  a.w = qw; a.cos_tab = cs; a.sin_tab = sn; a.ctx = ctx; a.positions = positions;
  a.B = B; a.H = Hq; a.T = 1; a.out_at_pos = 0; a.eps = eps; a.w_offset = w_offset;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_norm_rope_rows(a, S(st)); }), "qnorm_rope");
}

// ---- a4 -------------------------------------------------------------------
int vm_knorm_rope_append(vm_bf16* kc, int64_t kc_st, int64_t kc_sh, int64_t kc_sb, vm_bf16* vc,
                         int64_t vc_st, int64_t vc_sh, int64_t vc_sb, int64_t ctx,
                         const vm_bf16* k_raw, int64_t kr_sh, int64_t kr_sb, const vm_bf16* v_raw,
                         int64_t vr_sh, int64_t vr_sb, const vm_bf16* kw, const float* cs,
                         const float* sn, const int32_t* positions, int B, int Hk, int Dk, int Dv,
                         int half_rot, float eps, float w_offset, vm_stream st) {
  TRY(check_head_any(Dk, "knorm_rope_append", "Dk"));
  TRY(check_head_any(Dv, "knorm_rope_append", "Dv"));
  TRY(check_rot(Dk, half_rot, "knorm_rope_append"));
  REQUIRE(B >= 0 && Hk > 0 && ctx > 0, VM_E_ARG, "knorm_rope_append: B = %d, Hk = %d, Ctx = %lld",
          B, Hk, (long long)ctx);
  REQUIRE(kc && vc && k_raw && v_raw && kw && cs && sn && positions, VM_E_ARG,
          "knorm_rope_append: NULL pointer argument");
  for (int64_t v : {kc_st, kc_sh, kc_sb, vc_st, vc_sh, vc_sb, kr_sh, kr_sb, vr_sh, vr_sb})
    TRY(check_stride(v, "knorm_rope_append"));
  const bool tuned = Dk == vm::HEAD_DIM_ABI && Dv == Dk && half_rot == vm::HALF_ROT_ABI &&
                     kc_st == vc_st && kc_sh == vc_sh && kc_sb == vc_sb && kr_sh == vr_sh &&
                     kr_sb == vr_sb;
  if (!tuned) {  // the generic row kernel: K normed and rotated, V copied
    vm::RowAnyArgs g{};
    g.in = k_raw; g.in_sh = kr_sh; g.in_sb = kr_sb;
    g.out = kc; g.out_st = kc_st; g.out_sh = kc_sh; g.out_sb = kc_sb;
    g.in2 = v_raw; g.in2_sh = vr_sh; g.in2_sb = vr_sb;
    g.out2 = vc; g.out2_st = vc_st; g.out2_sh = vc_sh; g.out2_sb = vc_sb;
    g.w = kw; g.cos_tab = cs; g.sin_tab = sn; g.ctx = ctx; g.positions = positions;
    g.B = B; g.H = Hk; g.D = Dk; g.D2 = Dv; g.half = half_rot; g.out_at_pos = 1;
    g.eps = eps; g.w_offset = w_offset;
    return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_norm_rope_any(g, S(st)); }),
                      "knorm_rope_append");
  }
  vm::RowArgs a{};
  a.in = k_raw; a.in2 = v_raw; a.in_sh = kr_sh; a.in_sb = kr_sb;
  a.out = kc; a.out2 = vc; a.out_st = kc_st; a.out_sh = kc_sh; a.out_sb = kc_sb;
  a.w = kw; a.cos_tab = cs; a.sin_tab = sn; a.ctx = ctx; a.positions = positions;
  a.B = B; a.H = Hk; a.T = 1; a.out_at_pos = 1; a.eps = eps; a.w_offset = w_offset;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_norm_rope_rows(a, S(st)); }), "knorm_rope_append");
}

// ---- a5 -------------------------------------------------------------------
// the tuned split-KV decode's workspace (D = 256, groups up to 8)
static size_t tuned_decode_scratch_bytes(int B, int H, int Hk, int64_t ctx, int n_splits) {
  if (B <= 0 || H <= 0 || Hk <= 0 || H % Hk || ctx <= 0 || n_splits < 0) return 0;
  const int NW = vm::decode_stream_waves(B, Hk, n_splits);
  const int G = H / Hk;
  const size_t pm_end = decode_part_o_bytes(B, Hk, NW, G) + decode_part_ml_bytes(B, Hk, NW, G);
  return (pm_end + 255) / 256 * 256 + decode_geom_bytes(B);
}
// the generic decode's workspace: one (Dv + 2)-float partial row per split,
// sequence and head (the reference's O_partial, M_partial, L_partial)
static size_t generic_decode_scratch_bytes(int B, int H, int Hk, int Dv, int64_t ctx,
                                           int n_splits) {
  const int ns = vm::attn_any_splits(B, H, Hk, ctx, n_splits);
  return ((size_t)ns * B * H * (Dv + 2) * sizeof(float) + 255) / 256 * 256;
}

size_t vm_decode_scratch_bytes(int B, int H, int Hk, int D, int64_t ctx, int n_splits) {
  if (B <= 0 || H <= 0 || Hk <= 0 || H % Hk || ctx <= 0 || n_splits < 0) return 0;
  if (D < 16 || D > 512 || (D & (D - 1))) return 0;
  const size_t generic = generic_decode_scratch_bytes(B, H, Hk, D, ctx, n_splits);
  if (D != vm::HEAD_DIM_ABI || H / Hk > 8) return generic;
  return std::max(generic, tuned_decode_scratch_bytes(B, H, Hk, ctx, n_splits));
}

static int decode_common(vm::DecodeArgs& a, vm::CombineArgs& c, void* scratch, size_t scratch_bytes,
                         int B, int H, int Hk, int64_t ctx, int n_splits) {
  TRY(check_gqa(H, Hk));
  const int G = H / Hk;
  REQUIRE(G <= 8, VM_E_UNSUPPORTED, "decode: GQA group %d > 8 is not supported", G);
  REQUIRE(n_splits >= 0, VM_E_ARG, "decode: n_splits = %d", n_splits);
  REQUIRE(ctx > 0, VM_E_ARG, "decode: Ctx = %lld", (long long)ctx);
  REQUIRE((int64_t)B * ctx * Hk < ((int64_t)1 << 31), VM_E_UNSUPPORTED,
          "decode: B*Ctx*Hk = %lld token-heads exceeds 2^31", (long long)B * ctx * Hk);
  const int NW = vm::decode_stream_waves(B, Hk, n_splits);
  const size_t po = decode_part_o_bytes(B, Hk, NW, G), pm = decode_part_ml_bytes(B, Hk, NW, G);
  const size_t geo = (po + pm + 255) / 256 * 256;  // partition snapshot offset
  const size_t need = geo + decode_geom_bytes(B);
  REQUIRE(scratch != nullptr && scratch_bytes >= need, VM_E_SCRATCH,
          "decode: scratch of %zu bytes < %zu required (vm_decode_scratch_bytes)", scratch_bytes,
          need);
  TRY(check_aligned(scratch, "scratch"));
  char* sp = reinterpret_cast<char*>(scratch);
  a.part_o = reinterpret_cast<float*>(sp);
  a.part_ml = reinterpret_cast<float*>(sp + po);
  a.geom = reinterpret_cast<int32_t*>(sp + geo);
  a.B = B; a.Hk = Hk; a.G = G; a.NW = NW; a.min_chunk = vm::DECODE_MIN_CHUNK; a.ctx = ctx;
  c.part_o = a.part_o; c.part_ml = a.part_ml;
  c.geom = a.geom;
  c.B = B; c.Hk = Hk; c.G = G; c.NW = NW;
  c.advance = nullptr;
  return VM_OK;
}

int vm_decode_attention(vm_bf16* o, int64_t o_sh, int64_t o_sb, const vm_bf16* q, int64_t q_sh,
                        int64_t q_sb, const vm_bf16* kc, int64_t k_st, int64_t k_sh, int64_t k_sb,
                        const vm_bf16* vc, int64_t v_st, int64_t v_sh, int64_t v_sb,
                        int64_t ctx, const int32_t* lengths, int B, int H, int Hk, int Dk,
                        int Dv, int n_splits, void* scratch, size_t scratch_bytes,
                        vm_stream st) {
  TRY(check_head_any(Dk, "decode_attention", "Dk"));
  TRY(check_head_any(Dv, "decode_attention", "Dv"));
  REQUIRE(B >= 0, VM_E_ARG, "decode_attention: B = %d", B);
  REQUIRE(o && lengths, VM_E_ARG, "decode_attention: NULL pointer argument");
  TRY(check_aligned(o, "O"));
  TRY(check_aligned(q, "Q"));
  TRY(check_aligned(kc, "K"));
  TRY(check_aligned(vc, "V"));
  for (int64_t s : {o_sh, o_sb, q_sh, q_sb, k_st, k_sh, k_sb, v_st, v_sh, v_sb})
    TRY(check_stride(s, "decode"));
  TRY(check_gqa(H, Hk));
  REQUIRE(n_splits >= 0, VM_E_ARG, "decode: n_splits = %d", n_splits);
  REQUIRE(ctx > 0, VM_E_ARG, "decode: Ctx = %lld", (long long)ctx);
  const bool tuned = Dk == vm::HEAD_DIM_ABI && Dv == Dk && H / Hk <= 8 && k_st == v_st &&
                     k_sh == v_sh && k_sb == v_sb &&
                     (int64_t)B * ctx * Hk < ((int64_t)1 << 31);
  if (!tuned) {  // the generic split-KV kernel and its merge
    REQUIRE((int64_t)B * Hk <= 65535 && n_splits <= 65535, VM_E_UNSUPPORTED,
            "decode: B*Hk = %lld, n_splits = %d (at most 65535 each)", (long long)B * Hk,
            n_splits);
    const size_t need = generic_decode_scratch_bytes(B, H, Hk, Dv, ctx, n_splits);
    REQUIRE(scratch != nullptr && scratch_bytes >= need, VM_E_SCRATCH,
            "decode: scratch of %zu bytes < %zu required (vm_decode_scratch_bytes)",
            scratch_bytes, need);
    TRY(check_aligned(scratch, "scratch"));
    if (B == 0) return VM_OK;
    vm::AttnAnyArgs g{};
    g.q = q; g.q_st = 0; g.q_sh = q_sh; g.q_sb = q_sb;
    g.k = kc; g.k_st = k_st; g.k_sh = k_sh; g.k_sb = k_sb;
    g.v = vc; g.v_st = v_st; g.v_sh = v_sh; g.v_sb = v_sb;
    g.o = o; g.o_st = 0; g.o_sh = o_sh; g.o_sb = o_sb;
    g.k_lengths = lengths; g.q_lengths = nullptr;
    g.part = static_cast<float*>(scratch);
    g.B = B; g.H = H; g.Hk = Hk; g.Dk = Dk; g.Dv = Dv; g.L = 1;
    g.Lk = (int)std::min<int64_t>(ctx, INT32_MAX); g.causal = 0;
    g.n_split = vm::attn_any_splits(B, H, Hk, ctx, n_splits);
    g.split_keys = vm::attn_any_split_keys(ctx, g.n_split);
    g.scale = 1.0f / sqrtf((float)Dk);
    return hip_status(timed(VM_K_DECODE_SPLIT, S(st), [&] { return vm::launch_attn_any(g, S(st)); }),
                      "decode_attention");
  }
  const int64_t c_st = k_st, c_sh = k_sh, c_sb = k_sb;
  vm::DecodeArgs a{};
  vm::CombineArgs c{};
  TRY(decode_common(a, c, scratch, scratch_bytes, B, H, Hk, ctx, n_splits));
  if (B == 0) return VM_OK;
  a.q = q; a.q_sh = q_sh; a.q_sb = q_sb;
  // read-only here: the unfused operator appends nothing (k_new stays NULL)
  a.kc = const_cast<uint16_t*>(kc); a.vc = const_cast<uint16_t*>(vc);
  a.c_st = c_st; a.c_sh = c_sh; a.c_sb = c_sb;
  a.lengths = lengths;
  int rc = hip_status(timed(VM_K_DECODE_SPLIT, S(st), [&] { return vm::launch_decode(a, false, S(st)); }), "decode_attention split");
  if (rc) return rc;
  c.out = o; c.o_sh = o_sh; c.o_sb = o_sb; c.gate = nullptr;
  return hip_status(timed(VM_K_DECODE_COMBINE, S(st), [&] { return vm::launch_combine(c, S(st)); }), "decode_attention combine");
}

// ---- a6 -------------------------------------------------------------------
int vm_sigmoid_gate(vm_bf16* o, int64_t o_sh, int64_t o_sb, const vm_bf16* g, int64_t g_sh,
                    int64_t g_sb, int B, int H, int D, vm_stream st) {
  REQUIRE(D == vm::HEAD_DIM_ABI, VM_E_UNSUPPORTED, "sigmoid_gate: D = %d (need 256)", D);
  REQUIRE(B >= 0 && H >= 0, VM_E_ARG, "sigmoid_gate: B = %d, H = %d", B, H);
  TRY(check_aligned(o, "O"));
  TRY(check_aligned(g, "gate"));
  for (int64_t s : {o_sh, o_sb, g_sh, g_sb}) TRY(check_stride(s, "gate"));
  return hip_status(vm::launch_sigmoid_gate(o, o_sh, o_sb, g, g_sh, g_sb, B, H, S(st)),
                    "sigmoid_gate");
}

// ---- a7 -------------------------------------------------------------------
static int gated_attn_decode(vm_bf16* out, int64_t out_sb, const vm_bf16* qkv, int64_t qkv_sb,
                         vm_bf16* kc, vm_bf16* vc, int64_t c_st, int64_t c_sh, int64_t c_sb,
                         int64_t ctx, const vm_bf16* qw, const vm_bf16* kw, const float* cs,
                         const float* sn, int32_t* positions, int advance, int B, int Hq, int Hk,
                         int D, int half_rot, float eps, float w_offset, int n_splits,
                         void* scratch, size_t scratch_bytes, vm_stream st) {
  TRY(check_head(D, half_rot));
  REQUIRE(B >= 0, VM_E_ARG, "gated_attn_decode: B = %d", B);
  REQUIRE(out && qw && kw && cs && sn && positions, VM_E_ARG,
          "gated_attn_decode: NULL pointer argument");
  TRY(check_aligned(qkv, "qkv"));
  TRY(check_aligned(kc, "K_cache"));
  TRY(check_aligned(vc, "V_cache"));
  TRY(check_aligned(qw, "qw"));
  TRY(check_aligned(kw, "kw"));
  for (int64_t s : {out_sb, qkv_sb, c_st, c_sh, c_sb}) TRY(check_stride(s, "gated_attn_decode"));
  REQUIRE(qkv_sb >= (int64_t)(2 * Hq + 2 * Hk) * D || B <= 1, VM_E_DIM,
          "gated_attn_decode: qkv batch stride %lld < (2Hq+2Hk)*D = %lld", (long long)qkv_sb,
          (long long)(2 * Hq + 2 * Hk) * D);
  vm::DecodeArgs a{};
  vm::CombineArgs c{};
  TRY(decode_common(a, c, scratch, scratch_bytes, B, Hq, Hk, ctx, n_splits));
  if (B == 0) return VM_OK;
  const int64_t Dl = D;
  // a3 + a4 + a5: split-KV attention with the q norm+RoPE prologue fused; the
  // wave that covers each (b, hk)'s last token builds the new K/V row from the
  // raw projection, attends it and writes it to cache column positions[b]
  a.q = qkv; a.q_sh = 2 * Dl; a.q_sb = qkv_sb;
  a.qw = qw; a.kw = kw; a.cos_tab = cs; a.sin_tab = sn; a.eps = eps; a.w_offset = w_offset;
  a.kc = kc; a.vc = vc; a.c_st = c_st; a.c_sh = c_sh; a.c_sb = c_sb;
  a.lengths = positions;
  a.k_new = qkv + 2 * Hq * Dl; a.v_new = qkv + (2 * Hq + Hk) * Dl;
  a.new_sh = Dl; a.new_sb = qkv_sb;
  int rc = hip_status(timed(VM_K_DECODE_SPLIT, S(st), [&] { return vm::launch_decode(a, true, S(st)); }), "gated_attn_decode split");
  if (rc) return rc;
  // a5 merge + a6 gate, written as the Wo input (D, Hq, B); a12 advance fused
  c.out = out; c.o_sh = Dl; c.o_sb = out_sb;
  c.gate = qkv + Dl; c.g_sh = 2 * Dl; c.g_sb = qkv_sb;
  c.advance = advance ? positions : nullptr;
  return hip_status(timed(VM_K_DECODE_COMBINE, S(st), [&] { return vm::launch_combine(c, S(st)); }), "gated_attn_decode combine");
}

int vm_gated_attn_decode(vm_bf16* out, int64_t out_sb, const vm_bf16* qkv, int64_t qkv_sb,
                         vm_bf16* kc, vm_bf16* vc, int64_t c_st, int64_t c_sh, int64_t c_sb,
                         int64_t ctx, const vm_bf16* qw, const vm_bf16* kw, const float* cs,
                         const float* sn, int32_t* positions, int advance, int B, int Hq, int Hk,
                         int D, int half_rot, float eps, float w_offset, int n_splits,
                         void* scratch, size_t scratch_bytes, vm_stream st) {
  return gated_attn_decode(out, out_sb, qkv, qkv_sb, kc, vc, c_st, c_sh,
                           c_sb, ctx, qw, kw, cs, sn, positions, advance, B, Hq, Hk, D, half_rot,
                           eps, w_offset, n_splits, scratch, scratch_bytes, st);
}

// The same step with its workspace in the library's static per-GPU array
// (no allocation of any kind). Calls that overlap on one GPU share that array.
int vm_gated_attn_decode_noalloc(vm_bf16* out, int64_t out_sb, const vm_bf16* qkv,
                                 int64_t qkv_sb, vm_bf16* kc, vm_bf16* vc, int64_t c_st,
                                 int64_t c_sh, int64_t c_sb, int64_t ctx, const vm_bf16* qw,
                                 const vm_bf16* kw, const float* cs, const float* sn,
                                 int32_t* positions, int advance, int B, int Hq, int Hk, int D,
                                 int half_rot, float eps, float w_offset, int n_splits,
                                 vm_stream st) {
  REQUIRE(B >= 0 && Hq > 0 && Hk > 0 && Hq % Hk == 0 && ctx > 0 && n_splits >= 0, VM_E_ARG,
          "gated_attn_decode_noalloc: B = %d, Hq = %d, Hk = %d, Ctx = %lld, n_splits = %d", B,
          Hq, Hk, (long long)ctx, n_splits);
  TRY(check_head(D, half_rot));
  const size_t need = tuned_decode_scratch_bytes(B > 0 ? B : 1, Hq, Hk, ctx, n_splits);
  REQUIRE(need <= vm::DECODE_STATIC_SCRATCH_BYTES, VM_E_SCRATCH,
          "gated_attn_decode_noalloc: this step needs %zu bytes of workspace, more than the "
          "%zu-byte static workspace (use vm_gated_attn_decode with a caller buffer)",
          need, (size_t)vm::DECODE_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  TRY(hip_status(vm::decode_static_scratch(&ws), "gated_attn_decode_noalloc workspace"));
  return gated_attn_decode(out, out_sb, qkv, qkv_sb, kc, vc, c_st,
                           c_sh, c_sb, ctx, qw, kw, cs, sn, positions, advance, B, Hq, Hk, D,
                           half_rot, eps, w_offset, n_splits, ws, vm::DECODE_STATIC_SCRATCH_BYTES,
                           st);
}

int vm_advance_positions(int32_t* positions, int B, vm_stream st) {
  REQUIRE(positions || B == 0, VM_E_ARG, "advance_positions: NULL positions");
  REQUIRE(B >= 0, VM_E_ARG, "advance_positions: B = %d", B);
  return hip_status(vm::launch_advance(positions, B, S(st)), "advance");
}

// ---- a8 -------------------------------------------------------------------
int vm_attention_fwd(vm_bf16* o, int64_t o_st, int64_t o_sh, int64_t o_sb, const vm_bf16* q,
                     int64_t q_st, int64_t q_sh, int64_t q_sb, const vm_bf16* k, int64_t k_st,
                     int64_t k_sh, int64_t k_sb, const vm_bf16* v, int64_t v_st, int64_t v_sh,
                     int64_t v_sb, const int32_t* k_lengths, const int32_t* q_lengths, int B,
                     int H, int Hk, int Dk, int Dv, int L, int Lk, int causal, vm_stream st) {
  TRY(check_head_any(Dk, "attention", "Dk"));
  TRY(check_head_any(Dv, "attention", "Dv"));
  TRY(check_gqa(H, Hk));
  REQUIRE(B >= 0 && L >= 0 && Lk >= 0, VM_E_ARG, "attention: B = %d, L = %d, Lk = %d", B, L, Lk);
  TRY(check_aligned(o, "O"));
  TRY(check_aligned(q, "Q"));
  TRY(check_aligned(k, "K"));
  TRY(check_aligned(v, "V"));
  for (int64_t s : {o_st, o_sh, o_sb, q_st, q_sh, q_sb, k_st, k_sh, k_sb, v_st, v_sh, v_sb})
    TRY(check_stride(s, "attention"));
  if (B == 0 || L == 0) return VM_OK;
  REQUIRE(Lk > 0, VM_E_ARG, "attention: k_len must be >= 1 (Lk = 0)");
  // the MFMA kernel takes D = 256 (Qwen3.5), 128 and 64
  const bool tuned = (Dk == vm::HEAD_DIM_ABI || Dk == 128 || Dk == 64) && Dv == Dk && k_st == v_st &&
                     k_sh == v_sh && k_sb == v_sb && k_st < ((int64_t)1 << 25);
  if (!tuned) {  // the generic kernel
    REQUIRE((int64_t)B * Hk <= 65535, VM_E_UNSUPPORTED, "attention: B*Hk = %lld > 65535",
            (long long)B * Hk);
    vm::AttnAnyArgs g{};
    g.q = q; g.q_st = q_st; g.q_sh = q_sh; g.q_sb = q_sb;
    g.k = k; g.k_st = k_st; g.k_sh = k_sh; g.k_sb = k_sb;
    g.v = v; g.v_st = v_st; g.v_sh = v_sh; g.v_sb = v_sb;
    g.o = o; g.o_st = o_st; g.o_sh = o_sh; g.o_sb = o_sb;
    g.k_lengths = k_lengths; g.q_lengths = q_lengths; g.part = nullptr;
    g.B = B; g.H = H; g.Hk = Hk; g.Dk = Dk; g.Dv = Dv; g.L = L; g.Lk = Lk;
    g.causal = causal ? 1 : 0; g.n_split = 1; g.split_keys = Lk;
    g.scale = 1.0f / sqrtf((float)Dk);
    return hip_status(timed(VM_K_PREFILL, S(st), [&] { return vm::launch_attn_any(g, S(st)); }),
                      "attention");
  }
  const int64_t kv_st = k_st, kv_sh = k_sh, kv_sb = k_sb;
  vm::PrefillArgs a{};
  a.q = q; a.q_st = q_st; a.q_sh = q_sh; a.q_sb = q_sb;
  a.k = k; a.v = v; a.kv_st = kv_st; a.kv_sh = kv_sh; a.kv_sb = kv_sb;
  a.o = o; a.o_st = o_st; a.o_sh = o_sh; a.o_sb = o_sb;
  a.k_lengths = k_lengths; a.q_lengths = q_lengths; a.prior = nullptr;
  a.B = B; a.H = H; a.Hk = Hk; a.L = L; a.Lk = Lk; a.causal = causal ? 1 : 0; a.D = Dk;
  a.n_qt = (L + vm::PREFILL_ROWS_ABI - 1) / vm::PREFILL_ROWS_ABI;
  return hip_status(timed(VM_K_PREFILL, S(st), [&] { return vm::launch_prefill(a, S(st)); }), "attention");
}

// ---- a9 -------------------------------------------------------------------
static int prefill_row_common(int B, int T, int Hq, int Hk, int D, int half_rot, int64_t ctx,
                              const void* qkv, int64_t qkv_st, int64_t qkv_sb) {
  TRY(check_head(D, half_rot));
  TRY(check_gqa(Hq, Hk));
  REQUIRE(B >= 0 && T >= 0 && ctx > 0, VM_E_ARG, "prefill: B = %d, T = %d, Ctx = %lld", B, T,
          (long long)ctx);
  TRY(check_aligned(qkv, "qkv"));
  TRY(check_stride(qkv_st, "qkv_st"));
  TRY(check_stride(qkv_sb, "qkv_sb"));
  REQUIRE(qkv_st >= (int64_t)(2 * Hq + 2 * Hk) * D || T <= 1, VM_E_DIM,
          "prefill: qkv token stride %lld < (2Hq+2Hk)*D = %lld", (long long)qkv_st,
          (long long)(2 * Hq + 2 * Hk) * D);
  return VM_OK;
}

// Argument checks of the prefill K/V append (shared by vm_prefill_kv_append and
// vm_gated_attn_prefill, which fuses the append into its V^T kernel).
static int prefill_kv_append_check(vm_bf16* kc, vm_bf16* vc, int64_t c_st, int64_t c_sh,
                                   int64_t c_sb, int64_t ctx, const vm_bf16* qkv, int64_t qkv_st,
                                   int64_t qkv_sb, const vm_bf16* kw, const float* cs,
                                   const float* sn, int B, int T, int Hq, int Hk, int D,
                                   int half_rot) {
  TRY(prefill_row_common(B, T, Hq, Hk, D, half_rot, ctx, qkv, qkv_st, qkv_sb));
  REQUIRE(kc && vc && kw && cs && sn, VM_E_ARG, "prefill_kv_append: NULL pointer argument");
  for (int64_t s : {c_st, c_sh, c_sb}) TRY(check_stride(s, "cache"));
  return VM_OK;
}

int vm_prefill_kv_append(vm_bf16* kc, vm_bf16* vc, int64_t c_st, int64_t c_sh, int64_t c_sb,
                         int64_t ctx, const vm_bf16* qkv, int64_t qkv_st, int64_t qkv_sb,
                         const vm_bf16* kw, const float* cs, const float* sn, const int32_t* prior,
                         const int32_t* q_lengths, int B, int T, int Hq, int Hk, int D,
                         int half_rot, float eps, float w_offset, vm_stream st) {
  TRY(prefill_kv_append_check(kc, vc, c_st, c_sh, c_sb, ctx, qkv, qkv_st, qkv_sb, kw, cs, sn, B, T,
                              Hq, Hk, D, half_rot));
  const int64_t Dl = D;
  vm::RowArgs r{};
  r.in = qkv + 2 * Hq * Dl; r.in2 = qkv + (2 * Hq + Hk) * Dl;
  r.in_st = qkv_st; r.in_sh = Dl; r.in_sb = qkv_sb;
  r.out = kc; r.out2 = vc; r.out_st = c_st; r.out_sh = c_sh; r.out_sb = c_sb;
  r.w = kw; r.cos_tab = cs; r.sin_tab = sn; r.ctx = ctx; r.positions = nullptr;
  r.prior = prior; r.q_lengths = q_lengths;
  r.B = B; r.H = Hk; r.T = T; r.out_at_pos = 1; r.eps = eps; r.w_offset = w_offset;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_norm_rope_rows(r, S(st)); }), "prefill_kv_append");
}

int vm_prefill_q_norm_rope(vm_bf16* q_out, int64_t q_st, int64_t q_sh, int64_t q_sb,
                           const vm_bf16* qkv, int64_t qkv_st, int64_t qkv_sb, const vm_bf16* qw,
                           const float* cs, const float* sn, const int32_t* prior,
                           const int32_t* q_lengths, int B, int T, int Hq, int Hk, int D,
                           int half_rot, float eps, float w_offset, vm_stream st) {
  // ctx is not known here: positions prior[b]+t must lie inside the tables (caller's contract)
  TRY(prefill_row_common(B, T, Hq, Hk, D, half_rot, INT64_MAX, qkv, qkv_st, qkv_sb));
  REQUIRE(q_out && qw && cs && sn, VM_E_ARG, "prefill_q_norm_rope: NULL pointer argument");
  for (int64_t s : {q_st, q_sh, q_sb}) TRY(check_stride(s, "q_out"));
  const int64_t Dl = D;
  vm::RowArgs r{};
  r.in = qkv; r.in2 = nullptr; r.in_st = qkv_st; r.in_sh = 2 * Dl; r.in_sb = qkv_sb;
  r.out = q_out; r.out_st = q_st; r.out_sh = q_sh; r.out_sb = q_sb;
  r.w = qw; r.cos_tab = cs; r.sin_tab = sn; r.ctx = INT64_MAX; r.positions = nullptr;
  r.prior = prior; r.q_lengths = q_lengths;
  r.B = B; r.H = Hq; r.T = T; r.out_at_pos = 0; r.eps = eps; r.w_offset = w_offset;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_norm_rope_rows(r, S(st)); }), "prefill_q_norm_rope");
}

// ---- a11 ------------------------------------------------------------------
static int64_t prefill_vt_tiles(int64_t ctx) {
  return (ctx + vm::PREFILL_VT_TILE_KEYS - 1) / vm::PREFILL_VT_TILE_KEYS;
}

size_t vm_prefill_scratch_bytes(int B, int Hk, int D, int64_t ctx) {
  if (B <= 0 || Hk <= 0 || D != vm::HEAD_DIM_ABI || ctx <= 0) return 0;
  return (size_t)B * Hk * prefill_vt_tiles(ctx) * vm::PREFILL_VT_TILE_BYTES;
}

// vm_gated_attn_prefill and vm_gated_attn_prefill_staged (vt_rows set)
static int gated_attn_prefill(vm_bf16* out, int64_t out_st, int64_t out_sb, const vm_bf16* qkv,
                              int64_t qkv_st, int64_t qkv_sb, vm_bf16* kc, vm_bf16* vc,
                              int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                              const vm_bf16* qw, const vm_bf16* kw, const float* cs,
                              const float* sn, const int32_t* prior, const int32_t* q_lengths,
                              int B, int T, int Hq, int Hk, int D, int half_rot, float eps,
                              float w_offset, int32_t* vt_rows, void* scratch,
                              size_t scratch_bytes, vm_stream st) {
  // every argument is checked before anything is launched
  REQUIRE(out && qw, VM_E_ARG, "gated_attn_prefill: NULL pointer argument");
  TRY(check_aligned(out, "out"));
  TRY(check_aligned(qw, "qw"));
  TRY(check_aligned(kc, "K_cache"));
  TRY(check_aligned(vc, "V_cache"));
  TRY(check_stride(out_st, "out_st"));
  TRY(check_stride(out_sb, "out_sb"));
  const bool work = B > 0 && T > 0;
  if (work) {
    REQUIRE(ctx < (int64_t)1 << 31, VM_E_ARG, "gated_attn_prefill: Ctx too large");
    REQUIRE(c_st < ((int64_t)1 << 25), VM_E_ARG,
            "gated_attn_prefill: cache token stride too large");
    const size_t need = vm_prefill_scratch_bytes(B, Hk, D, ctx);
    REQUIRE(scratch != nullptr && scratch_bytes >= need, VM_E_SCRATCH,
            "gated_attn_prefill: scratch of %zu bytes < %zu required (vm_prefill_scratch_bytes)",
            scratch_bytes, need);
    REQUIRE(((uintptr_t)scratch & 255) == 0, VM_E_ARG,
            "gated_attn_prefill: scratch must be 256-byte aligned");
  }
  // a9's checks; its append runs inside the V^T kernel below
  TRY(prefill_kv_append_check(kc, vc, c_st, c_sh, c_sb, ctx, qkv, qkv_st, qkv_sb, kw, cs, sn, B, T,
                              Hq, Hk, D, half_rot));
  if (!work) return VM_OK;
  const int64_t Dl = D;
  vm::PrefillArgs a{};
  a.q = qkv; a.q_st = qkv_st; a.q_sh = 2 * Dl; a.q_sb = qkv_sb;
  a.qw = qw; a.kw = kw; a.cos_tab = cs; a.sin_tab = sn; a.eps = eps; a.w_offset = w_offset;
  a.k = kc; a.v = vc; a.kv_st = c_st; a.kv_sh = c_sh; a.kv_sb = c_sb;
  a.o = out; a.o_st = out_st; a.o_sh = Dl; a.o_sb = out_sb;
  a.gate = qkv + Dl; a.g_st = qkv_st; a.g_sh = 2 * Dl; a.g_sb = qkv_sb;
  a.k_lengths = nullptr; a.q_lengths = q_lengths; a.prior = prior;
  a.B = B; a.H = Hq; a.Hk = Hk; a.L = T; a.Lk = (int)ctx; a.causal = 1;
  a.n_qt = (T + vm::PREFILL_ROWS_ABI - 1) / vm::PREFILL_ROWS_ABI;
  // one kernel: the chunk's K/V appended to the cache (a9) and the attended V
  // (prior + chunk) as V^T tiles in the workspace
  vm::VtArgs t{};
  t.v = vc; t.v_st = c_st; t.v_sh = c_sh; t.v_sb = c_sb;
  t.vt = reinterpret_cast<uint16_t*>(scratch); t.vt_tiles = (int)prefill_vt_tiles(ctx);
  t.prior = prior; t.q_lengths = q_lengths; t.vt_rows = vt_rows;
  t.B = B; t.Hk = Hk; t.L = T; t.ctx = ctx;
  t.kc = kc; t.k_raw = qkv + 2 * Hq * Dl; t.v_raw = qkv + (2 * Hq + Hk) * Dl;
  t.raw_st = qkv_st; t.raw_sh = Dl; t.raw_sb = qkv_sb;
  t.kw = kw; t.cos_tab = cs; t.sin_tab = sn; t.eps = eps; t.w_offset = w_offset;
  TRY(hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_vt_transpose(t, S(st)); }),
                 "gated_attn_prefill append"));
  a.vt = t.vt; a.vt_tiles = t.vt_tiles;
  return hip_status(timed_ext(VM_K_PREFILL, S(st),
                              [&](hipEvent_t t0, hipEvent_t t1) { return vm::launch_prefill_fused(a, S(st), t0, t1); }),
                    "gated_attn_prefill");
}

int vm_gated_attn_prefill(vm_bf16* out, int64_t out_st, int64_t out_sb, const vm_bf16* qkv,
                          int64_t qkv_st, int64_t qkv_sb, vm_bf16* kc, vm_bf16* vc, int64_t c_st,
                          int64_t c_sh, int64_t c_sb, int64_t ctx, const vm_bf16* qw,
                          const vm_bf16* kw, const float* cs, const float* sn,
                          const int32_t* prior, const int32_t* q_lengths, int B, int T, int Hq,
                          int Hk, int D, int half_rot, float eps, float w_offset, void* scratch,
                          size_t scratch_bytes, vm_stream st) {
  return gated_attn_prefill(out, out_st, out_sb, qkv, qkv_st, qkv_sb, kc, vc, c_st, c_sh, c_sb, ctx,
                            qw, kw, cs, sn, prior, q_lengths, B, T, Hq, Hk, D, half_rot, eps,
                            w_offset, nullptr, scratch, scratch_bytes, st);
}

int vm_gated_attn_prefill_staged(vm_bf16* out, int64_t out_st, int64_t out_sb, const vm_bf16* qkv,
                                 int64_t qkv_st, int64_t qkv_sb, vm_bf16* kc, vm_bf16* vc,
                                 int64_t c_st, int64_t c_sh, int64_t c_sb, int64_t ctx,
                                 const vm_bf16* qw, const vm_bf16* kw, const float* cs,
                                 const float* sn, const int32_t* prior, const int32_t* q_lengths,
                                 int B, int T, int Hq, int Hk, int D, int half_rot, float eps,
                                 float w_offset, int32_t* vt_rows, void* vt, size_t vt_bytes,
                                 vm_stream st) {
  REQUIRE(vt_rows != nullptr, VM_E_ARG, "gated_attn_prefill_staged: NULL vt_rows");
  REQUIRE(((uintptr_t)vt_rows & 3) == 0, VM_E_ARG,
          "gated_attn_prefill_staged: vt_rows must be 4-byte aligned");
  return gated_attn_prefill(out, out_st, out_sb, qkv, qkv_st, qkv_sb, kc, vc, c_st, c_sh, c_sb, ctx,
                            qw, kw, cs, sn, prior, q_lengths, B, T, Hq, Hk, D, half_rot, eps,
                            w_offset, vt_rows, vt, vt_bytes, st);
}

// ---- f2: the rest of the decode step ----------------------------------------
static int check_rows(int M, int N, int64_t st, const char* what, const char* name) {
  REQUIRE(M > 0 && M % 8 == 0 && M <= 16384, VM_E_UNSUPPORTED,
          "%s: M = %d (a multiple of 8, at most 16384)", what, M);
  REQUIRE(N >= 0, VM_E_ARG, "%s: N = %d", what, N);
  TRY(check_stride(st, name));
  REQUIRE(N <= 1 || st >= M, VM_E_DIM, "%s: column stride %s = %lld < M = %d", what, name,
          (long long)st, M);
  return VM_OK;
}

int vm_rms_norm(vm_bf16* y, int64_t y_st, const vm_bf16* x, int64_t x_st, const vm_bf16* w, int M,
                int N, float eps, float offset, vm_stream st) {
  TRY(check_aligned(y, "Y"));
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(w, "W"));
  TRY(check_rows(M, N, y_st, "rms_norm", "y_st"));
  TRY(check_rows(M, N, x_st, "rms_norm", "x_st"));
  vm::NormArgs a{};
  a.y = y; a.y_st = y_st; a.x = x; a.x_st = x_st; a.w = w;
  a.M = M; a.N = N; a.offset = offset; a.eps = eps;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_rms_norm(a, S(st)); }), "rms_norm");
}

int vm_fused_add_rms_norm(vm_bf16* y, int64_t y_st, vm_bf16* xo, int64_t xo_st, const vm_bf16* x,
                          int64_t x_st, const vm_bf16* dx, int64_t dx_st, const vm_bf16* w, int M,
                          int N, float eps, float offset, vm_stream st) {
  TRY(check_aligned(y, "Y"));
  TRY(check_aligned(xo, "X_out"));
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(dx, "dX"));
  TRY(check_aligned(w, "W"));
  TRY(check_rows(M, N, y_st, "fused_add_rms_norm", "y_st"));
  TRY(check_rows(M, N, xo_st, "fused_add_rms_norm", "xo_st"));
  TRY(check_rows(M, N, x_st, "fused_add_rms_norm", "x_st"));
  TRY(check_rows(M, N, dx_st, "fused_add_rms_norm", "dx_st"));
  REQUIRE(xo != x || xo_st == x_st, VM_E_ARG,
          "fused_add_rms_norm: X_out aliases X with a different column stride");
  vm::NormArgs a{};
  a.y = y; a.y_st = y_st; a.xo = xo; a.xo_st = xo_st; a.x = x; a.x_st = x_st;
  a.dx = dx; a.dx_st = dx_st; a.w = w;
  a.M = M; a.N = N; a.offset = offset; a.eps = eps;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_rms_norm(a, S(st)); }),
                    "fused_add_rms_norm");
}

int vm_silu_mul(vm_bf16* mid, int64_t mid_st, const vm_bf16* gu, int64_t gu_st, int I, int N,
                vm_stream st) {
  TRY(check_aligned(mid, "mid"));
  TRY(check_aligned(gu, "gu"));
  REQUIRE(I > 0 && I % 8 == 0, VM_E_UNSUPPORTED, "silu_mul: I = %d (a multiple of 8)", I);
  REQUIRE(N >= 0, VM_E_ARG, "silu_mul: N = %d", N);
  TRY(check_stride(mid_st, "mid_st"));
  TRY(check_stride(gu_st, "gu_st"));
  REQUIRE(N <= 1 || (mid_st >= I && gu_st >= 2 * (int64_t)I), VM_E_DIM,
          "silu_mul: column strides (mid %lld, gu %lld) below (I, 2I) = (%d, %d)",
          (long long)mid_st, (long long)gu_st, I, 2 * I);
  vm::SiluMulArgs a{};
  a.mid = mid; a.mid_st = mid_st; a.gu = gu; a.gu_st = gu_st; a.I = I; a.N = N;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_silu_mul(a, S(st)); }), "silu_mul");
}

int vm_embed(vm_bf16* x, int64_t x_st, const vm_bf16* e, int64_t e_st, const int32_t* ids, int D,
             int B, int vocab, vm_stream st) {
  TRY(check_aligned(x, "x"));
  TRY(check_aligned(e, "E"));
  REQUIRE(ids || B == 0, VM_E_ARG, "embed: ids is NULL");
  REQUIRE(D > 0 && D % 8 == 0, VM_E_UNSUPPORTED, "embed: D = %d (a multiple of 8)", D);
  REQUIRE(B >= 0 && vocab > 0, VM_E_ARG, "embed: B = %d, vocab = %d", B, vocab);
  TRY(check_stride(x_st, "x_st"));
  TRY(check_stride(e_st, "e_st"));
  REQUIRE((B <= 1 || x_st >= D) && (vocab <= 1 || e_st >= D), VM_E_DIM,
          "embed: column strides (x %lld, E %lld) below D = %d", (long long)x_st, (long long)e_st, D);
  vm::EmbedArgs a{};
  a.x = x; a.x_st = x_st; a.e = e; a.e_st = e_st; a.ids = ids; a.D = D; a.B = B; a.vocab = vocab;
  return hip_status(vm::launch_embed(a, S(st)), "embed");
}

int vm_generation_advance(int32_t* tokens_out, const int32_t* col_offsets, int32_t* step,
                          int32_t* positions, const int32_t* result, int B, int max_new,
                          vm_stream st) {
  REQUIRE(step, VM_E_ARG, "generation_advance: step is NULL");
  REQUIRE(B >= 0 && B <= 1 << 20, VM_E_ARG, "generation_advance: B = %d", B);
  REQUIRE(B == 0 || (tokens_out && col_offsets && positions && result), VM_E_ARG,
          "generation_advance: NULL pointer argument");
  REQUIRE(max_new >= 0, VM_E_ARG, "generation_advance: max_new = %d", max_new);
  vm::AdvanceArgs a{};
  a.tokens_out = tokens_out; a.col_offsets = col_offsets; a.step = step; a.positions = positions;
  a.result = result; a.B = B; a.max_new = max_new;
  return hip_status(vm::launch_gen_advance(a, S(st)), "generation_advance");
}

// ---- f3: lm_head_argmax ------------------------------------------------------
size_t vm_lm_head_argmax_scratch_bytes(int K, int N, int B) {
  if (K <= 0 || N <= 0 || B < 0) return 0;
  return (size_t)vm::lm_head_waves() * (size_t)B * (sizeof(float) + sizeof(int32_t));
}

int vm_lm_head_argmax(int32_t* result, const vm_bf16* x, int64_t x_st, const vm_bf16* w,
                      int64_t w_st, int K, int N, int B, void* scratch, size_t scratch_bytes,
                      vm_stream st) {
  REQUIRE(result || B == 0, VM_E_ARG, "lm_head_argmax: Result is NULL");
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(w, "W"));
  REQUIRE(K > 0 && K % 64 == 0, VM_E_UNSUPPORTED, "lm_head_argmax: K = %d (a multiple of 64)",
          K);
  REQUIRE(N > 0 && B >= 0, VM_E_ARG, "lm_head_argmax: N = %d, B = %d", N, B);
  TRY(check_stride(x_st, "x_st"));
  TRY(check_stride(w_st, "w_st"));
  REQUIRE((B <= 1 || x_st >= K) && (N <= 1 || w_st >= K), VM_E_DIM,
          "lm_head_argmax: column strides (X %lld, W %lld) below K = %d", (long long)x_st,
          (long long)w_st, K);
  if (B == 0) return VM_OK;
  const size_t need = vm_lm_head_argmax_scratch_bytes(K, N, B);
  REQUIRE(scratch != nullptr && scratch_bytes >= need, VM_E_SCRATCH,
          "lm_head_argmax: scratch of %zu bytes < %zu required (vm_lm_head_argmax_scratch_bytes)",
          scratch_bytes, need);
  REQUIRE(((uintptr_t)scratch & 15) == 0, VM_E_ARG, "lm_head_argmax: scratch must be 16-byte aligned");
  vm::LmHeadArgs a{};
  a.x = x; a.x_st = x_st; a.w = w; a.w_st = w_st; a.K = K; a.N = N; a.B = B;
  a.NW = vm::lm_head_waves();
  a.pmax = reinterpret_cast<float*>(scratch);
  a.pidx = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(scratch) +
                                      (size_t)a.NW * B * sizeof(float));
  a.result = result;
  return hip_status(timed(VM_K_LM_HEAD, S(st), [&] { return vm::launch_lm_head_argmax(a, S(st)); }),
                    "lm_head_argmax");
}

// ---- f1: linear ------------------------------------------------------------
static int linear_check(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  REQUIRE(M > 0 && N > 0 && K > 0, VM_E_ARG, "linear: M = %d, N = %d, K = %d", M, N, K);
  REQUIRE(ldw >= K && ldx >= K && ldy >= M, VM_E_DIM,
          "linear: leading dimensions (W %lld, x %lld, y %lld) below (K, K, M) = (%d, %d, %d)",
          (long long)ldw, (long long)ldx, (long long)ldy, K, K, M);
  return VM_OK;
}

size_t vm_linear_workspace_bytes(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  if (linear_check(M, N, K, ldw, ldx, ldy) != VM_OK) return (size_t)-1;
  size_t n = 0;
  if (vm::linear_workspace(M, N, K, ldw, ldx, ldy, &n, g_err, sizeof g_err) != VM_OK)
    return (size_t)-1;
  return n;
}

int vm_linear_tune(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  TRY(linear_check(M, N, K, ldw, ldx, ldy));
  return vm::linear_tune(M, N, K, ldw, ldx, ldy, g_err, sizeof g_err);
}

int vm_linear_plan_state(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  return vm::linear_plan_state(M, N, K, ldw, ldx, ldy);
}

int vm_linear(vm_bf16* y, int64_t ldy, const vm_bf16* x, int64_t ldx, const vm_bf16* w,
              int64_t ldw, int M, int N, int K, void* workspace, size_t workspace_bytes,
              vm_stream st) {
  TRY(linear_check(M, N, K, ldw, ldx, ldy));
  REQUIRE(y && x && w, VM_E_ARG, "linear: NULL pointer argument");
  return vm::linear_run(y, ldy, x, ldx, w, ldw, M, N, K, workspace, workspace_bytes, S(st), g_err,
                        sizeof g_err);
}

// ---- f4: the linear-attention layer parts -----------------------------------
namespace {
int check_dn_heads(int Dk, int Dv, int Hk, int Hv, int B, const char* what) {
  REQUIRE(Dk == 128 && Dv == 128, VM_E_UNSUPPORTED,
          "%s: Dk = %d, Dv = %d; the kernels are built for Dk = Dv = 128", what, Dk, Dv);
  REQUIRE(Hk > 0 && Hv > 0 && B >= 0, VM_E_ARG, "%s: Hk = %d, Hv = %d, B = %d", what, Hk, Hv, B);
  REQUIRE(Hv % Hk == 0, VM_E_DIM, "value heads (%d) is not a multiple of key heads (%d)", Hv, Hk);
  return VM_OK;
}
// the operators' generic forms: Dk, Dv multiples of 16 up to 256
int check_dn_heads_any(int Dk, int Dv, int Hk, int Hv, int B, const char* what) {
  REQUIRE(Dk >= 16 && Dk <= 256 && Dk % 16 == 0 && Dv >= 16 && Dv <= 256 && Dv % 16 == 0,
          VM_E_UNSUPPORTED, "%s: Dk = %d, Dv = %d (multiples of 16 up to 256)", what, Dk, Dv);
  REQUIRE(Hk > 0 && Hv > 0 && B >= 0, VM_E_ARG, "%s: Hk = %d, Hv = %d, B = %d", what, Hk, Hv, B);
  REQUIRE(Hv % Hk == 0, VM_E_DIM, "value heads (%d) is not a multiple of key heads (%d)", Hv, Hk);
  REQUIRE((int64_t)B <= 65535, VM_E_UNSUPPORTED, "%s: B = %d > 65535", what, B);
  return VM_OK;
}
bool dn_tuned(int Dk, int Dv) { return Dk == 128 && Dv == 128; }
// the state out either is the state in (in place) or does not overlap it
int check_alias(const void* in, const void* out, size_t bytes, const char* what) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(in), b = reinterpret_cast<uintptr_t>(out);
  REQUIRE(a == b || a + bytes <= b || b + bytes <= a, VM_E_ARG,
          "%s: state out partially overlaps state in (alias exactly or not at all)", what);
  return VM_OK;
}
int check_align8(const void* p, int64_t stride, const char* name) {
  REQUIRE(p != nullptr, VM_E_ARG, "%s is NULL", name);
  REQUIRE((reinterpret_cast<uintptr_t>(p) & 7u) == 0 && stride >= 0 && stride % 4 == 0, VM_E_ARG,
          "%s must be 8-byte aligned with a sequence stride that is a multiple of 4", name);
  return VM_OK;
}
int check_conv(int D, int K, int B, int T, const char* what) {
  REQUIRE(D > 0 && D % 8 == 0, VM_E_UNSUPPORTED, "%s: D = %d must be a positive multiple of 8",
          what, D);
  REQUIRE(K >= 1 && K <= 8, VM_E_UNSUPPORTED, "%s: kernel size K = %d outside 1..8", what, K);
  REQUIRE(B >= 0 && T >= 0, VM_E_ARG, "%s: B = %d, T = %d", what, B, T);
  return VM_OK;
}
}  // namespace

int vm_causal_conv1d(vm_bf16* y, int64_t y_sb, const vm_bf16* x, int64_t x_sb,
                     const vm_bf16* s_in, vm_bf16* s_out, int64_t s_cs, int64_t s_sb,
                     const vm_bf16* w, int64_t w_cs, const vm_bf16* bias, int D, int K, int B,
                     int act, vm_stream st) {
  TRY(check_conv(D, K, B, 1, "causal_conv1d"));
  if (B == 0) return VM_OK;
  TRY(check_aligned(y, "Y"));
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(s_in, "S"));
  TRY(check_aligned(s_out, "S_out"));
  TRY(check_aligned(w, "Weight"));
  if (bias) TRY(check_aligned(bias, "Bias"));
  for (int64_t v : {y_sb, x_sb, s_cs, s_sb, w_cs}) TRY(check_stride(v, "causal_conv1d"));
  REQUIRE(s_cs >= D && w_cs >= D && (B <= 1 || (s_sb >= s_cs * K && y_sb >= D && x_sb >= D)),
          VM_E_DIM, "causal_conv1d: strides below the extents (D = %d, K = %d)", D, K);
  TRY(check_alias(s_in, s_out, (size_t)((B - 1) * s_sb + (K - 1) * s_cs + D) * 2, "causal_conv1d"));
  vm::Conv1dArgs a{};
  a.y = y; a.y_sb = y_sb; a.x = x; a.x_sb = x_sb; a.s_in = s_in; a.s_out = s_out;
  a.s_cs = s_cs; a.s_sb = s_sb; a.w = w; a.w_cs = w_cs; a.bias = bias;
  a.D = D; a.K = K; a.T = 1; a.B = B; a.act = act ? 1 : 0;
  return hip_status(timed(VM_K_CONV, S(st), [&] { return vm::launch_conv1d_update(a, S(st)); }),
                    "causal_conv1d");
}

int vm_causal_conv1d_sequence(vm_bf16* y, int64_t y_st, int64_t y_sb, const vm_bf16* x,
                              int64_t x_st, int64_t x_sb, const vm_bf16* w, int64_t w_cs,
                              const vm_bf16* bias, const vm_bf16* s_in, vm_bf16* s_out,
                              int64_t s_cs, int64_t s_sb, int D, int K, int T, int B, int act,
                              vm_stream st) {
  TRY(check_conv(D, K, B, T, "causal_conv1d_sequence"));
  if (B == 0 || T == 0) return VM_OK;
  TRY(check_aligned(y, "Y"));
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(w, "Weight"));
  if (bias) TRY(check_aligned(bias, "Bias"));
  if (s_in) TRY(check_aligned(s_in, "S"));
  if (s_out) TRY(check_aligned(s_out, "S_out"));
  for (int64_t v : {y_st, y_sb, x_st, x_sb, w_cs, s_cs, s_sb})
    TRY(check_stride(v, "causal_conv1d_sequence"));
  REQUIRE(w_cs >= D && (T <= 1 || (y_st >= D && x_st >= D)) &&
              (B <= 1 || (y_sb >= y_st * T && x_sb >= x_st * T)),
          VM_E_DIM, "causal_conv1d_sequence: strides below the extents (D = %d, T = %d)", D, T);
  if (s_in || s_out)
    REQUIRE(s_cs >= D && (B <= 1 || s_sb >= s_cs * K), VM_E_DIM,
            "causal_conv1d_sequence: state strides below (D, K) = (%d, %d)", D, K);
  if (s_in && s_out)
    TRY(check_alias(s_in, s_out, (size_t)((B - 1) * s_sb + (K - 1) * s_cs + D) * 2,
                    "causal_conv1d_sequence"));
  vm::Conv1dArgs a{};
  a.y = y; a.y_st = y_st; a.y_sb = y_sb; a.x = x; a.x_st = x_st; a.x_sb = x_sb;
  a.s_in = s_in; a.s_out = s_out; a.s_cs = s_cs; a.s_sb = s_sb; a.w = w; a.w_cs = w_cs;
  a.bias = bias; a.D = D; a.K = K; a.T = T; a.B = B; a.act = act ? 1 : 0;
  return hip_status(timed(VM_K_CONV, S(st), [&] { return vm::launch_conv1d_sequence(a, S(st)); }),
                    "causal_conv1d_sequence");
}

int vm_fused_deltanet_decode(vm_bf16* o, int64_t o_sb, const vm_bf16* q, int64_t q_sb,
                             const vm_bf16* k, int64_t k_sb, const vm_bf16* v, int64_t v_sb,
                             const vm_bf16* alpha, int64_t a_sb, const vm_bf16* beta_raw,
                             int64_t b_sb, const vm_bf16* z, int64_t z_sb, const float* a_log,
                             const float* dt_bias, const vm_bf16* norm_w, const float* s_in,
                             float* s_out, int Dk, int Dv, int Hk, int Hv, int B, float eps,
                             vm_stream st) {
  TRY(check_dn_heads_any(Dk, Dv, Hk, Hv, B, "fused_deltanet_decode"));
  if (B == 0) return VM_OK;
  REQUIRE(o && v && z && alpha && beta_raw && a_log && dt_bias && norm_w, VM_E_ARG,
          "fused_deltanet_decode: NULL pointer argument");
  TRY(check_align8(q, q_sb, "Q_raw"));
  TRY(check_align8(k, k_sb, "K_raw"));
  TRY(check_aligned(s_in, "S"));
  TRY(check_aligned(s_out, "S_out"));
  REQUIRE(B <= 1 || (q_sb >= (int64_t)Hk * Dk && k_sb >= (int64_t)Hk * Dk &&
                     v_sb >= (int64_t)Hv * Dv && z_sb >= (int64_t)Hv * Dv &&
                     o_sb >= (int64_t)Hv * Dv && a_sb >= Hv && b_sb >= Hv),
          VM_E_DIM, "fused_deltanet_decode: sequence strides below the head extents");
  const size_t sbytes = (size_t)B * Hv * Dk * Dv * sizeof(float);
  TRY(check_alias(s_in, s_out, sbytes, "fused_deltanet_decode"));
  vm::DeltaFusedArgs a{};
  a.o = o; a.o_sb = o_sb; a.q = q; a.q_sb = q_sb; a.k = k; a.k_sb = k_sb; a.v = v; a.v_sb = v_sb;
  a.z = z; a.z_sb = z_sb; a.alpha = alpha; a.a_sb = a_sb; a.beta = beta_raw; a.b_sb = b_sb;
  a.a_log = a_log; a.dt_bias = dt_bias; a.norm_w = norm_w; a.s_in = s_in; a.s_out = s_out;
  a.Hk = Hk; a.Hv = Hv; a.B = B; a.eps = eps;
  if (!dn_tuned(Dk, Dv))
    return hip_status(timed(VM_K_DELTANET, S(st),
                            [&] { return vm::launch_deltanet_any(nullptr, &a, Dk, Dv, S(st)); }),
                      "fused_deltanet_decode");
  return hip_status(
      timed(VM_K_DELTANET, S(st), [&] { return vm::launch_deltanet_fused_decode(a, S(st)); }),
      "fused_deltanet_decode");
}

static int deltanet_seq(float* o, const float* q, const float* k, const float* v,
                        const float* beta, const float* gate, const float* s_in, float* s_out,
                        int Dk, int Dv, int T, int Hk, int Hv, int B, vm_stream st,
                        const char* what) {
  TRY(check_dn_heads_any(Dk, Dv, Hk, Hv, B, what));
  REQUIRE(T >= 0, VM_E_ARG, "%s: T = %d", what, T);
  if (B == 0) return VM_OK;
  TRY(check_aligned(s_in, "S"));
  TRY(check_aligned(s_out, "S_out"));
  TRY(check_alias(s_in, s_out, (size_t)B * Hv * Dk * Dv * sizeof(float), what));
  if (T > 0) {
    TRY(check_aligned(o, "O"));
    TRY(check_aligned(q, "Q"));
    TRY(check_aligned(k, "K"));
    TRY(check_aligned(v, "V"));
    REQUIRE(beta && gate, VM_E_ARG, "%s: NULL Beta or Gate", what);
  }
  vm::DeltaSeqArgs a{};
  a.o = o; a.q = q; a.k = k; a.v = v; a.beta = beta; a.gate = gate; a.s_in = s_in;
  a.s_out = s_out; a.T = T; a.Hk = Hk; a.Hv = Hv; a.B = B;
  if (!dn_tuned(Dk, Dv))
    return hip_status(timed(VM_K_DELTANET, S(st),
                            [&] { return vm::launch_deltanet_any(&a, nullptr, Dk, Dv, S(st)); }),
                      what);
  return hip_status(
      timed(VM_K_DELTANET, S(st), [&] { return vm::launch_deltanet_sequence(a, S(st)); }), what);
}

int vm_deltanet_recurrent_decode(float* o, const float* q, const float* k, const float* v,
                                 const float* beta, const float* gate, const float* s_in,
                                 float* s_out, int Dk, int Dv, int Hk, int Hv, int B,
                                 vm_stream st) {
  return deltanet_seq(o, q, k, v, beta, gate, s_in, s_out, Dk, Dv, 1, Hk, Hv, B, st,
                      "deltanet_recurrent_decode");
}

int vm_deltanet_sequence(float* o, const float* q, const float* k, const float* v,
                         const float* beta, const float* gate, const float* s_in, float* s_out,
                         int Dk, int Dv, int T, int Hk, int Hv, int B, vm_stream st) {
  return deltanet_seq(o, q, k, v, beta, gate, s_in, s_out, Dk, Dv, T, Hk, Hv, B, st,
                      "deltanet_sequence");
}

size_t vm_deltanet_sequence_workspace_bytes(int T, int Hv, int B) {
  if (T < 0 || Hv <= 0 || B < 0) return (size_t)-1;
  return vm::deltanet_chunk_workspace_bytes(T, Hv, B);
}

namespace {
// the chunked recurrence; with g.y set, the gated RMSNorm fused into its output
// phase (o unused)
int deltanet_chunked(const char* what, float* o, const float* q, const float* k, const float* v,
                     const float* beta, const float* gate, const float* s_in, float* s_out, int Dk,
                     int Dv, int T, int Hk, int Hv, int B, void* workspace, size_t workspace_bytes,
                     const vm::GatedNormArgs& g, vm_stream st) {
  TRY(check_dn_heads(Dk, Dv, Hk, Hv, B, what));
  REQUIRE(T >= 0, VM_E_ARG, "%s: T = %d", what, T);
  if (B == 0) return VM_OK;
  TRY(check_aligned(s_in, "S"));
  TRY(check_aligned(s_out, "S_out"));
  TRY(check_alias(s_in, s_out, (size_t)B * Hv * Dk * Dv * sizeof(float), what));
  if (T > 0) {
    if (!g.y) TRY(check_aligned(o, "O"));
    TRY(check_aligned(q, "Q"));
    TRY(check_aligned(k, "K"));
    TRY(check_aligned(v, "V"));
    REQUIRE(beta && gate, VM_E_ARG, "%s: NULL Beta or Gate", what);
    const size_t need = vm::deltanet_chunk_workspace_bytes(T, Hv, B);
    REQUIRE(workspace && workspace_bytes >= need && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
            VM_E_SCRATCH, "%s: workspace of %zu bytes (256-byte aligned) < %zu required "
            "(vm_deltanet_sequence_workspace_bytes)", what, workspace_bytes, need);
  }
  vm::DeltaChunkArgs a{};
  a.s.o = o; a.s.q = q; a.s.k = k; a.s.v = v; a.s.beta = beta; a.s.gate = gate; a.s.s_in = s_in;
  a.s.s_out = s_out; a.s.T = T; a.s.Hk = Hk; a.s.Hv = Hv; a.s.B = B;
  a.ws = static_cast<float*>(workspace);
  a.g = g;
  return hip_status(
      timed(VM_K_DELTANET, S(st), [&] { return vm::launch_deltanet_sequence_chunked(a, S(st)); }),
      what);
}
}  // namespace

int vm_deltanet_sequence_chunked(float* o, const float* q, const float* k, const float* v,
                                 const float* beta, const float* gate, const float* s_in,
                                 float* s_out, int Dk, int Dv, int T, int Hk, int Hv, int B,
                                 void* workspace, size_t workspace_bytes, vm_stream st) {
  const vm::GatedNormArgs none{};
  return deltanet_chunked("deltanet_sequence_chunked", o, q, k, v, beta, gate, s_in, s_out, Dk, Dv,
                          T, Hk, Hv, B, workspace, workspace_bytes, none, st);
}

int vm_deltanet_sequence_chunked_gated_norm(vm_bf16* y, int64_t y_st, int64_t y_sb,
                                            const vm_bf16* z, int64_t z_st, int64_t z_sb,
                                            const vm_bf16* norm_w, float eps, const float* q,
                                            const float* k, const float* v, const float* beta,
                                            const float* gate, const float* s_in, float* s_out,
                                            int Dk, int Dv, int T, int Hk, int Hv, int B,
                                            void* workspace, size_t workspace_bytes, vm_stream st) {
  const char* what = "deltanet_sequence_chunked_gated_norm";
  TRY(check_dn_heads(Dk, Dv, Hk, Hv, B, what));
  REQUIRE(T >= 0, VM_E_ARG, "%s: T = %d", what, T);
  if (B > 0 && T > 0) {
    REQUIRE(y && z && norm_w, VM_E_ARG, "%s: NULL Y, Z or NormWeight", what);
    for (const void* p : {(const void*)y, (const void*)z, (const void*)norm_w})
      REQUIRE((reinterpret_cast<uintptr_t>(p) & 1u) == 0, VM_E_ARG, "%s: Y, Z and NormWeight must "
              "be 2-byte aligned", what);
    REQUIRE(y_st >= 0 && y_sb >= 0 && z_st >= 0 && z_sb >= 0, VM_E_ARG, "%s: negative stride",
            what);
    REQUIRE((T <= 1 || (y_st >= (int64_t)Hv * Dv && z_st >= (int64_t)Hv * Dv)) &&
                (B <= 1 || (y_sb >= y_st * T && z_sb >= z_st * T)),
            VM_E_DIM, "%s: strides below the extents", what);
  }
  vm::GatedNormArgs g{};
  g.z = z; g.z_st = z_st; g.z_sb = z_sb; g.norm_w = norm_w; g.y = y; g.y_st = y_st; g.y_sb = y_sb;
  g.T = T; g.Hv = Hv; g.B = B; g.eps = eps;
  return deltanet_chunked(what, nullptr, q, k, v, beta, gate, s_in, s_out, Dk, Dv, T, Hk, Hv, B,
                          workspace, workspace_bytes, g, st);
}

int vm_deltanet_prefill_prep(float* qe, float* ke, float* ve, float* beta, float* gate,
                             const vm_bf16* cv, int64_t cv_st, int64_t cv_sb, const vm_bf16* ab,
                             int64_t ab_st, int64_t ab_sb, const float* a_log,
                             const float* dt_bias, int Dk, int Dv, int Hk, int Hv, int T, int B,
                             vm_stream st) {
  TRY(check_dn_heads(Dk, Dv, Hk, Hv, B, "deltanet_prefill_prep"));
  REQUIRE(T >= 0, VM_E_ARG, "deltanet_prefill_prep: T = %d", T);
  if (B == 0 || T == 0) return VM_OK;
  REQUIRE(qe && ke && ve && beta && gate && ab && a_log && dt_bias, VM_E_ARG,
          "deltanet_prefill_prep: NULL pointer argument");
  TRY(check_align8(cv, cv_st, "conv output"));
  REQUIRE(cv_sb % 4 == 0, VM_E_ARG, "deltanet_prefill_prep: conv sequence stride %% 4 != 0");
  for (const float* p : {qe, ke, ve})
    REQUIRE((reinterpret_cast<uintptr_t>(p) & 7u) == 0, VM_E_ARG,
            "deltanet_prefill_prep: fp32 outputs must be 8-byte aligned");
  const int64_t n = 2LL * Hk * Dk + (int64_t)Hv * Dv;
  REQUIRE((T <= 1 || (cv_st >= n && ab_st >= 2LL * Hv)) &&
              (B <= 1 || (cv_sb >= cv_st * T && ab_sb >= ab_st * T)),
          VM_E_DIM, "deltanet_prefill_prep: strides below the extents (n = %lld)", (long long)n);
  vm::DeltaPrepArgs a{};
  a.cv = cv; a.cv_st = cv_st; a.cv_sb = cv_sb; a.ab = ab; a.ab_st = ab_st; a.ab_sb = ab_sb;
  a.a_log = a_log; a.dt_bias = dt_bias; a.qe = qe; a.ke = ke; a.ve = ve; a.beta = beta;
  a.gate = gate; a.T = T; a.Hk = Hk; a.Hv = Hv; a.B = B;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_deltanet_prep(a, S(st)); }),
                    "deltanet_prefill_prep");
}

int vm_deltanet_conv_prep(float* qe, float* ke, float* ve, float* beta, float* gate,
                          const vm_bf16* x, int64_t x_st, int64_t x_sb, const vm_bf16* w,
                          int64_t w_cs, const vm_bf16* bias, const vm_bf16* s_in, vm_bf16* s_out,
                          int64_t s_cs, int64_t s_sb, int K, const vm_bf16* ab, int64_t ab_st,
                          int64_t ab_sb, const float* a_log, const float* dt_bias, int Dk, int Dv,
                          int Hk, int Hv, int T, int B, vm_stream st) {
  TRY(check_dn_heads(Dk, Dv, Hk, Hv, B, "deltanet_conv_prep"));
  const int D = 2 * Hk * Dk + Hv * Dv;
  TRY(check_conv(D, K, B, T, "deltanet_conv_prep"));
  if (B == 0 || T == 0) return VM_OK;
  REQUIRE(qe && ke && ve && beta && gate && ab && a_log && dt_bias, VM_E_ARG,
          "deltanet_conv_prep: NULL pointer argument");
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(w, "Weight"));
  if (bias) TRY(check_aligned(bias, "Bias"));
  if (s_in) TRY(check_aligned(s_in, "S"));
  if (s_out) TRY(check_aligned(s_out, "S_out"));
  for (const float* p : {qe, ke, ve})
    REQUIRE((reinterpret_cast<uintptr_t>(p) & 15u) == 0, VM_E_ARG,
            "deltanet_conv_prep: fp32 outputs must be 16-byte aligned");
  for (int64_t v : {x_st, x_sb, w_cs, s_cs, s_sb}) TRY(check_stride(v, "deltanet_conv_prep"));
  REQUIRE(ab_st >= 0 && ab_sb >= 0, VM_E_ARG, "deltanet_conv_prep: negative ab stride");
  REQUIRE(w_cs >= D && (T <= 1 || (x_st >= D && ab_st >= 2LL * Hv)) &&
              (B <= 1 || (x_sb >= x_st * T && ab_sb >= ab_st * T)),
          VM_E_DIM, "deltanet_conv_prep: strides below the extents (n = %d, T = %d)", D, T);
  if (s_in || s_out)
    REQUIRE(s_cs >= D && (B <= 1 || s_sb >= s_cs * K), VM_E_DIM,
            "deltanet_conv_prep: state strides below (n, K) = (%d, %d)", D, K);
  if (s_in && s_out)
    TRY(check_alias(s_in, s_out, (size_t)((B - 1) * s_sb + (K - 1) * s_cs + D) * 2,
                    "deltanet_conv_prep"));
  vm::ConvPrepArgs a{};
  a.c.x = x; a.c.x_st = x_st; a.c.x_sb = x_sb; a.c.s_in = s_in; a.c.s_out = s_out;
  a.c.s_cs = s_cs; a.c.s_sb = s_sb; a.c.w = w; a.c.w_cs = w_cs; a.c.bias = bias;
  a.c.D = D; a.c.K = K; a.c.T = T; a.c.B = B; a.c.act = 1;
  a.p.ab = ab; a.p.ab_st = ab_st; a.p.ab_sb = ab_sb; a.p.a_log = a_log; a.p.dt_bias = dt_bias;
  a.p.qe = qe; a.p.ke = ke; a.p.ve = ve; a.p.beta = beta; a.p.gate = gate;
  a.p.T = T; a.p.Hk = Hk; a.p.Hv = Hv; a.p.B = B;
  return hip_status(timed(VM_K_CONV, S(st), [&] { return vm::launch_deltanet_conv_prep(a, S(st)); }),
                    "deltanet_conv_prep");
}

int vm_gated_rms_norm(vm_bf16* y, int64_t y_st, int64_t y_sb, const float* o, const vm_bf16* z,
                      int64_t z_st, int64_t z_sb, const vm_bf16* norm_w, int Dv, int Hv, int T,
                      int B, float eps, vm_stream st) {
  REQUIRE(Dv == 128, VM_E_UNSUPPORTED, "gated_rms_norm: Dv = %d; built for 128", Dv);
  REQUIRE(Hv > 0 && T >= 0 && B >= 0, VM_E_ARG, "gated_rms_norm: Hv = %d, T = %d, B = %d", Hv,
          T, B);
  if (B == 0 || T == 0) return VM_OK;
  REQUIRE(o && norm_w && (reinterpret_cast<uintptr_t>(o) & 7u) == 0, VM_E_ARG,
          "gated_rms_norm: O must be 8-byte aligned");
  for (const void* p : {(const void*)y, (const void*)z})
    REQUIRE(p && (reinterpret_cast<uintptr_t>(p) & 3u) == 0, VM_E_ARG,
            "gated_rms_norm: Y and Z must be 4-byte aligned");
  REQUIRE(y_st % 2 == 0 && y_sb % 2 == 0 && z_st % 2 == 0 && z_sb % 2 == 0, VM_E_ARG,
          "gated_rms_norm: strides must be even");
  REQUIRE((T <= 1 || (y_st >= (int64_t)Hv * Dv && z_st >= (int64_t)Hv * Dv)) &&
              (B <= 1 || (y_sb >= y_st * T && z_sb >= z_st * T)),
          VM_E_DIM, "gated_rms_norm: strides below the extents");
  vm::GatedNormArgs a{};
  a.o = o; a.z = z; a.z_st = z_st; a.z_sb = z_sb; a.norm_w = norm_w; a.y = y; a.y_st = y_st;
  a.y_sb = y_sb; a.T = T; a.Hv = Hv; a.B = B; a.eps = eps;
  return hip_status(timed(VM_K_ROWS, S(st), [&] { return vm::launch_gated_rms_norm(a, S(st)); }),
                    "gated_rms_norm");
}

// ---- linear! + fused_add_rms_norm! in one call -------------------------------
size_t vm_linear_add_rms_norm_workspace_bytes(int M, int N, int K, int64_t ldw, int64_t lda) {
  if (linear_check(M, N, K, ldw, lda, M) != VM_OK) return (size_t)-1;
  size_t n = 0;
  if (vm::linear_add_norm_workspace(M, N, K, ldw, lda, &n, g_err, sizeof g_err) != VM_OK)
    return (size_t)-1;
  return n;
}

int vm_linear_add_rms_norm(vm_bf16* y, int64_t y_st, vm_bf16* x, int64_t x_st, const vm_bf16* a,
                           int64_t lda, const vm_bf16* w, int64_t ldw, const vm_bf16* norm_w,
                           int M, int N, int K, float eps, float offset, void* workspace,
                           size_t workspace_bytes, vm_stream st) {
  TRY(linear_check(M, N, K, ldw, lda, M));
  TRY(check_rows(M, N, y_st, "linear_add_rms_norm", "y_st"));
  TRY(check_rows(M, N, x_st, "linear_add_rms_norm", "x_st"));
  TRY(check_aligned(y, "Y"));
  TRY(check_aligned(x, "X"));
  TRY(check_aligned(norm_w, "W_norm"));
  REQUIRE(a && w, VM_E_ARG, "linear_add_rms_norm: NULL pointer argument");
  return vm::linear_add_norm_run(y, y_st, x, x_st, a, lda, w, ldw, norm_w, M, N, K, eps, offset,
                                 workspace, workspace_bytes, S(st), g_err, sizeof g_err);
}

// ---- linear! + the MLP's silu .* mul in one call -----------------------------
size_t vm_linear_silu_mul_workspace_bytes(int I, int N, int K, int64_t ldw, int64_t ldx) {
  if (I <= 0 || I % 8 != 0 || linear_check(2 * I, N, K, ldw, ldx, 2 * (int64_t)I) != VM_OK)
    return (size_t)-1;
  size_t n = 0;
  if (vm::linear_silu_mul_workspace(I, N, K, ldw, ldx, &n, g_err, sizeof g_err) != VM_OK)
    return (size_t)-1;
  return n;
}

int vm_linear_silu_mul(vm_bf16* mid, int64_t mid_st, const vm_bf16* x, int64_t ldx,
                       const vm_bf16* w, int64_t ldw, int I, int N, int K, void* workspace,
                       size_t workspace_bytes, vm_stream st) {
  REQUIRE(I > 0 && I % 8 == 0, VM_E_UNSUPPORTED, "linear_silu_mul: I = %d (a multiple of 8)", I);
  TRY(linear_check(2 * I, N, K, ldw, ldx, 2 * (int64_t)I));
  TRY(check_aligned(mid, "mid"));
  TRY(check_stride(mid_st, "mid_st"));
  REQUIRE(N <= 1 || mid_st >= I, VM_E_DIM, "linear_silu_mul: mid column stride %lld below I = %d",
          (long long)mid_st, I);
  REQUIRE(x && w, VM_E_ARG, "linear_silu_mul: NULL pointer argument");
  return vm::linear_silu_mul_run(mid, mid_st, x, ldx, w, ldw, I, N, K, workspace, workspace_bytes,
                                 S(st), g_err, sizeof g_err);
}

// ---- linear! + causal_conv1d! in one call -------------------------------------
size_t vm_linear_causal_conv1d_workspace_bytes(int M, int N, int K, int64_t ldw, int64_t ldx,
                                               int64_t ldy) {
  if (linear_check(M, N, K, ldw, ldx, ldy) != VM_OK) return (size_t)-1;
  size_t n = 0;
  if (vm::linear_conv_workspace(M, N, K, ldw, ldx, ldy, &n, g_err, sizeof g_err) != VM_OK)
    return (size_t)-1;
  return n;
}

int vm_linear_causal_conv1d(vm_bf16* y, int64_t ldy, const vm_bf16* x, int64_t ldx,
                            const vm_bf16* w, int64_t ldw, int M, int N, int K, vm_bf16* yc,
                            int64_t yc_sb, const vm_bf16* s_in, vm_bf16* s_out, int64_t s_cs,
                            int64_t s_sb, const vm_bf16* conv_w, int64_t conv_w_cs,
                            const vm_bf16* conv_b, int D, int Kc, int act, void* workspace,
                            size_t workspace_bytes, vm_stream st) {
  TRY(linear_check(M, N, K, ldw, ldx, ldy));
  TRY(check_conv(D, Kc, N, 1, "linear_causal_conv1d"));
  REQUIRE(M % 8 == 0 && D <= M, VM_E_DIM,
          "linear_causal_conv1d: the conv's D = %d channels must lie within the projection's M = %d "
          "(a multiple of 8)", D, M);
  REQUIRE(x && w, VM_E_ARG, "linear_causal_conv1d: NULL pointer argument");
  TRY(check_aligned(y, "y"));
  TRY(check_aligned(yc, "Y"));
  TRY(check_aligned(s_in, "S"));
  TRY(check_aligned(s_out, "S_out"));
  TRY(check_aligned(conv_w, "Weight"));
  if (conv_b) TRY(check_aligned(conv_b, "Bias"));
  for (int64_t v : {ldy, yc_sb, s_cs, s_sb, conv_w_cs}) TRY(check_stride(v, "linear_causal_conv1d"));
  REQUIRE(s_cs >= D && conv_w_cs >= D && (N <= 1 || (s_sb >= s_cs * Kc && yc_sb >= D)), VM_E_DIM,
          "linear_causal_conv1d: strides below the extents (D = %d, K = %d)", D, Kc);
  TRY(check_alias(s_in, s_out, (size_t)((N - 1) * s_sb + (Kc - 1) * s_cs + D) * 2,
                  "linear_causal_conv1d"));
  vm::Conv1dArgs c{};
  c.y = yc; c.y_sb = yc_sb; c.s_in = s_in; c.s_out = s_out; c.s_cs = s_cs; c.s_sb = s_sb;
  c.w = conv_w; c.w_cs = conv_w_cs; c.bias = conv_b; c.D = D; c.K = Kc; c.T = 1; c.B = N;
  c.act = act ? 1 : 0;
  return vm::linear_conv_run(y, ldy, x, ldx, w, ldw, M, N, K, c, workspace, workspace_bytes,
                             S(st), g_err, sizeof g_err);
}

int vm_linear_deltanet_decode(vm_bf16* o, int64_t o_sb, vm_bf16* y, int64_t ldy, vm_bf16* yc,
                              int64_t yc_sb, const vm_bf16* x, int64_t ldx, const vm_bf16* w,
                              int64_t ldw, int M, int K, const vm_bf16* ring_in, vm_bf16* ring_out,
                              int64_t s_cs, int64_t s_sb, const vm_bf16* conv_w,
                              int64_t conv_w_cs, const vm_bf16* conv_b, int Kc, const float* a_log,
                              const float* dt_bias, const vm_bf16* norm_w, const float* s_in,
                              float* s_out, int Dk, int Dv, int Hk, int Hv, int B, float eps,
                              void* workspace, size_t workspace_bytes, vm_stream st) {
  const char* what = "linear_deltanet_decode";
  TRY(check_dn_heads(Dk, Dv, Hk, Hv, B, what));
  if (B == 0) return VM_OK;
  TRY(linear_check(M, B, K, ldw, ldx, ldy));
  const int D = 2 * Hk * Dk + Hv * Dv;
  TRY(check_conv(D, Kc, B, 1, what));
  REQUIRE(M == D + Hv * Dv + 2 * Hv, VM_E_DIM,
          "%s: the projection has M = %d rows, not [q | k | v | z | alpha | beta] = %d", what, M,
          D + Hv * Dv + 2 * Hv);
  REQUIRE(o && x && w && a_log && dt_bias && norm_w, VM_E_ARG, "%s: NULL pointer argument", what);
  TRY(check_aligned(y, "y"));
  TRY(check_aligned(yc, "Y"));
  TRY(check_aligned(ring_in, "S_ring"));
  TRY(check_aligned(ring_out, "S_ring_out"));
  TRY(check_aligned(conv_w, "Weight"));
  if (conv_b) TRY(check_aligned(conv_b, "Bias"));
  TRY(check_aligned(s_in, "S"));
  TRY(check_aligned(s_out, "S_out"));
  for (int64_t v : {ldy, yc_sb, s_cs, s_sb, conv_w_cs}) TRY(check_stride(v, what));
  REQUIRE(s_cs >= D && conv_w_cs >= D && (B <= 1 || (s_sb >= s_cs * Kc && yc_sb >= D)), VM_E_DIM,
          "%s: strides below the extents (D = %d, K = %d)", what, D, Kc);
  REQUIRE(B <= 1 || o_sb >= (int64_t)Hv * Dv, VM_E_DIM, "%s: O's sequence stride < Hv Dv", what);
  TRY(check_alias(ring_in, ring_out, (size_t)((B - 1) * s_sb + (Kc - 1) * s_cs + D) * 2, what));
  TRY(check_alias(s_in, s_out, (size_t)B * Hv * Dk * Dv * sizeof(float), what));
  vm::Conv1dArgs c{};
  c.y = yc; c.y_sb = yc_sb; c.s_in = ring_in; c.s_out = ring_out; c.s_cs = s_cs; c.s_sb = s_sb;
  c.w = conv_w; c.w_cs = conv_w_cs; c.bias = conv_b; c.D = D; c.K = Kc; c.T = 1; c.B = B;
  c.act = 1;
  vm::DeltaFusedArgs f{};
  f.o = o; f.o_sb = o_sb;
  f.q = yc; f.k = yc + (int64_t)Hk * Dk; f.v = yc + 2LL * Hk * Dk;
  f.q_sb = f.k_sb = f.v_sb = yc_sb;
  f.z = y + D; f.alpha = y + D + (int64_t)Hv * Dv; f.beta = f.alpha + Hv;
  f.z_sb = f.a_sb = f.b_sb = ldy;
  f.a_log = a_log; f.dt_bias = dt_bias; f.norm_w = norm_w; f.s_in = s_in; f.s_out = s_out;
  f.Hk = Hk; f.Hv = Hv; f.B = B; f.eps = eps;
  return vm::linear_dn_decode_run(y, ldy, x, ldx, w, ldw, M, B, K, c, f, workspace,
                                  workspace_bytes, S(st), g_err, sizeof g_err);
}

// ---- synthetic inputs ------------------------------------------------------
int vm_fill_normal_bf16(vm_bf16* dst, int64_t n, uint64_t seed, float scale, float shift,
                        vm_stream st) {
  REQUIRE(dst || n == 0, VM_E_ARG, "fill_normal: NULL destination");
  REQUIRE(n >= 0, VM_E_ARG, "fill_normal: n = %lld", (long long)n);
  return hip_status(vm::launch_fill_normal(dst, n, seed, scale, shift, S(st)), "fill_normal");
}

}  // extern "C"

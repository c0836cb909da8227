// linear.cpp — y = W^T x for the projections around the gated-attention block
// (src/linear.jl:22-79): the qkv projection before it and Wo after it
// (src/llm/qwen35.jl:194, :206, :296, :316-317). Host code only.
//
// Like the reference's cuBLASLt path, one plan per problem is built on first
// use and cached for the process (linear.jl:17-38): hipBLASLt matmul
// descriptor, matrix layouts and an algorithm, bf16 A/B/D with fp32 compute and
// fp32 scaling (linear.jl:29). A plan built on first use takes the heuristic's
// first algorithm, as the reference does, and costs no device allocation and no
// synchronisation, so the first call of a shape may be captured. linear_tune
// (vm_linear_tune) is the one call that times the heuristic's top candidates
// and keeps the fastest (tune_algo below): it allocates scratch buffers and
// waits for the timing runs, and belongs at model load. Column-major view, as in
// the reference: x :: (K, N) with column stride ldx, W :: (K, M) (K-major) with
// column stride ldw, y :: (M, N) with column stride ldy, so
//     D (M x N) = op(A) B,  A = W (K x M, op = transpose), B = x (K x N).
// The workspace comes from the caller (the reference takes it from the ambient
// arena, linear.jl:62-66), so a warm call allocates nothing and can be
// captured. A problem hipBLASLt has no algorithm for (remembered as such, as
// the reference remembers `nothing`), a view whose column strides are not
// multiples of 8 elements or whose pointers are not 16-byte aligned, and a
// call the library refuses run on the library's own general GEMM kernel
// (gemm.hip): the role of the reference's mul! fallback for problems without
// an Lt algorithm and for anything not a plain CuMatrix (linear.jl:59-61,
// :67). It needs no workspace.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "kernels.h"

namespace vm {

namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
  bool ok = false;
  int pick = -1;  // the heuristic candidate kept once tuned (0 = its first); -1: not tuned
};

using Key = std::tuple<int, int, int, int, int64_t, int64_t, int64_t>;  // dev, M, N, K, ldw, ldx, ldy

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Plan> g_plans;

const char* status_name(hipblasStatus_t s) {
  switch (s) {
    case HIPBLAS_STATUS_SUCCESS: return "success";
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "alloc failed";
    case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
    case HIPBLAS_STATUS_ARCH_MISMATCH: return "arch mismatch";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
    default: return "error";
  }
}

// The heuristic ranks candidates by a model, and on MI355X its first pick can
// be a third slower than the best of its own top candidates (M x N x K =
// 18432 x 4096 x 2560: 381 against 286 us). So linear_tune times up to NTUNE
// candidates on scratch buffers of the problem's shape (N(0,1) bf16 data, on
// a private stream) and keeps the fastest. The heuristic's first is kept
// unless another beats it by 3% or more, so close calls do not flip from
// process to process.
// Problems of fewer than COLD_N columns (decode batches) are memory-bound and
// a model's step streams their weights from HBM: timed on one weight buffer,
// the buffer stays in the 256 MB last-level cache and the ranking is wrong (a
// pick made that way ran 30.1 us in a decode step, the heuristic's first 25.5,
// another candidate 23.5). They are timed on rotating copies of the weights
// that together exceed that cache, 2 x copies launches per candidate after a
// warm-up pass, queued back to back so that the GPU, not the host, sets the
// time. Larger problems: one warm-up and three timed runs on one buffer.
// VM_LINEAR_TUNE=0 keeps the first always. If any step fails (for example an
// allocation while a stream of the device is being captured), the plan keeps
// the first and the error is cleared. Returns the chosen index into `cand`.
constexpr int NTUNE = 48;  // 16 gave a 0.7% slower model prefill
constexpr int COLD_N = 256;
constexpr size_t COLD_BYTES = (size_t)768 << 20;  // rotated weights: 3x the last-level cache
int tune_algo(hipblasLtHandle_t h, const Plan& p, const hipblasLtMatmulHeuristicResult_t* res,
              const int* cand, int nc, int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  const char* env = getenv("VM_LINEAR_TUNE");
  if (nc < 2 || (env && strcmp(env, "0") == 0)) return 0;
  size_t wsmax = 0;
  for (int i = 0; i < nc; ++i) wsmax = std::max(wsmax, (size_t)res[cand[i]].workspaceSize);
  const size_t abytes = ((size_t)ldw * M * 2 + 255) & ~(size_t)255;  // one copy, 256-B aligned
  const int copies =
      N < COLD_N ? (int)std::min<size_t>(64, std::max<size_t>(2, COLD_BYTES / abytes + 1)) : 1;
  const int warm = copies > 1 ? copies : 1, timed = copies > 1 ? 2 * copies : 3;
  void *A = nullptr, *B = nullptr, *D = nullptr, *W = nullptr;
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int best = 0;
  bool ok = hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess &&
            hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess &&
            hipMalloc(&A, abytes * copies) == hipSuccess &&
            hipMalloc(&B, (size_t)ldx * N * 2) == hipSuccess &&
            hipMalloc(&D, (size_t)ldy * N * 2) == hipSuccess &&
            (wsmax == 0 || hipMalloc(&W, wsmax) == hipSuccess) &&
            launch_fill_normal(static_cast<uint16_t*>(A), (int64_t)(abytes / 2) * copies, 0x51u, 1.0f,
                               0.0f, st) == hipSuccess &&
            launch_fill_normal(static_cast<uint16_t*>(B), (int64_t)ldx * N, 0x52u, 1.0f, 0.0f, st) ==
                hipSuccess;
  if (ok) {
    const float alpha = 1.0f, beta = 0.0f;
    float t_first = -1.f, t_best = -1.f;
    for (int i = 0; i < nc && ok; ++i) {
      const hipblasLtMatmulHeuristicResult_t& r = res[cand[i]];
      bool run_ok = true;
      for (int rep = 0; rep < warm + timed && run_ok; ++rep) {
        if (rep == warm) run_ok = hipEventRecord(e0, st) == hipSuccess;
        const void* a = static_cast<const char*>(A) + abytes * (size_t)(rep % copies);
        run_ok = run_ok && hipblasLtMatmul(h, p.desc, &alpha, a, p.a, B, p.b, &beta, D, p.d, D, p.d,
                                           &r.algo, W, r.workspaceSize, st) == HIPBLAS_STATUS_SUCCESS;
      }
      float ms = 0.f;
      run_ok = run_ok && hipEventRecord(e1, st) == hipSuccess &&
               hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
      if (!run_ok) {
        if (i == 0) ok = false;  // the first must run: it is the fallback
        continue;
      }
      if (i == 0) t_first = ms;
      if (t_best < 0.f || ms < t_best) {
        t_best = ms;
        best = i;
      }
    }
    if (!ok || t_first <= 1.03f * t_best) best = 0;
  }
  if (A) (void)hipFree(A);
  if (B) (void)hipFree(B);
  if (D) (void)hipFree(D);
  if (W) (void)hipFree(W);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (st) (void)hipStreamDestroy(st);
  if (!ok) {
    (void)hipGetLastError();
    best = 0;
  }
  return best;
}

// The heuristic's candidates for a plan's problem, within the workspace cap
// (the cap preference alone does not bound what it returns): up to NTUNE, in
// its ranking, as indices into res. Returns their count (0 on failure).
constexpr int NREQ = 64;
int candidates(hipblasLtHandle_t h, const Plan& p, hipblasLtMatmulHeuristicResult_t (&res)[NREQ],
               int (&cand)[NTUNE], hipblasStatus_t* status) {
  hipblasLtMatmulPreference_t pref = nullptr;
  hipblasStatus_t s = hipblasLtMatmulPreferenceCreate(&pref);
  const uint64_t cap = LINEAR_MAX_WORKSPACE_BYTES;
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap,
                                              sizeof cap);
  int n_res = 0;
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, NREQ, res, &n_res);
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  int nc = 0;
  for (int i = 0; s == HIPBLAS_STATUS_SUCCESS && i < n_res && nc < NTUNE; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= cap) cand[nc++] = i;
  *status = s;
  return nc;
}

// Finds, or builds with the heuristic's first algorithm, the plan of one
// problem on the current device (host work only: descriptors and the heuristic
// query; no device allocation, no synchronisation). Returns 0, or a VM_E_* /
// hipError_t code with `err` set. g_mu must be held.
int find_plan(int dev, int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy, Plan** out,
              hipblasLtHandle_t* handle, char* err, size_t errn) {
  const Key key{dev, M, N, K, ldw, ldx, ldy};
  hipblasLtHandle_t h;
  auto hit = g_handles.find(dev);
  if (hit == g_handles.end()) {
    hipblasStatus_t s = hipblasLtCreate(&h);
    if (s != HIPBLAS_STATUS_SUCCESS) {
      snprintf(err, errn, "linear: hipblasLtCreate: %s", status_name(s));
      return VM_E_UNSUPPORTED;
    }
    g_handles[dev] = h;
  } else {
    h = hit->second;
  }
  *handle = h;
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    if (!it->second.ok) {
      snprintf(err, errn, "linear: hipBLASLt has no algorithm for M = %d, N = %d, K = %d", M, N, K);
      return VM_E_UNSUPPORTED;
    }
    *out = &it->second;
    return VM_OK;
  }
  Plan p;
  hipblasStatus_t s = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta);
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, M, ldw);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, N, ldx);
  if (s == HIPBLAS_STATUS_SUCCESS) s = hipblasLtMatrixLayoutCreate(&p.d, HIP_R_16BF, M, N, ldy);
  hipblasLtMatmulHeuristicResult_t res[NREQ];
  int cand[NTUNE];
  const int nc = s == HIPBLAS_STATUS_SUCCESS ? candidates(h, p, res, cand, &s) : 0;
  if (nc > 0) {
    p.algo = res[cand[0]].algo;
    p.workspace = res[cand[0]].workspaceSize;
    p.ok = true;
  }
  auto& slot = g_plans[key];  // remembered either way (linear.jl:20-21)
  slot = p;
  if (!slot.ok) {
    snprintf(err, errn, "linear: hipBLASLt has no algorithm for M = %d, N = %d, K = %d (%s)", M,
             N, K, status_name(s));
    return VM_E_UNSUPPORTED;
  }
  *out = &slot;
  return VM_OK;
}

int get_plan(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy, const Plan** out,
             char* err, size_t errn) {
  int dev = 0;
  hipError_t he = hipGetDevice(&dev);
  if (he != hipSuccess) {
    snprintf(err, errn, "linear: hipGetDevice: %s", hipGetErrorString(he));
    return (int)he;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  Plan* p = nullptr;
  hipblasLtHandle_t h;
  const int rc = find_plan(dev, M, N, K, ldw, ldx, ldy, &p, &h, err, errn);
  if (rc == VM_OK) *out = p;
  return rc;
}

// Narrow problems run on the library's own split-K MFMA kernel (launch_gemv):
// every N <= 16, and N <= 32 when M <= 4096 (the short, deep out projections
// and the MLP's down projection). Measured under graph replay on MI355X with
// the weights cold (rotating copies larger than the 256 MB last-level cache),
// against the GEMM library's pick: N = 1..16 faster on every decode shape
// (18432 x 2560 gate-up: 25 vs 56 us), at N = 32 faster for 2560 x 4096 (11.1
// vs 12.4 us) and 2560 x 9216 (15.6 vs 20.5 us) and 3-6% slower for the
// wide 10-18K-row projections, which stay on the library. Its loads need
// 16-byte aligned columns of W and x and 8-byte aligned columns of y.
bool gemv_shape(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  const bool narrow = N <= 16 || (N <= 32 && M <= 4096);
  return narrow && K % 64 == 0 && M % 4 == 0 && ldw % 8 == 0 && ldx % 8 == 0 && ldy % 4 == 0;
}
bool gemv_aligned(const void* y, const void* x, const void* w) {
  return ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0) && ((uintptr_t)y % 8 == 0);
}

// views the GEMM library is not asked to take (see the file comment)
bool general_strides(int64_t ldw, int64_t ldx, int64_t ldy) {
  return (ldw % 8) != 0 || (ldx % 8) != 0 || (ldy % 8) != 0;
}
bool general_view(const void* y, const void* x, const void* w, int64_t ldw, int64_t ldx,
                  int64_t ldy) {
  return general_strides(ldw, ldx, ldy) || ((uintptr_t)x % 16) != 0 || ((uintptr_t)w % 16) != 0 ||
         ((uintptr_t)y % 16) != 0;
}

int run_gemm_any(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
                 int64_t ldw, int M, int N, int K, hipStream_t st, char* err, size_t errn) {
  GemmAnyArgs a{};
  a.w = w;
  a.x = x;
  a.y = y;
  a.ldw = ldw;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  const hipError_t e = launch_gemm_any(a, st);
  if (e != hipSuccess) {
    snprintf(err, errn, "linear (general kernel): %s", hipGetErrorString(e));
    return (int)e;
  }
  return VM_OK;
}

}  // namespace

int linear_tune(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy, char* err, size_t errn) {
  if (general_strides(ldw, ldx, ldy)) return VM_OK;  // the general kernel: nothing to tune
  if (gemv_shape(M, N, K, ldw, ldx, ldy)) {
    // aligned views run the GEMV, which has nothing to tune; the plan stays
    // the heuristic's first (it only serves misaligned views)
    const Plan* p = nullptr;
    const int rc = get_plan(M, N, K, ldw, ldx, ldy, &p, err, errn);
    return rc == VM_E_UNSUPPORTED ? VM_OK : rc;
  }
  int dev = 0;
  hipError_t he = hipGetDevice(&dev);
  if (he != hipSuccess) {
    snprintf(err, errn, "linear: hipGetDevice: %s", hipGetErrorString(he));
    return (int)he;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  Plan* p = nullptr;
  hipblasLtHandle_t h;
  int rc = find_plan(dev, M, N, K, ldw, ldx, ldy, &p, &h, err, errn);
  if (rc == VM_E_UNSUPPORTED) return VM_OK;  // the general kernel: nothing to tune
  if (rc != VM_OK || p->pick >= 0) return rc;
  hipblasLtMatmulHeuristicResult_t res[NREQ];
  int cand[NTUNE];
  hipblasStatus_t s;
  const int nc = candidates(h, *p, res, cand, &s);
  if (nc == 0) {
    p->pick = 0;  // keeps what it has
    return VM_OK;
  }
  // relaxed capture mode for this thread meanwhile, so that the scratch
  // allocations cannot invalidate a capture running on another stream
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
  const int k = tune_algo(h, *p, res, cand, nc, M, N, K, ldw, ldx, ldy);
  if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
  p->algo = res[cand[k]].algo;
  p->workspace = res[cand[k]].workspaceSize;
  p->pick = k;
  return VM_OK;
}

int linear_plan_state(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_plans.find(Key{dev, M, N, K, ldw, ldx, ldy});
  if (it == g_plans.end() || !it->second.ok) return -2;
  return it->second.pick;
}

int linear_workspace(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy, size_t* bytes,
                     char* err, size_t errn) {
  if (general_strides(ldw, ldx, ldy)) {
    // the GEMV (which takes y columns in steps of 4) or the general kernel,
    // which needs no workspace
    *bytes = gemv_shape(M, N, K, ldw, ldx, ldy) ? gemv_workspace_bytes(M, K) : 0;
    return VM_OK;
  }
  const Plan* p = nullptr;
  const int rc = get_plan(M, N, K, ldw, ldx, ldy, &p, err, errn);
  if (gemv_shape(M, N, K, ldw, ldx, ldy)) {
    // the GEMM library covers misaligned views of the same shape
    *bytes = std::max(gemv_workspace_bytes(M, K), rc == VM_OK ? p->workspace : (size_t)0);
    return VM_OK;
  }
  if (rc == VM_OK) *bytes = p->workspace;
  if (rc == VM_E_UNSUPPORTED) {  // the general kernel needs no workspace
    *bytes = 0;
    return VM_OK;
  }
  return rc;
}

int linear_run(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
               int64_t ldw, int M, int N, int K, void* workspace, size_t workspace_bytes,
               hipStream_t st, char* err, size_t errn) {
  if (gemv_shape(M, N, K, ldw, ldx, ldy) && gemv_aligned(y, x, w)) {
    const size_t need = gemv_workspace_bytes(M, K);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need ||
                     (uintptr_t)workspace % 16 != 0)) {
      snprintf(err, errn,
               "linear: workspace of %zu bytes (16-byte aligned) < %zu required "
               "(vm_linear_workspace_bytes)", workspace_bytes, need);
      return VM_E_SCRATCH;
    }
    GemvArgs a{};
    a.w = w;
    a.w_st = ldw;
    a.x = x;
    a.x_st = ldx;
    a.y = y;
    a.y_st = ldy;
    a.M = M;
    a.N = N;
    a.K = K;
    a.part = static_cast<float*>(workspace);
    const hipError_t e = launch_gemv(a, st);
    if (e != hipSuccess) {
      snprintf(err, errn, "linear: %s", hipGetErrorString(e));
      return (int)e;
    }
    return VM_OK;
  }
  if (general_view(y, x, w, ldw, ldx, ldy))
    return run_gemm_any(y, ldy, x, ldx, w, ldw, M, N, K, st, err, errn);
  const Plan* p = nullptr;
  int rc = get_plan(M, N, K, ldw, ldx, ldy, &p, err, errn);
  if (rc == VM_E_UNSUPPORTED) return run_gemm_any(y, ldy, x, ldx, w, ldw, M, N, K, st, err, errn);
  if (rc != VM_OK) return rc;
  if (p->workspace > 0 && (workspace == nullptr || workspace_bytes < p->workspace)) {
    snprintf(err, errn, "linear: workspace of %zu bytes < %zu required (vm_linear_workspace_bytes)",
             workspace_bytes, p->workspace);
    return VM_E_SCRATCH;
  }
  hipblasLtHandle_t h;
  {
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(g_mu);
    h = g_handles[dev];
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t s = hipblasLtMatmul(h, p->desc, &alpha, w, p->a, x, p->b, &beta, y, p->d, y,
                                            p->d, &p->algo, workspace, p->workspace, st);
  if (s != HIPBLAS_STATUS_SUCCESS) {
    // the plan's algorithm refused these operands (e.g. a misaligned view):
    // the general kernel, as the reference's mul! (linear.jl:60)
    return run_gemm_any(y, ldy, x, ldx, w, ldw, M, N, K, st, err, errn);
  }
  return VM_OK;
}

namespace {
size_t round256(size_t n) { return (n + 255) / 256 * 256; }
}  // namespace

int linear_add_norm_workspace(int M, int N, int K, int64_t ldw, int64_t lda, size_t* bytes,
                              char* err, size_t errn) {
  const size_t hbytes = round256((size_t)M * N * sizeof(uint16_t));  // a bf16 y, ld M
  if (gemv_shape(M, N, K, ldw, lda, M)) {
    const size_t part = gemv_workspace_bytes(M, K);
    // a split plan needs its partials; a single-slice one a bf16 y (and the
    // GEMM library's path for a misaligned view of the same shape: below)
    size_t lin = 0;
    const int rc = linear_workspace(M, N, K, ldw, lda, M, &lin, err, errn);
    *bytes = std::max(std::max(part, hbytes), (rc == VM_OK ? round256(lin) + hbytes : 0));
    return VM_OK;
  }
  size_t lin = 0;
  const int rc = linear_workspace(M, N, K, ldw, lda, M, &lin, err, errn);
  if (rc != VM_OK) return rc;
  *bytes = round256(lin) + hbytes;
  return VM_OK;
}

int linear_add_norm_run(uint16_t* yn, int64_t yn_st, uint16_t* x, int64_t x_st, const uint16_t* a,
                        int64_t lda, const uint16_t* w, int64_t ldw, const uint16_t* nw, int M,
                        int N, int K, float eps, float offset, void* workspace,
                        size_t workspace_bytes, hipStream_t st, char* err, size_t errn) {
  size_t need = 0;
  int rc = linear_add_norm_workspace(M, N, K, ldw, lda, &need, err, errn);
  if (rc != VM_OK) return rc;
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    snprintf(err, errn,
             "linear_add_rms_norm: workspace of %zu bytes (256-byte aligned) < %zu required "
             "(vm_linear_add_rms_norm_workspace_bytes)", workspace_bytes, need);
    return VM_E_SCRATCH;
  }
  NormArgs na{};
  na.y = yn;
  na.y_st = yn_st;
  na.xo = x;
  na.xo_st = x_st;
  na.x = x;
  na.x_st = x_st;
  na.w = nw;
  na.M = M;
  na.N = N;
  na.offset = offset;
  na.eps = eps;
  uint16_t* h = static_cast<uint16_t*>(workspace);  // the bf16 y when one is formed
  if (gemv_shape(M, N, K, ldw, lda, M) && gemv_aligned(h, a, w)) {
    GemvArgs g{};
    g.w = w;
    g.w_st = ldw;
    g.x = a;
    g.x_st = lda;
    g.y = h;
    g.y_st = M;
    g.M = M;
    g.N = N;
    g.K = K;
    g.part = static_cast<float*>(workspace);
    GemvPlan p{};
    hipError_t e = launch_gemv_partials(g, &p, st);
    if (e == hipSuccess && p.S2 > 1) {
      na.dpart = g.part;
      na.dpart_ss = (int64_t)32 * M;
      na.dpart_cs = M;
      na.S2 = p.S2;
    } else {
      na.dx = h;
      na.dx_st = M;
    }
    if (e == hipSuccess) e = launch_rms_norm(na, st);
    if (e != hipSuccess) {
      snprintf(err, errn, "linear_add_rms_norm: %s", hipGetErrorString(e));
      return (int)e;
    }
    return VM_OK;
  }
  // the GEMM library's path: y into the workspace after the plan's own space
  size_t lin = 0;
  rc = linear_workspace(M, N, K, ldw, lda, M, &lin, err, errn);
  if (rc != VM_OK) return rc;
  h = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + round256(lin));
  rc = linear_run(h, M, a, lda, w, ldw, M, N, K, workspace, lin, st, err, errn);
  if (rc != VM_OK) return rc;
  na.dx = h;
  na.dx_st = M;
  const hipError_t e = launch_rms_norm(na, st);
  if (e != hipSuccess) {
    snprintf(err, errn, "linear_add_rms_norm: %s", hipGetErrorString(e));
    return (int)e;
  }
  return VM_OK;
}

// ---- linear! + silu .* mul (the MLP's gate-up half, qwen35.jl:234-243) -------
namespace {
// the stream-K path: a decode batch, whole 64-k groups, aligned columns
bool sk_shape(int M, int N, int K, int64_t ldw, int64_t ldx) {
  return N >= 1 && N <= 32 && K > 0 && K % 64 == 0 && M % 8 == 0 && ldw % 8 == 0 && ldx % 8 == 0;
}
}  // namespace

int linear_silu_mul_workspace(int I, int N, int K, int64_t ldw, int64_t ldx, size_t* bytes,
                              char* err, size_t errn) {
  const int M = 2 * I;
  if (sk_shape(M, N, K, ldw, ldx)) {
    // the stream-K partials; a misaligned view takes the two-call path below
    // in the same workspace
    size_t lin = 0;
    const int rc = linear_workspace(M, N, K, ldw, ldx, M, &lin, err, errn);
    const size_t two = rc == VM_OK ? round256(lin) + round256((size_t)M * N * sizeof(uint16_t)) : 0;
    *bytes = std::max(round256(gemv_sk_workspace_bytes(M, K)), two);
    return VM_OK;
  }
  size_t lin = 0;
  const int rc = linear_workspace(M, N, K, ldw, ldx, M, &lin, err, errn);
  if (rc != VM_OK) return rc;
  *bytes = round256(lin) + round256((size_t)M * N * sizeof(uint16_t));
  return VM_OK;
}

int linear_silu_mul_run(uint16_t* mid, int64_t mid_st, const uint16_t* x, int64_t ldx,
                        const uint16_t* w, int64_t ldw, int I, int N, int K, void* workspace,
                        size_t workspace_bytes, hipStream_t st, char* err, size_t errn) {
  const int M = 2 * I;
  size_t need = 0;
  int rc = linear_silu_mul_workspace(I, N, K, ldw, ldx, &need, err, errn);
  if (rc != VM_OK) return rc;
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    snprintf(err, errn,
             "linear_silu_mul: workspace of %zu bytes (256-byte aligned) < %zu required "
             "(vm_linear_silu_mul_workspace_bytes)", workspace_bytes, need);
    return VM_E_SCRATCH;
  }
  if (sk_shape(M, N, K, ldw, ldx) && (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0) {
    GemvSkArgs g{};
    g.w = w;
    g.w_st = ldw;
    g.x = x;
    g.x_st = ldx;
    g.part = static_cast<float*>(workspace);
    g.M = M;
    g.N = N;
    g.K = K;
    g.p = gemv_sk_plan(M, K);
    SiluMulSkArgs a{};
    a.mid = mid;
    a.mid_st = mid_st;
    a.part = g.part;
    a.I = I;
    a.N = N;
    a.p = g.p;
    hipError_t e = launch_gemv_sk(g, st);
    if (e == hipSuccess) e = launch_silu_mul_sk(a, st);
    if (e != hipSuccess) {
      snprintf(err, errn, "linear_silu_mul: %s", hipGetErrorString(e));
      return (int)e;
    }
    return VM_OK;
  }
  // linear! into a bf16 gu after the plan's own space, then silu .* mul
  size_t lin = 0;
  rc = linear_workspace(M, N, K, ldw, ldx, M, &lin, err, errn);
  if (rc != VM_OK) return rc;
  uint16_t* gu = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + round256(lin));
  rc = linear_run(gu, M, x, ldx, w, ldw, M, N, K, workspace, lin, st, err, errn);
  if (rc != VM_OK) return rc;
  SiluMulArgs a{};
  a.mid = mid;
  a.mid_st = mid_st;
  a.gu = gu;
  a.gu_st = M;
  a.I = I;
  a.N = N;
  const hipError_t e = launch_silu_mul(a, st);
  if (e != hipSuccess) {
    snprintf(err, errn, "linear_silu_mul: %s", hipGetErrorString(e));
    return (int)e;
  }
  return VM_OK;
}

// ---- linear! + causal_conv1d! (the DeltaNet layer's decode step, qwen35.jl:212-223)
int linear_conv_workspace(int M, int N, int K, int64_t ldw, int64_t ldx, int64_t ldy,
                          size_t* bytes, char* err, size_t errn) {
  size_t lin = 0;
  const int rc = linear_workspace(M, N, K, ldw, ldx, ldy, &lin, err, errn);
  if (sk_shape(M, N, K, ldw, ldx)) {
    // a misaligned view takes linear! + the conv in the same workspace
    *bytes = std::max(round256(gemv_sk_workspace_bytes(M, K)), rc == VM_OK ? lin : (size_t)0);
    return VM_OK;
  }
  if (rc != VM_OK) return rc;
  *bytes = lin;
  return VM_OK;
}

int linear_conv_run(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx, const uint16_t* w,
                    int64_t ldw, int M, int N, int K, Conv1dArgs conv, void* workspace,
                    size_t workspace_bytes, hipStream_t st, char* err, size_t errn) {
  size_t need = 0;
  int rc = linear_conv_workspace(M, N, K, ldw, ldx, ldy, &need, err, errn);
  if (rc != VM_OK) return rc;
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    snprintf(err, errn,
             "linear_causal_conv1d: workspace of %zu bytes (256-byte aligned) < %zu required "
             "(vm_linear_causal_conv1d_workspace_bytes)", workspace_bytes, need);
    return VM_E_SCRATCH;
  }
  hipError_t e = hipSuccess;
  if (sk_shape(M, N, K, ldw, ldx) && ldy % 8 == 0 && (uintptr_t)x % 16 == 0 &&
      (uintptr_t)w % 16 == 0 && (uintptr_t)y % 16 == 0) {
    // the stream-K GEMV; the conv kernel adds each channel's partials, stores
    // the bf16 projection and convolves its first D channels
    GemvSkArgs g{};
    g.w = w;
    g.w_st = ldw;
    g.x = x;
    g.x_st = ldx;
    g.part = static_cast<float*>(workspace);
    g.M = M;
    g.N = N;
    g.K = K;
    g.p = gemv_sk_plan(M, K);
    Conv1dSkArgs a{};
    a.c = conv;
    a.yp = y;
    a.yp_sb = ldy;
    a.part = g.part;
    a.G = g.p.G;
    a.chunk = g.p.chunk;
    a.M = M;
    e = launch_gemv_sk(g, st);
    if (e == hipSuccess) e = launch_conv1d_update_sk(a, st);
  } else {
    size_t lin = 0;
    rc = linear_workspace(M, N, K, ldw, ldx, ldy, &lin, err, errn);
    if (rc != VM_OK) return rc;
    rc = linear_run(y, ldy, x, ldx, w, ldw, M, N, K, workspace, lin, st, err, errn);
    if (rc != VM_OK) return rc;
    conv.x = y;
    conv.x_sb = ldy;
    e = launch_conv1d_update(conv, st);
  }
  if (e != hipSuccess) {
    snprintf(err, errn, "linear_causal_conv1d: %s", hipGetErrorString(e));
    return (int)e;
  }
  return VM_OK;
}

int linear_dn_decode_run(uint16_t* y, int64_t ldy, const uint16_t* x, int64_t ldx,
                         const uint16_t* w, int64_t ldw, int M, int N, int K, Conv1dArgs conv,
                         const DeltaFusedArgs& f, void* workspace, size_t workspace_bytes,
                         hipStream_t st, char* err, size_t errn) {
  size_t need = 0;
  int rc = linear_conv_workspace(M, N, K, ldw, ldx, ldy, &need, err, errn);
  if (rc != VM_OK) return rc;
  if (workspace == nullptr || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) {
    snprintf(err, errn,
             "linear_deltanet_decode: workspace of %zu bytes (256-byte aligned) < %zu required "
             "(vm_linear_causal_conv1d_workspace_bytes)", workspace_bytes, need);
    return VM_E_SCRATCH;
  }
  const int R = f.Hv / f.Hk;
  hipError_t e = hipSuccess;
  if (sk_shape(M, N, K, ldw, ldx) && (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 &&
      (R == 1 || R == 2 || R == 4) && M == conv.D + f.Hv * 128 + 2 * f.Hv) {  // Dv = 128
    GemvSkArgs g{};
    g.w = w;
    g.w_st = ldw;
    g.x = x;
    g.x_st = ldx;
    g.part = static_cast<float*>(workspace);
    g.M = M;
    g.N = N;
    g.K = K;
    g.p = gemv_sk_plan(M, K);
    DeltaDecodeSkArgs a{};
    a.f = f;
    a.c = conv;
    a.part = g.part;
    a.G = g.p.G;
    a.chunk = g.p.chunk;
    e = launch_gemv_sk(g, st);
    if (e == hipSuccess) e = launch_deltanet_decode_sk(a, st);
  } else {
    rc = linear_conv_run(y, ldy, x, ldx, w, ldw, M, N, K, conv, workspace, workspace_bytes, st, err,
                         errn);
    if (rc != VM_OK) return rc;
    e = launch_deltanet_fused_decode(f, st);
  }
  if (e != hipSuccess) {
    snprintf(err, errn, "linear_deltanet_decode: %s", hipGetErrorString(e));
    return (int)e;
  }
  return VM_OK;
}

}  // namespace vm

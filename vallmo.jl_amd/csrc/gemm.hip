// gemm.hip — y = W^T x for the problems and views linear.cpp does not give the
// GEMM library: the role of the reference's mul! fallback (src/linear.jl:59-61,
// :67). Same column-major view as linear.cpp: x :: (K, N) with column stride
// ldx, W :: (K, M) (K-major) with column stride ldw, y :: (M, N) with column
// stride ldy, bf16 in and out, fp32 accumulation, one bf16 rounding (round to
// nearest even) per output. Any M, N, K >= 0, any strides >= the column lengths and
// 2-byte alignment only: an operand chunk of 8 k that lies inside the matrix
// and starts on a 16-byte boundary is one 16-byte load, any other is gathered
// element by element (bounds-checked 2-byte loads).
//
// One workgroup (4 waves) per 64 x 64 output tile; wave (wm, wn) owns the
// 32 x 32 block (wm, wn) on v_mfma_f32_32x32x16_bf16. Per 32-deep K step the
// tile's 64 W columns and 64 x columns (32 k each) are gathered into LDS rows
// of 32 contiguous k (+8 pad: the b128 operand reads of one cycle fall on
// distinct banks), the reads past K, M or N filled with zeros.
#include "common.h"
#include "kernels.h"

namespace vm {

namespace {
constexpr int GT = 64;        // output tile edge
constexpr int GK = 32;        // k per step
constexpr int GROW = GK + 8;  // LDS row, bf16

__global__ __launch_bounds__(256) void gemm_any_kernel(GemmAnyArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[GT][GROW], Bs[GT][GROW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t m0 = (int64_t)blockIdx.x * GT, n0 = (int64_t)blockIdx.y * GT;
  // gather: thread t fills row t / 4 (an m of A, an n of B), k 8 (t % 4) .. +7
  const int gr = t >> 2, gk = 8 * (t & 3);
  const int64_t am = m0 + gr, bn = n0 + gr;
  const uint16_t* ap = a.w + (am < a.M ? am : 0) * a.ldw;
  const uint16_t* bp = a.x + (bn < a.N ? bn : 0) * a.ldx;
  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  // 8 elements k .. k + 7 of one operand column (zeros past its end)
  auto chunk = [&](const uint16_t* p, bool live, int64_t k) __attribute__((always_inline)) {
    if (live && k + 8 <= a.K && ((uintptr_t)(p + k) & 15u) == 0)
      return *reinterpret_cast<const uint4*>(p + k);
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (live && k + e < a.K) ? p[k + e] : (uint16_t)0;
    return make_uint4(v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16),
                      v[4] | ((uint32_t)v[5] << 16), v[6] | ((uint32_t)v[7] << 16));
  };
  for (int64_t k0 = 0; k0 < a.K; k0 += GK) {
    const uint4 av = chunk(ap, am < a.M, k0 + gk);
    const uint4 bv = chunk(bp, bn < a.N, k0 + gk);
    __syncthreads();  // the previous step's operand reads are done
    *reinterpret_cast<uint4*>(&As[gr][gk]) = av;
    *reinterpret_cast<uint4*>(&Bs[gr][gk]) = bv;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GK; kk += 16) {
      // A lane l: row l % 32, k 8 (l / 32) .. +7; B lane l: column l % 32, same k
      const uint4 av4 = *reinterpret_cast<const uint4*>(&As[32 * wm + (lane & 31)][kk + 8 * (lane >> 5)]);
      const uint4 bv4 = *reinterpret_cast<const uint4*>(&Bs[32 * wn + (lane & 31)][kk + 8 * (lane >> 5)]);
      acc = mfma32(av4, bv4, acc);
    }
  }
  // D lane l reg j: row 8 (j / 4) + 4 (l / 32) + j % 4, column l % 32
  const int64_t n = n0 + 32 * wn + (lane & 31);
  if (n >= a.N) return;
  uint16_t* yc = a.y + n * a.ldy;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int64_t m = m0 + 32 * wm + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
    if (m < a.M) yc[m] = f2bf(acc[j]);
  }
}
}  // namespace

hipError_t launch_gemm_any(const GemmAnyArgs& a, hipStream_t st) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  const int64_t gm = (a.M + GT - 1) / GT, gn = (a.N + GT - 1) / GT;
  if (gm > 0x7fffffff || gn > 65535) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(gemm_any_kernel, dim3((unsigned)gm, (unsigned)gn), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace vm

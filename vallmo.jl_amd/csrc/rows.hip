// rows.hip — per-row kernels of the gated-attention path: RoPE tables, per-head
// RMSNorm + partial RoPE (decode and prefill flavours, with the cache append),
// the elementwise sigmoid gate, the device clock, and the seeded bf16 N(0,1)
// generator used for synthetic inputs.
//
// Row layout: one wave64 per (head, token) row of D = 256; lane l holds
// d = 4l .. 4l+3 (one 8-byte load). The rotate-half partner of d < 32 is
// d + 32, i.e. lane l ^ 8, so RoPE is one xor-8 shuffle.
#include "common.h"
#include "kernels.h"

namespace vm {

// ---------------------------------------------------------------------------
// a1: rope_tables (src/llm/qwen35.jl:115-119). inv_freq in f64 -> f32, angle
// as an f32 product, cos/sin evaluated in f64 and rounded once to f32.
__global__ void rope_tables_kernel(float* __restrict__ cos_tab, float* __restrict__ sin_tab,
                                   int half, int64_t ctx, double theta) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= ctx * half) return;
  int i = (int)(idx % half);
  int64_t t = idx / half;
  float inv = (float)pow(theta, -((double)i / (double)half));
  float ang = inv * (float)t;
  cos_tab[idx] = (float)cos((double)ang);
  sin_tab[idx] = (float)sin((double)ang);
}

// Generic row kernel. Row r -> (b, h, t) with t fastest. Position (0-based)
// of the row: decode = positions[b]-1 (T = 1), prefill = prior[b] + t.
// The output row index along the token axis is the position when
// out_at_pos (cache append) and t otherwise (q prologue / in-place q).
__global__ __launch_bounds__(256) void norm_rope_rows_kernel(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)a.B * a.H * a.T;
  if (row >= nrows) return;
  const int t = (int)(row % a.T);
  const int h = (int)((row / a.T) % a.H);
  const int b = (int)(row / ((int64_t)a.T * a.H));
  int pos;
  if (a.positions) {
    pos = a.positions[b] - 1;
  } else {
    if (a.q_lengths && t >= a.q_lengths[b]) return;
    pos = (a.prior ? a.prior[b] : 0) + t;
  }
  if (pos < 0 || pos >= a.ctx) return;  // out-of-contract position: write nothing
  const int64_t orow = a.out_at_pos ? (int64_t)pos : (int64_t)t;
  const uint16_t* src = a.in + b * a.in_sb + h * a.in_sh + t * a.in_st;
  uint16_t* dst = a.out + b * a.out_sb + h * a.out_sh + orow * a.out_st;
  float x[4];
  load_row4(src, lane, x);
  norm_rope_row(x, a.w, a.cos_tab + (int64_t)pos * HALF_ROT, a.sin_tab + (int64_t)pos * HALF_ROT,
                a.eps, a.w_offset, lane);
  store_row4(dst, lane, x);
  if (a.in2) {  // V rides along: plain copy into the same cache column
    const uint16_t* s2 = a.in2 + b * a.in_sb + h * a.in_sh + t * a.in_st;
    uint16_t* d2 = a.out2 + b * a.out_sb + h * a.out_sh + orow * a.out_st;
    *reinterpret_cast<uint2*>(d2 + 4 * lane) = *reinterpret_cast<const uint2*>(s2 + 4 * lane);
  }
}

// ---------------------------------------------------------------------------
// a6: O .*= sigmoid.(G) in place; one thread per 8 elements.
__global__ void sigmoid_gate_kernel(uint16_t* __restrict__ o, int64_t o_sh, int64_t o_sb,
                                    const uint16_t* __restrict__ g, int64_t g_sh, int64_t g_sb,
                                    int B, int H) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = HEAD_DIM / 8;
  if (idx >= (int64_t)B * H * per_row) return;
  int c = (int)(idx % per_row);
  int h = (int)((idx / per_row) % H);
  int b = (int)(idx / ((int64_t)per_row * H));
  uint16_t* op = o + b * o_sb + h * o_sh + 8 * c;
  const uint16_t* gp = g + b * g_sb + h * g_sh + 8 * c;
  float ov[8], gv[8];
  unpack8(load16(op), ov);
  unpack8(load16(gp), gv);
#pragma unroll
  for (int j = 0; j < 8; ++j) ov[j] *= sigmoidf(gv[j]);
  *reinterpret_cast<uint4*>(op) = pack8(ov);
}

// a12: advance! — the device clock.
__global__ void advance_kernel(int32_t* positions, int B) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) positions[i] += 1;
}

// ---------------------------------------------------------------------------
// Seeded N(0,1): SplitMix64 counter stream, Box-Muller in f64, -> f32 -> bf16.
__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__global__ void fill_normal_kernel(uint16_t* __restrict__ dst, int64_t n, uint64_t seed,
                                   float scale, float shift) {
  int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // pair index
  if (2 * k >= n) return;
  double u1 = (double)(splitmix64_at(seed, 2 * k) >> 11) * 0x1.0p-53;
  double u2 = (double)(splitmix64_at(seed, 2 * k + 1) >> 11) * 0x1.0p-53;
  double r = sqrt(-2.0 * log(1.0 - u1));
  double th = 6.283185307179586 * u2;
  double z0 = r * cos(th) * (double)scale + (double)shift;
  double z1 = r * sin(th) * (double)scale + (double)shift;
  dst[2 * k] = f2bf((float)z0);
  if (2 * k + 1 < n) dst[2 * k + 1] = f2bf((float)z1);
}

// ---------------------------------------------------------------------------
hipError_t launch_rope_tables(float* c, float* s, int half, int64_t ctx, double theta,
                              hipStream_t st) {
  int64_t n = ctx * half;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_tables_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     c, s, half, ctx, theta);
  return hipGetLastError();
}
hipError_t launch_norm_rope_rows(const RowArgs& a, hipStream_t st) {
  int64_t rows = (int64_t)a.B * a.H * a.T;
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(norm_rope_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, a);
  return hipGetLastError();
}
hipError_t launch_sigmoid_gate(uint16_t* o, int64_t o_sh, int64_t o_sb, const uint16_t* g,
                               int64_t g_sh, int64_t g_sb, int B, int H, hipStream_t st) {
  int64_t n = (int64_t)B * H * (HEAD_DIM / 8);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(sigmoid_gate_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     o, o_sh, o_sb, g, g_sh, g_sb, B, H);
  return hipGetLastError();
}
hipError_t launch_advance(int32_t* positions, int B, hipStream_t st) {
  if (B == 0) return hipSuccess;
  hipLaunchKernelGGL(advance_kernel, dim3((B + 255) / 256), dim3(256), 0, st, positions, B);
  return hipGetLastError();
}
hipError_t launch_fill_normal(uint16_t* dst, int64_t n, uint64_t seed, float scale, float shift,
                              hipStream_t st) {
  int64_t pairs = (n + 1) / 2;
  if (pairs == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, st,
                     dst, n, seed, scale, shift);
  return hipGetLastError();
}

}  // namespace vm

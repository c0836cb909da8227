// step.hip — the rest of one decode step around the attention block, re-designed
// for CDNA4: RMSNorm (src/kernels/rms_norm.jl:3-57), the fused residual add +
// RMSNorm (src/kernels/residual_norm.jl:4-60), the MLP's silu(gate) * up
// (src/llm/qwen35.jl:234-243), the embedding gather (qwen35.jl:251), the engine's
// clock advance (src/llm/generate.jl:82-88) and the fused lm-head GEMV + argmax
// (src/kernels/lm_head_topk.jl:27-147).
//
// The row kernels move 16-byte chunks of 8 bf16, compute in fp32 and round once
// to bf16 (round to nearest even). The lm head is HBM-bound: every weight byte is
// read once, by bf16 MFMAs that multiply a 32-column vocab tile by a 32-column
// batch tile; the logits never leave the registers.
#include "common.h"
#include "kernels.h"

namespace vm {

namespace {

constexpr int RT = 256;      // threads of a row kernel's workgroup
constexpr int RCHUNK = 8;    // 16-byte chunks per thread: rows of up to 256 * 8 * 8 = 16384

// Sum over the 64 lanes (DPP row shifts and broadcasts, no LDS), the same
// value in every lane.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the workgroup's 256 threads, in every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum_dpp(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ void load8f(const uint16_t* p, float* f) { unpack8(load16(p), f); }

}  // namespace

// ---- RMSNorm, optionally fused with the residual add before it. One workgroup
// (or, for many columns, one wave) per column n: x' = x + dx in fp32 (FUSED; stored rounded to bf16 into xo, which
// may be x itself), rstd = 1 / sqrt(sum(x'^2) / M + eps) over the fp32 x', then
// y = x' * rstd * (w + offset) -- on the stored, rounded x' when fused, as the
// reference reloads it (residual_norm.jl:36-41).
// DPART (FUSED only): dx from a split GEMV's fp32 slices (a.dpart), else a.dx
template <bool FUSED, bool DPART, int NT, int RCHUNK, typename Reduce>
__device__ __forceinline__ void rms_norm_row(const NormArgs& a, int n, int t, Reduce reduce) {
  const int nc = a.M / 8;
  const uint16_t* x = a.x + (int64_t)n * a.x_st;
  float v[RCHUNK][8];
  float ss = 0.f;
  // the norm weight first: its loads are in flight with the row's (a load after
  // the block reduction would add a memory latency to this latency-bound kernel)
  float w[RCHUNK][8];
#pragma unroll
  for (int i = 0; i < RCHUNK; ++i)
    if (t + NT * i < nc) load8f(a.w + 8 * (t + NT * i), w[i]);
#pragma unroll
  for (int i = 0; i < RCHUNK; ++i) {
    const int c = t + NT * i;
    if (c < nc) {
      load8f(x + 8 * c, v[i]);
      if (FUSED) {
        float d[8];
        if constexpr (DPART) {  // a split GEMV's slices, summed in slice order, rounded
          // up to 8 slices' loads issued together, then added in slice order
          const float* p = a.dpart + (int64_t)n * a.dpart_cs + 8 * c;
          float4 lo = *reinterpret_cast<const float4*>(p), hi = *reinterpret_cast<const float4*>(p + 4);
          for (int k0 = 1; k0 < a.S2; k0 += 8) {
            float4 l2[8], h2[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
              if (k0 + k < a.S2) {
                l2[k] = *reinterpret_cast<const float4*>(p + (k0 + k) * a.dpart_ss);
                h2[k] = *reinterpret_cast<const float4*>(p + (k0 + k) * a.dpart_ss + 4);
              }
#pragma unroll
            for (int k = 0; k < 8; ++k)
              if (k0 + k < a.S2) {
                lo.x += l2[k].x; lo.y += l2[k].y; lo.z += l2[k].z; lo.w += l2[k].w;
                hi.x += h2[k].x; hi.y += h2[k].y; hi.z += h2[k].z; hi.w += h2[k].w;
              }
          }
          const float s8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
          unpack8(pack8(s8), d);  // the bf16 h the reference stores
        } else {
          load8f(a.dx + (int64_t)n * a.dx_st + 8 * c, d);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float s = v[i][j] + d[j];
          ss += s * s;
          v[i][j] = s;
        }
        const uint4 r = pack8(v[i]);
        *reinterpret_cast<uint4*>(a.xo + (int64_t)n * a.xo_st + 8 * c) = r;
        unpack8(r, v[i]);  // the rounded x' the reference reloads
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += v[i][j] * v[i][j];
      }
    }
  }
  ss = reduce(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)a.M + a.eps);
#pragma unroll
  for (int i = 0; i < RCHUNK; ++i) {
    const int c = t + NT * i;
    if (c < nc) {
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = v[i][j] * rstd * (w[i][j] + a.offset);
      *reinterpret_cast<uint4*>(a.y + (int64_t)n * a.y_st + 8 * c) = pack8(y);
    }
  }
}

template <bool FUSED, bool DPART>
__global__ __launch_bounds__(RT) void rms_norm_kernel(NormArgs a) {
  __shared__ float red[4];
  rms_norm_row<FUSED, DPART, RT, vm::RCHUNK>(a, blockIdx.x, threadIdx.x,
                                             [&](float v) { return block_sum(v, red); });
}
// the same with one wave per column, four columns per workgroup, for many
// columns (a prefill's T x B tokens) of at most 64 x 8 x 8 = 4096: no workgroup
// barrier, and RC (= M / 512 rounded up) chunks per lane, so the registers and
// the waves a SIMD holds follow M
template <bool FUSED, bool DPART, int RC>
__global__ __launch_bounds__(RT) void rms_norm_wave_kernel(NormArgs a) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= a.N) return;
  rms_norm_row<FUSED, DPART, 64, RC>(a, n, threadIdx.x & 63,
                                     [](float v) { return wave_sum_dpp(v); });
}

hipError_t launch_rms_norm(const NormArgs& a, hipStream_t st) {
  if (a.N == 0) return hipSuccess;
  const int mode = a.dpart ? 2 : (a.dx ? 1 : 0);  // dx: none, a bf16 row, fp32 slices
  if (a.N >= 256 && a.M <= 64 * 8 * 8 && mode != 2) {
    const dim3 grid((unsigned)((a.N + 3) / 4));
    switch ((a.M / 8 + 63) / 64) {
#define X(rc)                                                                         \
  case rc:                                                                            \
    if (mode == 1)                                                                    \
      hipLaunchKernelGGL((rms_norm_wave_kernel<true, false, rc>), grid, dim3(RT), 0, st, a); \
    else                                                                              \
      hipLaunchKernelGGL((rms_norm_wave_kernel<false, false, rc>), grid, dim3(RT), 0, st, a); \
    break;
      X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)
#undef X
      default: return hipErrorInvalidValue;
    }
  } else if (mode == 2) {
    hipLaunchKernelGGL((rms_norm_kernel<true, true>), dim3(a.N), dim3(RT), 0, st, a);
  } else if (mode == 1) {
    hipLaunchKernelGGL((rms_norm_kernel<true, false>), dim3(a.N), dim3(RT), 0, st, a);
  } else {
    hipLaunchKernelGGL((rms_norm_kernel<false, false>), dim3(a.N), dim3(RT), 0, st, a);
  }
  return hipGetLastError();
}

// ---- mid = silu(gate) .* up, gate / up the two halves of the packed gate-up
// projection of each column (qwen35.jl:237-239); fp32, one rounding.
__global__ __launch_bounds__(RT) void silu_mul_kernel(SiluMulArgs a) {
  const int nc = a.I / 8;
  const int64_t idx = (int64_t)blockIdx.x * RT + threadIdx.x;
  if (idx >= (int64_t)nc * a.N) return;
  const int n = (int)(idx / nc), c = (int)(idx % nc);
  const uint16_t* g = a.gu + (int64_t)n * a.gu_st + 8 * c;
  float gf[8], uf[8], m[8];
  load8f(g, gf);
  load8f(g + a.I, uf);
#pragma unroll
  for (int j = 0; j < 8; ++j) m[j] = gf[j] / (1.0f + __expf(-gf[j])) * uf[j];
  *reinterpret_cast<uint4*>(a.mid + (int64_t)n * a.mid_st + 8 * c) = pack8(m);
}

hipError_t launch_silu_mul(const SiluMulArgs& a, hipStream_t st) {
  const int64_t n = (int64_t)(a.I / 8) * a.N;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + RT - 1) / RT)), dim3(RT), 0, st, a);
  return hipGetLastError();
}

// ---- x[:, b] = E[:, ids[b]] (ids 1-based; ids outside 1..vocab read the
// nearest valid column rather than past the table).
__global__ __launch_bounds__(RT) void embed_kernel(EmbedArgs a) {
  const int b = blockIdx.x;
  int id = a.ids[b] - 1;
  id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
  const uint16_t* e = a.e + (int64_t)id * a.e_st;
  uint16_t* x = a.x + (int64_t)b * a.x_st;
  for (int c = threadIdx.x; c < a.D / 8; c += RT)
    *reinterpret_cast<uint4*>(x + 8 * c) = load16(e + 8 * c);
}

hipError_t launch_embed(const EmbedArgs& a, hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3(a.B), dim3(RT), 0, st, a);
  return hipGetLastError();
}

// ---- advance!: tokens_out[step, b] = result[b] (column-major (max_new, B),
// column b at col_offsets[b]), then step += 1 and positions[b] += 1. A step
// outside 1..max_new harvests nothing (the reference's bounds contract).
__global__ __launch_bounds__(RT) void gen_advance_kernel(AdvanceArgs a) {
  const int s = *a.step;  // every thread reads it before thread 0 moves it
  for (int b = threadIdx.x; b < a.B; b += RT) {
    if (s >= 1 && s <= a.max_new) a.tokens_out[(int64_t)(s - 1) + a.col_offsets[b]] = a.result[b];
    a.positions[b] += 1;
  }
  __syncthreads();
  if (threadIdx.x == 0) *a.step = s + 1;
}

hipError_t launch_gen_advance(const AdvanceArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(gen_advance_kernel, dim3(1), dim3(RT), 0, st, a);
  return hipGetLastError();
}

// ---- lm head: Result[b] = argmax_v W[:, v] . X[:, b] (1-based, ties to the
// smallest v), without writing the logits.
//
// Wave w takes the vocab columns [w cols, (w + 1) cols) in balanced passes of up
// to four 32-column tiles, and one 32-column batch tile (blockIdx.y). The tiles
// stream through the wave's own LDS in groups of 64 k, double buffered, by direct
// global->LDS loads of 1 KB each (8 columns x 128 contiguous bytes), so every
// weight byte is read once, in whole lines. Per 16-deep k step one 32x32x16
// bf16 MFMA per tile: A = W^T (lane (j, h): column v0 + j, k + 8h .. +7, from
// LDS), B = X (lane (j, h): column b0 + j, the same k, staged the same way), so
// lane (j, h) ends with the logits of batch column b0 + j at vocab rows
// 8 (r / 4) + 4 h + r % 4 of the tile. The wave keeps a running (max, smallest
// index) per batch column; the combine kernel folds the waves' partials.
namespace {

constexpr int LM_TB = 2048;  // bf16 of one staged tile: 32 columns x 64 k (4 KB)

// (v, i) beats (bv, bi): larger, or equal with the smaller index
__device__ __forceinline__ bool lm_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Direct global->LDS loads of k0 .. k0 + 63 of one 32-column tile of a K-major
// matrix (column c at m + c * st), columns c0 .. c0 + 31 clamped to < n:
// instruction i moves columns 8i .. 8i + 7, 128 contiguous bytes each (1 KB per
// instruction, non-temporal); column c's 16-byte chunk q lands at position
// q ^ (c & 7) of its 128-byte row (conflict-free operand reads).
__device__ __forceinline__ void lm_dma_tile(uint16_t* dst, const uint16_t* m, int64_t st, int c0,
                                            int n, int k0, int lane) {
  const int cl = lane >> 3, p = lane & 7;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 8 * i + cl;
    const uint16_t* src = m + (int64_t)min(c0 + c, n - 1) * st + k0 + 8 * (p ^ (c & 7));
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst + 512 * i),
                                     16, 0, 2);
  }
}
// A product's operands: W (K x M rows... K-major, column m at w + m * w_st, m <
// nw) and X (K x B, column b at x + b * x_st, b < nx).
struct MmSrc {
  const uint16_t* w;
  int64_t w_st;
  int nw;
  const uint16_t* x;
  int64_t x_st;
  int nx;
};
// a group: the T weight tiles at v0, then the batch tile at b0 (slot T)
template <int T>
__device__ __forceinline__ void lm_dma(uint16_t* buf, const MmSrc& m, int v0, int b0, int k0,
                                       int lane) {
#pragma unroll
  for (int t = 0; t < T; ++t) lm_dma_tile(buf + t * LM_TB, m.w, m.w_st, v0 + 32 * t, m.nw, k0, lane);
  lm_dma_tile(buf + T * LM_TB, m.x, m.x_st, b0, m.nx, k0, lane);
}

// The products of one staged group: step s of tile t reads lane (j, h)'s A
// operand, column j k 16s + 8h .. +7, from LDS. The reads are issued from asm
// (a compiler-visible read would first drain every load in flight, the other
// buffer's included) one step ahead, each released by a counted wait tied to
// its registers.
typedef unsigned int lm_u32x4 __attribute__((ext_vector_type(4)));  // asm register operand
template <int T>
__device__ __forceinline__ void lm_read(lm_u32x4 (&w)[T], const uint16_t* buf, int j, int h, int s) {
  const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)buf;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t addr = base + 2u * (uint32_t)(t * LM_TB + 64 * j + 8 * ((2 * s + h) ^ (j & 7)));
    asm volatile("ds_read_b128 %0, %1" : "=v"(w[t]) : "v"(addr));
  }
}
template <int N, int T>
__device__ __forceinline__ void lm_take(lm_u32x4 (&w)[T]) {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
  for (int t = 0; t < T; ++t) asm volatile("" : "+v"(w[t]));
}
template <int T>
__device__ __forceinline__ void lm_mult(const uint16_t* buf, int j, int h, f32x16 (&acc)[T]) {
  // slots 0 .. T-1: the weight tiles (A operands), slot T: the batch tile (B)
  lm_u32x4 w0[T + 1], w1[T + 1];
  lm_read<T + 1>(w0, buf, j, h, 0);
  lm_read<T + 1>(w1, buf, j, h, 1);
  lm_take<T + 1, T + 1>(w0);
#pragma unroll
  for (int t = 0; t < T; ++t)
    acc[t] = mfma32(__builtin_bit_cast(uint4, w0[t]), __builtin_bit_cast(uint4, w0[T]), acc[t]);
  lm_read<T + 1>(w0, buf, j, h, 2);
  lm_take<T + 1, T + 1>(w1);
#pragma unroll
  for (int t = 0; t < T; ++t)
    acc[t] = mfma32(__builtin_bit_cast(uint4, w1[t]), __builtin_bit_cast(uint4, w1[T]), acc[t]);
  lm_read<T + 1>(w1, buf, j, h, 3);
  lm_take<T + 1, T + 1>(w0);
#pragma unroll
  for (int t = 0; t < T; ++t)
    acc[t] = mfma32(__builtin_bit_cast(uint4, w0[t]), __builtin_bit_cast(uint4, w0[T]), acc[t]);
  lm_take<0, T + 1>(w1);
#pragma unroll
  for (int t = 0; t < T; ++t)
    acc[t] = mfma32(__builtin_bit_cast(uint4, w1[t]), __builtin_bit_cast(uint4, w1[T]), acc[t]);
}

// one object per buffer: reads of one are seen not to alias the loads landing in
// the other (no drain of every load in flight before each read)
__shared__ __attribute__((aligned(16))) uint16_t lm_buf0[4][5 * LM_TB];
__shared__ __attribute__((aligned(16))) uint16_t lm_buf1[4][5 * LM_TB];

// acc[t] = W^T X over k = k0 .. k1 - 1 (multiples of 64) for the T 32-row tiles
// at v0 and the 32-column batch tile at b0, in groups of 64 k, double buffered.
// Lane (j, h) ends with batch column b0 + j at rows 8 (r / 4) + 4 h + r % 4 of
// each tile.
template <int T>
__device__ __forceinline__ void mm_tiles(const MmSrc& m, int v0, int bt0, int k0, int k1, int lane,
                                         f32x16 (&acc)[T]) {
  const int j = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  uint16_t* b0 = lm_buf0[wv];
  uint16_t* b1 = lm_buf1[wv];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
  constexpr int PER = 4 * (T + 1);  // loads per group
  const int G = (k1 - k0) / 64;      // groups, >= 1
  lm_dma<T>(b0, m, v0, bt0, k0, lane);
  int g = 0;
  // steady state, no branch in the body: groups g (in b0) and g + 1 (into b1),
  // then g + 2 into b0 again
  for (; g + 2 < G; g += 2) {
    lm_dma<T>(b1, m, v0, bt0, k0 + 64 * (g + 1), lane);
    wait_vmcnt<PER>();
    lm_mult<T>(b0, j, h, acc);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // b0's reads are in: refill it
    lm_dma<T>(b0, m, v0, bt0, k0 + 64 * (g + 2), lane);
    wait_vmcnt<PER>();
    lm_mult<T>(b1, j, h, acc);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  if (g + 1 < G) {  // the last two groups
    lm_dma<T>(b1, m, v0, bt0, k0 + 64 * (g + 1), lane);
    wait_vmcnt<PER>();
    lm_mult<T>(b0, j, h, acc);
    wait_vmcnt<0>();
    lm_mult<T>(b1, j, h, acc);
  } else {          // the last group
    wait_vmcnt<0>();
    lm_mult<T>(b0, j, h, acc);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the next call refills both
}

// One lm-head pass: T tiles (vocab columns v0 .. v0 + 32T - 1) over all of K,
// then the running (max, index) of this lane's batch column, in vocab order.
template <int T>
__device__ __forceinline__ void lm_pass(const LmHeadArgs& a, int v0, int vend, int bt0, int lane,
                                        float& best, int& besti) {
  const int h = lane >> 5;
  const MmSrc m{a.w, a.w_st, a.N, a.x, a.x_st, a.B};
  f32x16 acc[T];
  mm_tiles<T>(m, v0, bt0, 0, a.K, lane, acc);
  // lane (j, h): rows 8 (r / 4) + 4 h + r % 4 of each tile, increasing in r
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int v = v0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
      const float l = v < vend ? acc[t][r] : -INFINITY;
      if (lm_better(l, v, best, besti)) {
        best = l;
        besti = v;
      }
    }
  }
}

}  // namespace

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void lm_head_split_kernel(LmHeadArgs a) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int j = lane & 31, h = lane >> 5;
  const int b0 = 32 * blockIdx.y;
  const int vbeg = w * a.cols, vend = min(vbeg + a.cols, a.N);
  float best = -INFINITY;
  int besti = 0x7fffffff;
  const bool xok = b0 + j < a.B;  // padded batch columns re-read the last one (not stored)
  // the wave's tiles in balanced passes of at most four
  const int ntiles = vend > vbeg ? (vend - vbeg + 31) / 32 : 0;
  const int npass = (ntiles + 3) / 4;
  int v0 = vbeg;
  for (int p = 0; p < npass; ++p) {
    const int rem = ntiles - (v0 - vbeg) / 32;
    const int t_p = (rem + npass - p - 1) / (npass - p);
    switch (t_p) {
      case 4: lm_pass<4>(a, v0, vend, b0, lane, best, besti); break;
      case 3: lm_pass<3>(a, v0, vend, b0, lane, best, besti); break;
      case 2: lm_pass<2>(a, v0, vend, b0, lane, best, besti); break;
      default: lm_pass<1>(a, v0, vend, b0, lane, best, besti); break;
    }
    v0 += 32 * t_p;
  }
  // the two lane halves hold the same batch column: fold them
  const auto pv = __builtin_amdgcn_permlane32_swap(__float_as_uint(best), __float_as_uint(best), false, false);
  const auto pi = __builtin_amdgcn_permlane32_swap((unsigned)besti, (unsigned)besti, false, false);
  const float ov = __uint_as_float(h ? pv[0] : pv[1]);  // the other half's value
  const int oi = (int)(h ? pi[0] : pi[1]);
  if (lm_better(ov, oi, best, besti)) {
    best = ov;
    besti = oi;
  }
  if (h == 0 && xok) {
    a.pmax[(int64_t)w * a.B + b0 + j] = best;
    a.pidx[(int64_t)w * a.B + b0 + j] = besti;
  }
}

// ---- y = W^T x for a narrow x (N <= 32 columns; linear.cpp picks which): the decode step's projections (linear!, src/linear.jl:40-57, at N = B). HBM-bound like the lm
// head and built the same way: one 32-column batch tile, 32-row weight tiles
// staged through LDS by 1-KB direct loads, bf16 MFMAs, fp32 sums. Workgroup
// (tile group tg, K slice s2) takes T <= 2 tiles; its four waves split the
// slice's 64-deep k groups in four contiguous runs and add their sums through
// LDS (the staging buffers, free by then). With S2 > 1 slices the workgroups
// write fp32 partials, summed in slice order by gemv_reduce_kernel
// (deterministic).
//
// A wave's run is short (a few groups: the whole launch streams ~100 KB per
// CU), so the groups stream through a ring of three slots (12 KB each, 144 KB
// per workgroup): the first three are issued at once and each slot is refilled
// as soon as its products have read it, two groups in flight behind the one
// being multiplied. A run of up to three groups then costs one memory latency.
namespace {

// one object per slot (the reads of one are seen not to alias the loads
// landing in the others)
__shared__ __attribute__((aligned(16))) uint16_t gv_buf0[4][3 * LM_TB];
__shared__ __attribute__((aligned(16))) uint16_t gv_buf1[4][3 * LM_TB];
__shared__ __attribute__((aligned(16))) uint16_t gv_buf2[4][3 * LM_TB];

// wait until at most `left` groups (of PER loads each) issued after the one
// about to be multiplied are still in flight
template <int PER>
__device__ __forceinline__ void gv_wait(int left) {
  if (left >= 2) wait_vmcnt<2 * PER>();
  else if (left == 1) wait_vmcnt<PER>();
  else wait_vmcnt<0>();
}

// group g of the run (in slot S): wait for it, multiply, refill the slot with
// group g + 3
template <int T, int S>
__device__ __forceinline__ void gv_group(uint16_t* buf, const MmSrc& m, int v0, int k0, int g,
                                         int G, int j, int h, int lane, f32x16 (&acc)[T]) {
  constexpr int PER = 4 * (T + 1);
  gv_wait<PER>(min(G - 1 - g, 2));
  lm_mult<T>(buf, j, h, acc);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's reads are in: refill it
  if (g + 3 < G) lm_dma<T>(buf, m, v0, 0, k0 + 64 * (g + 3), lane);
}

// acc[t] = W^T X over k = k0 .. k1 - 1 (multiples of 64, k1 > k0) for the T
// 32-row tiles at v0 and the batch tile, through the three-slot ring (lane
// layout of mm_tiles)
template <int T>
__device__ __forceinline__ void gv_tiles(const MmSrc& m, int v0, int k0, int k1, int lane,
                                         f32x16 (&acc)[T]) {
  const int j = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  uint16_t* b0 = gv_buf0[wv];
  uint16_t* b1 = gv_buf1[wv];
  uint16_t* b2 = gv_buf2[wv];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
  const int G = (k1 - k0) / 64;
  lm_dma<T>(b0, m, v0, 0, k0, lane);
  if (G > 1) lm_dma<T>(b1, m, v0, 0, k0 + 64, lane);
  if (G > 2) lm_dma<T>(b2, m, v0, 0, k0 + 128, lane);
  for (int g = 0; g < G; g += 3) {
    gv_group<T, 0>(b0, m, v0, k0, g, G, j, h, lane, acc);
    if (g + 1 < G) gv_group<T, 1>(b1, m, v0, k0, g + 1, G, j, h, lane, acc);
    if (g + 2 < G) gv_group<T, 2>(b2, m, v0, k0, g + 2, G, j, h, lane, acc);
  }
}

template <int T>
__device__ __forceinline__ void gemv_wg(const GemvArgs& a, int tg, int s2, int lane) {
  const int wv = threadIdx.x >> 6, j = lane & 31, h = lane >> 5;
  const int v0 = 32 * T * tg;
  // this workgroup's k groups, then this wave's run of them
  const int gw0 = s2 * a.gps, gw1 = min(gw0 + a.gps, a.G);
  const int per = (gw1 - gw0 + 3) / 4;
  const int g0 = min(gw0 + wv * per, gw1), g1 = min(g0 + per, gw1);
  const MmSrc m{a.w, a.w_st, a.M, a.x, a.x_st, a.N};
  f32x16 acc[T];
  if (g1 > g0) {
    gv_tiles<T>(m, v0, 64 * g0, 64 * g1, lane, acc);
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
  }
  // the four waves' sums through LDS: wave w's tile t, register r, lane l at
  // [w][t][r][l] (floats, 32 KB at T = 2, in the first two slots); then wave t
  // adds tile t of all four
  static_assert(4 * 2 * 16 * 64 * sizeof(float) <= 2 * sizeof(gv_buf0), "reduction space");
  float* red = reinterpret_cast<float*>(gv_buf0[0]);
  __syncthreads();  // every wave is done with the staging buffers
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[((wv * T + t) * 16 + r) * 64 + lane] = acc[t][r];
  __syncthreads();
  if (wv >= T || j >= a.N) return;
  const int t = wv;
  float o[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float v = red[((0 * T + t) * 16 + r) * 64 + lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) v += red[((w * T + t) * 16 + r) * 64 + lane];
    o[r] = v;
  }
  // lane (j, h): rows 8q + 4h .. +3 of the tile, q = 0..3, for batch column j
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = v0 + 32 * t + 8 * q + 4 * h;
    if (row >= a.M) continue;
    if (a.S2 == 1) {
      const uint2 v = make_uint2(pack2(o[4 * q], o[4 * q + 1]), pack2(o[4 * q + 2], o[4 * q + 3]));
      *reinterpret_cast<uint2*>(a.y + (int64_t)j * a.y_st + row) = v;
    } else {
      *reinterpret_cast<float4*>(a.part + ((int64_t)s2 * 32 + j) * a.M + row) =
          make_float4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
    }
  }
}

}  // namespace

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemv_kernel(GemvArgs a) {
  const int lane = threadIdx.x & 63;
  const int tg = blockIdx.x / a.S2, s2 = blockIdx.x % a.S2;
  if (a.T == 2) gemv_wg<2>(a, tg, s2, lane);
  else gemv_wg<1>(a, tg, s2, lane);
}

// y[:, b] rows 4i .. 4i + 3 = the slices' partials added in slice order
__global__ __launch_bounds__(256) void gemv_reduce_kernel(GemvArgs a) {
  const int q4 = a.M / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)q4 * a.N) return;
  const int b = (int)(idx / q4), row = 4 * (int)(idx % q4);
  float4 s = *reinterpret_cast<const float4*>(a.part + (int64_t)b * a.M + row);
  for (int k = 1; k < a.S2; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(a.part + ((int64_t)k * 32 + b) * a.M + row);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  *reinterpret_cast<uint2*>(a.y + (int64_t)b * a.y_st + row) =
      make_uint2(pack2(s.x, s.y), pack2(s.z, s.w));
}

// The split: T tiles per workgroup and S2 K slices, from a cost model of
// one workgroup per CU (the staging buffers take the CU's LDS): the launch runs
// in ceil(workgroups / CUs) rounds, a round lasts as long as its waves take to
// stream their groups ((T + 1) tiles of 4 KB each, plus about two groups of
// pipeline fill), and S2 > 1 adds the partials' write and read spread over all
// waves. The smallest cost wins (ties: fewer slices, then wider tile groups).
GemvPlan gemv_plan(int M, int K, int waves) {
  const int tiles = (M + 31) / 32, G = K / 64;
  const int cus = max(1, waves / 4);
  GemvPlan best{1, 1, G, tiles};
  double best_cost = 1e300;
  for (int T : {2, 1}) {
    const int ntg = (tiles + T - 1) / T;
    for (int S2 = 1; S2 <= G; ++S2) {
      const int gps = (G + S2 - 1) / S2;
      if ((G + gps - 1) / gps != S2) continue;  // every slice non-empty
      const int rounds = (ntg * S2 + cus - 1) / cus;
      const int per = (gps + 3) / 4;
      double cost = (double)rounds * (per + 2) * (T + 1) * 4096.0;
      if (S2 > 1) cost += 2.0 * S2 * 32.0 * M * 4.0 / (4.0 * cus);
      if (cost < best_cost * (1 - 1e-9)) {
        best_cost = cost;
        best = GemvPlan{T, S2, gps, ntg};
      }
    }
  }
  return best;
}

size_t gemv_workspace_bytes(int M, int K) {
  const GemvPlan p = gemv_plan(M, K, lm_head_waves());
  return p.S2 > 1 ? (size_t)p.S2 * 32 * (size_t)M * sizeof(float) : 0;
}

hipError_t launch_gemv_partials(GemvArgs a, GemvPlan* plan, hipStream_t st) {
  const GemvPlan p = gemv_plan(a.M, a.K, lm_head_waves());
  *plan = p;
  a.T = p.T;
  a.S2 = p.S2;
  a.gps = p.gps;
  a.G = a.K / 64;
  hipLaunchKernelGGL(gemv_kernel, dim3(p.ntg * p.S2), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_gemv(GemvArgs a, hipStream_t st) {
  const GemvPlan p = gemv_plan(a.M, a.K, lm_head_waves());
  a.T = p.T;
  a.S2 = p.S2;
  a.gps = p.gps;
  a.G = a.K / 64;
  hipLaunchKernelGGL(gemv_kernel, dim3(p.ntg * p.S2), dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.S2 == 1) return e;
  const int64_t n = (int64_t)(a.M / 4) * a.N;
  hipLaunchKernelGGL(gemv_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ---- y = W^T x for the wide decode projections (N <= 32 batch columns, M of
// thousands of rows), stream-K over the weight: the unit of work is one 64-k
// group of one 128-row group of W (16 KB), numbered row-group-major. Workgroup
// b takes units [b chunk, (b + 1) chunk); its wave v computes the 32-row tile
// 4 rg + v of each unit, so the four waves share the unit's batch tile (32
// columns x 64 k, 4 KB), each DMAing a quarter of it into the workgroup's slot.
// The batch tile then costs a quarter of the weight bytes in L2 traffic (the
// narrow kernel above loads one per one or two weight tiles, which is what
// keeps it from the streaming rate at these sizes). Tiles stream through LDS
// by 1-KB direct loads, one barrier per unit; a unit's slot is refilled after
// the next barrier, once every wave has read it. A workgroup writes one fp32
// partial per row group it touches into slot (b + rg); the consumer adds a
// row's slots in workgroup order (gemv_sk_sum4, common.h), so results are
// bitwise repeatable.
constexpr int SK_NB = 4;   // ring slots per wave (three units in flight)
constexpr int SK_TE = 2048;  // bf16 of one staged 32 x 64 tile (4 KB)

namespace {

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemv_sk_kernel(GemvSkArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t wring[4][SK_NB][SK_TE];
  __shared__ __attribute__((aligned(16))) uint16_t xring[SK_NB][SK_TE];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int j = lane & 31, h = lane >> 5;
  const int G = a.p.G;
  const int u0 = blockIdx.x * a.p.chunk;
  if (u0 >= a.p.U) return;  // the whole workgroup
  const int u1 = min(u0 + a.p.chunk, a.p.U);
  const int n = u1 - u0;
  // unit u into ring slot s: this wave's weight tile (4 loads) and rows
  // 8 wv .. 8 wv + 7 of the batch tile (1 load; the batch stays in L2, so the
  // default cache policy)
  auto issue = [&](int u, int s) __attribute__((always_inline)) {
    const int rg = u / G, g = u - rg * G;
    lm_dma_tile(wring[wv][s], a.w, a.w_st, 32 * (4 * rg + wv), a.M, 64 * g, lane);
    const int c = 8 * wv + (lane >> 3), p = lane & 7;
    const uint16_t* src = a.x + (int64_t)min(c, a.N - 1) * a.x_st + 64 * g + 8 * (p ^ (c & 7));
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(&xring[s][512 * wv]),
                                     16, 0, 0);
  };
  int issued = 0;
  for (; issued < SK_NB - 1 && issued < n; ++issued) issue(u0 + issued, issued);
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  int rcur = u0 / G;
  // this wave's partial of row group rg: lane (j, h) holds batch column j at
  // rows 8 q + 4 h .. +3 of the tile (the 32x32x16 MFMA's D layout)
  auto flush = [&](int rg) __attribute__((always_inline)) {
    float* dst = a.part + (((int64_t)(blockIdx.x + rg) * 4 + wv) * 32 + j) * 32 + 4 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(dst + 8 * q) =
          make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
  };
  for (int i = 0; i < n; ++i) {
    // this wave's loads of unit i are in (loads retire in order; the partial
    // stores issued later only make the count conservative), then every
    // wave's: the barrier also tells that unit i - 1's slot is read
    if (issued - i - 1 >= SK_NB - 2) wait_vmcnt<5 * (SK_NB - 2)>(); else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (issued < n) {
      issue(u0 + issued, issued % SK_NB);
      ++issued;
    }
    const int s = i % SK_NB;
    const int rg = (u0 + i) / G;
    if (rg != rcur) {
      flush(rcur);
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.f;
      rcur = rg;
    }
    // operands from asm reads (a compiler-visible read would first drain every
    // load in flight), released by one counted wait tied to their registers
    lm_u32x4 wa[4], xb[4];
    const uint32_t wbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)wring[wv][s];
    const uint32_t xbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)xring[s];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const uint32_t off = 2u * (uint32_t)(64 * j + 8 * ((2 * st + h) ^ (j & 7)));
      asm volatile("ds_read_b128 %0, %1" : "=v"(wa[st]) : "v"(wbase + off));
      asm volatile("ds_read_b128 %0, %1" : "=v"(xb[st]) : "v"(xbase + off));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int st = 0; st < 4; ++st) asm volatile("" : "+v"(wa[st]), "+v"(xb[st]));
#pragma unroll
    for (int st = 0; st < 4; ++st)
      acc = mfma32(__builtin_bit_cast(uint4, wa[st]), __builtin_bit_cast(uint4, xb[st]), acc);
  }
  flush(rcur);
}

// ---- mid = silu(gate) .* up (qwen35.jl:237-239) from the gate-up projection's
// stream-K partials: gate and up rounded to bf16 first, as the reference stores
// them in gu, then one fp32 evaluation and one rounding, as silu_mul_kernel.
__global__ __launch_bounds__(RT) void silu_mul_sk_kernel(SiluMulSkArgs a) {
  const int nc = a.I / 8;
  const int64_t idx = (int64_t)blockIdx.x * RT + threadIdx.x;
  if (idx >= (int64_t)nc * a.N) return;
  const int n = (int)(idx / nc), i = 8 * (int)(idx % nc);
  const int G = a.p.G, ch = a.p.chunk;
  const float4 g0 = gemv_sk_sum4(a.part, G, ch, i, n), g1 = gemv_sk_sum4(a.part, G, ch, i + 4, n);
  const float4 u0 = gemv_sk_sum4(a.part, G, ch, a.I + i, n);
  const float4 u1 = gemv_sk_sum4(a.part, G, ch, a.I + i + 4, n);
  const float g8[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  const float u8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
  float gf[8], uf[8], m[8];
  unpack8(pack8(g8), gf);
  unpack8(pack8(u8), uf);
#pragma unroll
  for (int k = 0; k < 8; ++k) m[k] = gf[k] / (1.0f + __expf(-gf[k])) * uf[k];
  *reinterpret_cast<uint4*>(a.mid + (int64_t)n * a.mid_st + i) = pack8(m);
}

}  // namespace

GemvSkPlan gemv_sk_plan(int M, int K) {
  GemvSkPlan p;
  p.G = K / 64;
  p.RG = (M + 127) / 128;
  p.U = p.RG * p.G;
  const int wgs = max(1, lm_head_waves() / 4);  // one workgroup per CU
  p.chunk = max(1, (p.U + wgs - 1) / wgs);
  p.nwg = p.U > 0 ? (p.U + p.chunk - 1) / p.chunk : 0;
  return p;
}

size_t gemv_sk_workspace_bytes(int M, int K) {
  const GemvSkPlan p = gemv_sk_plan(M, K);
  return p.U > 0 ? (size_t)(p.nwg + p.RG - 1) * 4 * 1024 * sizeof(float) : 0;
}

hipError_t launch_gemv_sk(const GemvSkArgs& a, hipStream_t st) {
  if (a.p.U == 0 || a.N == 0) return hipSuccess;
  hipLaunchKernelGGL(gemv_sk_kernel, dim3(a.p.nwg), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_silu_mul_sk(const SiluMulSkArgs& a, hipStream_t st) {
  const int64_t n = (int64_t)(a.I / 8) * a.N;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(silu_mul_sk_kernel, dim3((unsigned)((n + RT - 1) / RT)), dim3(RT), 0, st, a);
  return hipGetLastError();
}

// One workgroup per batch column: the best of the NW partials (ties to the
// smallest index), stored 1-based.
__global__ __launch_bounds__(256) void lm_head_combine_kernel(LmHeadArgs a) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int b = blockIdx.x, t = threadIdx.x;
  float best = -INFINITY;
  int besti = 0x7fffffff;
  for (int w = t; w < a.NW; w += 256) {
    const float v = a.pmax[(int64_t)w * a.B + b];
    const int i = a.pidx[(int64_t)w * a.B + b];
    if (lm_better(v, i, best, besti)) {
      best = v;
      besti = i;
    }
  }
  sv[t] = best;
  si[t] = besti;
  __syncthreads();
  for (int s = 128; s >= 1; s >>= 1) {
    if (t < s && lm_better(sv[t + s], si[t + s], sv[t], si[t])) {
      sv[t] = sv[t + s];
      si[t] = si[t + s];
    }
    __syncthreads();
  }
  if (t == 0) a.result[b] = si[0] == 0x7fffffff ? 1 : si[0] + 1;
}

int lm_head_waves() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  return 4 * cus;  // one wave per SIMD
}

hipError_t launch_lm_head_argmax(LmHeadArgs a, hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  const int tiles = (a.N + 31) / 32;
  a.cols = 32 * ((tiles + a.NW - 1) / a.NW);
  hipLaunchKernelGGL(lm_head_split_kernel, dim3(a.NW / 4, (a.B + 31) / 32), dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lm_head_combine_kernel, dim3(a.B), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace vm

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
// per column n: x' = x + dx in fp32 (FUSED; stored rounded to bf16 into xo, which
// may be x itself), rstd = 1 / sqrt(sum(x'^2) / M + eps) over the fp32 x', then
// y = x' * rstd * (w + offset) -- on the stored, rounded x' when fused, as the
// reference reloads it (residual_norm.jl:36-41).
template <bool FUSED>
__global__ __launch_bounds__(RT) void rms_norm_kernel(NormArgs a) {
  __shared__ float red[4];
  const int n = blockIdx.x, t = threadIdx.x;
  const int nc = a.M / 8;
  const uint16_t* x = a.x + (int64_t)n * a.x_st;
  float v[RCHUNK][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < RCHUNK; ++i) {
    const int c = t + RT * i;
    if (c < nc) {
      load8f(x + 8 * c, v[i]);
      if (FUSED) {
        float d[8];
        load8f(a.dx + (int64_t)n * a.dx_st + 8 * c, d);
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
  ss = block_sum(ss, red);
  const float rstd = 1.0f / sqrtf(ss / (float)a.M + a.eps);
#pragma unroll
  for (int i = 0; i < RCHUNK; ++i) {
    const int c = t + RT * i;
    if (c < nc) {
      float w[8], y[8];
      load8f(a.w + 8 * c, w);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = v[i][j] * rstd * (w[j] + a.offset);
      *reinterpret_cast<uint4*>(a.y + (int64_t)n * a.y_st + 8 * c) = pack8(y);
    }
  }
}

hipError_t launch_rms_norm(const NormArgs& a, hipStream_t st) {
  if (a.N == 0) return hipSuccess;
  if (a.dx)
    hipLaunchKernelGGL(rms_norm_kernel<true>, dim3(a.N), dim3(RT), 0, st, a);
  else
    hipLaunchKernelGGL(rms_norm_kernel<false>, dim3(a.N), dim3(RT), 0, st, a);
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
// Wave w takes the vocab columns [w cols, (w + 1) cols) in passes of up to four
// 32-column tiles and one 32-column batch tile (blockIdx.y). Per 16-deep k step
// one 32x32x16 bf16 MFMA per tile: A = W^T (lane (j, h): column v0 + j, k + 8h
// .. +7, one 16-byte load), B = X (lane (j, h): column b0 + j, the same k), so
// lane (j, h) ends with the logits of batch column b0 + j at vocab rows
// 8 (r / 4) + 4 h + r % 4 of the tile. Each weight byte is read once. The next
// four k steps' loads are in flight while the current ones multiply. The wave
// keeps a running (max, smallest index) per batch column; LmCombine folds the
// waves' partials.
namespace {

constexpr int LM_KG = 4;  // k steps (of 16) per load group
constexpr int LM_T = 4;   // vocab tiles per pass

struct LmGroup {
  uint4 w[LM_T][LM_KG];
  uint4 x[LM_KG];
};

// the loads of k steps k0 .. k0 + 63; this lane's 8 values start at k + 8h
// (already in wcol0 / xcol; K is a multiple of 8, so a slice is all in or out)
__device__ __forceinline__ void lm_load(LmGroup& g, const LmHeadArgs& a, const uint16_t* wcol0,
                                        const uint16_t* xcol, int h, int k0, int ntile,
                                        const int (&vok)[LM_T]) {
#pragma unroll
  for (int s = 0; s < LM_KG; ++s) {
    const int k = k0 + 16 * s;
    const bool kin = k + 8 * h < a.K;
    g.x[s] = kin ? load16(xcol + k) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < LM_T; ++t) {
      if (t < ntile)
        g.w[t][s] = (kin && vok[t]) ? load16_nt(wcol0 + (int64_t)(32 * t) * a.w_st + k)
                                    : make_uint4(0, 0, 0, 0);
    }
  }
}

// (v, i) beats (bv, bi): larger, or equal with the smaller index
__device__ __forceinline__ bool lm_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
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
  const bool xok = b0 + j < a.B;  // padded batch lanes read column b0 (not stored)
  const uint16_t* xcol = a.x + (int64_t)(xok ? b0 + j : b0) * a.x_st + 8 * h;
  for (int v0 = vbeg; v0 < vend; v0 += 32 * LM_T) {
    const int ntile = min(LM_T, (vend - v0 + 31) / 32);  // uniform
    int vok[LM_T];
#pragma unroll
    for (int t = 0; t < LM_T; ++t) vok[t] = v0 + 32 * t + j < a.N;
    // column v0 + 32 t + j of this lane, clamped into the table
    const uint16_t* wcol0 = a.w + (int64_t)min(v0 + j, a.N - 1) * a.w_st + 8 * h;
    f32x16 acc[LM_T];
#pragma unroll
    for (int t = 0; t < LM_T; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
    // two register groups in turn: one multiplies while the other's loads land
    constexpr int KS = 16 * LM_KG;
    auto mult = [&](const LmGroup& g) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < LM_KG; ++s)
#pragma unroll
        for (int t = 0; t < LM_T; ++t)
          if (t < ntile) acc[t] = mfma32(g.w[t][s], g.x[s], acc[t]);
    };
    LmGroup g0, g1;
    lm_load(g0, a, wcol0, xcol, h, 0, ntile, vok);
    for (int k0 = 0; k0 < a.K; k0 += 2 * KS) {
      if (k0 + KS < a.K) lm_load(g1, a, wcol0, xcol, h, k0 + KS, ntile, vok);
      mult(g0);
      if (k0 + 2 * KS < a.K) lm_load(g0, a, wcol0, xcol, h, k0 + 2 * KS, ntile, vok);
      if (k0 + KS < a.K) mult(g1);
    }
    // the tiles' logits, in increasing vocab order within each lane half
#pragma unroll
    for (int t = 0; t < LM_T; ++t) {
      if (t < ntile) {
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

// decode.hip — split-KV flash-decoding for one new token per sequence
// (the work of src/kernels/attention_decode.jl:14-181, re-designed for CDNA4).
//
// Work partition ("stream-K"): the token-heads of the batch, sum_b len_b * Hk,
// are cut into NW equal contiguous chunks, one per wave, so every wave streams
// the same number of K/V bytes whatever the ragged lengths are (lengths are read
// on the device, so a captured graph replays correctly as they grow). A chunk
// may span several (sequence b, kv head hk) segments; the wave emits one
// partial (unnormalised O, shift m, sum l) per segment it touches, into slot
// w + (b*Hk + hk), which is unique because consecutive waves cover
// non-decreasing segment ranges. The combine kernel merges a segment's slots.
//
// Per wave, 16-token steps on bf16 MFMA with the GQA group (G <= 8 query heads
// sharing hk) on the N = 16 side, so each K/V byte is read from HBM once:
//   S^T[tok][head] = K[tok][:] . Q[head][:]    16x16x32; A = K straight from HBM
//                                                (16 B per lane), B = Q in registers
//   O^T[d][head]  += V^T[d][tok] . P^T[tok][head]   16x16x16
// S^T already sits in the lanes/slots of the P^T operand. V^T comes from the
// natural-layout V fragments through a 16x16x32 MFMA against a 0/1 selection
// matrix (bf16 * 1.0 plus exact zeros is exact in fp32), so no LDS is used.
// K/V fragments are triple-buffered in registers (one wave per SIMD): steps
// i+1 and i+2 are in flight while step i computes.
//
// Softmax: with QK-norm the logits are bounded, |s| <= |q~| * sqrt(D) *
// max|kw + w_offset|, so the fused path uses that bound as a fixed per-head
// shift when it is <= 64 (log2 units); otherwise, and for the unfused operator,
// a running max rescaled lazily (only when it grows by > 8).
#include "common.h"
#include "kernels.h"

namespace vm {

constexpr int DSTEP = 16;                 // tokens per step
constexpr float D_RESCALE_SLACK = 8.0f;
constexpr float D_STATIC_LIMIT = 64.0f;

__device__ __forceinline__ f32x4 mfma16k16(const uint2& a, const uint2& b, f32x4 c) {
  typedef short s16x4v __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4v, a),
                                                  __builtin_bit_cast(s16x4v, b), c, 0, 0, 0);
}

// chunk of the stream partition (token-heads per wave), identical in both kernels
__device__ __forceinline__ int stream_chunk(int W, int NW, int min_chunk) {
  int c = (W + NW - 1) / NW;
  c = max(c, min_chunk);
  return (c + DSTEP - 1) / DSTEP * DSTEP;
}

__device__ __forceinline__ int clamp_len(const int32_t* lengths, int b, int64_t ctx) {
  int64_t l = lengths[b];
  l = l < 0 ? 0 : (l > ctx ? ctx : l);
  return (int)l;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

struct StepBuf {
  uint4 k[8], v[8];
};

__device__ __forceinline__ void load_step(StepBuf& s, const uint16_t* kb, const uint16_t* vb,
                                          int64_t row, int64_t c_st) {
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) s.k[kk] = load16(kb + row * c_st + 32 * kk);
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) s.v[kk] = load16(vb + row * c_st + 32 * kk);
}

__device__ __forceinline__ void compute_step(StepBuf& s, int t, int hi, int n, int g,
                                             const uint4 (&qop)[8], const uint4 (&sel)[2],
                                             f32x4 (&acc)[16], float& m_run, float& l_part) {
  if (t + DSTEP > hi && t + n >= hi) {
    // rows past the range may hold anything: p = 0 must meet finite v
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) s.v[kk] = make_uint4(0, 0, 0, 0);
  }
  f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) sc = mfma16(s.k[kk], qop[kk], sc);
  if (t + DSTEP > hi) {
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = (t + 4 * g + j < hi) ? sc[j] : -INFINITY;
  }
  // running max in log2 units, rescaled lazily: only when it grows by more
  // than D_RESCALE_SLACK (never, when m_run starts at the QK-norm bound)
  float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
  mx = wave_max_xor(mx, 16);
  mx = wave_max_xor(mx, 32) * LOG2E;
  const float m_new = fmaxf(m_run, mx);  // finite: token t is valid
  const bool need = m_new > m_run + D_RESCALE_SLACK;
  if (__ballot(need) != 0ull) {
    const float m_use = need ? m_new : m_run;
    const float alpha = (m_use == m_run) ? 1.0f : fast_exp2(m_run - m_use);
    l_part *= alpha;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= alpha;
    m_run = m_use;
  }
  const float m_eff = m_run;
  float p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = fast_exp2(__builtin_fmaf(sc[j], LOG2E, -m_eff));
  l_part += (p[0] + p[1]) + (p[2] + p[3]);
  const uint2 pop = make_uint2(pack2(p[0], p[1]), pack2(p[2], p[3]));
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 tv = mfma16(s.v[kk], sel[h], zero);  // V[t+4g+j][32kk+16h+n], exact
      const uint2 vt = make_uint2(
          (__float_as_uint(tv[0]) >> 16) | (__float_as_uint(tv[1]) & 0xffff0000u),
          (__float_as_uint(tv[2]) >> 16) | (__float_as_uint(tv[3]) & 0xffff0000u));
      acc[2 * kk + h] = mfma16k16(vt, pop, acc[2 * kk + h]);
    }
  }
}

template <bool FUSED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void decode_stream_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int G = a.G, Hk = a.Hk;
  if (a.counter && blockIdx.x == 0 && threadIdx.x == 0) a.counter[0] = 0;  // for the merge

  // ---- stream partition: total work and this wave's chunk [gw0, gw1)
  int W = 0;
  for (int b0 = 0; b0 < a.B; b0 += 64) {
    int v = (b0 + lane < a.B) ? clamp_len(a.lengths, b0 + lane, a.ctx) : 0;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    W += v;
  }
  W *= Hk;
  const int chunk = stream_chunk(W, a.NW, a.min_chunk);
  const int gw0 = w * chunk;
  if (gw0 >= W) return;
  const int gw1 = min(gw0 + chunk, W);

  // ---- locate the segment holding gw0: first b whose prefix (token-heads) passes it
  int b = 0, seg_b_start = 0;
  {
    int pre = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
      const int len = (b0 + lane < a.B) ? clamp_len(a.lengths, b0 + lane, a.ctx) : 0;
      const int incl = wave_incl_scan(len * Hk, lane) + pre;
      const uint64_t m = __ballot(b0 + lane < a.B && incl > gw0);
      if (m != 0ull) {
        const int fl = __ffsll((unsigned long long)m) - 1;
        b = b0 + fl;
        seg_b_start = __shfl(incl - len * Hk, fl, 64);
        break;
      }
      pre = __shfl(incl, 63, 64);
    }
  }
  int len = clamp_len(a.lengths, b, a.ctx);
  int hk = (gw0 - seg_b_start) / len;

  // 0/1 selection operands for the V transpose: Sel_h[8g+j][n] = (8g+j == n+16h)
  uint4 sel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = (8 * g + 2 * j == n + 16 * h) ? 0x3F80u : 0u;
      const uint32_t hi = (8 * g + 2 * j + 1 == n + 16 * h) ? 0x3F80u : 0u;
      e[j] = lo | (hi << 16);
    }
    sel[h] = make_uint4(e[0], e[1], e[2], e[3]);
  }
  float kbound = 0.f;
  if (FUSED) {
    // |k~| <= sqrt(D) * max|kw + w_offset| (+ bf16 rounding of the cached rows)
    const uint2 wv = *reinterpret_cast<const uint2*>(a.kw + 4 * lane);  // d = 4*lane .. +3
    float wm = fmaxf(fmaxf(fabsf(__uint_as_float(wv.x << 16) + a.w_offset),
                           fabsf(__uint_as_float(wv.x & 0xffff0000u) + a.w_offset)),
                     fmaxf(fabsf(__uint_as_float(wv.y << 16) + a.w_offset),
                           fabsf(__uint_as_float(wv.y & 0xffff0000u) + a.w_offset)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) wm = fmaxf(wm, __shfl_xor(wm, o, 64));
    kbound = 16.0f * wm * 1.01f;
  }

  int pos = gw0;
  while (true) {
    const int seg_start = seg_b_start + hk * len;
    const int lo = pos - seg_start;
    const int hi = min(gw1 - seg_start, len);

    // ---- Q operand for (b, hk): lane (n, g) holds q[head n][32kk + 8g + j] / 16
    uint4 qop[8];
    float qn2 = 0.f;
    {
      const int nn = n < G ? n : 0;
      const uint16_t* qp =
          a.q + (int64_t)b * a.q_sb + (int64_t)(hk * G + nn) * a.q_sh + 8 * g;
      float x[8][8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) unpack8(load16(qp + 32 * kk), x[kk]);
      if (FUSED) {
        // qnorm_rope_fwd (src/kernels/qknorm_rope_append.jl:25-57) on the fly
        float ss = 0.f;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
          for (int j = 0; j < 8; ++j) ss += x[kk][j] * x[kk][j];
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        const float r = 1.0f / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          float wf[8];
          unpack8(load16(a.qw + 32 * kk + 8 * g), wf);
#pragma unroll
          for (int j = 0; j < 8; ++j) x[kk][j] = x[kk][j] * r * (wf[j] + a.w_offset);
        }
        const int p = len - 1;  // fused decode: lengths are the positions
        const float* cs = a.cos_tab + (int64_t)p * HALF_ROT + 8 * g;
        const float* sn = a.sin_tab + (int64_t)p * HALF_ROT + 8 * g;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float c = cs[j], si = sn[j];
          const float x1 = x[0][j], x2 = x[1][j];
          x[0][j] = x1 * c - x2 * si;
          x[1][j] = x2 * c + x1 * si;
        }
      }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[kk][j] *= QK_SCALE;
          qn2 += x[kk][j] * x[kk][j];
        }
        qop[kk] = pack8(x[kk]);
        if (n >= G) qop[kk] = make_uint4(0, 0, 0, 0);
      }
      qn2 += __shfl_xor(qn2, 16, 64);
      qn2 += __shfl_xor(qn2, 32, 64);
    }
    float m_run = -INFINITY;
    bool use_static = false;
    if (FUSED) {
      const float bound = sqrtf(qn2) * 1.01f * kbound * LOG2E;
      use_static = __ballot(n < G && !(bound <= D_STATIC_LIMIT)) == 0ull;
      if (use_static) m_run = bound;
    }

    // ---- stream tokens [lo, hi) of (b, hk), double-buffered 16-token steps
    f32x4 acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float l_part = 0.f;
    const uint16_t* kb = a.kc + (int64_t)b * a.c_sb + (int64_t)hk * a.c_sh + 8 * g;
    const uint16_t* vb = a.vc + (int64_t)b * a.c_sb + (int64_t)hk * a.c_sh + 8 * g;
    const int64_t last = a.ctx - 1;
    // three register stages: two 16-token steps in flight while one computes;
    // one loop for both shifts (with the static bound m_run never moves)
    StepBuf s0, s1, s2;
    load_step(s0, kb, vb, min((int64_t)(lo + n), last), a.c_st);
    if (lo + DSTEP < hi) load_step(s1, kb, vb, min((int64_t)(lo + DSTEP + n), last), a.c_st);
    for (int t = lo; t < hi; t += 3 * DSTEP) {
      if (t + 2 * DSTEP < hi)
        load_step(s2, kb, vb, min((int64_t)(t + 2 * DSTEP + n), last), a.c_st);
      compute_step(s0, t, hi, n, g, qop, sel, acc, m_run, l_part);
      if (t + 3 * DSTEP < hi)
        load_step(s0, kb, vb, min((int64_t)(t + 3 * DSTEP + n), last), a.c_st);
      if (t + DSTEP < hi) compute_step(s1, t + DSTEP, hi, n, g, qop, sel, acc, m_run, l_part);
      if (t + 4 * DSTEP < hi)
        load_step(s1, kb, vb, min((int64_t)(t + 4 * DSTEP + n), last), a.c_st);
      if (t + 2 * DSTEP < hi)
        compute_step(s2, t + 2 * DSTEP, hi, n, g, qop, sel, acc, m_run, l_part);
    }

    // ---- partial for (w, segment): slot w + b*Hk + hk
    float l_tot = l_part + __shfl_xor(l_part, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    const int64_t slot = (int64_t)w + (int64_t)b * Hk + hk;
    if (n < G) {
      float* dst = a.part_o + (slot * G + n) * HEAD_DIM + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 16; ++dt)
        *reinterpret_cast<float4*>(dst + 16 * dt) =
            make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
      if (g == 0) {
        a.part_ml[2 * (slot * G + n)] = m_run;
        a.part_ml[2 * (slot * G + n) + 1] = l_tot;
      }
    }

    pos = seg_start + hi;
    if (pos >= gw1) break;
    if (++hk == Hk) {  // next sequence with a non-empty cache
      hk = 0;
      seg_b_start += Hk * len;
      do {
        ++b;
        len = clamp_len(a.lengths, b, a.ctx);
      } while (len == 0 && b + 1 < a.B);
    }
  }
}

// Log-sum-exp merge of a segment's partials (src/kernels/attention_decode.jl:91-132)
// and the sigmoid gate (src/llm/qwen35.jl:205). One workgroup per (16-wide d
// chunk, head of the group, hk, b); thread (sg, dd) merges slots w_first+sg,
// +16, ..., then an LDS merge over the 16 groups. With `advance`, the last
// workgroup to finish bumps positions[b] (src/llm/generate.jl:82-88).
__global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgs a) {
  const int chunk16 = blockIdx.x & 15, n = blockIdx.x >> 4, hk = blockIdx.y, b = blockIdx.z;
  const int sg = threadIdx.x >> 4, dd = threadIdx.x & 15;
  const int d = chunk16 * 16 + dd;
  int W = 0, pre_b = 0;
  for (int i = 0; i < a.B; ++i) {
    const int l = clamp_len(a.lengths, i, a.ctx);
    W += l;
    if (i < b) pre_b += l;
  }
  W *= a.Hk;
  const int len = clamp_len(a.lengths, b, a.ctx);
  const int seg_start = pre_b * a.Hk + hk * len;
  const int chunk = stream_chunk(W, a.NW, a.min_chunk);
  float M = -INFINITY, L = 0.f, O = 0.f;
  if (len > 0) {
    const int w_first = seg_start / chunk, w_last = (seg_start + len - 1) / chunk;
    const int64_t base = (int64_t)b * a.Hk + hk;
    for (int w = w_first + sg; w <= w_last; w += 16) {
      const int64_t r = (w + base) * a.G + n;
      const float m = a.part_ml[2 * r], l = a.part_ml[2 * r + 1];
      const float o = a.part_o[r * HEAD_DIM + d];
      const float mn = fmaxf(M, m);
      const float c1 = fast_exp2(M - mn), c2 = fast_exp2(m - mn);
      L = L * c1 + l * c2;
      O = O * c1 + o * c2;
      M = mn;
    }
  }
  __shared__ float sM[16][16], sL[16][16], sO[16][16];
  sM[sg][dd] = M;
  sL[sg][dd] = L;
  sO[sg][dd] = O;
  __syncthreads();
  if (sg == 0) {
    float Mf = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) Mf = fmaxf(Mf, sM[i][dd]);
    float Lf = 0.f, Of = 0.f;
    if (Mf > -INFINITY) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float c = fast_exp2(sM[i][dd] - Mf);
        Lf += sL[i][dd] * c;
        Of += sO[i][dd] * c;
      }
    }
    float out = Lf > 0.f ? Of / Lf : 0.f;  // no valid key: o = 0 (attention_decode.jl:126-128)
    const int h = hk * a.G + n;
    if (a.gate) out *= sigmoidf(bf2f(a.gate[(int64_t)b * a.g_sb + (int64_t)h * a.g_sh + d]));
    a.out[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d] = f2bf(out);
  }
  if (a.advance) {
    // every workgroup has read lengths (== positions) above; the last one to
    // arrive advances the clock
    __syncthreads();
    if (threadIdx.x == 0) {
      __threadfence();
      const int total = (int)(gridDim.x * gridDim.y * gridDim.z);
      const int prev = atomicAdd(a.counter, 1);
      if (prev == total - 1) {
        __threadfence();
        for (int i = 0; i < a.B; ++i) a.advance[i] += 1;
        a.counter[0] = 0;
      }
    }
  }
}

int decode_stream_waves(int B, int Hk, int n_splits) {
  int nw;
  if (n_splits > 0) {
    nw = n_splits * B * Hk;
  } else {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 256;
    nw = cus * 4;  // one wave per SIMD
  }
  return (nw + 3) / 4 * 4;
}

hipError_t launch_decode(const DecodeArgs& a, bool fused_q, hipStream_t st) {
  if (a.B == 0 || a.Hk == 0) return hipSuccess;
  dim3 grid(a.NW / 4);
  if (fused_q)
    hipLaunchKernelGGL(decode_stream_kernel<true>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(decode_stream_kernel<false>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs& a, hipStream_t st) {
  if (a.B == 0 || a.Hk == 0) return hipSuccess;
  dim3 grid(16 * a.G, a.Hk, a.B);
  hipLaunchKernelGGL(decode_combine_kernel, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace vm

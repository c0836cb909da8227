// decode.hip — split-KV flash-decoding for one new token per sequence
// (the work of src/kernels/attention_decode.jl:148-266, re-designed for CDNA4).
//
// Work unit: a workgroup of 4 waves owns `split` consecutive cache columns of one
// (sequence b, kv head hk); each wave streams split/4 of them in 32-token steps.
// The GQA group (G <= 16 query heads sharing hk) is the N = 16 side of a
// 16x16x32 bf16 MFMA, so every K/V byte is read from HBM once for the group.
//
//   S^T[tok][head] = K[tok][:] . Q[head][:]   A = K fragment straight from HBM
//                                              (16 B per lane), B = Q in registers
//   O^T[d][head]  += V^T[d][tok] . P^T[tok][head]
//
// The S^T accumulator already sits in the lanes/slots the P^T operand needs
// (token slot permutation {4g..4g+3, 16+4g..16+4g+3}), and V^T is produced
// from natural-layout V fragments by a 16x16x32 MFMA against a 0/1 selection
// matrix: bf16 * 1.0 summed with exact zeros is exact in fp32, so the transpose
// is lossless and needs no LDS. Partials (unnormalised O, running max m, sum l)
// are merged across the 4 waves in LDS, then across splits by the combine
// kernel, which also applies the sigmoid gate (src/llm/qwen35.jl:205).
#include "common.h"
#include "kernels.h"

namespace vm {

constexpr int SACC_STRIDE = HEAD_DIM + 16;  // LDS row pad: conflict-free for G <= 4

template <bool FUSED>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  extern __shared__ float smem[];
  const int s = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  // lengths beyond the capacity are out of contract; clamp so every access stays in bounds
  const int len = (int)min((int64_t)a.lengths[b], a.ctx);
  const int64_t wg_begin = (int64_t)s * a.split;
  if (wg_begin >= len) return;  // the combine kernel only reads active splits

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int G = a.G;
  const int per_wave = a.split >> 2;
  const int64_t w_begin = wg_begin + (int64_t)wave * per_wave;
  const int64_t w_end = min(w_begin + (int64_t)per_wave, (int64_t)len);

  // ---- Q operand: lane (n, g) holds q[head n][32kk + 8g + j], pre-scaled by 1/16.
  uint4 qop[8];
  {
    const int nn = n < G ? n : 0;
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(hk * G + nn) * a.q_sh + 8 * g;
    float x[8][8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) unpack8(load16(qp + 32 * kk), x[kk]);
    if (FUSED) {
      // qnorm_rope_fwd (src/kernels/qknorm_rope_append.jl:25-57) on the fly.
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
      const int pos = len - 1;  // fused decode: lengths are the positions
      const float* cs = a.cos_tab + (int64_t)pos * HALF_ROT + 8 * g;
      const float* sn = a.sin_tab + (int64_t)pos * HALF_ROT + 8 * g;
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
      for (int j = 0; j < 8; ++j) x[kk][j] *= QK_SCALE;
      qop[kk] = pack8(x[kk]);
      if (n >= G) qop[kk] = make_uint4(0, 0, 0, 0);
    }
  }

  // 0/1 selection operands for the V transpose: Sel_h[8g+j][n] = (8g+j == n+16h).
  uint4 sel[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t lo = (8 * g + 2 * j == n + 16 * h) ? 0x3F80u : 0u;
      uint32_t hi = (8 * g + 2 * j + 1 == n + 16 * h) ? 0x3F80u : 0u;
      e[j] = lo | (hi << 16);
    }
    sel[h] = make_uint4(e[0], e[1], e[2], e[3]);
  }

  f32x4 acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  const uint16_t* kb = a.kc + (int64_t)b * a.c_sb + (int64_t)hk * a.c_sh + 8 * g;
  const uint16_t* vb = a.vc + (int64_t)b * a.c_sb + (int64_t)hk * a.c_sh + 8 * g;
  const int64_t last_row = a.ctx - 1;

  for (int64_t t0 = w_begin; t0 < w_end; t0 += 32) {
    uint4 kf[2][8], vf[2][8];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int64_t row = min(t0 + 16 * tt + n, last_row);
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) kf[tt][kk] = load16(kb + row * a.c_st + 32 * kk);
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) vf[tt][kk] = load16(vb + row * a.c_st + 32 * kk);
    }
    if (t0 + 32 > w_end) {  // boundary step: rows past the range may hold anything
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        if (t0 + 16 * tt + n >= w_end)
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) vf[tt][kk] = make_uint4(0, 0, 0, 0);
    }

    float sv[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) c = mfma16(kf[tt][kk], qop[kk], c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t tok = t0 + 16 * tt + 4 * g + j;
        sv[tt][j] = tok < w_end ? c[j] * LOG2E : -INFINITY;
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(sv[0][0], sv[0][1]), fmaxf(sv[0][2], sv[0][3])),
                     fmaxf(fmaxf(sv[1][0], sv[1][1]), fmaxf(sv[1][2], sv[1][3])));
    mx = wave_max_xor(mx, 16);
    mx = wave_max_xor(mx, 32);
    const float m_new = fmaxf(m_run, mx);  // finite: token t0 is always valid
    const float alpha = fast_exp2(m_run - m_new);
    float p[2][4], psum = 0.f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[tt][j] = fast_exp2(sv[tt][j] - m_new);
        psum += p[tt][j];
      }
    l_part = l_part * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= alpha;

    uint4 pop;
    pop.x = pack2(p[0][0], p[0][1]);
    pop.y = pack2(p[0][2], p[0][3]);
    pop.z = pack2(p[1][0], p[1][1]);
    pop.w = pack2(p[1][2], p[1][3]);

#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4 t0v = mfma16(vf[0][kk], sel[h], zero);
        const f32x4 t1v = mfma16(vf[1][kk], sel[h], zero);
        uint4 vt;  // exact bf16 values: truncation is lossless
        vt.x = (__float_as_uint(t0v[0]) >> 16) | (__float_as_uint(t0v[1]) & 0xffff0000u);
        vt.y = (__float_as_uint(t0v[2]) >> 16) | (__float_as_uint(t0v[3]) & 0xffff0000u);
        vt.z = (__float_as_uint(t1v[0]) >> 16) | (__float_as_uint(t1v[1]) & 0xffff0000u);
        vt.w = (__float_as_uint(t1v[2]) >> 16) | (__float_as_uint(t1v[3]) & 0xffff0000u);
        acc[2 * kk + h] = mfma16(vt, pop, acc[2 * kk + h]);
      }
    }
  }

  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);

  // ---- merge the 4 waves of this split in LDS
  float* s_acc = smem;                                   // [4][G][SACC_STRIDE]
  float* s_m = smem + 4 * G * SACC_STRIDE;               // [4][16]
  float* s_l = s_m + 64;                                 // [4][16]
  if (n < G) {
    float* dst = s_acc + (wave * G + n) * SACC_STRIDE + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) dst[16 * dt + j] = acc[dt][j];
    if (g == 0) {
      s_m[wave * 16 + n] = m_run;
      s_l[wave * 16 + n] = l_tot;
    }
  }
  __syncthreads();
  const int d = threadIdx.x;
  const int64_t row0 = ((int64_t)(b * a.Hk + hk) * a.NS + s) * G;
  for (int hn = 0; hn < G; ++hn) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w * 16 + hn]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float c = fast_exp2(s_m[w * 16 + hn] - M);  // empty wave: exp2(-inf) = 0
      L += s_l[w * 16 + hn] * c;
      O += s_acc[(w * G + hn) * SACC_STRIDE + d] * c;
    }
    a.part_o[(row0 + hn) * HEAD_DIM + d] = O;
    if (d == 0) {
      a.part_ml[2 * (row0 + hn)] = M;
      a.part_ml[2 * (row0 + hn) + 1] = L;
    }
  }
}

// Log-sum-exp merge across splits (src/kernels/attention_decode.jl:225-266),
// one workgroup per (16-wide d chunk, head of the group, hk, b). Thread
// (sg, dd): splits s = sg, sg+16, ...; then an LDS merge over the 16 groups.
__global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgs a) {
  const int chunk = blockIdx.x & 15, n = blockIdx.x >> 4, hk = blockIdx.y, b = blockIdx.z;
  const int sg = threadIdx.x >> 4, dd = threadIdx.x & 15;
  const int d = chunk * 16 + dd;
  const int len = a.lengths[b];
  const int n_active = min((len + a.split - 1) / a.split, a.NS);
  const int64_t base = ((int64_t)(b * a.Hk + hk) * a.NS) * a.G + n;
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int s = sg; s < n_active; s += 16) {
    const int64_t r = base + (int64_t)s * a.G;
    const float m = a.part_ml[2 * r], l = a.part_ml[2 * r + 1];
    const float o = a.part_o[r * HEAD_DIM + d];
    const float mn = fmaxf(M, m);
    const float c1 = fast_exp2(M - mn), c2 = fast_exp2(m - mn);
    L = L * c1 + l * c2;
    O = O * c1 + o * c2;
    M = mn;
  }
  __shared__ float sM[16][16], sL[16][16], sO[16][16];
  sM[sg][dd] = M;
  sL[sg][dd] = L;
  sO[sg][dd] = O;
  __syncthreads();
  if (sg != 0) return;
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
  float out = Lf > 0.f ? Of / Lf : 0.f;  // no valid key: o = 0 (attention_decode.jl:261)
  const int h = hk * a.G + n;
  if (a.gate) out *= sigmoidf(bf2f(a.gate[(int64_t)b * a.g_sb + (int64_t)h * a.g_sh + d]));
  a.out[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + d] = f2bf(out);
}

int decode_split_tokens(int B, int Hk, int64_t ctx, int n_splits) {
  int64_t split;
  if (n_splits > 0) {
    split = (ctx + n_splits - 1) / n_splits;
  } else {
    // Aim for ~1024 workgroups (4 per CU) when every sequence is at capacity.
    split = (ctx * B * Hk + 1023) / 1024;
    if (split > 8192) split = 8192;
  }
  split = (split + DECODE_WG_TOKENS - 1) / DECODE_WG_TOKENS * DECODE_WG_TOKENS;
  if (split < DECODE_WG_TOKENS) split = DECODE_WG_TOKENS;
  return (int)split;
}

hipError_t launch_decode(const DecodeArgs& a, bool fused_q, hipStream_t st) {
  if (a.B == 0 || a.Hk == 0 || a.NS == 0) return hipSuccess;
  dim3 grid(a.NS, a.Hk, a.B);
  size_t lds = (size_t)(4 * a.G * SACC_STRIDE + 128) * sizeof(float);
  if (fused_q)
    hipLaunchKernelGGL(decode_split_kernel<true>, grid, dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL(decode_split_kernel<false>, grid, dim3(256), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs& a, hipStream_t st) {
  if (a.B == 0 || a.Hk == 0) return hipSuccess;
  dim3 grid(16 * a.G, a.Hk, a.B);
  hipLaunchKernelGGL(decode_combine_kernel, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace vm

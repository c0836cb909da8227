// deltanet.hip — the linear-attention layer parts of Qwen3.5 on gfx950: the
// depthwise causal conv1d (one decode step with its ring state, and the whole
// sequence) and the gated delta-rule recurrence (the fused decode step, the
// plain step and the whole sequence), plus the prefill's prep (l2 norms, gates)
// and its gated-RMSNorm epilogue.
//
// Reference: src/kernels/causal_conv1d.jl, src/kernels/deltanet_recurrent.jl,
// src/kernels/deltanet_fused.jl and their call sites in src/llm/qwen35.jl
// (decode!: :210-232, forward: :320-365).
//
// The recurrence: per (value head, sequence) a state S (Dk x Dv, fp32) with
//   S = decay S;  delta = beta (v - S^T k);  S += k delta^T;  o = S^T q.
// Every column of S evolves on its own given k, q, and its v entry, so the
// kernels split the columns over waves with no cross-wave traffic: wave w
// owns 2 NI columns; lane (j = lane % 32, h = lane / 32) holds rows 4j .. 4j+3
// of columns 2 NI w + 2 i + h, i < NI (one 16-byte load per i: two adjacent
// 512-byte columns per load instruction, 1 KB contiguous). The column sums
// S^T k and S^T q are butterfly reduce-scatters over the 32 lanes of a half:
// NI partial sums per lane become one full sum per lane group. The state is
// read once and written once per step (the reference makes two passes).
#include "common.h"
#include "kernels.h"

namespace vm {

namespace {

constexpr int DN_D = 128;  // Dk = Dv (Qwen3.5: deltanet.jl:12, qwen35.jl:19)

// v[l ^ M] within each 32-lane half: DPP quad permutes for M = 1, 2, the
// swizzle unit's bitmask mode (and 0x1f, xor M) for M = 4, 8, 16.
template <int M>
__device__ __forceinline__ float xor32(float v) {
  const int x = __float_as_int(v);
  if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
  if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
  return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x1F | (M << 10)));
}

__device__ __forceinline__ float half_sum(float v) {
  v += xor32<16>(v);
  v += xor32<8>(v);
  v += xor32<4>(v);
  v += xor32<2>(v);
  return v + xor32<1>(v);
}

// One scatter level over mask bit M: N values (index m + (N/2) * bit for the
// kept half) -> N / 2, each summed with the partner lane's matching value.
template <int M, int N>
__device__ __forceinline__ void scatter_level(float (&p)[16], bool bit) {
#pragma unroll
  for (int m = 0; m < N / 2; ++m) {
    const float keep = bit ? p[m + N / 2] : p[m];
    const float send = bit ? p[m] : p[m + N / 2];
    p[m] = keep + xor32<M>(send);
  }
}
template <int M>
__device__ __forceinline__ float sum_masks(float v) {  // plain sums over masks M, M/2, .., 1
  if constexpr (M >= 1) return sum_masks<M / 2>(v + xor32<M>(v));
  else return v;
}
template <int N, int M>
__device__ __forceinline__ float rs_level(float (&p)[16], int j) {
  if constexpr (N == 1) {
    return sum_masks<M>(p[0]);
  } else {
    scatter_level<M, N>(p, (j & M) != 0);
    return rs_level<N / 2, M / 2>(p, j);
  }
}
// p[0 .. NI-1]: this lane's partial sums of its NI columns. Scatter levels on
// masks 16, 8, .. (log2 NI of them) halve the values held, plain sums on the
// rest of the mask bits finish: every lane then holds the sum over the 32 lanes
// of its half for column index i = j >> (5 - log2 NI).
template <int NI>
__device__ __forceinline__ float reduce_scatter(float (&p)[16], int j) {
  static_assert(NI == 16 || NI == 8 || NI == 4 || NI == 2, "NI");
  return rs_level<NI, 16>(p, j);
}

// The sum of column index i sits in lanes (i << SH) .. of each half: lane
// (j, h) fetches index i of its own half.
template <int NI>
__device__ __forceinline__ float column_value(float v, int i, int h) {
  constexpr int SH = NI == 16 ? 1 : NI == 8 ? 2 : NI == 4 ? 3 : 4;
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i << SH));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32 + (i << SH)));
  return h ? hi : lo;
}

// One delta step of this lane's slice s[i][0..3] (rows 4j.., column index i):
// returns o = S'^T q for column index j >> SH (the lane group's column).
template <int NI>
__device__ __forceinline__ float delta_step(float (&s)[16][4], const float (&kn)[4],
                                            const float (&qn)[4], float v_col, float beta,
                                            float decay, int j, int h) {
  float p[16];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) s[i][e] *= decay;
    p[i] = s[i][0] * kn[0] + s[i][1] * kn[1] + s[i][2] * kn[2] + s[i][3] * kn[3];
  }
  const float acc = reduce_scatter<NI>(p, j);
  const float delta = beta * (v_col - acc);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float d = column_value<NI>(delta, i, h);
#pragma unroll
    for (int e = 0; e < 4; ++e) s[i][e] += kn[e] * d;
    p[i] = s[i][0] * qn[0] + s[i][1] * qn[1] + s[i][2] * qn[2] + s[i][3] * qn[3];
  }
  return reduce_scatter<NI>(p, j);
}

template <int NI>
__device__ __forceinline__ void load_state(float (&s)[16][4], const float* base, int w, int lane) {
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const f32x4 t = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4*>(base + (int64_t)(2 * NI * w + 2 * i) * DN_D + 4 * lane));
    s[i][0] = t[0];
    s[i][1] = t[1];
    s[i][2] = t[2];
    s[i][3] = t[3];
  }
}
template <int NI>
__device__ __forceinline__ void store_state(const float (&s)[16][4], float* base, int w, int lane) {
#pragma unroll
  for (int i = 0; i < NI; ++i)
    __builtin_nontemporal_store(f32x4{s[i][0], s[i][1], s[i][2], s[i][3]},
                                reinterpret_cast<f32x4*>(base + (int64_t)(2 * NI * w + 2 * i) * DN_D + 4 * lane));
}

__device__ __forceinline__ void load4_bf16(const uint16_t* p, float (&x)[4]) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  x[0] = __uint_as_float(u.x << 16);
  x[1] = __uint_as_float(u.x & 0xffff0000u);
  x[2] = __uint_as_float(u.y << 16);
  x[3] = __uint_as_float(u.y & 0xffff0000u);
}

}  // namespace

// ---- fused_deltanet_decode! (deltanet_fused.jl:27-141): one block of four
// waves per (value head, sequence), 32 columns per wave (NI = 16).
__global__ __launch_bounds__(256) void deltanet_fused_decode_kernel(DeltaFusedArgs a) {
  constexpr int NI = 16;
  const int hv = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, j = lane & 31, h = lane >> 5;
  const int hk = hv / (a.Hv / a.Hk);
  const int64_t sb = ((int64_t)b * a.Hv + hv) * DN_D * DN_D;
  float s[16][4];
  load_state<NI>(s, a.s_in + sb, w, lane);
  float q[4], k[4];
  load4_bf16(a.q + b * a.q_sb + hk * DN_D + 4 * j, q);
  load4_bf16(a.k + b * a.k_sb + hk * DN_D + 4 * j, k);
  const int col = 2 * NI * w + 2 * (j >> 1) + h;  // this lane group's column
  const float v_col = bf2f(a.v[b * a.v_sb + hv * DN_D + col]);
  const float z_col = bf2f(a.z[b * a.z_sb + hv * DN_D + col]);
  const float w_col = bf2f(a.norm_w[col]);
  // per-value-head gates (deltanet_fused.jl:52-59)
  const float spi = bf2f(a.alpha[b * a.a_sb + hv]) + a.dt_bias[hv];
  const float sp = spi > 20.0f ? spi : logf(1.0f + expf(spi));
  const float decay = expf(-expf(a.a_log[hv]) * sp);
  const float beta = accurate_sigmoid(bf2f(a.beta[b * a.b_sb + hv]));
  // l2 norms over the shared qk head (deltanet_fused.jl:61-71)
  const float qss = half_sum(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  const float kss = half_sum(k[0] * k[0] + k[1] * k[1] + k[2] * k[2] + k[3] * k[3]);
  const float qsc = 1.0f / sqrtf(qss + 1e-6f) / sqrtf((float)DN_D);
  const float ksc = 1.0f / sqrtf(kss + 1e-6f);
  float qn[4], kn[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    qn[e] = q[e] * qsc;
    kn[e] = k[e] * ksc;
  }
  const float out = delta_step<NI>(s, kn, qn, v_col, beta, decay, j, h);
  store_state<NI>(s, a.s_out + sb, w, lane);
  // gated RMSNorm over the Dv columns (deltanet_fused.jl:98-105): lanes with j
  // even hold each column once
  __shared__ float red[4];
  const float ss = half_sum((j & 1) ? 0.f : out * out);
  const float wave_ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0)) +
                        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 32));
  if (lane == 0) red[w] = wave_ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rstd = 1.0f / sqrtf(tot / (float)DN_D + a.eps);
  if ((j & 1) == 0)
    a.o[b * a.o_sb + hv * DN_D + col] = f2bf(out * rstd * w_col * accurate_silu(z_col));
}

// ---- the DeltaNet layer's decode step after its projection in one kernel
// (qwen35.jl:212-232): one workgroup of 4 R waves per (qk head hk, sequence),
// R = Hv / Hk value heads. First every thread takes 4-channel groups of the
// projection [q | k | v | z | alpha | beta] of this head: the stream-K
// partials summed in workgroup order and rounded to bf16 (the value linear!
// stores), then for q, k and v the conv step as conv1d_update_sk_kernel
// (ring shift, silu, bf16), into LDS, the channels' ring columns written
// (each channel has one owner: the qk head's q and k, its R heads' v). The
// state loads are issued first and land meanwhile. Then wave group j runs
// fused_deltanet_decode! for value head hk R + j as deltanet_fused_decode_kernel,
// its inputs from LDS: bit for bit the results of linear_causal_conv1d
// followed by fused_deltanet_decode, one launch and the bf16 projection and
// conv output round trips fewer.
namespace {
__device__ __forceinline__ void unpack4(const uint2& u, float (&x)[4]) {
  x[0] = __uint_as_float(u.x << 16);
  x[1] = __uint_as_float(u.x & 0xffff0000u);
  x[2] = __uint_as_float(u.y << 16);
  x[3] = __uint_as_float(u.y & 0xffff0000u);
}
}  // namespace

template <int KC, int R>
__global__ __launch_bounds__(256 * R) void deltanet_decode_sk_kernel(DeltaDecodeSkArgs a) {
  constexpr int NI = 16;
  const DeltaFusedArgs& f = a.f;
  const Conv1dArgs& c = a.c;
  const int hk = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int j = tid >> 8, t = tid & 255;  // value head hk R + j; thread t of its group
  const int lane = t & 63, w = t >> 6, jl = lane & 31, h = lane >> 5;
  const int hv = hk * R + j;
  const int64_t sb = ((int64_t)b * f.Hv + hv) * DN_D * DN_D;
  float s[16][4];
  load_state<NI>(s, f.s_in + sb, w, lane);
  // LDS: q, k, v[R], z[R] (DN_D each), alpha[R], beta[R]
  __shared__ float xs[(2 + 2 * R) * DN_D + 2 * R];
  __shared__ float red[R][4];
  constexpr int XA = (2 + 2 * R) * DN_D;
  for (int g = tid; g < 64 + 64 * R; g += 256 * R) {
    int ch, xo;  // projection channel and LDS slot of the group's first element
    if (g < 64) {  // q (g < 32) or k of head hk
      ch = (g < 32 ? 0 : f.Hk * DN_D) + hk * DN_D + 4 * (g & 31);
      xo = (g >> 5) * DN_D + 4 * (g & 31);
    } else if (g < 64 + 32 * R) {  // v of head hk R + jj
      const int jj = (g - 64) >> 5;
      ch = 2 * f.Hk * DN_D + (hk * R + jj) * DN_D + 4 * (g & 31);
      xo = (2 + jj) * DN_D + 4 * (g & 31);
    } else {  // z of head hk R + jj
      const int jj = (g - 64 - 32 * R) >> 5;
      ch = c.D + (hk * R + jj) * DN_D + 4 * (g & 31);
      xo = (2 + R + jj) * DN_D + 4 * (g & 31);
    }
    const float4 sum = gemv_sk_sum4(a.part, a.G, a.chunk, ch, b);
    const uint2 xr = make_uint2(pack2(sum.x, sum.y), pack2(sum.z, sum.w));  // bf16 projection
    float x4[4];
    if (g < 64 + 32 * R) {
      uint2 raw[KC];
#pragma unroll
      for (int i = 0; i < KC - 1; ++i)
        raw[i] = *reinterpret_cast<const uint2*>(c.s_in + b * c.s_sb + (int64_t)(i + 1) * c.s_cs + ch);
      raw[KC - 1] = xr;
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KC; ++i) {
        float v[4], wf[4];
        unpack4(raw[i], v);
        unpack4(*reinterpret_cast<const uint2*>(c.w + (int64_t)i * c.w_cs + ch), wf);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += v[e] * wf[e];
      }
#pragma unroll
      for (int i = 0; i < KC; ++i)
        *reinterpret_cast<uint2*>(c.s_out + b * c.s_sb + (int64_t)i * c.s_cs + ch) = raw[i];
      if (c.bias) {
        float bf4[4];
        unpack4(*reinterpret_cast<const uint2*>(c.bias + ch), bf4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += bf4[e];
      }
      if (c.act) {
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = accurate_silu(acc[e]);
      }
      unpack4(make_uint2(pack2(acc[0], acc[1]), pack2(acc[2], acc[3])), x4);  // bf16 conv output
    } else {
      unpack4(xr, x4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) xs[xo + e] = x4[e];
  }
  if (tid < 2 * R) {  // alpha (tid < R) and beta of head hk R + tid % R
    const int ch = c.D + f.Hv * DN_D + (tid < R ? 0 : f.Hv) + hk * R + tid % R;
    xs[XA + tid] = __uint_as_float(pack2(gemv_sk_sum1(a.part, a.G, a.chunk, ch, b), 0.f) << 16);
  }
  __syncthreads();
  float q[4], k[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    q[e] = xs[4 * jl + e];
    k[e] = xs[DN_D + 4 * jl + e];
  }
  const int col = 2 * NI * w + 2 * (jl >> 1) + h;  // this lane group's column
  const float v_col = xs[(2 + j) * DN_D + col];
  const float z_col = xs[(2 + R + j) * DN_D + col];
  const float w_col = bf2f(f.norm_w[col]);
  const float spi = xs[XA + j] + f.dt_bias[hv];
  const float sp = spi > 20.0f ? spi : logf(1.0f + expf(spi));
  const float decay = expf(-expf(f.a_log[hv]) * sp);
  const float beta = accurate_sigmoid(xs[XA + R + j]);
  const float qss = half_sum(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  const float kss = half_sum(k[0] * k[0] + k[1] * k[1] + k[2] * k[2] + k[3] * k[3]);
  const float qsc = 1.0f / sqrtf(qss + 1e-6f) / sqrtf((float)DN_D);
  const float ksc = 1.0f / sqrtf(kss + 1e-6f);
  float qn[4], kn[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    qn[e] = q[e] * qsc;
    kn[e] = k[e] * ksc;
  }
  const float out = delta_step<NI>(s, kn, qn, v_col, beta, decay, jl, h);
  store_state<NI>(s, f.s_out + sb, w, lane);
  const float ss = half_sum((jl & 1) ? 0.f : out * out);
  const float wave_ss = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0)) +
                        __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 32));
  if (lane == 0) red[j][w] = wave_ss;
  __syncthreads();
  const float tot = red[j][0] + red[j][1] + red[j][2] + red[j][3];
  const float rstd = 1.0f / sqrtf(tot / (float)DN_D + f.eps);
  if ((jl & 1) == 0)
    f.o[b * f.o_sb + hv * DN_D + col] = f2bf(out * rstd * w_col * accurate_silu(z_col));
}

// ---- deltanet_sequence! (deltanet_recurrent.jl:109-198) and, at T = 1,
// deltanet_recurrent_decode! (:15-95): fp32 inputs already normed and gated.
// Grid (columns / (2 NI * 4), Hv, B), four independent waves per block; the
// state stays in registers across the T steps, the next step's inputs load
// while the current one computes.
template <int NI>
__global__ __launch_bounds__(256) void deltanet_sequence_kernel(DeltaSeqArgs a) {
  const int hv = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);  // wave index within the head
  const int hk = hv / (a.Hv / a.Hk);
  const int64_t sb = ((int64_t)b * a.Hv + hv) * DN_D * DN_D;
  constexpr int SH = NI == 16 ? 1 : NI == 8 ? 2 : NI == 4 ? 3 : 4;
  const int col = 2 * NI * w + 2 * (j >> SH) + h;
  float s[16][4];
  load_state<NI>(s, a.s_in + sb, w, lane);
  const float* qp = a.q + ((int64_t)b * a.Hk + hk) * a.T * DN_D + 4 * j;
  const float* kp = a.k + ((int64_t)b * a.Hk + hk) * a.T * DN_D + 4 * j;
  const float* vp = a.v + ((int64_t)b * a.Hv + hv) * a.T * DN_D + col;
  const float* bp = a.beta + (int64_t)b * a.T * a.Hv + hv;
  const float* gp = a.gate + (int64_t)b * a.T * a.Hv + hv;
  float* op = a.o + ((int64_t)b * a.Hv + hv) * a.T * DN_D + col;
  float4 qv = *reinterpret_cast<const float4*>(qp);
  float4 kv = *reinterpret_cast<const float4*>(kp);
  float v_col = *vp, beta = *bp, gate = *gp;
  for (int t = 0; t < a.T; ++t) {
    const float qn[4] = {qv.x, qv.y, qv.z, qv.w};
    const float kn[4] = {kv.x, kv.y, kv.z, kv.w};
    const float vc = v_col, bt = beta, decay = expf(gate);
    if (t + 1 < a.T) {  // the next step's inputs
      const int64_t o4 = (int64_t)(t + 1) * DN_D;
      qv = *reinterpret_cast<const float4*>(qp + o4);
      kv = *reinterpret_cast<const float4*>(kp + o4);
      v_col = vp[o4];
      beta = bp[(int64_t)(t + 1) * a.Hv];
      gate = gp[(int64_t)(t + 1) * a.Hv];
    }
    const float out = delta_step<NI>(s, kn, qn, vc, bt, decay, j, h);
    if ((j & ((1 << SH) - 1)) == 0) op[(int64_t)t * DN_D] = out;
  }
  store_state<NI>(s, a.s_out + sb, w, lane);
}

// ---- the chunked form of deltanet_sequence! ---------------------------------
// Over a chunk of C tokens (G the in-chunk cumulative log decay, gamma = exp G,
// D_ij = gamma_i / gamma_j) the recurrence's per-token corrections delta_i =
// beta_i (v_i - alpha_i S_{i-1}^T k_i) satisfy the lower-triangular system
//     (I + L) delta = beta V - (beta gamma K) S_0,   L_ij = beta_i D_ij k_i.k_j (i > j)
// so delta = U - W S_0 with U = (I + L)^-1 beta V, W = (I + L)^-1 beta gamma K;
// then O = gamma Q S_0 + M delta with M_ij = D_ij q_i.k_j (j <= i), and
// S_C = gamma_C S_0 + K~^T delta with K~_j = (gamma_C / gamma_j) k_j (exact
// algebra of the sequential update; fp32 throughout). Three launches:
// Phase 1 (deltanet_chunk_kernel, chunk-parallel): the Gram K K^T and the
// products [U | W] = T [beta V | beta gamma K] with T = (I + L)^-1 on the bf16
// MFMA in split precision (see phase 3), T itself by fp32 forward
// substitution, and the operands of the state chain (-W, K~^T split, U,
// gamma_C) written in the operand orders phase 2 loads them in, 16 bytes per
// lane, so phase 2 reads 1 KB contiguous per wave load.
// Phase 2 (deltanet_scan_kernel, sequential over chunks): one workgroup per 16
// state columns of a value head; per chunk 24 split-precision MFMAs per wave
// (delta, then the state, fp32 accumulators), writing each chunk's start state
// S_0 and its delta for phase 3, the next chunk's operands loading into a
// second register set meanwhile. The state and delta pass between the waves
// through LDS split and transposed ([column][k]), so that a B operand is one
// 16-byte read.
// Phase 3 (deltanet_out_kernel, chunk-parallel): Q K^T, M and O = gamma Q S_0 +
// M delta on the bf16 MFMA (v_mfma_f32_16x16x32_bf16) in split precision:
// each fp32 operand x is hi = bf16(x) and lo = bf16(x - hi), and a product is
// hi hi + hi lo + lo hi with fp32 accumulation (about 2^-16 relative per
// product), then either O (fp32, the operator's output) or, fused, the layer's
// gated RMSNorm with z (qwen35.jl:360-364) in bf16. The scan writes S_0 and
// delta already split, in that MFMA's B operand order.
namespace {
constexpr int DC = 64;   // chunk length
constexpr int CBW = 16;  // state columns per scan workgroup
// per (chunk, value head, sequence) unit of the scan's operands, floats
// (-W and K~^T split into bf16 hi / lo in the A operand order of
// v_mfma_f32_16x16x32_bf16, 8 bf16 per lane: lane l element j = A[16 tile + l %
// 16][32 ks + 8 (l / 16) + j]; U fp32 in accumulator order)
constexpr int UO_W = 0;      // -W:   [w 4][ks 4][hl 2][lane][8] bf16, A[i = r][k = dk]
constexpr int UO_K = 8192;   // K~^T: [d 8][ks 2][hl 2][lane][8] bf16, A[i = dk][k = r]
constexpr int UO_U = 16384;  // U:    [cb 8][w 4][lane][4] floats, D[r][dv] tiles
constexpr int UO_G = 24576;  // gamma_C
constexpr int UNIT = 24640;  // floats per unit (98 560 B, a multiple of 256)
// per (chunk, value head, sequence), written by the scan for phase 3, in
// float-sized units: S_0 and delta split into bf16 hi and lo parts, in the B
// operand order of v_mfma_f32_16x16x32_bf16 for column block cb and 32-deep k
// step ks: [cb 8][ks][hl 2][lane 64][8] bf16 with lane l element j =
// X[32 ks + 8 (l / 16) + j][16 cb + l % 16] (hl 0: hi, 1: lo); ks < 4 for S_0
// (k = dk), ks < 2 for delta (k = the chunk's token)
constexpr int S0_UNIT = DN_D * DN_D;
constexpr int DL_UNIT = DC * DN_D;

// the chunk's inclusive cumulative log decay (wave 0, one token per lane; log
// decays below -110 are taken as -110: expf underflows to exactly 0 below
// about -104, so every decay the recurrence applies is unchanged, while the
// cumulative sums stay finite; a -inf log decay, e.g. from softplus
// overflowing in log1p(exp(x)) at x > 88.7, would make their differences NaN)
__device__ __forceinline__ float chunk_cumsum(const DeltaSeqArgs& q, int b, int hv, int t0, int n,
                                              int t) {
  const int64_t g = ((int64_t)b * q.T + t0 + min(t, n - 1)) * q.Hv + hv;  // in bounds
  const float gt = t < n ? fmaxf(q.gate[g], -110.0f) : 0.f;
  float G = gt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_up(G, off);
    if (t >= off) G += o;
  }
  return G;
}
}  // namespace

// the (chunk, value head, sequence) workspaces of the three phases
__host__ __device__ __forceinline__ int64_t dn_units_floats(int NC) { return (int64_t)(NC + 1) * UNIT; }
__host__ __device__ __forceinline__ int64_t dn_s0_floats(int NC) { return (int64_t)(NC + 1) * S0_UNIT; }
__host__ __device__ __forceinline__ int64_t dn_dl_floats(int NC) { return (int64_t)(NC + 1) * DL_UNIT; }
__device__ __forceinline__ float* dn_units(const DeltaChunkArgs& a, int b, int hv, int NC) {
  return a.ws + ((int64_t)b * a.s.Hv + hv) * dn_units_floats(NC);
}
__device__ __forceinline__ float* dn_s0(const DeltaChunkArgs& a, int b, int hv, int NC) {
  return a.ws + (int64_t)a.s.B * a.s.Hv * dn_units_floats(NC) +
         ((int64_t)b * a.s.Hv + hv) * dn_s0_floats(NC);
}
__device__ __forceinline__ float* dn_dl(const DeltaChunkArgs& a, int b, int hv, int NC) {
  return a.ws + (int64_t)a.s.B * a.s.Hv * (dn_units_floats(NC) + dn_s0_floats(NC)) +
         ((int64_t)b * a.s.Hv + hv) * dn_dl_floats(NC);
}

namespace {
// 4 fp32 values as bf16 hi and lo parts (x = hi + lo to about 2^-16), 4 each
__device__ __forceinline__ void split4(const f32x4& x, uint2& hi, uint2& lo) {
  hi = make_uint2(pack2(x[0], x[1]), pack2(x[2], x[3]));
  lo = make_uint2(pack2(x[0] - __uint_as_float(hi.x << 16), x[1] - __uint_as_float(hi.x & 0xffff0000u)),
                  pack2(x[2] - __uint_as_float(hi.y << 16), x[3] - __uint_as_float(hi.y & 0xffff0000u)));
}
__device__ __forceinline__ void split8(const f32x4& a, const f32x4& b, uint4& hi, uint4& lo) {
  uint2 h0, l0, h1, l1;
  split4(a, h0, l0);
  split4(b, h1, l1);
  hi = make_uint4(h0.x, h0.y, h1.x, h1.y);
  lo = make_uint4(l0.x, l0.y, l1.x, l1.y);
}
// acc += A B in split precision (hi hi + hi lo + lo hi) on v_mfma_f32_16x16x32_bf16
// (A lane l = A[l % 16][8 (l / 16) + j], B lane l = B[8 (l / 16) + j][l % 16], D
// lane l reg r = D[4 (l / 16) + r][l % 16])
__device__ __forceinline__ f32x4 mfma_x3(const uint4& ah, const uint4& al, const uint4& bh,
                                         const uint4& bl, f32x4 acc) {
  acc = mfma16(al, bh, acc);
  acc = mfma16(ah, bl, acc);
  return mfma16(ah, bh, acc);
}
constexpr int KSW = DN_D + 4;  // LDS row of K (floats; 16-byte aligned, banks skewed)
constexpr int LSW = DC + 4;    // LDS row of L (floats)
constexpr int TW = DC + 8;     // LDS row of T hi / lo (bf16)
}  // namespace

// One workgroup per (chunk, value head, sequence). Wave w forms Gram row block
// w into L (L[i][j] = beta_i gamma_i / gamma_j k_i . k_j below the diagonal),
// then wave 3 solves (I + L) T = I, lane c for column c, in fp32 (row i + 1 of
// L read from LDS while row i is reduced), and stores T split into bf16 hi /
// lo over L, while waves 0-2 write K~^T and gather their operands of the
// products below. Then waves 0, 1 form U = T (beta V) (value columns 64 w ..)
// in the scan's accumulator order, and waves 2, 3 form W^T = (beta gamma K)^T
// T^T (key columns 64 (w - 2) ..): their A operand lane l of tile ct gathers
// key column 32 (ct / 2) + 4 (ct % 2) + 8 ((l % 16) / 4) + l % 4, so that
// result tiles 2 h, 2 h + 1, lane l reg r hold W[i][32 h + 8 (l / 16) + 4 (tile
// % 2) + r]: 8 consecutive keys per lane, the -W operand order of the scan.
// (three waves per SIMD: the phases are latency-bound, and three workgroups fit a CU's LDS)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void deltanet_chunk_kernel(DeltaChunkArgs a) {
  const DeltaSeqArgs& q = a.s;
  const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z, t = threadIdx.x;
  const int lane = t & 63, l16 = lane & 15, r4 = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: scalar branches
  const int hk = hv / (q.Hv / q.Hk);
  const int t0 = c * DC, n = min(DC, q.T - t0);
  const int NC = (q.T + DC - 1) / DC;
  float* u = dn_units(a, b, hv, NC) + (int64_t)c * UNIT;
  if (c == 0) {  // unit NC: the identity chunk (all zero, gamma_C = 1), the scan's pad
    float* id = u + (int64_t)NC * UNIT;
    for (int i = t; i < UNIT / 4; i += 256)
      reinterpret_cast<float4*>(id)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();
    if (t == 0) id[UO_G] = 1.f;
  }
  // K rows, and L, later T (hi, lo) in its place: ~52 KB, three workgroups per CU
  __shared__ __attribute__((aligned(16))) float Ks[DC * KSW];
  __shared__ __attribute__((aligned(16))) float LT[DC * TW];
  static_assert(sizeof(LT) >= DC * LSW * sizeof(float), "L");
  __shared__ __attribute__((aligned(16))) float Gs[DC], Bs[DC], Es[DC], Ek[DC];
  uint16_t* const Th = reinterpret_cast<uint16_t*>(LT);
  uint16_t* const Tl = Th + DC * TW;
  const float* kp = q.k + (((int64_t)b * q.Hk + hk) * q.T + t0) * DN_D;
  {  // K: float4 t + 256 m = (row, column group) ((t + 256 m) / 32, t % 32), all loads in flight at once
    float4 kv[DC / 8];
#pragma unroll
    for (int m = 0; m < DC / 8; ++m)
      kv[m] = *reinterpret_cast<const float4*>(kp + min((t >> 5) + 8 * m, n - 1) * DN_D + 4 * (t & 31));
    float bt = 0.f;
    if (t < 64) {  // wave 0: beta, gates, inclusive cumulative sum of the log decay
      bt = q.beta[((int64_t)b * q.T + t0 + min(t, n - 1)) * q.Hv + hv];
      const float G = chunk_cumsum(q, b, hv, t0, n, t);
      Gs[t] = G;
      Bs[t] = t < n ? bt : 0.f;
      Es[t] = expf(G);
      Ek[t] = expf(__shfl(G, DC - 1) - G);  // gamma_C / gamma_t
    }
#pragma unroll
    for (int m = 0; m < DC / 8; ++m) {  // rows past the end read as 0
      const int r = (t >> 5) + 8 * m;
      *reinterpret_cast<float4*>(&Ks[r * KSW + 4 * (t & 31)]) = r < n ? kv[m] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __syncthreads();
  {  // Gram tiles (w, jt), jt <= w: lane l reg r = k_i . k_j, i = 16 w + 4 (l / 16) + r, j = 16 jt + l % 16
    uint4 ah[4], al[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const float* kr = &Ks[(16 * w + l16) * KSW + 32 * ks + 8 * r4];
      split8(*reinterpret_cast<const f32x4*>(kr), *reinterpret_cast<const f32x4*>(kr + 4), ah[ks], al[ks]);
    }
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      if (jt > w) break;
      f32x4 G = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const float* kr = &Ks[(16 * jt + l16) * KSW + 32 * ks + 8 * r4];
        uint4 bh, bl;
        split8(*reinterpret_cast<const f32x4*>(kr), *reinterpret_cast<const f32x4*>(kr + 4), bh, bl);
        G = mfma_x3(ah[ks], al[ks], bh, bl, G);
      }
      const int j = 16 * jt + l16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * w + 4 * r4 + r;
        LT[i * LSW + j] = i > j ? Bs[i] * expf(Gs[i] - Gs[j]) * G[r] : 0.f;
      }
    }
  }
  __syncthreads();
  // the products' operands from V or K (rows j = 32 ks + 8 (l / 16) + e of R),
  // scaled and split: waves 0, 1 B = beta_j V[j][64 w + 16 ct + l % 16] (rows past
  // the end: beta = 0), waves 2, 3 A = beta_j gamma_j K[j][key column]
  const bool uw = w < 2;
  uint4 rh[2][4], rl[2][4];  // [ks][ct]
  auto gather = [&]() __attribute__((always_inline)) {
    const float* vp = q.v + (((int64_t)b * q.Hv + hv) * q.T + t0) * DN_D + 64 * (w & 1) + l16;
    // gathered key column of tile ct: 64 (w % 2) + 32 (ct / 2) + 4 (ct % 2) + pc
    const int pc = 64 * (w & 1) + 8 * (l16 >> 2) + (l16 & 3);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int j0 = 32 * ks + 8 * r4;
      f32x4 s0 = *reinterpret_cast<const f32x4*>(&Bs[j0]), s1 = *reinterpret_cast<const f32x4*>(&Bs[j0 + 4]);
      if (!uw) {
        s0 = s0 * *reinterpret_cast<const f32x4*>(&Es[j0]);
        s1 = s1 * *reinterpret_cast<const f32x4*>(&Es[j0 + 4]);
      }
      f32x4 r0[4], r1[4];
      if (uw) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            r0[ct][e] = vp[(int64_t)min(j0 + e, n - 1) * DN_D + 16 * ct];
            r1[ct][e] = vp[(int64_t)min(j0 + 4 + e, n - 1) * DN_D + 16 * ct];
          }
      } else {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            r0[ct][e] = Ks[(j0 + e) * KSW + pc + 32 * (ct >> 1) + 4 * (ct & 1)];
            r1[ct][e] = Ks[(j0 + 4 + e) * KSW + pc + 32 * (ct >> 1) + 4 * (ct & 1)];
          }
      }
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) split8(r0[ct] * s0, r1[ct] * s1, rh[ks][ct], rl[ks][ct]);
    }
  };
  if (w == 3) {
    // (I + L) T = I: lane c holds column c (rows above c stay 0, T[c][c] = 1).
    // The float4s of L's rows 1 .. 63 (j < i) are read in order through a ring
    // of SD registers, SD ahead of their use (the cursor (pi, pj) is a
    // constant once the loops are unrolled). All four lanes of a float4 enter
    // the sums: the ones at j >= i hold L's zeros above the diagonal (the Gram
    // tiles on it are written whole) times x[j] = 0, and a load whose every
    // register is used keeps the allocator from reloading into one in flight.
    constexpr int SD = 12;
    float x[DC];
#pragma unroll
    for (int i = 0; i < DC; ++i) x[i] = 0.f;
    f32x4 ring[SD];
    int pi = 1, pj = 0;  // next float4 to read: row pi, columns 4 pj ..
#pragma unroll
    for (int d = 0; d < SD; ++d) {
      ring[d] = *reinterpret_cast<const f32x4*>(&LT[pi * LSW + 4 * pj]);
      if (4 * (pj + 1) < pi) ++pj; else { ++pi; pj = 0; }
    }
    x[0] = lane == 0 ? 1.f : 0.f;
    int idx = 0;
#pragma unroll
    for (int i = 1; i < DC; ++i) {
      float acc[4] = {i == lane ? 1.f : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j4 = 0; 4 * j4 < i; ++j4) {
        const f32x4 l4 = ring[idx % SD];
        if (pi < DC) {
          ring[idx % SD] = *reinterpret_cast<const f32x4*>(&LT[pi * LSW + 4 * pj]);
          if (4 * (pj + 1) < pi) ++pj; else { ++pi; pj = 0; }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] -= l4[e] * x[4 * j4 + e];
        ++idx;
      }
      x[i] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    // T rows, split: columns (c & ~1, c | 1) as one pair, lane c even stores the
    // hi pair, odd the lo pair (L is dead: every read of it is above)
#pragma unroll
    for (int i = 0; i < DC; ++i) {
      const float xo = __shfl_xor(x[i], 1);
      const float x0 = (lane & 1) ? xo : x[i], x1 = (lane & 1) ? x[i] : xo;
      const uint32_t hi = pack2(x0, x1);
      const uint32_t lo = pack2(x0 - __uint_as_float(hi << 16), x1 - __uint_as_float(hi & 0xffff0000u));
      *reinterpret_cast<uint32_t*>(((lane & 1) ? Tl : Th) + i * TW + (lane & ~1)) = (lane & 1) ? lo : hi;
    }
  } else {
    // K~^T split, in operand order: slot f = (tile d, ks) = (f / 128, (f / 64) % 2),
    // lane f % 64: dk 16 d + l % 16, r = 32 ks + 8 (l / 16) + j
    uint16_t* const kt = reinterpret_cast<uint16_t*>(u + UO_K);
    for (int f = t; f < 1024; f += 192) {
      const int l = f & 63, dk = 16 * (f >> 7) + (l & 15), r0 = 32 * ((f >> 6) & 1) + 8 * (l >> 4);
      f32x4 v0, v1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v0[e] = Ek[r0 + e] * Ks[(r0 + e) * KSW + dk];
        v1[e] = Ek[r0 + 4 + e] * Ks[(r0 + 4 + e) * KSW + dk];
      }
      uint4 hi, lo;
      split8(v0, v1, hi, lo);
      *reinterpret_cast<uint4*>(kt + ((2 * (f >> 6) + 0) * 64 + l) * 8) = hi;
      *reinterpret_cast<uint4*>(kt + ((2 * (f >> 6) + 1) * 64 + l) * 8) = lo;
    }
    if (t == 0) u[UO_G] = expf(Gs[DC - 1]);
    gather();
  }
  __syncthreads();
  if (w == 3) gather();
  f32x4 acc[4][4];  // [row tile][column tile] (U) or [column tile][row tile] (W^T)
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int j0 = 32 * ks + 8 * r4;
    uint4 th[4], tl[4];  // T[16 rt + l % 16][j0 ..]
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      th[rt] = *reinterpret_cast<const uint4*>(&Th[(16 * rt + l16) * TW + j0]);
      tl[rt] = *reinterpret_cast<const uint4*>(&Tl[(16 * rt + l16) * TW + j0]);
    }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        if (uw)
          acc[rt][ct] = mfma_x3(th[rt], tl[rt], rh[ks][ct], rl[ks][ct], acc[rt][ct]);
        else
          acc[ct][rt] = mfma_x3(rh[ks][ct], rl[ks][ct], th[rt], tl[rt], acc[ct][rt]);
      }
  }
  if (uw) {  // U tile (rt, column block 4 w + ct): lane l reg r = U[16 rt + 4 (l / 16) + r][..]
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        *reinterpret_cast<f32x4*>(u + UO_U + (((4 * w + ct) * 4 + rt) * 64 + lane) * 4) = acc[rt][ct];
  } else {  // -W, row tile rt, k step ks = 2 (w - 2) + h: tiles 2 h, 2 h + 1 hold
            // lane l's dk 32 ks + 8 (l / 16) + j, j < 4 and j >= 4
    uint16_t* const wm = reinterpret_cast<uint16_t*>(u + UO_W);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int ks = 2 * (w - 2) + h;
        uint4 hi, lo;
        split8(-acc[2 * h][rt], -acc[2 * h + 1][rt], hi, lo);
        *reinterpret_cast<uint4*>(wm + (((rt * 4 + ks) * 2 + 0) * 64 + lane) * 8) = hi;
        *reinterpret_cast<uint4*>(wm + (((rt * 4 + ks) * 2 + 1) * 64 + lane) * 8) = lo;
      }
  }
}

namespace {
// a chunk's operands, split by the step that consumes them: step A (the delta
// products) and step B (the state products); bf16 hi / lo pairs [.][hl]
struct ScanOpsA {
  uint4 w[4][2];  // -W rows 16 w .., k step ks
  f32x4 u;
};
struct ScanOpsB {
  uint4 k[2][2][2];  // K~^T tiles 2 w + x, k step ks
  float gl;
};
__device__ __forceinline__ void scan_load_a(ScanOpsA& o, const float* unit, int w, int cb,
                                            int lane) {
  const uint16_t* wm = reinterpret_cast<const uint16_t*>(unit + UO_W);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
      o.w[ks][hl] = *reinterpret_cast<const uint4*>(wm + (((w * 4 + ks) * 2 + hl) * 64 + lane) * 8);
  o.u = *reinterpret_cast<const f32x4*>(unit + UO_U + ((cb * 4 + w) * 64 + lane) * 4);
}
__device__ __forceinline__ void scan_load_b(ScanOpsB& o, const float* unit, int w, int lane) {
  const uint16_t* kt = reinterpret_cast<const uint16_t*>(unit + UO_K);
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        o.k[x][ks][hl] =
            *reinterpret_cast<const uint4*>(kt + ((((2 * w + x) * 2 + ks) * 2 + hl) * 64 + lane) * 8);
  o.gl = unit[UO_G];
}
// an accumulator tile (lane (r4, n) rows 16 d + 4 r4 + e, column n) split into
// the phase-3 B operand order: k step d / 2, lane 16 (2 (d % 2) + r4 / 2) + n,
// elements 4 (r4 % 2) .. +3 (ks: this tile's k step; blk: the block's base)
__device__ __forceinline__ void store_split(uint16_t* blk, int ks, int half, const uint2& hi,
                                            const uint2& lo, int lane) {
  const int r4 = lane >> 4, n = lane & 15;
  const int l2 = 16 * (2 * half + (r4 >> 1)) + n;
  *reinterpret_cast<uint2*>(blk + ((ks * 2 + 0) * 64 + l2) * 8 + 4 * (r4 & 1)) = hi;
  *reinterpret_cast<uint2*>(blk + ((ks * 2 + 1) * 64 + l2) * 8 + 4 * (r4 & 1)) = lo;
}
constexpr int SSW = DN_D + 8;  // LDS row (one state column) of S hi / lo, bf16
constexpr int DSW = DC + 8;    // LDS row (one state column) of delta hi / lo, bf16
// the scan's LDS: S and delta split, transposed: X[k][column c] at [c][k]
struct ScanLds {
  uint16_t sh[CBW * SSW], sl[CBW * SSW], dh[CBW * DSW], dl[CBW * DSW];
};
// accumulator tile rows k0 + 4 (l / 16) .. +3 of column l % 16, split, into LDS
__device__ __forceinline__ void lds_put(uint16_t* h, uint16_t* l, int ld, int k0, const uint2& hi,
                                        const uint2& lo, int lane) {
  const int o = (lane & 15) * ld + k0 + 4 * (lane >> 4);
  *reinterpret_cast<uint2*>(h + o) = hi;
  *reinterpret_cast<uint2*>(l + o) = lo;
}
// one chunk: S_0 out for phase 3, delta = U - W S_0 (step A), delta out, then
// S = gamma_C S_0 + K~^T delta (step B). s0 / dl: this chunk's S_0 and delta
// blocks of this workgroup's column block (bf16 hi / lo, see S0_UNIT). B
// operand of k step ks, lane l: X[32 ks + 8 (l / 16) + j][l % 16], one LDS read
// each of hi and lo.
__device__ __forceinline__ void scan_chunk(const ScanOpsA& oa, const ScanOpsB& ob, f32x4 (&St)[2],
                                           ScanLds& sm, uint16_t* s0, uint16_t* dl, int w,
                                           int lane) {
  const int row4 = lane >> 4, col = lane & 15;
#pragma unroll
  for (int x = 0; x < 2; ++x) {  // rows 16 (2 w + x) ..
    uint2 hi, lo;
    split4(St[x], hi, lo);
    store_split(s0, w, x, hi, lo, lane);
  }
  f32x4 dacc = oa.u;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int o = col * SSW + 32 * ks + 8 * row4;
    dacc = mfma_x3(oa.w[ks][0], oa.w[ks][1], *reinterpret_cast<const uint4*>(&sm.sh[o]),
                   *reinterpret_cast<const uint4*>(&sm.sl[o]), dacc);
  }
  {  // delta rows 16 w ..
    uint2 hi, lo;
    split4(dacc, hi, lo);
    store_split(dl, w >> 1, w & 1, hi, lo, lane);
    lds_put(sm.dh, sm.dl, DSW, 16 * w, hi, lo, lane);
  }
  __syncthreads();
  f32x4 s0v = St[0] * ob.gl, s1v = St[1] * ob.gl;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int o = col * DSW + 32 * ks + 8 * row4;
    const uint4 bh = *reinterpret_cast<const uint4*>(&sm.dh[o]);
    const uint4 bl = *reinterpret_cast<const uint4*>(&sm.dl[o]);
    s0v = mfma_x3(ob.k[0][ks][0], ob.k[0][ks][1], bh, bl, s0v);
    s1v = mfma_x3(ob.k[1][ks][0], ob.k[1][ks][1], bh, bl, s1v);
  }
  St[0] = s0v;
  St[1] = s1v;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    uint2 hi, lo;
    split4(St[x], hi, lo);
    lds_put(sm.sh, sm.sl, SSW, 16 * (2 * w + x), hi, lo, lane);
  }
  __syncthreads();
}
}  // namespace

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void deltanet_scan_kernel(DeltaChunkArgs a) {
  const DeltaSeqArgs& q = a.s;
  const int HB = q.Hv * q.B;
  // the 8 column blocks of a head share an XCD (workgroup id mod 8) when HB % 8 == 0
  const int head = blockIdx.x % HB, cb = blockIdx.x / HB;
  const int hv = head % q.Hv, b = head / q.Hv;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row4 = lane >> 4, col = lane & 15;
  __shared__ __attribute__((aligned(16))) ScanLds sm;
  const int dv0 = cb * CBW;
  const int64_t sb = ((int64_t)b * q.Hv + hv) * DN_D * DN_D;
  f32x4 St[2];  // state tiles d = 2w, 2w + 1: lane l reg e = S[16 d + 4 (l / 16) + e][l % 16]
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int d = 2 * w + x;
    St[x] = *reinterpret_cast<const f32x4*>(q.s_in + sb + (int64_t)(dv0 + col) * DN_D + 16 * d +
                                            4 * row4);
    uint2 hi, lo;
    split4(St[x], hi, lo);
    lds_put(sm.sh, sm.sl, SSW, 16 * d, hi, lo, lane);
  }
  const int NC = (q.T + DC - 1) / DC;
  const float* units = dn_units(a, b, hv, NC);
  // phase 3's inputs of this column block: chunk c at + c * unit + cb * block
  uint16_t* s0b = reinterpret_cast<uint16_t*>(dn_s0(a, b, hv, NC) + cb * (S0_UNIT / 8));
  uint16_t* dlb = reinterpret_cast<uint16_t*>(dn_dl(a, b, hv, NC) + cb * (DL_UNIT / 8));
  // Two register sets, chunks in pairs, each set reloaded two chunks ahead right
  // after its chunk; chunk indices past the end read the identity unit (an odd
  // count pads with it; its S_0 and delta go to the spare slot NC). Branch-free,
  // so the compiler's waits count exactly.
  ScanOpsA ax, ay;
  ScanOpsB bx, by;
  scan_load_a(ax, units, w, cb, lane);
  scan_load_b(bx, units, w, lane);
  scan_load_a(ay, units + (int64_t)min(1, NC) * UNIT, w, cb, lane);
  scan_load_b(by, units + (int64_t)min(1, NC) * UNIT, w, lane);
  // every prologue load complete (s_waitcnt vmcnt(0)): the loop is then entered
  // with no load in flight, and the compiler's count of the loads each wait in
  // the loop must see is the one its own body implies (else it takes the
  // prologue's order, where a register the loop reloads early was loaded last).
  // NC >= 1 (the launch returns before T = 0): a do-while has no guard branch
  // that the prologue's loads could be sunk past.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0x0f70);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  int c = 0;
  do {
    scan_chunk(ax, bx, St, sm, s0b + 2 * (int64_t)c * S0_UNIT, dlb + 2 * (int64_t)c * DL_UNIT, w,
               lane);
    const float* u2 = units + (int64_t)min(c + 2, NC) * UNIT;
    __builtin_amdgcn_sched_barrier(0);  // the reloads issue here, between the chunks
    scan_load_a(ax, u2, w, cb, lane);
    scan_load_b(bx, u2, w, lane);
    __builtin_amdgcn_sched_barrier(0);
    const int c1 = min(c + 1, NC);
    scan_chunk(ay, by, St, sm, s0b + 2 * (int64_t)c1 * S0_UNIT, dlb + 2 * (int64_t)c1 * DL_UNIT, w,
               lane);
    const float* u3 = units + (int64_t)min(c + 3, NC) * UNIT;
    __builtin_amdgcn_sched_barrier(0);
    scan_load_a(ay, u3, w, cb, lane);
    scan_load_b(by, u3, w, lane);
    __builtin_amdgcn_sched_barrier(0);
    c += 2;
  } while (c < NC);
#pragma unroll
  for (int x = 0; x < 2; ++x)
    *reinterpret_cast<f32x4*>(q.s_out + sb + (int64_t)(dv0 + col) * DN_D + 16 * (2 * w + x) +
                              4 * row4) = St[x];
}

// Phase 3: one workgroup per (chunk, value head, sequence). First each wave w
// forms rows 16 w .. 16 w + 15 of M and of gamma Q into LDS, split into bf16
// hi and lo parts: lane l holds q row i = 16 w + l % 16 at columns 32 ks + 8
// (l / 16) .. +7 (ks < 4), the B operand of P^T = K Q^T, whose result tiles
// (tile jt: lane l reg r = P[i][16 jt + 4 (l / 16) + r]) are masked and
// decayed into M. Then wave w forms output columns 32 w .. 32 w + 31 (the
// scan's column blocks 2 w, 2 w + 1) of all 64 rows: its S_0 and delta
// operands (the scan's split blocks) are loaded once the first phase is done,
// and gamma Q and M come from LDS. Each product is hi hi + hi lo + lo hi on
// v_mfma_f32_16x16x32_bf16 (A lane l = A[l % 16][8 (l / 16) + j], B lane l =
// B[8 (l / 16) + j][l % 16], D lane l reg r = D[4 (l / 16) + r][l % 16]). The
// output tile is staged through LDS, so that a thread then holds 32
// contiguous columns of one row: O, or with NORM y = o rstd norm_w silu(z)
// (the layer's gated norm, as gated_rms_norm_kernel) in bf16.
constexpr int OQW = DN_D + 8;  // LDS row of gamma Q hi / lo (bf16; 16-byte aligned, banks skewed)
constexpr int OMW = DC + 8;    // LDS row of M hi / lo (bf16)
constexpr int OOW = DN_D + 4;  // LDS row of the output tile (floats)
template <bool NORM>
__global__ __launch_bounds__(256) void deltanet_out_kernel(DeltaChunkArgs a) {
  const DeltaSeqArgs& q = a.s;
  const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z, t = threadIdx.x;
  const int lane = t & 63, w = t >> 6, l16 = lane & 15, r4 = lane >> 4;
  const int hk = hv / (q.Hv / q.Hk);
  const int t0 = c * DC, n = min(DC, q.T - t0);
  const int NC = (q.T + DC - 1) / DC;
  __shared__ float Gs[DC];
  __shared__ __attribute__((aligned(16))) uint16_t Qhl[2][DC * OQW];  // gamma Q [i][dk] hi, lo
  uint16_t* const Qh = Qhl[0];
  uint16_t* const Ql = Qhl[1];
  __shared__ __attribute__((aligned(16))) uint16_t Mh[DC * OMW], Ml[DC * OMW];  // M [i][j]
  if (t < 64) Gs[t] = chunk_cumsum(q, b, hv, t0, n, t);
  const float* qp = q.q + (((int64_t)b * q.Hk + hk) * q.T + t0) * DN_D;
  const float* kp = q.k + (((int64_t)b * q.Hk + hk) * q.T + t0) * DN_D;
  {
    const int i = 16 * w + l16;  // this lane's q row
    f32x4 qv[8];                 // q[i][32 ks + 8 (l / 16) + 4 u .. +3] at qv[2 ks + u]
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        qv[2 * ks + u] = *reinterpret_cast<const f32x4*>(qp + (int64_t)min(i, n - 1) * DN_D + 32 * ks +
                                                         8 * r4 + 4 * u);
    uint4 qh[4], ql[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) split8(qv[2 * ks], qv[2 * ks + 1], qh[ks], ql[ks]);
    // P^T tiles: D[j][i] = sum_dk K[j][dk] Q[i][dk], A lane l = K[16 jt + l % 16][dk]
    f32x4 P[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) P[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint4 kh[4], kl[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const float* kr = kp + (int64_t)min(16 * jt + l16, n - 1) * DN_D + 32 * ks + 8 * r4;
        split8(*reinterpret_cast<const f32x4*>(kr), *reinterpret_cast<const f32x4*>(kr + 4), kh[jt],
               kl[jt]);
      }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) P[jt] = mfma_x3(kh[jt], kl[jt], qh[ks], ql[ks], P[jt]);
    }
    __syncthreads();  // Gs
    // M = P D on j <= i < n, j < n (rows or keys past the chunk: 0); lane l reg r
    // of tile jt is (i, j = 16 jt + 4 (l / 16) + r)
    const float Gi = Gs[i];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      f32x4 m;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jt + 4 * r4 + r;
        m[r] = (j <= i && i < n) ? P[jt][r] * expf(Gi - Gs[j]) : 0.f;
      }
      uint2 mh, ml;
      split4(m, mh, ml);
      *reinterpret_cast<uint2*>(&Mh[i * OMW + 16 * jt + 4 * r4]) = mh;
      *reinterpret_cast<uint2*>(&Ml[i * OMW + 16 * jt + 4 * r4]) = ml;
    }
    const float gi = i < n ? expf(Gi) : 0.f;  // gamma_i (rows past the chunk: 0)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint4 gh, gl;
      split8(qv[2 * ks] * gi, qv[2 * ks + 1] * gi, gh, gl);
      *reinterpret_cast<uint4*>(&Qh[i * OQW + 32 * ks + 8 * r4]) = gh;
      *reinterpret_cast<uint4*>(&Ql[i * OQW + 32 * ks + 8 * r4]) = gl;
    }
  }
  // this wave's B operands, column blocks 2 w + x: S_0 (ks < 4) and delta (ks < 2)
  const uint16_t* s0 = reinterpret_cast<const uint16_t*>(dn_s0(a, b, hv, NC) + (int64_t)c * S0_UNIT) +
                       2 * (2 * w) * (S0_UNIT / 8);
  const uint16_t* dl = reinterpret_cast<const uint16_t*>(dn_dl(a, b, hv, NC) + (int64_t)c * DL_UNIT) +
                       2 * (2 * w) * (DL_UNIT / 8);
  uint4 sb[2][4][2], db[2][2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        sb[x][ks][hl] = *reinterpret_cast<const uint4*>(s0 + 2 * x * (S0_UNIT / 8) + ((ks * 2 + hl) * 64 + lane) * 8);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
        db[x][ks][hl] = *reinterpret_cast<const uint4*>(dl + 2 * x * (DL_UNIT / 8) + ((ks * 2 + hl) * 64 + lane) * 8);
  }
  __syncthreads();
  // O = gamma Q S_0 + M delta: row tile rt, column block 2 w + x
  f32x4 O[4][2];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int x = 0; x < 2; ++x) O[rt][x] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    uint4 ah[4], al[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      ah[rt] = *reinterpret_cast<const uint4*>(&Qh[(16 * rt + l16) * OQW + 32 * ks + 8 * r4]);
      al[rt] = *reinterpret_cast<const uint4*>(&Ql[(16 * rt + l16) * OQW + 32 * ks + 8 * r4]);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int x = 0; x < 2; ++x)
        O[rt][x] = mfma_x3(ah[rt], al[rt], sb[x][ks][0], sb[x][ks][1], O[rt][x]);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    uint4 ah[4], al[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      ah[rt] = *reinterpret_cast<const uint4*>(&Mh[(16 * rt + l16) * OMW + 32 * ks + 8 * r4]);
      al[rt] = *reinterpret_cast<const uint4*>(&Ml[(16 * rt + l16) * OMW + 32 * ks + 8 * r4]);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int x = 0; x < 2; ++x)
        O[rt][x] = mfma_x3(ah[rt], al[rt], db[x][ks][0], db[x][ks][1], O[rt][x]);
  }
  // lane l reg r of O[rt][x] = O[16 rt + 4 (l / 16) + r][32 w + 16 x + l % 16]: the
  // tile goes through LDS (the gamma Q and M rows, free once every wave is past
  // its products) so that a thread then holds 32 contiguous columns of one row
  __syncthreads();
  float* Os = reinterpret_cast<float*>(&Qhl[0][0]);  // 2 x 17 KB >= 64 rows of OOW floats
  static_assert(sizeof(Qhl) >= DC * OOW * sizeof(float), "output tile");
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int x = 0; x < 2; ++x) Os[(16 * rt + 4 * r4 + r) * OOW + 32 * w + 16 * x + l16] = O[rt][x][r];
  __syncthreads();
  const int row = t >> 2, c0 = 32 * (t & 3);  // thread t: row t / 4, columns c0 .. c0 + 31
  float o[32];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(&Os[row * OOW + c0 + 4 * j]);
    o[4 * j] = v[0]; o[4 * j + 1] = v[1]; o[4 * j + 2] = v[2]; o[4 * j + 3] = v[3];
  }
  const int64_t tok = t0 + row;
  if constexpr (!NORM) {
    if (row < n) {
      float* op = q.o + (((int64_t)b * q.Hv + hv) * q.T + tok) * DN_D + c0;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        *reinterpret_cast<float4*>(op + 4 * j) = make_float4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
    }
  } else {
    const GatedNormArgs& g = a.g;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) ss += o[j] * o[j];
    ss += __shfl_xor(ss, 1);  // the row's four threads
    ss += __shfl_xor(ss, 2);
    const float rstd = 1.0f / sqrtf(ss / (float)DN_D + g.eps);
    if (row < n) {
      const uint16_t* z = g.z + (int64_t)b * g.z_sb + tok * g.z_st + hv * DN_D + c0;
      uint16_t* y = g.y + (int64_t)b * g.y_sb + tok * g.y_st + hv * DN_D + c0;
      if (((reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(y) |
            reinterpret_cast<uintptr_t>(g.norm_w)) & 15u) == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float zf[8], wf[8], yv[8];
          unpack8(*reinterpret_cast<const uint4*>(z + 8 * j), zf);
          unpack8(*reinterpret_cast<const uint4*>(g.norm_w + c0 + 8 * j), wf);
#pragma unroll
          for (int e = 0; e < 8; ++e) yv[e] = o[8 * j + e] * rstd * wf[e] * accurate_silu(zf[e]);
          *reinterpret_cast<uint4*>(y + 8 * j) = pack8(yv);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 32; ++j)
          y[j] = f2bf(o[j] * rstd * bf2f(g.norm_w[c0 + j]) * accurate_silu(bf2f(z[j])));
      }
    }
  }
}

// ---- the prefill's inputs to the recurrence (qwen35.jl:347-356): one wave per
// (token, head): q / k heads l2-normed (q also by 1/sqrt(Dk)) from the conv
// output, v heads widened to fp32, gates from the alpha | beta projection.
__global__ __launch_bounds__(256) void deltanet_prep_kernel(DeltaPrepArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nh = 2 * a.Hk + a.Hv;  // q heads, k heads, v heads
  const int64_t tok = wid / nh;    // b * T + t
  if (tok >= (int64_t)a.B * a.T) return;
  const int hh = (int)(wid % nh);
  const int b = (int)(tok / a.T), t = (int)(tok % a.T);
  const uint16_t* row = a.cv + (int64_t)b * a.cv_sb + (int64_t)t * a.cv_st + hh * DN_D;
  const float x0 = bf2f(row[2 * lane]), x1 = bf2f(row[2 * lane + 1]);
  if (hh < 2 * a.Hk) {
    const int hk = hh % a.Hk;
    float ss = x0 * x0 + x1 * x1;
    ss += __shfl_xor(ss, 32);
    ss = half_sum(ss);
    const float den = sqrtf(ss + 1e-6f);
    const bool isq = hh < a.Hk;
    const float sc = isq ? 1.0f / sqrtf((float)DN_D) : 1.0f;
    float* dst = (isq ? a.qe : a.ke) + (((int64_t)b * a.Hk + hk) * a.T + t) * DN_D;
    *reinterpret_cast<float2*>(dst + 2 * lane) = make_float2(x0 / den * sc, x1 / den * sc);
  } else {
    const int hv = hh - 2 * a.Hk;
    float* dst = a.ve + (((int64_t)b * a.Hv + hv) * a.T + t) * DN_D;
    *reinterpret_cast<float2*>(dst + 2 * lane) = make_float2(x0, x1);
    if (lane == 0) {
      const uint16_t* ab = a.ab + (int64_t)b * a.ab_sb + (int64_t)t * a.ab_st;
      const int64_t g = ((int64_t)b * a.T + t) * a.Hv + hv;
      a.beta[g] = accurate_sigmoid(bf2f(ab[a.Hv + hv]));
      a.gate[g] = -expf(a.a_log[hv]) * log1pf(expf(bf2f(ab[hv]) + a.dt_bias[hv]));
    }
  }
}

// The same, vectorised for aligned operands (the conv output 16-byte aligned
// with strides of whole 8-element chunks, fp32 outputs 16-byte aligned; the
// launcher checks): one wave per token, four heads per pass (16 lanes of 8
// channels per head: 16-byte reads, 32-byte writes), the q / k sums of squares
// reduced over each 16-lane group, then lane l takes the gates of heads l, l + 64,
// ... The one-wave-per-(token, head) kernel above issued 64 times the waves
// for 4-byte reads, and ran at 2 TB/s.
__global__ __launch_bounds__(256) void deltanet_prep_vec_kernel(DeltaPrepArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= (int64_t)a.B * a.T) return;
  const int b = (int)(tok / a.T), t = (int)(tok % a.T);
  const int nh = 2 * a.Hk + a.Hv, grp = lane >> 4, c = lane & 15;
  const uint16_t* row = a.cv + (int64_t)b * a.cv_sb + (int64_t)t * a.cv_st + 8 * c;
  const float qsc = 1.0f / sqrtf((float)DN_D);
  for (int h0 = 0; h0 < nh; h0 += 4) {
    const int hh = h0 + grp;  // uniform over the 16-lane group
    if (hh < nh) {
      float x[8];
      unpack8(*reinterpret_cast<const uint4*>(row + (int64_t)hh * DN_D), x);
      float* dst;
      float den = 1.0f, sc = 1.0f;
      if (hh < 2 * a.Hk) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
        ss += xor32<8>(ss);
        ss += xor32<4>(ss);
        ss += xor32<2>(ss);
        ss += xor32<1>(ss);
        den = sqrtf(ss + 1e-6f);
        const bool isq = hh < a.Hk;
        sc = isq ? qsc : 1.0f;
        dst = (isq ? a.qe : a.ke) + (((int64_t)b * a.Hk + (isq ? hh : hh - a.Hk)) * a.T + t) * DN_D;
      } else {
        dst = a.ve + (((int64_t)b * a.Hv + (hh - 2 * a.Hk)) * a.T + t) * DN_D;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = x[j] / den * sc;
      float4* d4 = reinterpret_cast<float4*>(dst + 8 * c);
      d4[0] = make_float4(x[0], x[1], x[2], x[3]);
      d4[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
  }
  const uint16_t* ab = a.ab + (int64_t)b * a.ab_sb + (int64_t)t * a.ab_st;
  for (int hv = lane; hv < a.Hv; hv += 64) {
    const int64_t gi = ((int64_t)b * a.T + t) * a.Hv + hv;
    a.beta[gi] = accurate_sigmoid(bf2f(ab[a.Hv + hv]));
    a.gate[gi] = -expf(a.a_log[hv]) * log1pf(expf(bf2f(ab[hv]) + a.dt_bias[hv]));
  }
}

// ---- the prefill's epilogue (qwen35.jl:360-364): one wave per (head, token):
// y = o rstd norm_w silu(z) in bf16, written in the out projection's input
// layout (Dv, Hv, T, B).
__global__ __launch_bounds__(256) void gated_rms_norm_kernel(GatedNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= (int64_t)a.B * a.T * a.Hv) return;
  const int hv = (int)(wid % a.Hv);
  const int64_t tok = wid / a.Hv;
  const int b = (int)(tok / a.T), t = (int)(tok % a.T);
  const float2 o = *reinterpret_cast<const float2*>(
      a.o + (((int64_t)b * a.Hv + hv) * a.T + t) * DN_D + 2 * lane);
  float ss = o.x * o.x + o.y * o.y;
  ss += __shfl_xor(ss, 32);
  ss = half_sum(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)DN_D + a.eps);
  const uint16_t* z = a.z + (int64_t)b * a.z_sb + (int64_t)t * a.z_st + hv * DN_D + 2 * lane;
  const float w0 = bf2f(a.norm_w[2 * lane]), w1 = bf2f(a.norm_w[2 * lane + 1]);
  const float y0 = o.x * rstd * w0 * accurate_silu(bf2f(z[0]));
  const float y1 = o.y * rstd * w1 * accurate_silu(bf2f(z[1]));
  *reinterpret_cast<uint32_t*>(a.y + (int64_t)b * a.y_sb + (int64_t)t * a.y_st + hv * DN_D +
                               2 * lane) = pack2(y0, y1);
}

// The same, vectorised for aligned z and y (16-byte aligned, strides of whole
// 8-element chunks): one wave per token, four heads per pass (16 lanes of 8
// channels: 32-byte o reads, 16-byte z reads and y writes).
__global__ __launch_bounds__(256) void gated_rms_norm_vec_kernel(GatedNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= (int64_t)a.B * a.T) return;
  const int b = (int)(tok / a.T), t = (int)(tok % a.T);
  const int grp = lane >> 4, c = lane & 15;
  float w[8];
  unpack8(*reinterpret_cast<const uint4*>(a.norm_w + 8 * c), w);
  for (int h0 = 0; h0 < a.Hv; h0 += 4) {
    const int hv = h0 + grp;
    if (hv < a.Hv) {
      const float4* op = reinterpret_cast<const float4*>(
          a.o + (((int64_t)b * a.Hv + hv) * a.T + t) * DN_D + 8 * c);
      const float4 o0 = op[0], o1 = op[1];
      const float o[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += o[j] * o[j];
      ss += xor32<8>(ss);
      ss += xor32<4>(ss);
      ss += xor32<2>(ss);
      ss += xor32<1>(ss);
      const float rstd = 1.0f / sqrtf(ss / (float)DN_D + a.eps);
      float z[8], y[8];
      unpack8(*reinterpret_cast<const uint4*>(a.z + (int64_t)b * a.z_sb + (int64_t)t * a.z_st +
                                              hv * DN_D + 8 * c), z);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = o[j] * rstd * w[j] * accurate_silu(z[j]);
      *reinterpret_cast<uint4*>(a.y + (int64_t)b * a.y_sb + (int64_t)t * a.y_st + hv * DN_D + 8 * c) =
          pack8(y);
    }
  }
}

// ---- causal_conv1d! (causal_conv1d.jl:7-61): one thread per 8 channels of one
// sequence. The ring's columns are all read before any is written, so the
// shifted ring may overwrite the one read (in place, as the reference runs it).
template <int K>
__global__ __launch_bounds__(256) void conv1d_update_kernel(Conv1dArgs a) {
  const int64_t c8 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (c8 * 8 >= a.D) return;
  const int d = (int)c8 * 8;
  uint4 raw[K];
#pragma unroll
  for (int i = 0; i < K - 1; ++i)
    raw[i] = *reinterpret_cast<const uint4*>(a.s_in + b * a.s_sb + (int64_t)(i + 1) * a.s_cs + d);
  raw[K - 1] = *reinterpret_cast<const uint4*>(a.x + b * a.x_sb + d);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < K; ++i) {
    float c[8], wf[8];
    unpack8(raw[i], c);
    unpack8(*reinterpret_cast<const uint4*>(a.w + (int64_t)i * a.w_cs + d), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += c[e] * wf[e];
  }
#pragma unroll
  for (int i = 0; i < K; ++i)
    *reinterpret_cast<uint4*>(a.s_out + b * a.s_sb + (int64_t)i * a.s_cs + d) = raw[i];
  if (a.bias) {
    float bf8[8];
    unpack8(*reinterpret_cast<const uint4*>(a.bias + d), bf8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += bf8[e];
  }
  if (a.act) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = accurate_silu(acc[e]);
  }
  *reinterpret_cast<uint4*>(a.y + b * a.y_sb + d) = pack8(acc);
}

// ---- linear! + causal_conv1d! (the decode step's in-projection and conv,
// qwen35.jl:212-223) from the projection's stream-K partials (gemv_sk_kernel,
// step.hip): thread = 8 channels of one sequence. Each thread adds its rows'
// partials in workgroup order, stores them rounded to bf16 as the projection's
// output (every channel: the conv's input, z, alpha, beta), and for the first
// D channels runs the conv step of conv1d_update_kernel on that bf16 input.
template <int K>
__global__ __launch_bounds__(256) void conv1d_update_sk_kernel(Conv1dSkArgs a) {
  const Conv1dArgs& c = a.c;
  const int64_t c8 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int b = blockIdx.y;
  if (c8 * 8 >= a.M) return;
  const int d = (int)c8 * 8;
  const float4 lo = gemv_sk_sum4(a.part, a.G, a.chunk, d, b);
  const float4 hi = gemv_sk_sum4(a.part, a.G, a.chunk, d + 4, b);
  const float s8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  const uint4 xr = pack8(s8);
  *reinterpret_cast<uint4*>(a.yp + b * a.yp_sb + d) = xr;
  if (d >= c.D) return;
  uint4 raw[K];
#pragma unroll
  for (int i = 0; i < K - 1; ++i)
    raw[i] = *reinterpret_cast<const uint4*>(c.s_in + b * c.s_sb + (int64_t)(i + 1) * c.s_cs + d);
  raw[K - 1] = xr;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < K; ++i) {
    float v[8], wf[8];
    unpack8(raw[i], v);
    unpack8(*reinterpret_cast<const uint4*>(c.w + (int64_t)i * c.w_cs + d), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e] * wf[e];
  }
#pragma unroll
  for (int i = 0; i < K; ++i)
    *reinterpret_cast<uint4*>(c.s_out + b * c.s_sb + (int64_t)i * c.s_cs + d) = raw[i];
  if (c.bias) {
    float bf8[8];
    unpack8(*reinterpret_cast<const uint4*>(c.bias + d), bf8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += bf8[e];
  }
  if (c.act) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = accurate_silu(acc[e]);
  }
  *reinterpret_cast<uint4*>(c.y + b * c.y_sb + d) = pack8(acc);
}

// ---- causal_conv1d_sequence! (causal_conv1d.jl:73-149): thread = 8 channels x
// a run of CONV_TC tokens of one sequence, the window of the last K inputs in
// registers. The left context of token 0 is the ring's columns 2..K (s_in:
// the suffix prefill of qwen35.jl:333-344) or zeros. Only the threads of run 0
// read s_in (CONV_TC >= K - 1), and they also write the seeded ring (the last
// K inputs of the context-extended sequence) after reading, so s_out may alias
// s_in.
namespace {
template <int K>
__device__ __forceinline__ uint4 conv_ext(const Conv1dArgs& a, int b, int d, int t) {
  // ext(t), t in [-(K-1), T): x[t] for t >= 0, else ring column K + t (0-based)
  if (t >= 0) return *reinterpret_cast<const uint4*>(a.x + b * a.x_sb + (int64_t)t * a.x_st + d);
  if (a.s_in)
    return *reinterpret_cast<const uint4*>(a.s_in + b * a.s_sb + (int64_t)(K + t) * a.s_cs + d);
  return make_uint4(0, 0, 0, 0);
}
}  // namespace

template <int K>
__global__ __launch_bounds__(256) void conv1d_sequence_kernel(Conv1dArgs a) {
  static_assert(CONV_TC >= K - 1, "run 0 must cover the context reads");
  const int64_t c8 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int run = blockIdx.y, b = blockIdx.z;
  if (c8 * 8 >= a.D) return;
  const int d = (int)c8 * 8;
  const int t0 = run * CONV_TC;
  const int t1 = min(t0 + CONV_TC, a.T);
  float wf[K][8];
#pragma unroll
  for (int i = 0; i < K; ++i)
    unpack8(*reinterpret_cast<const uint4*>(a.w + (int64_t)i * a.w_cs + d), wf[i]);
  float bias8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (a.bias) unpack8(*reinterpret_cast<const uint4*>(a.bias + d), bias8);
  float win[K][8];  // win[i] = ext(t - K + 1 + i) for the current t
#pragma unroll
  for (int i = 0; i < K - 1; ++i) unpack8(conv_ext<K>(a, b, d, t0 - K + 1 + i), win[i]);
  for (int t = t0; t < t1; ++t) {
    unpack8(conv_ext<K>(a, b, d, t), win[K - 1]);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < K; ++i) v += win[i][e] * wf[i][e];
      v += bias8[e];
      acc[e] = a.act ? accurate_silu(v) : v;
    }
    *reinterpret_cast<uint4*>(a.y + b * a.y_sb + (int64_t)t * a.y_st + d) = pack8(acc);
#pragma unroll
    for (int i = 0; i + 1 < K; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = win[i + 1][e];
  }
  if (run == 0 && a.s_out) {
    uint4 seed[K];  // column i = ext(T - K + i); every column read first (aliasing)
#pragma unroll
    for (int i = 0; i < K; ++i) seed[i] = conv_ext<K>(a, b, d, a.T - K + i);
#pragma unroll
    for (int i = 0; i < K; ++i)
      *reinterpret_cast<uint4*>(a.s_out + b * a.s_sb + (int64_t)i * a.s_cs + d) = seed[i];
  }
}

// ---- the prefill's conv and prep in one pass (qwen35.jl:333-356): thread = 8
// channels x a run of CONV_TC tokens as in conv1d_sequence_kernel, the 16
// lanes of a head's 128 channels in one 16-lane group. Per token the conv
// output is rounded to bf16 (the value the two-kernel form stores between the
// kernels), then each q / k head row is scaled by its inverse L2 norm (q also
// by Dk^-1/2) over the group, and the row is written fp32 to Q / K / V, head
// major, as deltanet_prep_vec_kernel writes it: bit for bit the two-kernel
// result, without the conv output's round trip through memory. Workgroup
// column 0 also writes beta and the gate of its run's tokens.
template <int K>
__global__ __launch_bounds__(256) void deltanet_conv_prep_kernel(ConvPrepArgs a) {
  static_assert(CONV_TC >= K - 1, "run 0 must cover the context reads");
  const Conv1dArgs& c = a.c;
  const DeltaPrepArgs& p = a.p;
  const int run = blockIdx.y, b = blockIdx.z;
  const int t0 = run * CONV_TC;
  const int t1 = min(t0 + CONV_TC, c.T);
  if (blockIdx.x == 0) {
    const uint16_t* ab = p.ab + (int64_t)b * p.ab_sb;
    for (int i = threadIdx.x; i < (t1 - t0) * p.Hv; i += 256) {
      const int t = t0 + i / p.Hv, hv = i % p.Hv;
      const int64_t gi = ((int64_t)b * p.T + t) * p.Hv + hv;
      p.beta[gi] = accurate_sigmoid(bf2f(ab[(int64_t)t * p.ab_st + p.Hv + hv]));
      p.gate[gi] = -expf(p.a_log[hv]) * log1pf(expf(bf2f(ab[(int64_t)t * p.ab_st + hv]) + p.dt_bias[hv]));
    }
  }
  const int64_t c8 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c8 * 8 >= c.D) return;  // whole heads: a 16-lane group is all in or all out
  const int d = (int)c8 * 8;
  const int hh = d / DN_D, dc = d % DN_D;
  float* dst;  // this lane's 8 columns of head hh, token 0
  if (hh < p.Hk)
    dst = p.qe + ((int64_t)b * p.Hk + hh) * p.T * DN_D + dc;
  else if (hh < 2 * p.Hk)
    dst = p.ke + ((int64_t)b * p.Hk + hh - p.Hk) * p.T * DN_D + dc;
  else
    dst = p.ve + ((int64_t)b * p.Hv + hh - 2 * p.Hk) * p.T * DN_D + dc;
  const bool qk = hh < 2 * p.Hk;
  const float sc = hh < p.Hk ? 1.0f / sqrtf((float)DN_D) : 1.0f;
  float wf[K][8];
#pragma unroll
  for (int i = 0; i < K; ++i)
    unpack8(*reinterpret_cast<const uint4*>(c.w + (int64_t)i * c.w_cs + d), wf[i]);
  float bias8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (c.bias) unpack8(*reinterpret_cast<const uint4*>(c.bias + d), bias8);
  float win[K][8];  // win[i] = ext(t - K + 1 + i) for the current t
#pragma unroll
  for (int i = 0; i < K - 1; ++i) unpack8(conv_ext<K>(c, b, d, t0 - K + 1 + i), win[i]);
  for (int t = t0; t < t1; ++t) {
    unpack8(conv_ext<K>(c, b, d, t), win[K - 1]);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < K; ++i) v += win[i][e] * wf[i][e];
      v += bias8[e];
      acc[e] = c.act ? accurate_silu(v) : v;
    }
    float x[8];
    unpack8(pack8(acc), x);  // the conv output, bf16
    float den = 1.0f;
    if (qk) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
      ss += xor32<8>(ss);
      ss += xor32<4>(ss);
      ss += xor32<2>(ss);
      ss += xor32<1>(ss);
      den = sqrtf(ss + 1e-6f);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = x[j] / den * sc;
    float4* d4 = reinterpret_cast<float4*>(dst + (int64_t)t * DN_D);
    d4[0] = make_float4(x[0], x[1], x[2], x[3]);
    d4[1] = make_float4(x[4], x[5], x[6], x[7]);
#pragma unroll
    for (int i = 0; i + 1 < K; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) win[i][e] = win[i + 1][e];
  }
  if (run == 0 && c.s_out) {
    uint4 seed[K];  // column i = ext(T - K + i); every column read first (aliasing)
#pragma unroll
    for (int i = 0; i < K; ++i) seed[i] = conv_ext<K>(c, b, d, c.T - K + i);
#pragma unroll
    for (int i = 0; i < K; ++i)
      *reinterpret_cast<uint4*>(c.s_out + b * c.s_sb + (int64_t)i * c.s_cs + d) = seed[i];
  }
}

// ---- launchers -----------------------------------------------------------
hipError_t launch_deltanet_fused_decode(const DeltaFusedArgs& a, hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  hipLaunchKernelGGL(deltanet_fused_decode_kernel, dim3(a.Hv, a.B), dim3(256), 0, st, a);
  return hipGetLastError();
}

#define VM_CONV_K_CASES(X) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8)

hipError_t launch_deltanet_decode_sk(const DeltaDecodeSkArgs& a, hipStream_t st) {
  if (a.f.B == 0) return hipSuccess;
  const int R = a.f.Hv / a.f.Hk;
  const dim3 grid(a.f.Hk, a.f.B);
#define DN_SK(kc, r) hipLaunchKernelGGL((deltanet_decode_sk_kernel<kc, r>), grid, dim3(256 * r), 0, st, a)
#define X(kc)                              \
  case kc:                                 \
    if (R == 1) DN_SK(kc, 1);              \
    else if (R == 2) DN_SK(kc, 2);         \
    else if (R == 4) DN_SK(kc, 4);         \
    else return hipErrorInvalidValue;      \
    break;
  switch (a.c.K) {
    VM_CONV_K_CASES(X)
    default: return hipErrorInvalidValue;
  }
#undef X
#undef DN_SK
  return hipGetLastError();
}

hipError_t launch_deltanet_sequence(const DeltaSeqArgs& a, hipStream_t st) {
  if (a.B == 0 || a.T == 0) {
    if (a.B > 0 && a.s_out != a.s_in)  // T = 0: the state passes through
      return hipMemcpyAsync(a.s_out, a.s_in, (size_t)a.B * a.Hv * DN_D * DN_D * sizeof(float),
                            hipMemcpyDeviceToDevice, st);
    return hipSuccess;
  }
  // few blocks (small B * Hv): 16 waves per head (NI = 4), else 4 (NI = 16)
  if ((int64_t)a.B * a.Hv >= 512) {
    hipLaunchKernelGGL(deltanet_sequence_kernel<16>, dim3(1, a.Hv, a.B), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL(deltanet_sequence_kernel<4>, dim3(4, a.Hv, a.B), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

size_t deltanet_chunk_workspace_bytes(int T, int Hv, int B) {
  const int NC = (T + DC - 1) / DC;  // each per (b, hv): the units (+ the identity), S_0, delta
  return (size_t)((dn_units_floats(NC) + dn_s0_floats(NC) + dn_dl_floats(NC)) * Hv * B) *
         sizeof(float);
}

hipError_t launch_deltanet_sequence_chunked(const DeltaChunkArgs& a, hipStream_t st) {
  const DeltaSeqArgs& q = a.s;
  if (q.B == 0 || q.T == 0) return launch_deltanet_sequence(q, st);  // state copy / no-op
  const int NC = (q.T + DC - 1) / DC;
  hipLaunchKernelGGL(deltanet_chunk_kernel, dim3(NC, q.Hv, q.B), dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(deltanet_scan_kernel, dim3(q.Hv * q.B * (DN_D / CBW)), dim3(256), 0, st, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.g.y)
    hipLaunchKernelGGL(deltanet_out_kernel<true>, dim3(NC, q.Hv, q.B), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(deltanet_out_kernel<false>, dim3(NC, q.Hv, q.B), dim3(256), 0, st, a);
  return hipGetLastError();
}

namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

hipError_t launch_deltanet_prep(const DeltaPrepArgs& a, hipStream_t st) {
  const int64_t toks = (int64_t)a.B * a.T;
  if (toks == 0) return hipSuccess;
  if (al16(a.cv) && a.cv_st % 8 == 0 && a.cv_sb % 8 == 0 && al16(a.qe) && al16(a.ke) && al16(a.ve)) {
    hipLaunchKernelGGL(deltanet_prep_vec_kernel, dim3((unsigned)((toks + 3) / 4)), dim3(256), 0, st, a);
  } else {
    const int64_t waves = toks * (2 * a.Hk + a.Hv);
    hipLaunchKernelGGL(deltanet_prep_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_gated_rms_norm(const GatedNormArgs& a, hipStream_t st) {
  const int64_t toks = (int64_t)a.B * a.T;
  if (toks == 0 || a.Hv == 0) return hipSuccess;
  if (al16(a.o) && al16(a.z) && al16(a.y) && al16(a.norm_w) && a.z_st % 8 == 0 && a.z_sb % 8 == 0 &&
      a.y_st % 8 == 0 && a.y_sb % 8 == 0) {
    hipLaunchKernelGGL(gated_rms_norm_vec_kernel, dim3((unsigned)((toks + 3) / 4)), dim3(256), 0, st, a);
  } else {
    const int64_t waves = toks * a.Hv;
    hipLaunchKernelGGL(gated_rms_norm_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}


hipError_t launch_conv1d_update(const Conv1dArgs& a, hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.D / 8 + 255) / 256), a.B);
  switch (a.K) {
#define X(k) \
  case k: hipLaunchKernelGGL(conv1d_update_kernel<k>, grid, dim3(256), 0, st, a); break;
    VM_CONV_K_CASES(X)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_conv1d_update_sk(const Conv1dSkArgs& a, hipStream_t st) {
  if (a.c.B == 0 || a.M == 0) return hipSuccess;
  const dim3 grid((unsigned)((a.M / 8 + 255) / 256), a.c.B);
  switch (a.c.K) {
#define X(k) \
  case k: hipLaunchKernelGGL(conv1d_update_sk_kernel<k>, grid, dim3(256), 0, st, a); break;
    VM_CONV_K_CASES(X)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_deltanet_conv_prep(const ConvPrepArgs& a, hipStream_t st) {
  if (a.c.B == 0 || a.c.T == 0) return hipSuccess;
  const int runs = (a.c.T + CONV_TC - 1) / CONV_TC;
  const dim3 grid((unsigned)((a.c.D / 8 + 255) / 256), runs, a.c.B);
  switch (a.c.K) {
#define X(k) \
  case k: hipLaunchKernelGGL(deltanet_conv_prep_kernel<k>, grid, dim3(256), 0, st, a); break;
    VM_CONV_K_CASES(X)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_conv1d_sequence(const Conv1dArgs& a, hipStream_t st) {
  if (a.B == 0 || a.T == 0) return hipSuccess;
  const int runs = (a.T + CONV_TC - 1) / CONV_TC;
  const dim3 grid((unsigned)((a.D / 8 + 255) / 256), runs, a.B);
  switch (a.K) {
#define X(k) \
  case k: hipLaunchKernelGGL(conv1d_sequence_kernel<k>, grid, dim3(256), 0, st, a); break;
    VM_CONV_K_CASES(X)
#undef X
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace vm

// generic.hip — the attention operators at head shapes outside the tuned
// kernels: qnorm_rope! and knorm_rope_append! (src/kernels/qknorm_rope_append.jl:
// 100-141), attention! (src/kernels/attention.jl:93-129) and decode_attention!
// (src/kernels/attention_decode.jl:134-200) for any power-of-two head dims from
// 16 to 512, Dk != Dv, any rotary half-width and any GQA group. The tuned
// kernels (rows.hip, prefill.hip, decode.hip) are built for Qwen3.5's head
// shape (D = 256, a 64-dim rotary part, groups up to 8; prefill.hip also
// D = 128 and 64); these take every other shape the reference's operators take. fp32 arithmetic on bf16 operands staged
// in LDS, one workgroup per 4 or 16 query rows: correct at any shape, not tuned.
// Likewise the DeltaNet operators (fused decode, recurrent decode, sequence)
// for Dk, Dv multiples of 16 up to 256 beside the tuned Dk = Dv = 128 kernels.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace vm {

namespace {

__device__ __forceinline__ float bfv(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

constexpr int AK = 32;  // keys per staged tile

}  // namespace

// ---- rows: one wave per (head, sequence) row; lane l holds d = l + 64 e. The
// rotate-half partner of d < 2 half is read raw and normed by the same lane, so
// every load of the row comes before its first store (Q is updated in place).
template <int E>
__global__ __launch_bounds__(256) void norm_rope_any_kernel(RowAnyArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)a.B * a.H) return;
  const int h = (int)(row % a.H), b = (int)(row / a.H);
  const int64_t pos = (int64_t)a.positions[b] - 1;
  if (pos < 0 || pos >= a.ctx) return;  // out-of-contract position: write nothing
  const uint16_t* src = a.in + b * a.in_sb + h * a.in_sh;
  uint16_t* dst = a.out + b * a.out_sb + h * a.out_sh + (a.out_at_pos ? pos * a.out_st : 0);
  const int D = a.D, half = a.half;
  float x[E], xp[E];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    x[e] = 0.f;
    xp[e] = 0.f;
    if (d < D) {
      x[e] = bfv(src[d]);
      if (d < 2 * half) xp[e] = bfv(src[d < half ? d + half : d - half]);
    }
    ss = fmaf(x[e], x[e], ss);
  }
  ss = wave_sum_all(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + a.eps);
  const float* cs = a.cos_tab + pos * half;
  const float* sn = a.sin_tab + pos * half;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int d = lane + 64 * e;
    if (d >= D) continue;
    float y = x[e] * r * (bfv(a.w[d]) + a.w_offset);
    if (d < 2 * half) {
      const bool first = d < half;
      const int i = first ? d : d - half;
      const float yp = xp[e] * r * (bfv(a.w[first ? d + half : d - half]) + a.w_offset);
      y = first ? y * cs[i] - yp * sn[i] : y * cs[i] + yp * sn[i];
    }
    dst[d] = f2bf(y);
  }
  if (a.in2) {  // V rides along: copied into the same cache column
    const uint16_t* s2 = a.in2 + b * a.in2_sb + h * a.in2_sh;
    uint16_t* d2 = a.out2 + b * a.out2_sb + h * a.out2_sh + pos * a.out2_st;
    for (int d = lane; d < a.D2; d += 64) d2[d] = s2[d];
  }
}

// ---- attention over staged tiles. Workgroup (row block, (b, kv head), split):
// rows rho = g L + t enumerate the group's G query heads x L queries, so the
// heads of a kv group share every staged K/V tile. A block holds RPB rows of
// TPR = 256 / RPB threads: RPB = 16 (16 threads per row, each scoring keys c
// and c + 16 of a 32-key tile over all of Dk) or, where a kv group has at most
// 4 rows (decode), RPB = 4 (64 threads per row, one wave: key c % 32 over half
// of Dk, the halves added across the wave). Each thread owns the output
// columns c + TPR i of its row. Online softmax per row over the row's threads.
// With part set (decode splits) it writes the unnormalised row, its max and
// its sum instead.
template <int RPB, int DVT, bool PREF>
__global__ __launch_bounds__(256) void attn_any_kernel(AttnAnyArgs a) {
  constexpr int TPR = 256 / RPB;                 // threads per row
  constexpr int KPT = TPR >= AK ? 1 : AK / TPR;  // keys scored per thread
  constexpr int DP = TPR >= AK ? TPR / AK : 1;   // parts of Dk per key
  constexpr int RX = (TPR < AK ? TPR : AK) / 2;  // first xor of the row reductions
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int Dk = a.Dk, Dv = a.Dv;
  const int qs_st = Dk + 4;  // floats per staged Q row (rows on distinct banks)
  const int ks_st = Dk + 8;  // bf16 per staged K row (the keys a row group reads: distinct banks)
  const int vs_st = Dv + 8;
  float* qs = reinterpret_cast<float*>(smem);
  uint16_t* ks = reinterpret_cast<uint16_t*>(qs + RPB * qs_st);
  uint16_t* vs = ks + AK * ks_st;
  float* ps = reinterpret_cast<float*>(vs + AK * vs_st);  // [RPB][AK + 1]
  const int G = a.H / a.Hk;
  const int hk = blockIdx.y % a.Hk, b = blockIdx.y / a.Hk, z = blockIdx.z;
  const int rows = G * a.L, rho0 = blockIdx.x * RPB;
  const int tid = threadIdx.x, r = tid / TPR, c = tid % TPR;
  const int k_len = min(a.k_lengths ? a.k_lengths[b] : a.Lk, a.Lk);
  const int q_len = min(a.q_lengths ? a.q_lengths[b] : a.L, a.L);
  const int off = k_len - q_len;  // queries are the suffix of the keys
  const int rho = rho0 + r;
  const int g = rho / a.L, t = rho % a.L;
  const bool active = rho < rows && t < q_len;
  const int h = hk * G + g;
  // the block's key range: this split's keys, up to its last row's causal limit
  int tmax = -1;
  for (int i = 0; i < RPB; ++i) {
    const int rr = rho0 + i;
    if (rr < rows && rr % a.L < q_len) tmax = max(tmax, rr % a.L);
  }
  if (tmax < 0 && a.part == nullptr) return;  // no row of this block is written
  const int kb0 = (int)min((int64_t)z * a.split_keys, (int64_t)k_len);
  int kb1 = (int)min((int64_t)kb0 + a.split_keys, (int64_t)k_len);
  if (a.causal) kb1 = min(kb1, max(kb0, off + tmax + 1));
  const int lim = a.causal ? min(kb1 - 1, t + off) : kb1 - 1;  // this row's last key
  // Q rows of the block, fp32
  for (int i = tid; i < RPB * Dk; i += 256) {
    const int rr = i / Dk, d = i % Dk, q_rho = rho0 + rr;
    float v = 0.f;
    if (q_rho < rows) {
      const int qg = q_rho / a.L, qt = q_rho % a.L;
      v = bfv(a.q[b * a.q_sb + (int64_t)(hk * G + qg) * a.q_sh + (int64_t)qt * a.q_st + d]);
    }
    qs[rr * qs_st + d] = v;
  }
  float m = -INFINITY, l = 0.f, acc[DVT];
#pragma unroll
  for (int i = 0; i < DVT; ++i) acc[i] = 0.f;
  const uint16_t* kbase = a.k + b * a.k_sb + (int64_t)hk * a.k_sh;
  const uint16_t* vbase = a.v + b * a.v_sb + (int64_t)hk * a.v_sh;
  const int key0 = c % AK, dpart = c / AK;    // DP > 1: this thread's key and Dk part
  // the thread's output columns c + TPR i: Dv is TPR * DVT, or (DVT = 1) less
  // than TPR, where threads c >= Dv own none (they read column 0, store nothing)
  const bool col_ok = c < Dv;
  const int dlen = Dk / DP, dbeg = DP > 1 ? dpart * dlen : 0;
  // PREF (decode, bound by its loads): the tiles go through registers, one tile
  // ahead: thread tid holds 16-byte chunks tid + 256 n of the tile's K (then V)
  // rows, n < Dk / 64 (Dv / 64). Otherwise each tile is loaded after the
  // barrier (fewer registers, more workgroups per CU for the products).
  const int kc8 = Dk / 8, vc8 = Dv / 8;
  constexpr int NPF = PREF ? 8 : 1;
  uint4 kr[NPF], vr8[NPF];
  auto fetch = [&](int j0) {
#pragma unroll
    for (int n = 0; n < NPF; ++n) {
      const int i = tid + 256 * n;
      kr[n] = make_uint4(0u, 0u, 0u, 0u);
      vr8[n] = make_uint4(0u, 0u, 0u, 0u);
      if (i < AK * kc8) {
        const int j = j0 + i / kc8;
        if (j < kb1) kr[n] = *reinterpret_cast<const uint4*>(kbase + (int64_t)j * a.k_st + 8 * (i % kc8));
      }
      if (i < AK * vc8) {
        const int j = j0 + i / vc8;
        if (j < kb1) vr8[n] = *reinterpret_cast<const uint4*>(vbase + (int64_t)j * a.v_st + 8 * (i % vc8));
      }
    }
  };
  if constexpr (PREF) {
    if (kb0 < kb1) fetch(kb0);
  }
  for (int j0 = kb0; j0 < kb1; j0 += AK) {
    __syncthreads();  // the previous tile's reads are done (and Q is staged)
    if constexpr (PREF) {
#pragma unroll
      for (int n = 0; n < NPF; ++n) {
        const int i = tid + 256 * n;
        if (i < AK * kc8) *reinterpret_cast<uint4*>(ks + (i / kc8) * ks_st + 8 * (i % kc8)) = kr[n];
        if (i < AK * vc8) *reinterpret_cast<uint4*>(vs + (i / vc8) * vs_st + 8 * (i % vc8)) = vr8[n];
      }
      if (j0 + AK < kb1) fetch(j0 + AK);  // in flight during this tile's products
    } else {
      for (int i = tid; i < AK * kc8; i += 256) {
        const int key = i / kc8, ch = i % kc8, j = j0 + key;
        uint4 u = make_uint4(0u, 0u, 0u, 0u);
        if (j < kb1) u = *reinterpret_cast<const uint4*>(kbase + (int64_t)j * a.k_st + 8 * ch);
        *reinterpret_cast<uint4*>(ks + key * ks_st + 8 * ch) = u;
      }
      for (int i = tid; i < AK * vc8; i += 256) {
        const int key = i / vc8, ch = i % vc8, j = j0 + key;
        uint4 u = make_uint4(0u, 0u, 0u, 0u);
        if (j < kb1) u = *reinterpret_cast<const uint4*>(vbase + (int64_t)j * a.v_st + 8 * ch);
        *reinterpret_cast<uint4*>(vs + key * vs_st + 8 * ch) = u;
      }
    }
    __syncthreads();
    // scores: keys key0 + TPR x (x < KPT) over dims dbeg .. dbeg + dlen - 1
    float sc[KPT];
    const uint32_t* kp[KPT];
    const float* qr = qs + r * qs_st + dbeg;
#pragma unroll
    for (int x = 0; x < KPT; ++x) {
      sc[x] = 0.f;
      kp[x] = reinterpret_cast<const uint32_t*>(ks + (DP > 1 ? key0 : c + TPR * x) * ks_st + dbeg);
    }
    for (int d2 = 0; d2 < dlen / 2; ++d2) {
      const float qa = qr[2 * d2], qb = qr[2 * d2 + 1];  // one q read for the thread's keys
#pragma unroll
      for (int x = 0; x < KPT; ++x) {
        const uint32_t u = kp[x][d2];
        sc[x] = fmaf(qa, bf_lo(u), sc[x]);
        sc[x] = fmaf(qb, bf_hi(u), sc[x]);
      }
    }
    if (DP > 1) {
#pragma unroll
      for (int x = 0; x < KPT; ++x) sc[x] += __shfl_xor(sc[x], AK, 64);  // the other half of Dk
    }
    float bm = -INFINITY;
#pragma unroll
    for (int x = 0; x < KPT; ++x) {
      const int key = DP > 1 ? key0 : c + TPR * x;
      sc[x] = active && j0 + key <= lim ? sc[x] * a.scale : -INFINITY;
      bm = fmaxf(bm, sc[x]);
    }
#pragma unroll
    for (int x = RX; x >= 1; x >>= 1) bm = fmaxf(bm, __shfl_xor(bm, x, 64));
    const float mn = fmaxf(m, bm);
    float corr = 1.f, ls = 0.f;
#pragma unroll
    for (int x = 0; x < KPT; ++x) {
      const float p = mn != -INFINITY ? expf(sc[x] - mn) : 0.f;
      ls += p;
      sc[x] = p;
    }
    if (mn != -INFINITY) corr = expf(m - mn);  // 0 while m is still -inf
#pragma unroll
    for (int x = RX; x >= 1; x >>= 1) ls += __shfl_xor(ls, x, 64);
    l = l * corr + ls;
    m = mn;
    if (DP == 1 || dpart == 0) {
#pragma unroll
      for (int x = 0; x < KPT; ++x) ps[r * (AK + 1) + (DP > 1 ? key0 : c + TPR * x)] = sc[x];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < DVT; ++i) acc[i] *= corr;
    for (int kk = 0; kk < AK; ++kk) {
      const float p = ps[r * (AK + 1) + kk];
      const uint16_t* vr = vs + kk * vs_st + (col_ok ? c : 0);
#pragma unroll
      for (int i = 0; i < DVT; ++i) acc[i] = fmaf(p, bfv(vr[TPR * i]), acc[i]);
    }
  }
  if (!active) return;
  if (a.part == nullptr) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;  // no key: o = 0 (attention.jl:86)
    uint16_t* orow = a.o + b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)t * a.o_st;
    if (col_ok) {
#pragma unroll
      for (int i = 0; i < DVT; ++i) orow[c + TPR * i] = f2bf(acc[i] * inv);
    }
  } else {
    float* pr = a.part + (((int64_t)z * a.B + b) * a.H + h) * (Dv + 2);
    if (col_ok) {
#pragma unroll
      for (int i = 0; i < DVT; ++i) pr[c + TPR * i] = acc[i];
    }
    if (c == 0) {
      pr[Dv] = m;
      pr[Dv + 1] = l;
    }
  }
}

// The decode splits merged per (b, head), in split order
// (attention_decode.jl:85-132): o = sum_z e^(m_z - m) acc_z / sum_z e^(m_z - m) l_z.
__global__ __launch_bounds__(256) void attn_any_combine_kernel(AttnAnyArgs a) {
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int Dv = a.Dv;
  const int64_t zst = (int64_t)a.B * a.H * (Dv + 2);
  const float* p0 = a.part + ((int64_t)b * a.H + h) * (Dv + 2);
  float mx = -INFINITY;
  for (int z = 0; z < a.n_split; ++z) mx = fmaxf(mx, p0[z * zst + Dv]);
  float sum = 0.f;
  if (mx != -INFINITY)
    for (int z = 0; z < a.n_split; ++z) {
      const float mz = p0[z * zst + Dv];
      if (mz != -INFINITY) sum += p0[z * zst + Dv + 1] * expf(mz - mx);
    }
  const float inv = sum > 0.f ? 1.0f / sum : 0.f;
  uint16_t* orow = a.o + b * a.o_sb + (int64_t)h * a.o_sh;
  for (int d = threadIdx.x; d < Dv; d += 256) {
    float o = 0.f;
    if (mx != -INFINITY)
      for (int z = 0; z < a.n_split; ++z) {
        const float mz = p0[z * zst + Dv];
        if (mz != -INFINITY) o += p0[z * zst + d] * expf(mz - mx);
      }
    orow[d] = f2bf(o * inv);
  }
}

// ---- the DeltaNet operators at head dims outside the tuned kernels (Dk, Dv
// multiples of 16 up to 256; src/kernels/deltanet_fused.jl:109-141,
// deltanet_recurrent.jl:72-198 tile any Dk by 16). One workgroup of 16 waves
// per (value head, sequence): wave w owns value columns j0 .. j0 + nc - 1 (j0 =
// w nc, nc = Dv / 16) and keeps their state in registers, lane l rows l + 64 e.
// Per column: S *= decay, delta = beta (v - S^T k), S += k delta^T, o = S^T q
// (the reference's two passes in one: every state element is read and written
// once per step).
namespace {

constexpr int DN_NC = 16;  // columns per wave at Dv = 256

template <int KE, int NC>
__device__ __forceinline__ void dn_any_load(float (&s)[DN_NC][KE], const float* base, int Dk,
                                            int j0, int nc, int lane) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      const int i = lane + 64 * e;
      s[c][e] = c < nc && i < Dk ? base[(int64_t)(j0 + c) * Dk + i] : 0.f;
    }
  }
}
template <int KE, int NC>
__device__ __forceinline__ void dn_any_store(const float (&s)[DN_NC][KE], float* base, int Dk,
                                             int j0, int nc, int lane) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      const int i = lane + 64 * e;
      if (c < nc && i < Dk) base[(int64_t)(j0 + c) * Dk + i] = s[c][e];
    }
  }
}
// one delta step on the wave's NC columns (NC a power of two >= the wave's
// columns; the extra ones hold zeros and are never stored), in phases so that
// the columns' independent cross-lane sums overlap; vv: lane c holds v of
// column j0 + c; o[c] (every lane) the column's output
template <int KE, int NC>
__device__ __forceinline__ void dn_any_step(float (&s)[DN_NC][KE], const float (&k)[KE],
                                            const float (&q)[KE], float vv, float decay,
                                            float beta, float (&o)[DN_NC]) {
  float ks[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    ks[c] = 0.f;
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      s[c][e] *= decay;
      ks[c] = fmaf(s[c][e], k[e], ks[c]);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
    for (int c = 0; c < NC; ++c) ks[c] += __shfl_xor(ks[c], m, 64);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float delta = beta * (__shfl(vv, c, 64) - ks[c]);
    float os = 0.f;
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      s[c][e] = fmaf(k[e], delta, s[c][e]);
      os = fmaf(s[c][e], q[e], os);
    }
    o[c] = os;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
    for (int c = 0; c < NC; ++c) o[c] += __shfl_xor(o[c], m, 64);
}
// lane c's copy of o[c] (registers are not indexable by lane)
template <int NC>
__device__ __forceinline__ float dn_pick(const float (&o)[DN_NC], int lane) {
  float r = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) r = lane == c ? o[c] : r;
  return r;
}

}  // namespace

// deltanet_sequence! and, at T = 1, deltanet_recurrent_decode!: fp32 inputs
// already normed and gated (decay = exp(gate)), the state carried in registers
template <int KE, int NC>
__global__ __launch_bounds__(1024) void deltanet_any_seq_kernel(DeltaSeqArgs a, int Dk, int Dv) {
  const int hv = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nc = Dv / 16, j0 = w * nc;
  const int hk = hv / (a.Hv / a.Hk);
  const int64_t sb = ((int64_t)b * a.Hv + hv) * Dv * Dk;
  float s[DN_NC][KE], o[DN_NC] = {};
  dn_any_load<KE, NC>(s, a.s_in + sb, Dk, j0, nc, lane);
  for (int t = 0; t < a.T; ++t) {
    const int64_t qk = (((int64_t)b * a.Hk + hk) * a.T + t) * Dk;
    const int64_t vo = (((int64_t)b * a.Hv + hv) * a.T + t) * Dv;
    const int64_t g = ((int64_t)b * a.T + t) * a.Hv + hv;
    float q[KE], k[KE];
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      const int i = lane + 64 * e;
      q[e] = i < Dk ? a.q[qk + i] : 0.f;
      k[e] = i < Dk ? a.k[qk + i] : 0.f;
    }
    const float vv = lane < nc ? a.v[vo + j0 + lane] : 0.f;
    dn_any_step<KE, NC>(s, k, q, vv, expf(a.gate[g]), a.beta[g], o);
    if (lane < nc) a.o[vo + j0 + lane] = dn_pick<NC>(o, lane);
  }
  dn_any_store<KE, NC>(s, a.s_out + sb, Dk, j0, nc, lane);
}

// fused_deltanet_decode!: raw bf16 q, k (l2-normed here, q also by 1/sqrt(Dk)),
// the gates from alpha and beta_raw, then the gated RMSNorm with silu(z)
// (deltanet_fused.jl:27-105)
template <int KE, int NC>
__global__ __launch_bounds__(1024) void deltanet_any_fused_kernel(DeltaFusedArgs a, int Dk, int Dv) {
  const int hv = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int nc = Dv / 16, j0 = w * nc;
  const int hk = hv / (a.Hv / a.Hk);
  const int64_t sb = ((int64_t)b * a.Hv + hv) * Dv * Dk;
  float s[DN_NC][KE], o[DN_NC] = {};
  dn_any_load<KE, NC>(s, a.s_in + sb, Dk, j0, nc, lane);
  float q[KE], k[KE], qss = 0.f, kss = 0.f;
#pragma unroll
  for (int e = 0; e < KE; ++e) {
    const int i = lane + 64 * e;
    q[e] = i < Dk ? bfv(a.q[b * a.q_sb + (int64_t)hk * Dk + i]) : 0.f;
    k[e] = i < Dk ? bfv(a.k[b * a.k_sb + (int64_t)hk * Dk + i]) : 0.f;
    qss = fmaf(q[e], q[e], qss);
    kss = fmaf(k[e], k[e], kss);
  }
  qss = wave_sum_all(qss);
  kss = wave_sum_all(kss);
  const float qsc = 1.0f / sqrtf(qss + 1e-6f) / sqrtf((float)Dk);
  const float ksc = 1.0f / sqrtf(kss + 1e-6f);
#pragma unroll
  for (int e = 0; e < KE; ++e) {
    q[e] *= qsc;
    k[e] *= ksc;
  }
  const float spi = bfv(a.alpha[b * a.a_sb + hv]) + a.dt_bias[hv];
  const float sp = spi > 20.0f ? spi : logf(1.0f + expf(spi));
  const float decay = expf(-expf(a.a_log[hv]) * sp);
  const float beta = accurate_sigmoid(bfv(a.beta[b * a.b_sb + hv]));
  const float vv = lane < nc ? bfv(a.v[b * a.v_sb + (int64_t)hv * Dv + j0 + lane]) : 0.f;
  dn_any_step<KE, NC>(s, k, q, vv, decay, beta, o);
  dn_any_store<KE, NC>(s, a.s_out + sb, Dk, j0, nc, lane);
  // gated RMSNorm over the Dv columns
  __shared__ float red[16];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) ss = fmaf(o[c], o[c], ss);  // columns past nc hold 0
  if (lane == 0) red[w] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < 16; ++i) tot += red[i];
  const float rstd = 1.0f / sqrtf(tot / (float)Dv + a.eps);
  if (lane < nc) {
    const int j = j0 + lane;
    const float z = bfv(a.z[b * a.z_sb + (int64_t)hv * Dv + j]);
    a.o[b * a.o_sb + (int64_t)hv * Dv + j] =
        f2bf(dn_pick<NC>(o, lane) * rstd * bfv(a.norm_w[j]) * accurate_silu(z));
  }
}

// ---- launchers ---------------------------------------------------------------
hipError_t launch_norm_rope_any(const RowAnyArgs& a, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H;
  if (rows == 0) return hipSuccess;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  switch (a.D <= 64 ? 1 : a.D / 64) {
    case 1: hipLaunchKernelGGL(norm_rope_any_kernel<1>, grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL(norm_rope_any_kernel<2>, grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL(norm_rope_any_kernel<4>, grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL(norm_rope_any_kernel<8>, grid, block, 0, st, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// rows per block: 4 where a kv group has at most 4 rows (decode at G <= 4), else 16
static int attn_any_rpb(const AttnAnyArgs& a) { return (a.H / a.Hk) * a.L <= 4 ? 4 : 16; }

static size_t attn_any_lds(int rpb, int Dk, int Dv) {
  return (size_t)rpb * (Dk + 4) * 4 + (size_t)AK * (Dk + 8) * 2 + (size_t)AK * (Dv + 8) * 2 +
         (size_t)rpb * (AK + 1) * 4;
}

int attn_any_splits(int B, int H, int Hk, int64_t ctx, int n_splits) {
  if (n_splits > 0) return n_splits;  // the reference's fixed split count
  const int G = H / Hk;
  const int rpb = G <= 4 ? 4 : 16;  // rows per workgroup at L = 1 (attn_any_rpb)
  const int64_t blocks = (int64_t)B * Hk * ((G + rpb - 1) / rpb);
  int64_t s = (1024 + blocks - 1) / blocks;  // about four workgroups per CU
  s = std::min<int64_t>(s, (ctx + 127) / 128);  // at least 128 keys per split
  return (int)std::max<int64_t>(1, s);
}

int attn_any_split_keys(int64_t ctx, int n_split) {
  // tile-aligned split boundaries (attention_decode.jl:159)
  const int64_t per = (ctx + n_split - 1) / n_split;
  return (int)std::max<int64_t>(AK, (per + AK - 1) / AK * AK);
}

template <int RPB, int DVT, bool PREF>
static hipError_t launch_attn_any_p(const AttnAnyArgs& a, dim3 grid, size_t lds, hipStream_t st) {
  if (lds > 65536) {  // lift the dynamic-LDS cap of the current device for this kernel
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&attn_any_kernel<RPB, DVT, PREF>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((attn_any_kernel<RPB, DVT, PREF>), grid, dim3(256), lds, st, a);
  return hipGetLastError();
}
// decode (split partials, one query per row) prefetches its tiles
template <int RPB, int DVT>
static hipError_t launch_attn_any_t(const AttnAnyArgs& a, dim3 grid, size_t lds, hipStream_t st) {
  return a.part ? launch_attn_any_p<RPB, DVT, true>(a, grid, lds, st)
                : launch_attn_any_p<RPB, DVT, false>(a, grid, lds, st);
}

hipError_t launch_attn_any(const AttnAnyArgs& a, hipStream_t st) {
  if (a.B == 0 || a.L == 0) return hipSuccess;
  const int G = a.H / a.Hk, rpb = attn_any_rpb(a);
  const dim3 grid((unsigned)((G * a.L + rpb - 1) / rpb), (unsigned)(a.Hk * a.B),
                  (unsigned)(a.part ? a.n_split : 1));
  const size_t lds = attn_any_lds(rpb, a.Dk, a.Dv);
  hipError_t e;
  if (rpb == 16) {
    switch (a.Dv / 16) {  // DVT = Dv / 16 columns per thread
      case 1: e = launch_attn_any_t<16, 1>(a, grid, lds, st); break;
      case 2: e = launch_attn_any_t<16, 2>(a, grid, lds, st); break;
      case 4: e = launch_attn_any_t<16, 4>(a, grid, lds, st); break;
      case 8: e = launch_attn_any_t<16, 8>(a, grid, lds, st); break;
      case 16: e = launch_attn_any_t<16, 16>(a, grid, lds, st); break;
      case 32: e = launch_attn_any_t<16, 32>(a, grid, lds, st); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (a.Dv <= 64 ? 1 : a.Dv / 64) {  // DVT = ceil(Dv / 64) columns per thread
      case 1: e = launch_attn_any_t<4, 1>(a, grid, lds, st); break;
      case 2: e = launch_attn_any_t<4, 2>(a, grid, lds, st); break;
      case 4: e = launch_attn_any_t<4, 4>(a, grid, lds, st); break;
      case 8: e = launch_attn_any_t<4, 8>(a, grid, lds, st); break;
      default: return hipErrorInvalidValue;
    }
  }
  if (e != hipSuccess || a.part == nullptr) return e;
  hipLaunchKernelGGL(attn_any_combine_kernel, dim3((unsigned)(a.B * a.H)), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_deltanet_any(const DeltaSeqArgs* seq, const DeltaFusedArgs* fused, int Dk,
                               int Dv, hipStream_t st) {
  const int B = seq ? seq->B : fused->B, Hv = seq ? seq->Hv : fused->Hv;
  if (B == 0) return hipSuccess;
  const dim3 grid((unsigned)Hv, (unsigned)B), block(1024);
  int ncp = 1;  // the wave's columns, rounded up to a power of two
  while (ncp < Dv / 16) ncp *= 2;
#define DN_ANY(ke, nc)                                                                       \
  if (seq)                                                                                   \
    hipLaunchKernelGGL((deltanet_any_seq_kernel<ke, nc>), grid, block, 0, st, *seq, Dk, Dv); \
  else                                                                                       \
    hipLaunchKernelGGL((deltanet_any_fused_kernel<ke, nc>), grid, block, 0, st, *fused, Dk, Dv);
#define DN_NCS(ke)                              \
  switch (ncp) {                                \
    case 1: DN_ANY(ke, 1); break;               \
    case 2: DN_ANY(ke, 2); break;               \
    case 4: DN_ANY(ke, 4); break;               \
    case 8: DN_ANY(ke, 8); break;               \
    case 16: DN_ANY(ke, 16); break;             \
    default: return hipErrorInvalidValue;       \
  }
  switch ((Dk + 63) / 64) {
    case 1: DN_NCS(1); break;
    case 2: DN_NCS(2); break;
    case 3: DN_NCS(3); break;
    case 4: DN_NCS(4); break;
    default: return hipErrorInvalidValue;
  }
#undef DN_NCS
#undef DN_ANY
  return hipGetLastError();
}

}  // namespace vm

// prefill.hip — causal / non-causal GQA flash attention for prefill and chunked
// prefill (the work of src/kernels/attention.jl:12-91, re-designed for CDNA4),
// optionally fused with the q norm+RoPE prologue and the sigmoid-gate epilogue
// of forward(::AttnLayer) (src/llm/qwen35.jl:292-318).
//
// Workgroup = 4 waves = 128 query rows of one (head, sequence); wave w owns 32
// rows. Per 32-key step, all on 32x32x16 bf16 MFMA with fp32 accumulate:
//   S^T[key][row] = K[key][:] . Q[row][:]     A = K (LDS, ds_read_b128),
//                                             B = Q (registers, loaded once)
//   O^T[d][row]  += V^T[d][key] . P^T[key][row]   A = V^T (LDS, ds_read_b64_tr_b16),
//                                             B = P^T (the S^T accumulator, in place)
// The S^T accumulator layout (lane l: row l%32, keys 8(j/4)+4(l/32)+j%4) is the
// P^T operand layout up to a key permutation, which the V^T transpose reads
// reproduce, so P never leaves registers. K/V tiles are double-buffered in LDS
// with a 544-byte row pitch (bank-conflict-free for both read patterns).
// Softmax is exp2-based with the running max rescaled lazily (only when it
// grows by > 8, keeping p <= 256), and the fully-masked-row guard of the
// reference (o = 0 when l = 0).
#include "common.h"
#include "kernels.h"

namespace vm {

constexpr int PF_BM = 128;     // query rows per workgroup
constexpr int PF_BN = 32;      // keys per step
constexpr int LDS_ROW = 272;   // bf16 per LDS row: 256 + 16 pad (544 B)
constexpr float RESCALE_SLACK = 8.0f;

template <bool QRAW, bool GATE, bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][PF_BN * LDS_ROW];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][PF_BN * LDS_ROW];

  // ---- work item: heaviest query tiles first; the query heads of one
  // kv head land on the same XCD (workgroup id mod 8) when H*B % 8 == 0.
  const int HB = a.H * a.B;
  const int lin = blockIdx.x;
  const int qt = a.n_qt - 1 - lin / HB;
  const int rem = lin % HB;
  const int hb = (HB & 7) == 0 ? (rem & 7) * (HB >> 3) + (rem >> 3) : rem;
  const int b = hb / a.H, h = hb % a.H;
  const int hk = h / (a.H / a.Hk);

  // q_len > L is out of contract; clamp so rows past the tensor are never written
  const int q_len = a.q_lengths ? min(a.q_lengths[b], a.L) : a.L;
  const int r0 = qt * PF_BM;
  if (r0 >= q_len) return;
  int k_len;
  if (a.prior) k_len = a.prior[b] + q_len;
  else k_len = a.k_lengths ? a.k_lengths[b] : a.Lk;
  const int off = k_len - q_len;  // queries are the suffix of keys
  const int kend = CAUSAL ? min(k_len, off + r0 + PF_BM) : k_len;
  const int n_tiles = kend > 0 ? (kend + PF_BN - 1) / PF_BN : 0;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h2 = lane >> 5;
  const int row = r0 + 32 * wave + l32;                 // query row in the chunk
  const int wrow0 = r0 + 32 * wave, wrow1 = wrow0 + 31;  // this wave's rows

  // ---- Q operand: lane holds q[row][16kk + 8*h2 + j], pre-scaled by 1/16.
  uint4 qop[16];
  {
    const int qrow = min(row, a.L - 1);
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                         (int64_t)qrow * a.q_st + 8 * h2;
    if (QRAW) {
      float x[16][8];
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) unpack8(load16(qp + 16 * kk), x[kk]);
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x[kk][j] * x[kk][j];
      ss += __shfl_xor(ss, 32, 64);
      const float r = 1.0f / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        float wf[8];
        unpack8(load16(a.qw + 16 * kk + 8 * h2), wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[kk][j] = x[kk][j] * r * (wf[j] + a.w_offset);
      }
      const int64_t pos = min((int64_t)(a.prior ? a.prior[b] : 0) + qrow, (int64_t)a.Lk - 1);
      const float* cs = a.cos_tab + pos * HALF_ROT + 8 * h2;
      const float* sn = a.sin_tab + pos * HALF_ROT + 8 * h2;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float c = cs[16 * kk + j], si = sn[16 * kk + j];
          const float x1 = x[kk][j], x2 = x[kk + 2][j];
          x[kk][j] = x1 * c - x2 * si;
          x[kk + 2][j] = x2 * c + x1 * si;
        }
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[kk][j] *= QK_SCALE;
        qop[kk] = pack8(x[kk]);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        float x[8];
        unpack8(load16(qp + 16 * kk), x);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] *= QK_SCALE;
        qop[kk] = pack8(x);
      }
    }
  }

  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[i][j] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;

  const uint16_t* kbase = a.k + (int64_t)b * a.kv_sb + (int64_t)hk * a.kv_sh;
  const uint16_t* vbase = a.v + (int64_t)b * a.kv_sb + (int64_t)hk * a.kv_sh;

  // global -> registers: thread owns 16-byte chunks c = tid + 256*i of the tile
  uint4 kreg[4], vreg[4];
  auto load_tile = [&](int jt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int key = jt * PF_BN + (c >> 5);
      const int64_t krow = min(key, a.Lk - 1);
      const int col = (c & 31) * 8;
      kreg[i] = load16(kbase + krow * a.kv_st + col);
      vreg[i] = load16(vbase + krow * a.kv_st + col);
      if (key >= k_len) vreg[i] = make_uint4(0, 0, 0, 0);  // p = 0 must meet finite v
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int off_l = (c >> 5) * LDS_ROW + (c & 31) * 8;
      *reinterpret_cast<uint4*>(&Ks[buf][off_l]) = kreg[i];
      *reinterpret_cast<uint4*>(&Vs[buf][off_l]) = vreg[i];
    }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  const bool wave_live = wrow0 < q_len;
  // V^T read addressing (see ds_read_b64_tr_b16 in common.h)
  const int i16 = lane & 15, grp = lane >> 4;
  const int tr_key = 4 * (grp >> 1) + (i16 >> 2);
  const int tr_col = 16 * (grp & 1) + 4 * (i16 & 3);

  for (int jt = 0; jt < n_tiles; ++jt) {
    const int buf = jt & 1;
    const bool more = jt + 1 < n_tiles;
    if (more) load_tile(jt + 1);

    const bool skip = !wave_live || (CAUSAL && jt * PF_BN > off + wrow1);
    if (!skip) {
      const uint16_t* kl = &Ks[buf][l32 * LDS_ROW + 8 * h2];
      f32x16 sacc;
#pragma unroll
      for (int j = 0; j < 16; ++j) sacc[j] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) sacc = mfma32(load16(kl + 16 * kk), qop[kk], sacc);

      float sv[16];
      float mx = -INFINITY;
      const int key0 = jt * PF_BN + 4 * h2;
      const bool need_mask = (jt * PF_BN + PF_BN > k_len) ||
                             (CAUSAL && jt * PF_BN + PF_BN - 1 > off + wrow0);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = key0 + 8 * (j >> 2) + (j & 3);
        bool valid = true;
        if (need_mask) valid = key < k_len && (!CAUSAL || key <= row + off);
        sv[j] = valid ? sacc[j] * LOG2E : -INFINITY;
        mx = fmaxf(mx, sv[j]);
      }
      mx = wave_max_xor(mx, 32);
      const float m_new = fmaxf(m_run, mx);
      const bool need = m_new > m_run + RESCALE_SLACK;
      if (__ballot(need) != 0ull) {
        const float m_use = need ? m_new : m_run;
        const float alpha = (m_use == m_run) ? 1.0f : fast_exp2(m_run - m_use);
        l_part *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= alpha;
        m_run = m_use;
      }
      const float m_eff = m_run == -INFINITY ? 0.f : m_run;
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        sv[j] = fast_exp2(sv[j] - m_eff);
        psum += sv[j];
      }
      l_part += psum;
      uint4 pop[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        pop[ks].x = pack2(sv[8 * ks + 0], sv[8 * ks + 1]);
        pop[ks].y = pack2(sv[8 * ks + 2], sv[8 * ks + 3]);
        pop[ks].z = pack2(sv[8 * ks + 4], sv[8 * ks + 5]);
        pop[ks].w = pack2(sv[8 * ks + 6], sv[8 * ks + 7]);
      }
      const uint16_t* vl = &Vs[buf][0];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const uint16_t* p0 = vl + (16 * ks + tr_key) * LDS_ROW + 32 * dt + tr_col;
          const uint2 lo = lds_read_tr16(p0);
          const uint2 hi = lds_read_tr16(p0 + 8 * LDS_ROW);
          const uint4 vt = make_uint4(lo.x, lo.y, hi.x, hi.y);
          acc[dt] = mfma32(vt, pop[ks], acc[dt]);
        }
      }
    }
    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: normalise, gate, store (row-major d within each row)
  if (row >= q_len) return;
  float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;  // fully-masked row -> 0
  uint16_t* op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)row * a.o_st;
  const uint16_t* gp = nullptr;
  if (GATE) gp = a.gate + (int64_t)b * a.g_sb + (int64_t)h * a.g_sh + (int64_t)row * a.g_st;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int d0 = 32 * dt + 8 * jb + 4 * h2;
      float o4[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) o4[c] = acc[dt][4 * jb + c] * inv;
      if (GATE) {
        const uint2 gv = *reinterpret_cast<const uint2*>(gp + d0);
        o4[0] *= sigmoidf(__uint_as_float(gv.x << 16));
        o4[1] *= sigmoidf(__uint_as_float(gv.x & 0xffff0000u));
        o4[2] *= sigmoidf(__uint_as_float(gv.y << 16));
        o4[3] *= sigmoidf(__uint_as_float(gv.y & 0xffff0000u));
      }
      uint2 ov;
      ov.x = pack2(o4[0], o4[1]);
      ov.y = pack2(o4[2], o4[3]);
      *reinterpret_cast<uint2*>(op + d0) = ov;
    }
  }
}

hipError_t launch_prefill(const PrefillArgs& a, bool qraw, bool gate, hipStream_t st) {
  const int64_t nwg = (int64_t)a.n_qt * a.H * a.B;
  if (nwg == 0) return hipSuccess;
  dim3 grid((unsigned)nwg), block(256);
  if (qraw && gate && a.causal)
    hipLaunchKernelGGL((prefill_kernel<true, true, true>), grid, block, 0, st, a);
  else if (!qraw && !gate && a.causal)
    hipLaunchKernelGGL((prefill_kernel<false, false, true>), grid, block, 0, st, a);
  else if (!qraw && !gate && !a.causal)
    hipLaunchKernelGGL((prefill_kernel<false, false, false>), grid, block, 0, st, a);
  else if (qraw && gate && !a.causal)
    hipLaunchKernelGGL((prefill_kernel<true, true, false>), grid, block, 0, st, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

constexpr int prefill_rows_per_wg() { return PF_BM; }

}  // namespace vm

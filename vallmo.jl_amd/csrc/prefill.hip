// prefill.hip — causal / non-causal GQA flash attention for prefill and chunked
// prefill: the attention! operator (src/kernels/attention.jl:12-129, re-designed
// for CDNA4) on already-normalised q. The gated layer path with its fused
// prologue and epilogue is prefill_fused.hip.
//
// Workgroup = 4 waves = 128 query rows of one (head, sequence); wave w owns 32
// rows. Per 32-key tile, all on 32x32x16 bf16 MFMA with fp32 accumulate:
//   S^T[key][row] = K[key][:] . Q[row][:]         A = K (LDS, ds_read_b128),
//                                                 B = Q (registers, loaded once)
//   O^T[d][row]  += V^T[d][key] . P^T[key][row]   A = V^T (LDS, ds_read_b64_tr_b16),
//                                                 B = P^T (the S^T accumulator, in place)
// The S^T accumulator layout (lane l: row l%32, keys 8(j/4)+4(l/32)+j%4) is the
// P^T operand layout up to a key permutation that the V^T transpose reads
// reproduce, so P never leaves registers.
//
// K/V tiles stream through a 4-slot LDS ring filled by direct global->LDS
// loads (global_load_lds_dwordx4: no VGPR staging), issued two tiles ahead of
// use; each iteration issues QK of the next tile on the matrix cores before the
// softmax of the current one, so the VALU work runs under the MFMAs.
// Rows are 512 B with the 16-byte chunks XOR-swizzled by row (swz_pf below) so that
// both read patterns hit distinct banks.
//
// Softmax is exp2-based with an online running max, rescaled lazily (only when
// it grows by > 8 in log2 units; the final 1/l cancels the common scale). No
// weight bound is known to this operator, so there is no static shift. Rows
// with no valid key (k_len = 0, or a causal row before the first key) produce
// 0 (attention.jl:86).
#include "common.h"
#include "kernels.h"

namespace vm {

constexpr int PF_BM = 128;                   // query rows per workgroup
constexpr int PF_BN = 32;                    // keys per tile
constexpr float RESCALE_SLACK = 8.0f;

// Head dims D = 256 (Qwen3.5), 128 and 64. A tile is 32 rows of 2D bytes,
// loaded as 1-KB slots (D / 16 of them, D / 64 per wave), each slot 512 / D
// rows of D / 8 lanes. The swizzle below keeps 16-chunk blocks (masked to the
// row's 8 chunks at D = 64), so it serves every row width. Q is pre-scaled by
// 1/sqrt(D) where that is a power of two (1/16, 1/8: exact in bf16); at D = 128
// the 1/sqrt(128) goes into the exp2 factor.
template <int D> struct PfShape {
  static constexpr int TILE = PF_BN * D;           // bf16 per K (or V) tile
  static constexpr int RB = 2 * D;                 // bytes per row
  static constexpr int SPW = D / 64;               // 1-KB slots per wave and tile (K or V)
  static constexpr int RPS = 512 / D;              // rows per slot
  static constexpr int LPR = D / 8;                // lanes per row in a slot
  static constexpr int LOADS = 2 * SPW;            // vmem instructions per wave per tile
  static constexpr int KK = D / 16;                // 16-deep k-steps of QK
  static constexpr int DT = D / 32;                // 32-wide d-blocks of O
  static constexpr int CM = D / 8 < 16 ? D / 8 - 1 : 15;  // swizzle mask (chunks per row)
  static constexpr float QPRE = D == 256 ? QK_SCALE : D == 64 ? 0.125f : 1.0f;
  static constexpr float SL = D == 128 ? LOG2E * 0.08838834764831845f : LOG2E;  // 1/sqrt(128)
};

// Workgroup barrier without the release/acquire fences of __syncthreads(): those
// would wait for every outstanding load (vmcnt(0)), including the tiles still in
// flight. LDS visibility is established by each wave's explicit vmcnt wait on its
// own DMA before the barrier; the asm memory clobbers keep the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// chunk c of tile row r lives at chunk c ^ swz_pf(r), swz_pf(r) = 4(r & 3) + ((r >> 2) & 3):
// the 16 rows of each 16-lane group of a b128 K read, and the 4 rows x 64 B of
// each 32-lane half of a transposing V read, fall on distinct banks (gfx950 LDS:
// 64 banks of 4 bytes).
__device__ __forceinline__ int swz_pf(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

struct PrefillCtx {
  const uint16_t* kbase;   // K rows of (b, hk)
  const uint16_t* vbase;
  int64_t kv_st;
  int k_len, off, row, wrow0, wrow1, q_len, lane, wave;
  int krow_max;            // last row that may be read (finite data)
  int dma_off[4];          // per-lane element offsets of this wave's DMA slots
};

// Issue this wave's share (SPW K + SPW V instructions of 1 KB) of tile `jt`.
template <int D>
__device__ __forceinline__ void issue_tile(const PrefillCtx& c, int jt, uint16_t* kd,
                                           uint16_t* vd) {
  using Sh = PfShape<D>;
  const int row0 = jt * PF_BN;
  if (row0 + PF_BN - 1 <= c.krow_max) {
    // whole tile in range: uniform tile base + precomputed per-lane offsets
    const uint16_t* kt = c.kbase + (int64_t)row0 * c.kv_st;
    const uint16_t* vt = c.vbase + (int64_t)row0 * c.kv_st;
#pragma unroll
    for (int i = 0; i < Sh::SPW; ++i) {
      const int g = Sh::SPW * c.wave + i;  // 1-KB slot of the tile: rows RPS g ..
      __builtin_amdgcn_global_load_lds((const void*)(kt + c.dma_off[i]),
                                       (__attribute__((address_space(3))) void*)(kd + g * 512),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vt + c.dma_off[i]),
                                       (__attribute__((address_space(3))) void*)(vd + g * 512),
                                       16, 0, 0);
    }
  } else {
    // last tile: rows past the last readable row re-read it (their keys are masked)
    const int l = c.lane;
#pragma unroll
    for (int i = 0; i < Sh::SPW; ++i) {
      const int g = Sh::SPW * c.wave + i;
      const int r = Sh::RPS * g + l / Sh::LPR;
      const int chunk = (l % Sh::LPR) ^ (swz_pf(r) & Sh::CM);
      const int64_t key = min(row0 + r, c.krow_max);
      const int64_t go = key * c.kv_st + chunk * 8;
      __builtin_amdgcn_global_load_lds((const void*)(c.kbase + go),
                                       (__attribute__((address_space(3))) void*)(kd + g * 512),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(c.vbase + go),
                                       (__attribute__((address_space(3))) void*)(vd + g * 512),
                                       16, 0, 0);
    }
  }
}

// S^T = K Q^T for one tile: chunk 2kk+h2 of row l%32 sits at
// ((2kk+h2) ^ swz_pf) -> koff[kk&7] + 256*(kk>>3) bytes.
template <int D>
__device__ __forceinline__ f32x16 qk_tile(const uint16_t* kb, const uint4 (&qop)[16],
                                          const int (&koff)[8]) {
  constexpr int KK = PfShape<D>::KK;
  const char* kl = reinterpret_cast<const char*>(kb);
  uint4 kf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
    kf[kk] = *reinterpret_cast<const uint4*>(kl + koff[kk & 7] + 256 * (kk >> 3));
  f32x16 s;
#pragma unroll
  for (int j = 0; j < 16; ++j) s[j] = 0.f;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) s = mfma32(kf[kk], qop[kk], s);
  return s;
}

// Mask keys past k_len and (causal) past row + off with -inf.
template <bool CAUSAL>
__device__ __forceinline__ void mask_tile(const PrefillCtx& c, int jt, f32x16& s) {
  const int lim = CAUSAL ? min(c.k_len - 1, c.row + c.off) : c.k_len - 1;
  const int key0 = jt * PF_BN + 4 * (c.lane >> 5);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int key = key0 + 8 * (j >> 2) + (j & 3);
    s[j] = key <= lim ? s[j] : -INFINITY;
  }
}

// One pipelined iteration on ring slot SLOT = jt % 4: wait for tile jt+1, issue
// tile jt+3, then QK(jt+1) on the matrix cores while the VALU runs softmax(jt),
// then PV(jt). `sc` holds S^T of tile jt on entry and of tile jt+1 on exit.
template <bool CAUSAL, int SLOT, int D>
__device__ __forceinline__ void tile_step(const PrefillCtx& c, int jt, int n_tiles, int my_tiles,
                                          uint16_t* const (&K)[4], uint16_t* const (&V)[4],
                                          const uint4 (&qop)[16], f32x16 (&acc)[8], f32x16& sc,
                                          float& m_run, float& l_part, const int (&koff)[8],
                                          const int (&voff)[4][2]) {
  using Sh = PfShape<D>;
  // tiles jt+1 and jt+2 may be in flight; tile jt+1 must be resident for all waves
  if (jt + 2 < n_tiles)
    wait_vmcnt<Sh::LOADS>();
  else
    wait_vmcnt<0>();
  lds_barrier();
  if (jt + 3 < n_tiles) issue_tile<D>(c, jt + 3, K[(SLOT + 3) & 3], V[(SLOT + 3) & 3]);
  if (jt >= my_tiles) return;

  const bool need_mask = (jt * PF_BN + PF_BN > c.k_len) ||
                         (CAUSAL && jt * PF_BN + PF_BN - 1 > c.off + c.wrow0);
  if (need_mask) mask_tile<CAUSAL>(c, jt, sc);

  // S^T of the next tile (its slot is resident; past this wave's last tile the
  // result is simply unused)
  const f32x16 sn = qk_tile<D>(K[(SLOT + 1) & 3], qop, koff);

  float mx = sc[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) mx = fmaxf(mx, sc[j]);
  mx = wave_max_xor(mx, 32) * Sh::SL;
  const float m_new = fmaxf(m_run, mx);
  const bool need = m_new > m_run + RESCALE_SLACK;
  if (__ballot(need) != 0ull) {
    const float m_use = need ? m_new : m_run;
    const float alpha = (m_use == m_run) ? 1.0f : fast_exp2(m_run - m_use);
    l_part *= alpha;
#pragma unroll
    for (int i = 0; i < Sh::DT; ++i) acc[i] *= alpha;
    m_run = m_use;
  }
  const float m_eff = m_run == -INFINITY ? 0.f : m_run;
  float p[16], psum = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    p[j] = fast_exp2(__builtin_fmaf(sc[j], Sh::SL, -m_eff));
    psum += p[j];
  }
  l_part += psum;
  uint4 pop[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    pop[ks].x = pack2(p[8 * ks + 0], p[8 * ks + 1]);
    pop[ks].y = pack2(p[8 * ks + 2], p[8 * ks + 3]);
    pop[ks].z = pack2(p[8 * ks + 4], p[8 * ks + 5]);
    pop[ks].w = pack2(p[8 * ks + 6], p[8 * ks + 7]);
  }
  // O^T += V^T P^T; d-block dt, key half ks, row half hi at
  // voff[dt&3][hi] + 256*(dt>>2) + 16 RB ks bytes
  const char* vl = reinterpret_cast<const char*>(V[SLOT]);
#pragma unroll
  for (int dt = 0; dt < Sh::DT; ++dt) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const char* p0 = vl + 256 * (dt >> 2) + 16 * Sh::RB * ks;
      const uint2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(p0 + voff[dt & 3][0]));
      const uint2 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(p0 + voff[dt & 3][1]));
      acc[dt] = mfma32(make_uint4(lo.x, lo.y, hi.x, hi.y), pop[ks], acc[dt]);
    }
  }
  sc = sn;
}

// Ring of 4 tile slots; tiles 0..2 are issued by the caller.
template <bool CAUSAL, int D>
__device__ __forceinline__ void tile_loop(const PrefillCtx& c, int n_tiles, int my_tiles,
                                          uint16_t* const (&K)[4], uint16_t* const (&V)[4],
                                          const uint4 (&qop)[16], f32x16 (&acc)[8],
                                          float& m_run, float& l_part, const int (&koff)[8],
                                          const int (&voff)[4][2]) {
  // tile 0 resident (tiles 1 and 2 may still be in flight), then S^T of tile 0
  if (n_tiles > 2)
    wait_vmcnt<2 * PfShape<D>::LOADS>();
  else if (n_tiles > 1)
    wait_vmcnt<PfShape<D>::LOADS>();
  else
    wait_vmcnt<0>();
  lds_barrier();
  f32x16 sc;
  if (my_tiles > 0) sc = qk_tile<D>(K[0], qop, koff);
  for (int jt = 0; jt < n_tiles; jt += 4) {
    tile_step<CAUSAL, 0, D>(c, jt, n_tiles, my_tiles, K, V, qop, acc, sc, m_run, l_part,
                                 koff, voff);
    if (jt + 1 < n_tiles)
      tile_step<CAUSAL, 1, D>(c, jt + 1, n_tiles, my_tiles, K, V, qop, acc, sc, m_run,
                                   l_part, koff, voff);
    if (jt + 2 < n_tiles)
      tile_step<CAUSAL, 2, D>(c, jt + 2, n_tiles, my_tiles, K, V, qop, acc, sc, m_run,
                                   l_part, koff, voff);
    if (jt + 3 < n_tiles)
      tile_step<CAUSAL, 3, D>(c, jt + 3, n_tiles, my_tiles, K, V, qop, acc, sc, m_run,
                                   l_part, koff, voff);
  }
}

template <bool CAUSAL, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_kernel(PrefillArgs a) {
  using Sh = PfShape<D>;
  constexpr int TILE = Sh::TILE;
  __shared__ __attribute__((aligned(1024))) uint16_t K0[TILE], K1[TILE], K2[TILE], K3[TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t V0[TILE], V1[TILE], V2[TILE], V3[TILE];
  uint16_t* const K[4] = {K0, K1, K2, K3};
  uint16_t* const V[4] = {V0, V1, V2, V3};

  // ---- work item: heaviest query tiles first; the query heads of one
  // kv head land on the same XCD (workgroup id mod 8) when H*B % 8 == 0.
  const int HB = a.H * a.B;
  const int lin = blockIdx.x;
  const int qt = a.n_qt - 1 - lin / HB;
  const int rem = lin % HB;
  const int hb = (HB & 7) == 0 ? (rem & 7) * (HB >> 3) + (rem >> 3) : rem;
  const int b = hb / a.H, h = hb % a.H;
  const int hk = h / (a.H / a.Hk);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h2 = lane >> 5;
  const int r0 = qt * PF_BM;
  const int row = r0 + 32 * wave + l32;  // query row in the chunk

  // q rows first: they depend on nothing the length lookups below return, so
  // their HBM latency overlaps those lookups (rows past q_len are clamped
  // in-bounds and never used).
  const int qrow = min(row, a.L - 1);
  const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                       (int64_t)qrow * a.q_st + 8 * h2;
  uint4 qraw[16];
#pragma unroll
  for (int kk = 0; kk < Sh::KK; ++kk) qraw[kk] = load16(qp + 16 * kk);

  // q_len > L and k_len > Lk are out of contract; clamp so rows past the
  // tensors are never read or written
  const int q_len = a.q_lengths ? min(a.q_lengths[b], a.L) : a.L;
  if (r0 >= q_len) return;
  const int k_len = a.k_lengths ? max(0, min(a.k_lengths[b], a.Lk)) : a.Lk;
  const int off = k_len - q_len;  // queries are the suffix of keys
  const int kend = CAUSAL ? min(k_len, off + r0 + PF_BM) : k_len;
  const int n_tiles = kend > 0 ? (kend + PF_BN - 1) / PF_BN : 0;

  PrefillCtx c;
  c.kbase = a.k + (int64_t)b * a.kv_sb + (int64_t)hk * a.kv_sh;
  c.vbase = a.v + (int64_t)b * a.kv_sb + (int64_t)hk * a.kv_sh;
  c.kv_st = a.kv_st;
  c.k_len = k_len; c.off = off; c.row = row; c.q_len = q_len;
  c.wrow0 = r0 + 32 * wave; c.wrow1 = c.wrow0 + 31;
  c.lane = lane; c.wave = wave;
  c.krow_max = max(0, k_len - 1);  // rows past k_len are masked; read finite data
#pragma unroll
  for (int i = 0; i < Sh::SPW; ++i) {
    const int r = Sh::RPS * (Sh::SPW * wave + i) + lane / Sh::LPR;
    c.dma_off[i] = r * (int)a.kv_st + (((lane % Sh::LPR) ^ (swz_pf(r) & Sh::CM)) * 8);
  }

  // the first three tiles go out before the q operand is formed so their
  // latency overlaps it
  if (n_tiles > 0) issue_tile<D>(c, 0, K0, V0);
  if (n_tiles > 1) issue_tile<D>(c, 1, K1, V1);
  if (n_tiles > 2) issue_tile<D>(c, 2, K2, V2);
  // tiles this wave computes (causal: keys <= off + its last row)
  int my_tiles = c.wrow0 < q_len ? n_tiles : 0;
  if (CAUSAL && my_tiles > 0) my_tiles = max(0, min(n_tiles, (off + c.wrow1) / PF_BN + 1));

  // ---- Q operand: lane holds q[row][16kk + 8*h2 + j], pre-scaled by 1/16 at
  // D = 256 (a power of two: exact in bf16)
  uint4 qop[16];
#pragma unroll
  for (int kk = 0; kk < Sh::KK; ++kk) {
    float x[8];
    unpack8(qraw[kk], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] *= Sh::QPRE;
    qop[kk] = pack8(x);
  }

  // swizzled LDS read offsets (bytes). K: chunk c = 2kk + h2 of row l32 sits at
  // chunk c ^ S, S = swz_pf(l32) < 16, i.e. 16((2(kk&7) + h2) ^ S) + 256(kk>>3).
  // V^T: a transposing read by source lane i of 16-lane group m reads key row
  // rr = 8hi + 4(m>>1) + (i>>2) (+16 ks), d-chunk 4dt + u, u = 2(m&1) + ((i&3)>>1),
  // 8-byte half i&1; with S(rr) = 4(i>>2) + 2hi + (m>>1) the chunk lands at
  // 4((dt&3) ^ (i>>2)) + 16(dt>>2) + (u ^ (2hi + (m>>1))).
  int koff[8], voff[4][2];
  {
    const int sk = swz_pf(l32) & Sh::CM;
#pragma unroll
    for (int q = 0; q < 8; ++q) koff[q] = l32 * Sh::RB + 16 * ((2 * q + h2) ^ sk);
    const int m = lane >> 4, i = lane & 15;
    const int u = 2 * (m & 1) + ((i & 3) >> 1);
#pragma unroll
    for (int d3 = 0; d3 < 4; ++d3)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int rr = 8 * hi + 4 * (m >> 1) + (i >> 2);
        voff[d3][hi] = rr * Sh::RB + 16 * ((4 * d3 + u) ^ (swz_pf(rr) & Sh::CM)) + 8 * (i & 1);
      }
  }

  f32x16 acc[8];
#pragma unroll
  for (int i = 0; i < Sh::DT; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[i][j] = 0.f;
  float l_part = 0.f, m_run = -INFINITY;

  tile_loop<CAUSAL, D>(c, n_tiles, my_tiles, K, V, qop, acc, m_run, l_part, koff, voff);

  // ---- epilogue: normalise and store (row-major d within each row)
  if (row >= q_len) return;
  float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = l_tot > 0.f ? fast_rcp(l_tot) : 0.f;  // no valid key -> 0
  uint16_t* op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)row * a.o_st;
#pragma unroll
  for (int dt = 0; dt < Sh::DT; ++dt) {
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int d0 = 32 * dt + 8 * jb + 4 * h2;
      uint2 ov;
      ov.x = pack2(acc[dt][4 * jb + 0] * inv, acc[dt][4 * jb + 1] * inv);
      ov.y = pack2(acc[dt][4 * jb + 2] * inv, acc[dt][4 * jb + 3] * inv);
      *reinterpret_cast<uint2*>(op + d0) = ov;
    }
  }
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t st) {
  const int64_t nwg = (int64_t)a.n_qt * a.H * a.B;
  if (nwg == 0) return hipSuccess;
  dim3 grid((unsigned)nwg), block(256);
  if (a.D == 128) {
    if (a.causal)
      hipLaunchKernelGGL((prefill_kernel<true, 128>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((prefill_kernel<false, 128>), grid, block, 0, st, a);
  } else if (a.D == 64) {
    if (a.causal)
      hipLaunchKernelGGL((prefill_kernel<true, 64>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((prefill_kernel<false, 64>), grid, block, 0, st, a);
  } else if (a.causal) {
    hipLaunchKernelGGL((prefill_kernel<true, 256>), grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL((prefill_kernel<false, 256>), grid, block, 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace vm

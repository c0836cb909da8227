// prefill_fused.hip — the fused gated-attention prefill of forward(::AttnLayer)
// (src/llm/qwen35.jl:292-318): q norm + RoPE prologue, causal GQA flash attention
// over the cache (src/kernels/attention.jl:12-91), sigmoid-gate epilogue written in
// the Wo input layout. Re-designed for CDNA4:
//
// * Persistent workgroups. One workgroup per CU walks a static list of work
//   items (b, h, 128-row q-block), heaviest causal q-blocks first, in a
//   serpentine order (pass 0 forward, pass 1 backward, ...), so every CU gets
//   about the same number of key tiles and no second dispatch round exists.
//   Items of one pass that share a workgroup slot keep the same (b, h), so the
//   four query heads of a kv head stay on one XCD and share its L2.
// * Workgroup = 4 waves x 32 query rows, 32-key tiles, all on 32x32x16 bf16 MFMA
//   with fp32 accumulation:
//     S^T[key][row] = K[key][:] . Q[row][:]       A = K (LDS, ds_read_b128), B = Q (VGPRs)
//     O^T[d][row]  += V^T[d][key] . P^T[key][row] A = V^T (LDS, ds_read_b128),
//                                                 B = P^T (the S^T accumulator, packed)
//   V^T comes ready-made: vt_transpose_kernel (below) writes each 32-key tile of
//   the cached V as V^T in exactly the byte layout the MFMA reads from LDS, into a
//   caller-provided workspace, so the tiles are plain 16-KB copies and every V
//   operand is one b128 read (transposing LDS reads cost about 1.6x the time).
// * Three-stage software pipeline per iteration j: QK(j+1) on the matrix cores,
//   softmax(j) on the VALU and PV(j-1) on the matrix cores, in one straight-line
//   block whose instruction groups are pinned so the LDS reads run ahead of the
//   MFMAs that consume them and the softmax spreads over all 32 MFMAs.
// * K and V tiles stream through separate 4-slot LDS rings filled by direct
//   global->LDS loads; K(t) is issued three iterations before QK(t), V(t) three
//   before PV(t). Every iteration issues the same 8 loads per wave (past the
//   last tile, the last tile again), so the wait before each barrier is the
//   constant vmcnt(16).
// * Softmax: exp2 with the QK-norm bound as a static shift when it is <= 64 in
//   log2 units (no running max, no accumulator rescale), else an online max
//   rescaled lazily (only when it grows by > 8).
#include "common.h"
#include "kernels.h"

namespace vm {

namespace {

constexpr int FM = 128;                    // query rows per item
constexpr int FN = 32;                     // keys per tile
constexpr int FT = FN * HEAD_DIM;          // bf16 per K (or V) tile: 16 KB
constexpr int NS = 4;                      // ring slots (K and V each)
constexpr int DMA_PER_ITER = 8;            // load instructions per wave per iteration
constexpr float FSTATIC_LIMIT = 64.0f;
constexpr float FRESCALE_SLACK = 8.0f;
constexpr int SG_VALU = 0x002, SG_MFMA = 0x008, SG_DSR = 0x100;

#define FSGB(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)

__device__ __forceinline__ void fbarrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// chunk c of tile row r lives at chunk c ^ fswz(r): the 16 rows of each 16-lane
// group of a b128 K read and the 4 rows x 64 B of each 32-lane half of a
// transposing V read fall on distinct banks (64 banks of 4 bytes).
__device__ __forceinline__ int fswz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

struct FItem {
  int b, h, hk, qt;
};

__device__ __forceinline__ FItem item_at(const PrefillArgs& a, int i) {
  const int HB = a.H * a.B;
  const int r = i / HB;  // 0 = heaviest q-block
  const int rem = i % HB;
  // the 8 XCDs take workgroups round-robin: slot rem lands on XCD rem % 8; give
  // consecutive heads (one kv group) to the same XCD
  const int hb = (HB & 7) == 0 ? (rem & 7) * (HB >> 3) + (rem >> 3) : rem;
  FItem it;
  it.b = hb / a.H;
  it.h = hb % a.H;
  it.hk = it.h / (a.H / a.Hk);
  it.qt = a.n_qt - 1 - r;
  return it;
}

// item of pass p for workgroup w of P: even passes forward, odd passes backward
// over the q-block ranks (keeping the workgroup's (b, h) slot when P % HB == 0)
__device__ __forceinline__ int item_index(int p, int w, int P, int HB) {
  if ((p & 1) == 0) return p * P + w;
  if (P % HB == 0) return p * P + (P / HB - 1 - w / HB) * HB + w % HB;
  return p * P + (P - 1 - w);
}

// ---- V^T tiles. Tile t of (b, hk) holds keys 32t .. 32t+31 as 256 d-rows of 64
// bytes. Row d holds four 16-byte chunks; logical chunk c = 2ks + h carries the 8
// keys 16ks + {4h..4h+3, 8+4h..8+4h+3} -- the key order of the P^T operand that
// lane half h holds for key half ks -- and is stored at chunk c ^ ((d >> 2) & 3),
// so the 16 rows of a b128 read group fall on distinct banks. Byte offset of
// logical chunk c of row m of a 32-row d-block:
__device__ __forceinline__ int vt_chunk_offset(int m, int c) {
  return 64 * m + 16 * (c ^ ((m >> 2) & 3));
}

// One workgroup per (32-key tile, kv head, sequence): 16 KB of the cached V in
// (coalesced 16-byte rows), through LDS, out as one V^T tile (coalesced). Keys
// past the attended length repeat the last one (they are masked; V stays finite).
__global__ __launch_bounds__(256) void vt_transpose_kernel(VtArgs a) {
  const int t = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int q_len = a.q_lengths ? min(a.q_lengths[b], a.L) : a.L;
  const int64_t k_len = min((int64_t)(a.prior ? a.prior[b] : 0) + q_len, a.ctx);
  if ((int64_t)t * FN >= k_len) return;
  __shared__ __attribute__((aligned(16))) uint16_t tile[FN][HEAD_DIM + 8];  // 16-B row pad
  const int tid = threadIdx.x;
  const uint16_t* src = a.v + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
#pragma unroll
  for (int q = tid; q < FN * 32; q += 256) {
    const int row = q >> 5, c16 = q & 31;
    const int64_t key = min((int64_t)t * FN + row, k_len - 1);
    *reinterpret_cast<uint4*>(&tile[row][c16 * 8]) = load16(src + key * a.v_st + c16 * 8);
  }
  __syncthreads();
  uint16_t* dst = a.vt + ((int64_t)b * a.Hk + hk) * a.vt_tiles * FT + (int64_t)t * FT;
#pragma unroll
  for (int o = tid; o < HEAD_DIM * 4; o += 256) {
    const int d = o >> 2;
    const int c = (o & 3) ^ ((d >> 2) & 3);
    const int ks = c >> 1, h = c & 1;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int b0 = 2 * e, b1 = 2 * e + 1;
      const uint32_t lo = tile[16 * ks + 8 * (b0 >> 2) + 4 * h + (b0 & 3)][d];
      const uint32_t hi = tile[16 * ks + 8 * (b1 >> 2) + 4 * h + (b1 & 3)][d];
      w[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(dst + o * 8) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

struct FCtx {
  const uint16_t* kbase;
  const uint16_t* vtbase;  // V^T tiles of (b, hk): 16 KB each
  int64_t kv_st;
  int krow_max;   // last cache row that may be read
  int n_tiles;
  uint32_t row_bytes;   // cache row stride in bytes
  uint32_t dma_boff[4]; // per-lane byte offsets of this wave's 4 one-KB pieces of a tile
  int wave, lane;
};

// This wave's quarter of tile t (clamped to the last tile) of K or V into `dst`:
// piece i = rows 2g, 2g+1 (g = 4 wave + i) as 64 lanes x 16 B. A whole tile is a
// scalar base plus per-lane unsigned byte offsets (the scalar-base addressing
// form); the last tile re-reads the last readable row past it (its keys are
// masked, and V must stay finite).
__device__ __forceinline__ void issue_quarter(const FCtx& c, const uint16_t* base, int t,
                                              uint16_t* dst) {
  t = min(t, c.n_tiles - 1);
  const int row0 = t * FN;
  const char* src = reinterpret_cast<const char*>(base + (int64_t)row0 * c.kv_st);
  if (row0 + FN - 1 <= c.krow_max) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * c.wave + i;
      __builtin_amdgcn_global_load_lds((const void*)(src + c.dma_boff[i]),
                                       (__attribute__((address_space(3))) void*)(dst + g * 512),
                                       16, 0, 0);
    }
  } else {
    const int last = c.krow_max - row0;  // last readable row of the tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * c.wave + i;
      const int r = 2 * g + (c.lane >> 5);
      const uint32_t over = (uint32_t)max(0, r - last);
      __builtin_amdgcn_global_load_lds((const void*)(src + (c.dma_boff[i] - over * c.row_bytes)),
                                       (__attribute__((address_space(3))) void*)(dst + g * 512),
                                       16, 0, 0);
    }
  }
}

// This wave's quarter of V^T tile t (clamped to the last tile): 4 one-KB pieces,
// a plain copy (the transpose kernel wrote the LDS byte layout).
__device__ __forceinline__ void issue_quarter_vt(const FCtx& c, int t, uint16_t* dst) {
  t = min(t, c.n_tiles - 1);
  const char* src = reinterpret_cast<const char*>(c.vtbase + (int64_t)t * FT) + 16 * c.lane;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = 4 * c.wave + i;
    __builtin_amdgcn_global_load_lds((const void*)(src + 1024 * g),
                                     (__attribute__((address_space(3))) void*)(dst + g * 512),
                                     16, 0, 0);
  }
}

template <int N>
__device__ __forceinline__ void fwait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---- explicit ordering. Empty volatile asm statements keep their source order;
// passing a value through one pins the instruction that produced it before that
// point (and its consumers after), and a memory clobber pins LDS reads and tile
// loads. The steady-state iteration below is written as a fixed sequence of
// steps this way; the MFMAs themselves stay builtins, so the compiler still
// inserts the LDS waits and hazard NOPs they need.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void mem_fence_order() { asm volatile("" ::: "memory"); }
__device__ __forceinline__ void pin(f32x16& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_acc(f32x16& x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(uint4& x) {
  u32x4 t = __builtin_bit_cast(u32x4, x);
  asm volatile("" : "+v"(t));
  x = __builtin_bit_cast(uint4, t);
}
// max / sum with the lane 32 apart (wave64), on the VALU (no LDS instruction)
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

struct LdsRing {
  uint16_t* K[NS];
  uint16_t* V[NS];
};

// softmax of one S^T tile (this lane: row l%32, 16 keys) -> packed P^T operands
// Softmax of one S^T tile (this lane: row l%32, 16 keys), branch-free: the running
// shift m_run (log2 units) moves to the tile's row max only when that exceeds it
// by > FRESCALE_SLACK (lazy rescale); alpha = 2^(old - new) (1 when it stays) is
// applied to l_part here and to the accumulator by the caller. With m_run
// starting at the QK-norm bound the shift never moves (the bound dominates every
// logit), which is the static-shift case at the price of a row max per tile.
// Outputs the packed P^T operands.
__device__ __forceinline__ void softmax_tile(const f32x16& s, float& m_run, float& l_part,
                                             uint4 (&pop)[2], float& alpha) {
  float mx = fmaxf(s[0], s[1]);
#pragma unroll
  for (int j = 2; j < 16; j += 2) mx = fmaxf(mx, fmaxf(s[j], s[j + 1]));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * LOG2E;
  const float m_new = fmaxf(m_run, mx);
  const float m_use = m_new > m_run + FRESCALE_SLACK ? m_new : m_run;
  alpha = m_use == m_run ? 1.0f : fast_exp2(m_run - m_use);
  m_run = m_use;
  const float m_eff = m_use == -INFINITY ? 0.f : m_use;
  float p[16], psum = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    p[j] = fast_exp2(__builtin_fmaf(s[j], LOG2E, -m_eff));
    psum += p[j];
  }
  l_part = l_part * alpha + psum;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    pop[ks].x = pack2(p[8 * ks + 0], p[8 * ks + 1]);
    pop[ks].y = pack2(p[8 * ks + 2], p[8 * ks + 3]);
    pop[ks].z = pack2(p[8 * ks + 4], p[8 * ks + 5]);
    pop[ks].w = pack2(p[8 * ks + 6], p[8 * ks + 7]);
  }
}

struct WaveGeo {
  int row, wrow0, wrow1, off, k_len;
};

template <bool CAUSAL>
__device__ __forceinline__ bool tile_needs_mask(const WaveGeo& g, int j) {
  return (j * FN + FN > g.k_len) || (CAUSAL && j * FN + FN - 1 > g.off + g.wrow0);
}
template <bool CAUSAL>
__device__ __forceinline__ void mask_s(const WaveGeo& g, int j, int lane, f32x16& s) {
  const int lim = CAUSAL ? min(g.k_len - 1, g.row + g.off) : g.k_len - 1;
  const int key0 = j * FN + 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int key = key0 + 8 * (i >> 2) + (i & 3);
    s[i] = key <= lim ? s[i] : -INFINITY;
  }
}

// K fragments of one ring slot: chunk 2kk+h2 of row l%32 at koff[kk&7] + 256*(kk>>3)
__device__ __forceinline__ void read_kf(const uint16_t* kb, const int (&koff)[8], uint4 (&kf)[16]) {
  const char* kl = reinterpret_cast<const char*>(kb);
#pragma unroll
  for (int kk = 0; kk < 16; ++kk)
    kf[kk] = *reinterpret_cast<const uint4*>(kl + koff[kk & 7] + 256 * (kk >> 3));
}

struct WaveState {
  uint4 qop[16];
  f32x16 acc[8];
  f32x16 sc;       // S^T of the tile whose softmax runs next
  uint4 pprev[2];  // P^T of the tile whose PV runs next
  float m_run, l_part;
};

// LDS reads issued from inline asm, with explicit waits. While a direct
// global->LDS load is in flight the compiler's wait pass can only wait for all
// LDS reads (lgkmcnt(0)) before using any of them, which would serialise every
// MFMA behind the latest read; here the reads of the steady block are counted
// by hand instead (no other LDS or scalar-memory instruction runs in that block,
// and waits the compiler places elsewhere can only wait for more, never less).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
template <int OFF>
__device__ __forceinline__ u32x4 ds_b128(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// wait until at most N LDS reads are outstanding; the two fragments a step
// consumes are threaded through it so their MFMAs cannot be scheduled ahead of
// the wait (and no copy of them can be made before it)
template <int N>
__device__ __forceinline__ void lds_wait(u32x4& x, u32x4& y) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}

// The steady-state iteration (softmax(j), QK(j+1), PV(j-1)) as 16 fixed steps.
// Step k issues QK MFMA k (chain on S(j+1)) and PV MFMA k (chain pairs on the
// accumulator), the two b128 LDS reads of step k + AHEAD (K fragment and V^T
// fragment k+AHEAD), and a few VALU ops of softmax(j):
//   steps 0-1 row max, 2 cross-half max, 3 shift update, 4-11 two exps each,
//   12-14 bf16 packing and the row sum.
// QK and PV MFMAs alternate, so a dependent MFMA always has an independent one
// between it and its producer. Reads complete in issue order (2 per step), so
// the operands of step k are in once at most 2*AHEAD - 2 reads are outstanding.
constexpr int AHEAD = 3;
template <int J4>
__device__ __forceinline__ void steady_block(WaveState& st, const LdsRing& ring,
                                             const int (&koff)[8], const int (&vof)[2],
                                             float& alpha) {
  // K slot j+1 and V slot j-1 share one LDS object (see the ring layout)
  const uint32_t kb = lds_addr(ring.K[(J4 + 1) % NS]);
  const uint32_t vb = lds_addr(ring.V[(J4 + 3) % NS]);
  uint32_t ka[8], va[2];
#pragma unroll
  for (int q = 0; q < 8; ++q) ka[q] = kb + koff[q];
  va[0] = vb + vof[0];
  va[1] = vb + vof[1];
  // K fragment k: chunk 2k+h2 of row l%32 at koff[k&7] + 256*(k>>3)
  // V^T fragment v = 2dt+ks: d-row 32dt + l%32 at vof[ks] + 2048*dt
#define RK(k) (kf[k] = ds_b128<256 * ((k) >> 3)>(ka[(k) & 7]))
#define RV(v) (vf[v] = ds_b128<2048 * ((v) >> 1)>(va[(v) & 1]))

  f32x16 s = st.sc;
  pin(s);  // the softmax starts inside this block
  u32x4 kf[16], vf[16];
  RK(0); RV(0); RK(1); RV(1); RK(2); RV(2);

  f32x16 sn;
  float mx[8], m_eff = 0.f, psum = 0.f, p[16];
  uint4 pcur[2];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    // operands of step k: issued 3 per step, AHEAD steps back; the reads of
    // the AHEAD-1 later steps (3 each) may still be outstanding
    if (k <= 16 - AHEAD) {
      lds_wait<2 * (AHEAD - 1)>(kf[k], vf[k]);
    } else if (k == 14) {
      lds_wait<2>(kf[k], vf[k]);
    } else {
      lds_wait<0>(kf[k], vf[k]);
    }
    if (k == 0) {
      f32x16 z;
#pragma unroll
      for (int i = 0; i < 16; ++i) z[i] = 0.f;
      sn = mfma32(__builtin_bit_cast(uint4, kf[0]), st.qop[0], z);
    } else {
      sn = mfma32(__builtin_bit_cast(uint4, kf[k]), st.qop[k], sn);
    }
    pin_acc(sn);
    st.acc[k >> 1] = mfma32(__builtin_bit_cast(uint4, vf[k]), st.pprev[k & 1], st.acc[k >> 1]);
    pin_acc(st.acc[k >> 1]);
    switch (k + AHEAD) {
      case 3: RK(3); RV(3); break;
      case 4: RK(4); RV(4); break;
      case 5: RK(5); RV(5); break;
      case 6: RK(6); RV(6); break;
      case 7: RK(7); RV(7); break;
      case 8: RK(8); RV(8); break;
      case 9: RK(9); RV(9); break;
      case 10: RK(10); RV(10); break;
      case 11: RK(11); RV(11); break;
      case 12: RK(12); RV(12); break;
      case 13: RK(13); RV(13); break;
      case 14: RK(14); RV(14); break;
      case 15: RK(15); RV(15); break;
      default: break;
    }
    // softmax(j), a few VALU ops per step
    if (k == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) { mx[i] = fmaxf(s[2 * i], s[2 * i + 1]); pin(mx[i]); }
    } else if (k == 1) {
#pragma unroll
      for (int i = 4; i < 8; ++i) { mx[i] = fmaxf(s[2 * i], s[2 * i + 1]); pin(mx[i]); }
    } else if (k == 2) {
      mx[0] = fmaxf(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])),
                    fmaxf(fmaxf(mx[4], mx[5]), fmaxf(mx[6], mx[7])));
      mx[0] = xor32_max(mx[0]) * LOG2E;
      pin(mx[0]);
    } else if (k == 3) {
      // lazy shift update (never moves when m_run starts at the QK-norm bound)
      const float m_run = st.m_run;
      const float m_new = fmaxf(m_run, mx[0]);
      const float m_use = m_new > m_run + FRESCALE_SLACK ? m_new : m_run;
      alpha = m_use == m_run ? 1.0f : fast_exp2(m_run - m_use);
      st.m_run = m_use;
      m_eff = m_use == -INFINITY ? 0.f : m_use;
      pin(m_eff);
      pin(alpha);
    } else if (k < 12) {
      const int e = 2 * (k - 4);
      p[e] = fast_exp2(__builtin_fmaf(s[e], LOG2E, -m_eff));
      p[e + 1] = fast_exp2(__builtin_fmaf(s[e + 1], LOG2E, -m_eff));
      psum += p[e] + p[e + 1];
      pin(p[e]);
      pin(p[e + 1]);
      pin(psum);
    } else if (k == 12) {
      pcur[0].x = pack2(p[0], p[1]);
      pcur[0].y = pack2(p[2], p[3]);
      pcur[0].z = pack2(p[4], p[5]);
      pcur[0].w = pack2(p[6], p[7]);
      pin(pcur[0]);
    } else if (k == 13) {
      pcur[1].x = pack2(p[8], p[9]);
      pcur[1].y = pack2(p[10], p[11]);
      pcur[1].z = pack2(p[12], p[13]);
      pcur[1].w = pack2(p[14], p[15]);
      pin(pcur[1]);
    } else if (k == 14) {
      st.l_part = st.l_part * alpha + psum;
      pin(st.l_part);
    }
  }
#undef RK
#undef RV
  st.sc = sn;
  st.pprev[0] = pcur[0];
  st.pprev[1] = pcur[1];
}

// Iteration j of the pipeline on compile-time ring slots (slot = tile % NS).
// PV: PV(j-1) runs; SM: softmax(j) runs; QK: QK(j+1) runs.
template <bool CAUSAL, int J4, bool PV, bool SM, bool QK>
__device__ __forceinline__ void iter(WaveState& st, const FCtx& c, const LdsRing& ring,
                                     const WaveGeo& g, int j, const int (&koff)[8],
                                     const int (&vof)[2]) {
  // K(j+1) and V(j-1) landed for every wave (loads of iterations j-2, j-1 may
  // still be in flight), and every wave is past iteration j-1
  fwait_vmcnt<2 * DMA_PER_ITER>();
  fbarrier();
  issue_quarter(c, c.kbase, j + NS, ring.K[J4 % NS]);
  issue_quarter_vt(c, j + NS - 2, ring.V[(J4 + 2) % NS]);

  if (SM && tile_needs_mask<CAUSAL>(g, j)) mask_s<CAUSAL>(g, j, c.lane, st.sc);
  float alpha = 1.0f;

  if (QK && PV && SM) {
    steady_block<J4>(st, ring, koff, vof, alpha);
  } else {
    __builtin_amdgcn_sched_barrier(0);
    uint4 kf[16];
    if (QK) read_kf(ring.K[(J4 + 1) % NS], koff, kf);
    uint4 pcur[2];
    if (SM) softmax_tile(st.sc, st.m_run, st.l_part, pcur, alpha);
    f32x16 sn;
    if (QK) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sn[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) sn = mfma32(kf[kk], st.qop[kk], sn);
    }
    if (PV) {
      const char* vl = reinterpret_cast<const char*>(ring.V[(J4 + 3) % NS]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          // V^T fragment: d-rows 32dt.., key half ks
          const uint4 vfrag = *reinterpret_cast<const uint4*>(vl + vof[ks] + 2048 * dt);
          st.acc[dt] = mfma32(vfrag, st.pprev[ks], st.acc[dt]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (QK) st.sc = sn;
    if (SM) {
      st.pprev[0] = pcur[0];
      st.pprev[1] = pcur[1];
    }
  }
  if (SM && __ballot(alpha != 1.0f) != 0ull) {
    // the shift grew: what the accumulator holds (through PV(j-1), at the old
    // shift) moves to the new one (rare)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) st.acc[dt] *= alpha;
  }
}

template <bool CAUSAL>
__device__ __forceinline__ void run_tiles(WaveState& st, const FCtx& c, const LdsRing& ring,
                                          const WaveGeo& g, const int (&koff)[8],
                                          const int (&vof)[2]) {
  const int n = c.n_tiles;
  // iteration 0: softmax(0), QK(1); no PV yet
  iter<CAUSAL, 0, false, true, true>(st, c, ring, g, 0, koff, vof);
  // steady iterations 1 .. n-1 (QK(n) at j = n-1 reads a repeated tile; unused)
  int j = 1;
  for (; j + 3 < n; j += 4) {
    iter<CAUSAL, 1, true, true, true>(st, c, ring, g, j, koff, vof);
    iter<CAUSAL, 2, true, true, true>(st, c, ring, g, j + 1, koff, vof);
    iter<CAUSAL, 3, true, true, true>(st, c, ring, g, j + 2, koff, vof);
    iter<CAUSAL, 0, true, true, true>(st, c, ring, g, j + 3, koff, vof);
  }
  // remaining steady iterations, then the PV(n-1)-only iteration j = n
  const int rem = n - j;  // 0..3 steady iterations left
  if (rem >= 1) iter<CAUSAL, 1, true, true, true>(st, c, ring, g, j, koff, vof);
  if (rem >= 2) iter<CAUSAL, 2, true, true, true>(st, c, ring, g, j + 1, koff, vof);
  if (rem >= 3) iter<CAUSAL, 3, true, true, true>(st, c, ring, g, j + 2, koff, vof);
  switch (n & 3) {  // the last iteration is j = n, slot n % 4
    case 0: iter<CAUSAL, 0, true, false, false>(st, c, ring, g, n, koff, vof); break;
    case 1: iter<CAUSAL, 1, true, false, false>(st, c, ring, g, n, koff, vof); break;
    case 2: iter<CAUSAL, 2, true, false, false>(st, c, ring, g, n, koff, vof); break;
    default: iter<CAUSAL, 3, true, false, false>(st, c, ring, g, n, koff, vof); break;
  }
}

}  // namespace

template <bool CAUSAL, bool PERSIST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_fused_kernel(PrefillArgs a, int n_items, int P) {
  // four __shared__ objects A_s, each holding K slot s and V slot (s+2)%4: the two
  // loads issued in iteration j both go to A_{j%4}, its reads (K slot j+1, V slot
  // j-1) come from A_{(j+1)%4}, whose last loads finished three iterations back,
  // so the compiler can see that no read aliases a load in flight (one object for
  // the whole ring would make it drain every load before each read)
  __shared__ __attribute__((aligned(1024))) uint16_t A0[2 * FT], A1[2 * FT], A2[2 * FT], A3[2 * FT];
  LdsRing ring;
  ring.K[0] = A0; ring.K[1] = A1; ring.K[2] = A2; ring.K[3] = A3;
  ring.V[0] = A2 + FT; ring.V[1] = A3 + FT; ring.V[2] = A0 + FT; ring.V[3] = A1 + FT;

  // the wave index through readfirstlane: a scalar, so tile-load LDS addresses
  // (M0) are scalar arithmetic rather than hoisted vector registers
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h2 = lane >> 5;
  const int HB = a.H * a.B;

  // swizzled LDS read offsets (bytes). K: chunk c = 2kk + h2 of row l32 sits at
  // chunk c ^ fswz(l32). V^T: a transposing read by lane i of 16-lane group m
  // reads key row rr = 8hi + 4(m>>1) + (i>>2) (+16 ks), d-chunk 4dt + u with
  // u = 2(m&1) + ((i&3)>>1), 8-byte half i&1.
  int koff[8], vof[2];
  {
    const int sk = fswz(l32);
#pragma unroll
    for (int q = 0; q < 8; ++q) koff[q] = l32 * 512 + 16 * ((2 * q + h2) ^ sk);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) vof[ks] = vt_chunk_offset(l32, 2 * ks + h2);
  }
  // static bound on |k~| (rows of any kv head): sqrt(D) * max|kw + w_offset|
  float kbound;
  {
    const uint2 wv = *reinterpret_cast<const uint2*>(a.kw + 4 * lane);
    float wmax = fmaxf(fmaxf(fabsf(__uint_as_float(wv.x << 16) + a.w_offset),
                             fabsf(__uint_as_float(wv.x & 0xffff0000u) + a.w_offset)),
                       fmaxf(fabsf(__uint_as_float(wv.y << 16) + a.w_offset),
                             fabsf(__uint_as_float(wv.y & 0xffff0000u) + a.w_offset)));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) wmax = fmaxf(wmax, __shfl_xor(wmax, m, 64));
    kbound = 16.0f * wmax * 1.01f;  // + bf16 rounding of the cached rows
  }

  WaveState st;
  for (int p = 0; PERSIST || p < 1; ++p) {
    const int idx = PERSIST ? item_index(p, blockIdx.x, P, HB) : (int)blockIdx.x;
    if (idx >= n_items) break;
    const FItem it = item_at(a, idx);
    const int b = it.b, h = it.h;
    const int r0 = it.qt * FM;
    const int row = r0 + 32 * wave + l32;

    // raw q rows first: they depend on nothing the length lookups return
    const int qrow = min(row, a.L - 1);
    const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh +
                         (int64_t)qrow * a.q_st + 8 * h2;
    uint4 qraw[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) qraw[kk] = load16(qp + 16 * kk);

    const int q_len = a.q_lengths ? min(a.q_lengths[b], a.L) : a.L;
    if (r0 >= q_len) continue;  // uniform over the workgroup
    const int prior = a.prior ? a.prior[b] : 0;
    const int k_len = prior + q_len;  // queries are the suffix of the attended keys
    WaveGeo g;
    g.row = row;
    g.wrow0 = r0 + 32 * wave;
    g.wrow1 = g.wrow0 + 31;
    g.off = k_len - q_len;
    g.k_len = k_len;
    const int kend = CAUSAL ? min(k_len, g.off + r0 + FM) : k_len;

    FCtx c;
    c.kbase = a.k + (int64_t)b * a.kv_sb + (int64_t)it.hk * a.kv_sh;
    c.vtbase = a.vt + ((int64_t)b * a.Hk + it.hk) * a.vt_tiles * FT;
    c.kv_st = a.kv_st;
    c.krow_max = max(0, min(k_len, a.Lk) - 1);
    c.n_tiles = max(1, (kend + FN - 1) / FN);
    c.wave = wave;
    c.lane = lane;
    c.row_bytes = (uint32_t)(2 * a.kv_st);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 2 * (4 * wave + i) + (lane >> 5);
      c.dma_boff[i] = (uint32_t)r * c.row_bytes + (uint32_t)(((lane & 31) ^ fswz(r)) * 16);
    }
    // the other prologue operands, also ahead of the tile loads (loads complete
    // in order: the prologue math must not wait behind six tiles)
    // (qw is the same for every item: an opaque zero keeps the compiler from
    // hoisting these 64 registers out of the item loop and through the main loop)
    int opaque0 = 0;
    asm volatile("" : "+v"(opaque0));
    uint4 qwv[16];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) qwv[kk] = load16(a.qw + opaque0 + 16 * kk + 8 * h2);
    const int64_t pos = min((int64_t)prior + qrow, (int64_t)a.Lk - 1);
    float4 cv[4], sv[4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        cv[2 * kk + u] = *reinterpret_cast<const float4*>(a.cos_tab + pos * HALF_ROT + 8 * h2 + 16 * kk + 4 * u);
        sv[2 * kk + u] = *reinterpret_cast<const float4*>(a.sin_tab + pos * HALF_ROT + 8 * h2 + 16 * kk + 4 * u);
      }
    // pre-loop loads, in the order of the virtual iterations -4 .. -1 of the
    // pipeline: K(0), K(1), K(2)+V(0), K(3)+V(1)
    issue_quarter(c, c.kbase, 0, ring.K[0]);
    issue_quarter(c, c.kbase, 1, ring.K[1]);
    issue_quarter(c, c.kbase, 2, ring.K[2]);
    issue_quarter_vt(c, 0, ring.V[0]);
    issue_quarter(c, c.kbase, 3, ring.K[3]);
    issue_quarter_vt(c, 1, ring.V[1]);

    // ---- q prologue: qnorm_rope (src/kernels/qknorm_rope_append.jl:25-57) and
    // the 1/16 scale (exact in bf16); lane holds q[row][16kk + 8h2 + j]
    float qn2 = 0.f;
    {
      float x[16][8];
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) unpack8(qraw[kk], x[kk]);
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x[kk][j] * x[kk][j];
      ss += __shfl_xor(ss, 32, 64);
      const float rn = 1.0f / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
        float wf[8];
        unpack8(qwv[kk], wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[kk][j] = x[kk][j] * rn * (wf[j] + a.w_offset);
      }
      const float* cs = reinterpret_cast<const float*>(cv);
      const float* sn = reinterpret_cast<const float*>(sv);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float cc = cs[8 * kk + j], si = sn[8 * kk + j];
          const float x1 = x[kk][j], x2 = x[kk + 2][j];
          x[kk][j] = x1 * cc - x2 * si;
          x[kk + 2][j] = x2 * cc + x1 * si;
        }
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x[kk][j] *= QK_SCALE;
          qn2 += x[kk][j] * x[kk][j];
        }
        st.qop[kk] = pack8(x[kk]);
      }
    }
    qn2 += __shfl_xor(qn2, 32, 64);
    const float bound = sqrtf(qn2) * 1.01f * kbound * LOG2E;  // |q op| rounded to bf16
    const bool use_static = __ballot(!(bound <= FSTATIC_LIMIT)) == 0ull;
    st.m_run = use_static ? bound : -INFINITY;
    st.l_part = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 16; ++j) st.acc[i][j] = 0.f;

    // S^T(0): K(0) landed (K(1), K(2)+V(0), K(3)+V(1) may be in flight)
    fwait_vmcnt<20>();
    fbarrier();
    {
      uint4 kf[16];
      read_kf(ring.K[0], koff, kf);
#pragma unroll
      for (int i = 0; i < 16; ++i) st.sc[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) st.sc = mfma32(kf[kk], st.qop[kk], st.sc);
    }
    run_tiles<CAUSAL>(st, c, ring, g, koff, vof);

    // ---- epilogue: normalise, gate (sigmoid, src/kernels/kernels.jl:34), store
    // in the Wo input layout. Every gate load goes out before the first store.
    if (row < q_len) {
      const float l_tot = st.l_part + __shfl_xor(st.l_part, 32, 64);
      const float inv = l_tot > 0.f ? fast_rcp(l_tot) : 0.f;  // fully-masked row -> 0
      const uint16_t* gp = a.gate + (int64_t)b * a.g_sb + (int64_t)h * a.g_sh + (int64_t)row * a.g_st;
      uint2 gv[8][4];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
          gv[dt][jb] = *reinterpret_cast<const uint2*>(gp + 32 * dt + 8 * jb + 4 * h2);
      uint16_t* op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)row * a.o_st;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int d0 = 32 * dt + 8 * jb + 4 * h2;
          const uint2 g2 = gv[dt][jb];
          const float o0 = st.acc[dt][4 * jb + 0] * inv * sigmoidf(__uint_as_float(g2.x << 16));
          const float o1 = st.acc[dt][4 * jb + 1] * inv * sigmoidf(__uint_as_float(g2.x & 0xffff0000u));
          const float o2 = st.acc[dt][4 * jb + 2] * inv * sigmoidf(__uint_as_float(g2.y << 16));
          const float o3 = st.acc[dt][4 * jb + 3] * inv * sigmoidf(__uint_as_float(g2.y & 0xffff0000u));
          uint2 ov;
          ov.x = pack2(o0, o1);
          ov.y = pack2(o2, o3);
          *reinterpret_cast<uint2*>(op + d0) = ov;
        }
    }
    // the ring is reused by the next item: every load landed, every wave done
    fwait_vmcnt<0>();
    fbarrier();
  }
  fwait_vmcnt<0>();  // no LDS load may land after the workgroup is gone
}

hipError_t launch_vt_transpose(const VtArgs& a, hipStream_t st) {
  if (a.B == 0 || a.Hk == 0 || a.vt_tiles == 0) return hipSuccess;
  hipLaunchKernelGGL(vt_transpose_kernel, dim3(a.vt_tiles, a.Hk, a.B), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_prefill_fused(const PrefillArgs& a, hipStream_t st) {
  const int64_t n_items = (int64_t)a.n_qt * a.H * a.B;
  if (n_items == 0) return hipSuccess;
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    cus = n;
  }
  // one item per workgroup, heaviest first (the hardware hands the next item to
  // the first CU that frees up)
  const int P = (int)n_items;
  (void)cus;
  if (a.causal)
    hipLaunchKernelGGL((prefill_fused_kernel<true, false>), dim3(P), dim3(256), 0, st, a, (int)n_items, P);
  else
    hipLaunchKernelGGL((prefill_fused_kernel<false, false>), dim3(P), dim3(256), 0, st, a, (int)n_items, P);
  return hipGetLastError();
}

}  // namespace vm

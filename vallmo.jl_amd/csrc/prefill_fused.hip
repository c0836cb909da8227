// prefill_fused.hip — the fused gated-attention prefill of forward(::AttnLayer)
// (src/llm/qwen35.jl:292-318): q norm + RoPE prologue, causal GQA flash attention
// over the cache (src/kernels/attention.jl:12-91), sigmoid-gate epilogue written in
// the Wo input layout. Re-designed for CDNA4.
//
// One workgroup (4 waves, one per SIMD, the whole 160-KB LDS) per work item
// (b, h, 128-row q-block), heaviest causal q-blocks first (the hardware hands the
// next item to the first CU that frees up). All products are 32x32x16 bf16 MFMAs
// with fp32 accumulation, over 32-key tiles:
//     S^T[key][row] = K[key][:] . Q[row][:]       A = K fragment, B = Q^T fragment
//     O^T[d][row]  += V^T[d][key] . P^T[key][row] A = V^T fragment, B = P^T fragment
//
// Wave pairs: the two waves of a pair share 64 query rows. Wave e of the pair
// takes every other key tile (tiles t = e mod 2): QK of its tile for all 64 rows
// (each K fragment read from LDS feeds two MFMAs), the softmax of that tile, and
// PV of d-half e (d in 128e .. 128e+127) for all 64 rows over both tiles of the
// pair step (each V fragment feeds two MFMAs), its own tile's P^T first (read
// back before the barrier), the partner's through LDS. This halves the LDS
// operand traffic of one-wave-per-32-rows tiling (one b128 read per MFMA). K
// tiles stream through an 8-slot LDS ring by direct global->LDS loads (issued
// two pair steps ahead); V^T fragments come straight from the workspace into
// registers one pair step ahead (the V^T transpose kernel writes each 32-key tile
// fragment-major, so every fragment is one coalesced 1-KB load). Per pair step
// and wave: 64 MFMAs, 16 K reads, 8 P reads, 4 P writes, 16 V loads, 8 tile
// loads, 32 exponentials; a three-stage software pipeline (QK of the next tile,
// softmax of the current one, PV of the previous pair) with one barrier.
//
// Loads whose results feed MFMAs directly (V^T, K and P^T fragments) are issued
// from inline asm with counted waits (the compiler would drain every load in
// flight, including the tile loads two steps ahead, before each use). Each of
// these registers is loaded and consumed inside one straight-line pair step: V^T
// at the start of the step for that step's PV (the QK phase hides the latency),
// K four fragments ahead within the QK phase, P^T just before the PV; the
// consumer reads the value through the wait statement, so no copy of it can be
// placed before its data has landed.
//
// Softmax: a static shift. The QK-norm weights bound every logit (|q op| <=
// max|qw + w_offset|, |k~| <= 16 max|kw + w_offset|); when that bound is at most
// 64 in log2 units it is the shift for every row. Otherwise an exact row max is
// taken first by a QK-only pass over the same tiles and used as each row's shift.
#include "common.h"
#include "kernels.h"

namespace vm {

namespace {

constexpr int FM = 128;                    // query rows per item
constexpr int FN = 32;                     // keys per tile
constexpr int FT = FN * HEAD_DIM;          // bf16 per K (or V) tile: 16 KB
constexpr float FSTATIC_LIMIT = 64.0f;

__device__ __forceinline__ void fbarrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// chunk c of K tile row r lives at chunk c ^ fswz(r): the 16 rows of each 16-lane
// group of a b128 read fall on distinct banks (64 banks of 4 bytes).
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

// ---- V^T tiles. Tile t of (b, hk) holds keys 32t .. 32t+31 as 16 MFMA
// A-operand fragments of 1 KB, fragment f = 2 * dblk + ks (d-block dblk of 32
// d-rows, key half ks): lane l's 16 bytes (at 1024 f + 16 l) are the 8 keys
// 16 ks + {4h .. 4h+3, 8+4h .. 8+4h+3} (h = l / 32) of d-row 32 dblk + l % 32 --
// the key order of the P^T operand that lane half h holds for key half ks (the
// S^T accumulator layout).
//
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
    const int f = o >> 6, l = o & 63;
    const int d = 32 * (f >> 1) + (l & 31);
    const int k0 = 16 * (f & 1) + 4 * (l >> 5);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int u0 = 2 * e, u1 = 2 * e + 1;  // element u: key k0 + (u & 3) + 8 (u >> 2)
      const uint32_t lo = tile[k0 + (u0 & 3) + 8 * (u0 >> 2)][d];
      const uint32_t hi = tile[k0 + (u1 & 3) + 8 * (u1 >> 2)][d];
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

// This wave's quarter of K tile t (clamped to the last tile) into `dst`: piece
// i = rows 2g, 2g+1 (g = 4 wave + i) as 64 lanes x 16 B. A whole tile is a
// scalar base plus per-lane unsigned byte offsets (the scalar-base addressing
// form); the last tile re-reads the last readable row past it (its keys are
// masked).
__device__ __forceinline__ void issue_quarter(const FCtx& c, int t, uint16_t* dst) {
  t = min(t, c.n_tiles - 1);
  const int row0 = t * FN;
  const char* src = reinterpret_cast<const char*>(c.kbase + (int64_t)row0 * c.kv_st);
  // rows past the last readable one re-read it (they are masked); one code path,
  // so every step issues the same count of loads
  const int last = c.krow_max - row0;
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

template <int N>
__device__ __forceinline__ void fwait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// waits for the inline-asm loads: they order against the asm that consumes
// their registers by program order alone
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(f32x16& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_acc(uint4& x) {
  u32x4 t = __builtin_bit_cast(u32x4, x);
  asm volatile("" : "+a"(t));
  x = __builtin_bit_cast(uint4, t);
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// acc + (the two bf16 of w summed), the row sum of a packed P^T pair
__device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                         __builtin_bit_cast(bf16x2, 0x3f803f80u), acc, false);
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
template <int OFF>
__device__ __forceinline__ void ds_w128(uint32_t addr, const uint4& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(addr), "v"(__builtin_bit_cast(u32x4, v)),
               "i"(OFF));
}

// ---- asm loads into compiler registers and the waits that release them. A load
// defines its value; the wait takes it (tied) so every reader is placed after the
// wait; the waits count in issue order (loads of one kind complete in order).
template <int OFF>
__device__ __forceinline__ u32x4 ds_b128(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int IMM>
__device__ __forceinline__ u32x4 g_b128(const char* base, uint32_t off) {
  static_assert(IMM >= 0 && IMM < 4096, "global offset is 13-bit signed");
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(r) : "v"(off), "s"(base), "i"(IMM));
  return r;
}
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
template <int IMM>
__device__ __forceinline__ u32x2 g_b64(const void* p) {
  u32x2 r;
  asm volatile("global_load_dwordx2 %0, %1, off offset:%2" : "=v"(r) : "v"(p), "i"(IMM));
  return r;
}
template <int N>
__device__ __forceinline__ void vm_take8(u32x2 (&g)[4][4], int dq0) {
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(g[dq0][0]), "+v"(g[dq0][1]), "+v"(g[dq0][2]), "+v"(g[dq0][3]),
                 "+v"(g[dq0 + 1][0]), "+v"(g[dq0 + 1][1]), "+v"(g[dq0 + 1][2]), "+v"(g[dq0 + 1][3])
               : "n"(N));
}
// a 16-byte workspace load into v in place (tied: whatever read the old contents
// of v is placed before it, and nothing can read the new contents before vm_take)
template <int IMM>
__device__ __forceinline__ void g_b128_into(u32x4& v, const char* base, uint32_t off) {
  static_assert(IMM >= 0 && IMM < 4096, "global offset is 13-bit signed");
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "+v"(v) : "v"(off), "s"(base), "i"(IMM));
}
template <int N>
__device__ __forceinline__ void lgkm_take(u32x4& x, u32x4& y) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "n"(N));
}
template <int N>
__device__ __forceinline__ void lgkm_take(u32x4& x, u32x4& y, u32x4& z, u32x4& w) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(x), "+v"(y), "+v"(z), "+v"(w) : "n"(N));
}
template <int N>
__device__ __forceinline__ void vm_take(u32x4& x, u32x4& y, u32x4& z, u32x4& w) {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%4)" : "+v"(x), "+v"(y), "+v"(z), "+v"(w) : "n"(N));
}
// S^T[key][row] (+)= K fragment . Q^T (S in VGPRs, Q in AGPRs); the builtin would
// accumulate in AGPRs. A dependent product always has another MFMA between it and
// its producer (the two row blocks alternate), which needs no wait states.
__device__ __forceinline__ void mfma_qk0(f32x16& s, const u32x4& k, const uint4& q) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0"
               : "=&v"(s) : "v"(k), "a"(__builtin_bit_cast(u32x4, q)));
}
__device__ __forceinline__ void mfma_qk(f32x16& s, const u32x4& k, const uint4& q) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
               : "+v"(s) : "v"(k), "a"(__builtin_bit_cast(u32x4, q)));
}

// 11+ wait states before a VALU reads what an 8-pass MFMA wrote (threaded
// through the results so no reader moves above the padding)
__device__ __forceinline__ void mfma_drain(f32x16& s0, f32x16& s1) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(s0), "+v"(s1));
}

// Item geometry.
struct ItemGeo {
  int b, h, hk, r0, q_len, prior, k_len, off, kend;
};

__device__ __forceinline__ ItemGeo item_geo(const PrefillArgs& a, const FItem& it, bool causal) {
  ItemGeo ig;
  ig.b = it.b; ig.h = it.h; ig.hk = it.hk;
  ig.r0 = it.qt * FM;
  ig.q_len = a.q_lengths ? min(a.q_lengths[it.b], a.L) : a.L;
  ig.prior = a.prior ? a.prior[it.b] : 0;
  ig.k_len = ig.prior + ig.q_len;  // queries are the suffix of the attended keys
  ig.off = ig.k_len - ig.q_len;
  ig.kend = causal ? min(ig.k_len, ig.off + ig.r0 + FM) : ig.k_len;
  return ig;
}

__device__ __forceinline__ void init_fctx(FCtx& c, const PrefillArgs& a, const ItemGeo& ig,
                                          int wave, int lane) {
  c.kbase = a.k + (int64_t)ig.b * a.kv_sb + (int64_t)ig.hk * a.kv_sh;
  c.vtbase = a.vt + ((int64_t)ig.b * a.Hk + ig.hk) * a.vt_tiles * FT;
  c.kv_st = a.kv_st;
  c.krow_max = max(0, min(ig.k_len, a.Lk) - 1);
  // tiles never reach past the cache (prior + q_len > Lk is a caller error: the
  // keys past Lk were never appended), so neither do the V^T workspace reads
  c.n_tiles = max(1, (min(ig.kend, a.Lk) + FN - 1) / FN);
  c.wave = wave;
  c.lane = lane;
  c.row_bytes = (uint32_t)(2 * a.kv_st);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 2 * (4 * wave + i) + (lane >> 5);
    c.dma_boff[i] = (uint32_t)r * c.row_bytes + (uint32_t)(((lane & 31) ^ fswz(r)) * 16);
  }
}

// raw q row, norm weight, and RoPE table operands of this lane (row `row` of head h)
struct QLoads {
  uint4 qraw[16], qwv[16];
  float4 cv[4], sv[4];
};

__device__ __forceinline__ void q_load_raw(const PrefillArgs& a, int b, int h, int row, int h2,
                                           QLoads& ql) {
  const int qrow = min(row, a.L - 1);
  const uint16_t* qp = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qrow * a.q_st + 8 * h2;
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) ql.qraw[kk] = load16(qp + 16 * kk);
}
__device__ __forceinline__ void q_load_rest(const PrefillArgs& a, int row, int prior, int h2,
                                            QLoads& ql) {
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) ql.qwv[kk] = load16(a.qw + 16 * kk + 8 * h2);
  const int64_t pos = min((int64_t)prior + min(row, a.L - 1), (int64_t)a.Lk - 1);
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      ql.cv[2 * kk + u] = *reinterpret_cast<const float4*>(a.cos_tab + pos * HALF_ROT + 8 * h2 + 16 * kk + 4 * u);
      ql.sv[2 * kk + u] = *reinterpret_cast<const float4*>(a.sin_tab + pos * HALF_ROT + 8 * h2 + 16 * kk + 4 * u);
    }
}

// q rows of one 32-row block: qnorm_rope (src/kernels/qknorm_rope_append.jl:25-57)
// and the 1/16 scale, with the per-row 1/rms folded into that final scale (RoPE
// is linear); lane holds q[row][16kk + 8h2 + j]
__device__ __forceinline__ void q_prologue(const PrefillArgs& a, const QLoads& ql, uint4 (&qop)[16]) {
  float ss = 0.f;
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    float x[8];
    unpack8(ql.qraw[kk], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  }
  ss += __shfl_xor(ss, 32, 64);
  const float scale = QK_SCALE / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
  const float* cs = reinterpret_cast<const float*>(ql.cv);
  const float* sn = reinterpret_cast<const float*>(ql.sv);
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    if (kk == 2 || kk == 3) continue;  // rotated with d-steps 0, 1
    float x1[8], wf[8];
    unpack8(ql.qraw[kk], x1);
    unpack8(ql.qwv[kk], wf);
#pragma unroll
    for (int j = 0; j < 8; ++j) x1[j] *= wf[j] + a.w_offset;
    if (kk < 2) {
      // d-steps 0..3 carry the rotary dims: pairs (d, d + 32) = d-steps (kk, kk + 2)
      float x2[8];
      unpack8(ql.qraw[kk + 2], x2);
      unpack8(ql.qwv[kk + 2], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x2[j] *= wf[j] + a.w_offset;
        const float cc = cs[8 * kk + j], si = sn[8 * kk + j];
        const float r1 = x1[j] * cc - x2[j] * si;
        const float r2 = x2[j] * cc + x1[j] * si;
        x1[j] = r1;
        x2[j] = r2;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) x2[j] *= scale;
      qop[kk + 2] = pack8(x2);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) x1[j] *= scale;
    qop[kk] = pack8(x1);
  }
}

// ============================ pair path ============================

struct PairState {
  uint4 qop[2][16];     // Q^T operands of the pair's two 32-row blocks (held in AGPRs)
  f32x16 o[4][2];       // O^T of d-blocks 4e .. 4e+3 x the two row blocks (AGPRs)
  f32x16 s[2];          // S^T of this wave's current tile, per row block
  uint32_t pprev[2][8]; // packed P^T of this wave's tile of the previous step
  u32x4 v[16];          // V^T of the next PV: own tile (0..7) then the partner's,
                        // d-block 4e + ((k & 7) >> 1), key half k & 1
  float lsum[2];        // row sums over this wave's tiles (this lane's keys)
};

struct PairCtx {
  FCtx c;             // K tile loads
  const char* vt;     // V^T tiles of (b, hk)
  uint32_t voff;      // e * 8 KB + 16 lane: this lane's bytes of the wave's d-half
  int koffe[8];       // K fragment byte offsets in a ring object (this wave's half)
  uint32_t pxr;       // P exchange: this pair's region (tile-0 wave; tile-1 wave +4 KB)
  uint32_t pxw;       // P exchange: this wave's region
  float negm[2];      // minus the softmax shift of this lane's row in each row block
  const uint16_t* gate_row[2];  // gate logits of this lane's row in each row block
};

struct PairGeo {
  int prow0;   // first row of the pair
  int row[2];  // this lane's row in each row block
  int off, k_len;
};

// LDS objects: K ring slots 2s, 2s+1 in object s (halves), and the P exchange
// area (two buffers x four waves x 4 KB)
struct PairLds {
  uint16_t* ring;  // the four objects, 2 FT elements each
  uint16_t* PX;
  __device__ __forceinline__ uint16_t* obj(int j) const { return ring + j * (2 * FT); }
};

template <bool CAUSAL>
__device__ __forceinline__ bool pair_needs_mask(const PairGeo& g, int t) {
  return (t * FN + FN > g.k_len) || (CAUSAL && t * FN + FN - 1 > g.off + g.prow0);
}
template <bool CAUSAL>
__device__ __forceinline__ void pair_mask(const PairGeo& g, int t, int lane, f32x16 (&s)[2]) {
  const int key0 = t * FN + 4 * (lane >> 5);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int lim = CAUSAL ? min(g.k_len - 1, g.row[rb] + g.off) : g.k_len - 1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = key0 + 8 * (i >> 2) + (i & 3);
      s[rb][i] = key <= lim ? s[rb][i] : -INFINITY;
    }
  }
}

// softmax of elements j0, j0+1 of one row block with the shift: packed P^T word
// (bf16 pair) and the row sum of what was packed
__device__ __forceinline__ uint32_t pair_p2(const f32x16& s, int j0, float negm, float& lsum) {
  const float p0 = fast_exp2(__builtin_fmaf(s[j0], LOG2E, negm));
  const float p1 = fast_exp2(__builtin_fmaf(s[j0 + 1], LOG2E, negm));
  uint32_t w = pack2(p0, p1);
  pin(w);
  lsum = dot2_ones(w, lsum);
  pin(lsum);  // summed here, not deferred (which would keep every word live)
  return w;
}

__device__ __forceinline__ void k_addrs(const PairCtx& pc, const uint16_t* obj, uint32_t (&ka)[8]) {
  const uint32_t kb = lds_addr(obj);
#pragma unroll
  for (int q = 0; q < 8; ++q) ka[q] = kb + pc.koffe[q];
}

// QK of this wave's tile for both row blocks, as 8 pairs of K fragments (fragment
// kk: chunk 2kk + h2 of row l%32, at ka[kk & 7] + 256 (kk >> 3)), read 4 ahead.
// The caller issued reads 0..3 last (anything LDS older may be outstanding: the
// waits only need those to be done too). SM: softmax slice p (words 2p, 2p+1 of
// row block p >> 2) rides along pair p.
#define PRK(kk) (kf[kk] = ds_b128<256 * ((kk) >> 3)>(ka[(kk) & 7]))
template <int P, bool SM>
__device__ __forceinline__ void qk_pair(PairState& st, const PairCtx& pc, const uint32_t (&ka)[8],
                                        u32x4 (&kf)[16], const f32x16& s0, const f32x16& s1,
                                        uint32_t (&pw)[2][8]) {
  // LDS ops issued after read 2P+1 at this point: reads 2P+2, 2P+3
  constexpr int W = P < 7 ? 2 : 0;
  lgkm_take<W>(kf[2 * P], kf[2 * P + 1]);
  if constexpr (P == 0) {
    mfma_qk0(st.s[0], kf[0], st.qop[0][0]);
    mfma_qk0(st.s[1], kf[0], st.qop[1][0]);
  } else {
    mfma_qk(st.s[0], kf[2 * P], st.qop[0][2 * P]);
    mfma_qk(st.s[1], kf[2 * P], st.qop[1][2 * P]);
  }
  mfma_qk(st.s[0], kf[2 * P + 1], st.qop[0][2 * P + 1]);
  mfma_qk(st.s[1], kf[2 * P + 1], st.qop[1][2 * P + 1]);
  if constexpr (P < 6) {
    PRK(2 * P + 4);
    PRK(2 * P + 5);
  }
  if constexpr (SM) {
    constexpr int RB = P >> 2, W0 = (2 * P) & 7;
    pw[RB][W0] = pair_p2(RB == 0 ? s0 : s1, 2 * W0, pc.negm[RB], st.lsum[RB]);
    pw[RB][W0 + 1] = pair_p2(RB == 0 ? s0 : s1, 2 * W0 + 2, pc.negm[RB], st.lsum[RB]);
  }
}
template <bool SM>
__device__ __forceinline__ void qk_phase(PairState& st, const PairCtx& pc, const uint32_t (&ka)[8],
                                         u32x4 (&kf)[16], const f32x16& s0, const f32x16& s1,
                                         uint32_t (&pw)[2][8]) {
#define QP(p) qk_pair<p, SM>(st, pc, ka, kf, s0, s1, pw)
  QP(0); QP(1); QP(2); QP(3); QP(4); QP(5); QP(6); QP(7);
#undef QP
  mfma_drain(st.s[0], st.s[1]);
}

// this wave's P^T words of its tile to the exchange
__device__ __forceinline__ void p_publish(const PairCtx& pc, uint32_t pbuf, const uint32_t (&pw)[2][8]) {
  const uint32_t wa = pc.pxw + pbuf;
  ds_w128<0>(wa, make_uint4(pw[0][0], pw[0][1], pw[0][2], pw[0][3]));
  ds_w128<1024>(wa, make_uint4(pw[0][4], pw[0][5], pw[0][6], pw[0][7]));
  ds_w128<2048>(wa, make_uint4(pw[1][0], pw[1][1], pw[1][2], pw[1][3]));
  ds_w128<3072>(wa, make_uint4(pw[1][4], pw[1][5], pw[1][6], pw[1][7]));
}

// V^T of one PV position k (own tile for k < 8, the partner's after) into slot k
template <int K>
__device__ __forceinline__ void v_load(PairState& st, const char* vbo, const char* vbp, uint32_t vo0,
                                       uint32_t vo1) {
  g_b128_into<(K & 3) * 1024>(st.v[K], K < 8 ? vbo : vbp, (K & 4) ? vo1 : vo0);
}
__device__ __forceinline__ void v_tiles(const PairCtx& pc, int t_own, int t_part, const char*& vbo,
                                        const char*& vbp) {
  const int n = pc.c.n_tiles;
  vbo = pc.vt + (int64_t)min(t_own, n - 1) * (2 * FT);
  vbp = pc.vt + (int64_t)min(t_part, n - 1) * (2 * FT);
}

// Step 0: softmax of this wave's tile e, the V^T of step 1 (tiles e, 1-e; order:
// 4 V, the K loads of tiles 6, 7 into object 3, 12 V), QK of its tile 2+e (object
// 1), the P^T of tile e to the exchange (buffer 0).
template <bool CAUSAL>
__device__ __forceinline__ void pair_first(PairState& st, const PairCtx& pc, const PairLds& L,
                                           const PairGeo& g, int e, int lane) {
  fwait_vmcnt<8>();  // K(2), K(3) (K(4), K(5) may be in flight)
  fbarrier();
  if (pair_needs_mask<CAUSAL>(g, e)) pair_mask<CAUSAL>(g, e, lane, st.s);
  uint32_t ka[8];
  u32x4 kf[16];
  k_addrs(pc, L.obj(1), ka);
  PRK(0); PRK(1); PRK(2); PRK(3);
  const char *vbo, *vbp;
  v_tiles(pc, e, 1 - e, vbo, vbp);
  const uint32_t vo0 = pc.voff, vo1 = pc.voff + 4096;
  v_load<0>(st, vbo, vbp, vo0, vo1); v_load<1>(st, vbo, vbp, vo0, vo1);
  v_load<2>(st, vbo, vbp, vo0, vo1); v_load<3>(st, vbo, vbp, vo0, vo1);
  issue_quarter(pc.c, 6, L.obj(3));
  issue_quarter(pc.c, 7, L.obj(3) + FT);
  v_load<4>(st, vbo, vbp, vo0, vo1);   v_load<5>(st, vbo, vbp, vo0, vo1);
  v_load<6>(st, vbo, vbp, vo0, vo1);   v_load<7>(st, vbo, vbp, vo0, vo1);
  v_load<8>(st, vbo, vbp, vo0, vo1);   v_load<9>(st, vbo, vbp, vo0, vo1);
  v_load<10>(st, vbo, vbp, vo0, vo1);  v_load<11>(st, vbo, vbp, vo0, vo1);
  v_load<12>(st, vbo, vbp, vo0, vo1);  v_load<13>(st, vbo, vbp, vo0, vo1);
  v_load<14>(st, vbo, vbp, vo0, vo1);  v_load<15>(st, vbo, vbp, vo0, vo1);
  f32x16 s0 = st.s[0], s1 = st.s[1];
  pin(s0);
  pin(s1);
  uint32_t pw[2][8];
  qk_phase<true>(st, pc, ka, kf, s0, s1, pw);
  p_publish(pc, 0u, pw);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int q = 0; q < 8; ++q) st.pprev[rb][q] = pw[rb][q];
  lgkm_wait<0>();  // the P writes land before the next barrier
}

// One PV position k of a step: slot k on both row blocks (own tile with the P^T
// kept from the last step, the partner's with pf), then (LOAD) slot k's
// successor for the next step, the K loads after slot 3.
template <int K, bool LOAD>
__device__ __forceinline__ void pv_pos(PairState& st, const PairCtx& pc, const u32x4 (&pf)[4],
                                       const char* vbo, const char* vbp, uint32_t vo0, uint32_t vo1,
                                       int i, uint16_t* dma_dst) {
  constexpr int DQ = (K & 7) >> 1, KS = K & 1;
  uint4 p0, p1;
  if constexpr (K < 8) {
    p0 = make_uint4(st.pprev[0][4 * KS], st.pprev[0][4 * KS + 1], st.pprev[0][4 * KS + 2], st.pprev[0][4 * KS + 3]);
    p1 = make_uint4(st.pprev[1][4 * KS], st.pprev[1][4 * KS + 1], st.pprev[1][4 * KS + 2], st.pprev[1][4 * KS + 3]);
  } else {
    p0 = __builtin_bit_cast(uint4, pf[KS]);
    p1 = __builtin_bit_cast(uint4, pf[2 + KS]);
  }
  st.o[DQ][0] = mfma32(__builtin_bit_cast(uint4, st.v[K]), p0, st.o[DQ][0]);
  st.o[DQ][1] = mfma32(__builtin_bit_cast(uint4, st.v[K]), p1, st.o[DQ][1]);
  if constexpr (LOAD) {
    v_load<K>(st, vbo, vbp, vo0, vo1);
    if constexpr (K == 3) {
      issue_quarter(pc.c, 2 * i + 6, dma_dst);
      issue_quarter(pc.c, 2 * i + 7, dma_dst + FT);
    }
  }
}

// Steps 1 .. n_it-1 (ring slots from i at run time): PV of tiles 2i-2, 2i-1 from
// the V^T loaded last step (own tile first: its P^T is in registers; the
// partner's P^T was read at the start), each slot reloaded for step i+1 (tiles
// 2i, 2i+1; the K loads of tiles 2i+6, 2i+7 into object (i+3) % 4 after slot 3);
// then QK of this wave's tile 2i+2+e (object (i+1) % 4) with the softmax of its
// tile 2i+e riding along; its P^T to exchange buffer i & 1. (The last of these
// steps computes a QK nobody reads.)
template <bool CAUSAL>
__device__ __forceinline__ void pair_steady(PairState& st, const PairCtx& pc, const PairLds& L,
                                            const PairGeo& g, int i, int e, int lane) {
  // K(2i+2), K(2i+3) (loaded at step i-2) landed: only step i-1's 8 tile + 16 V
  // loads may still be in flight; every wave is past step i-1
  fwait_vmcnt<24>();
  fbarrier();
  if (pair_needs_mask<CAUSAL>(g, 2 * i + e)) pair_mask<CAUSAL>(g, 2 * i + e, lane, st.s);
  const uint32_t pbuf_r = ((i - 1) & 1) * 16384u, pbuf_w = (i & 1) * 16384u;
  u32x4 pf[4], kf[16];
  {
    const uint32_t prd = pc.pxr + pbuf_r + (1 - e) * 4096;
    pf[0] = ds_b128<0>(prd);
    pf[1] = ds_b128<1024>(prd);
    pf[2] = ds_b128<2048>(prd);
    pf[3] = ds_b128<3072>(prd);
  }
  uint32_t ka[8];
  k_addrs(pc, L.obj((i + 1) & 3), ka);
  PRK(0); PRK(1); PRK(2); PRK(3);
  const char *vbo, *vbp;
  v_tiles(pc, 2 * i + e, 2 * i + 1 - e, vbo, vbp);
  const uint32_t vo0 = pc.voff, vo1 = pc.voff + 4096;
  uint16_t* dma_dst = L.obj((i + 3) & 3);
  // slots 4g .. 4g+3 of step i-1 landed: loads issued after slot 4g+3 are its
  // 12 - 4g later V loads and its 8 tile loads (after slot 3), plus this step's
  // 4g V loads and (g > 0) 8 tile loads: 20 in every case
#define PVP(k) pv_pos<k, true>(st, pc, pf, vbo, vbp, vo0, vo1, i, dma_dst)
  vm_take<20>(st.v[0], st.v[1], st.v[2], st.v[3]);
  PVP(0); PVP(1); PVP(2); PVP(3);
  vm_take<20>(st.v[4], st.v[5], st.v[6], st.v[7]);
  PVP(4); PVP(5); PVP(6); PVP(7);
  vm_take<20>(st.v[8], st.v[9], st.v[10], st.v[11]);
  lgkm_take<4>(pf[0], pf[1], pf[2], pf[3]);  // only K reads 0..3 are younger
  PVP(8); PVP(9); PVP(10); PVP(11);
  vm_take<20>(st.v[12], st.v[13], st.v[14], st.v[15]);
  PVP(12); PVP(13); PVP(14); PVP(15);
#undef PVP
  f32x16 s0 = st.s[0], s1 = st.s[1];
  pin(s0);
  pin(s1);
  uint32_t pw[2][8];
  qk_phase<true>(st, pc, ka, kf, s0, s1, pw);
  p_publish(pc, pbuf_w, pw);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int q = 0; q < 8; ++q) st.pprev[rb][q] = pw[rb][q];
  lgkm_wait<0>();  // the P writes land before the next barrier
}

// Step n_it: PV of the last two tiles only; the epilogue's gate logits go out
// first (4 bf16 at d = 32 (4e + dq) + 8 jb + 4 h2 of this lane's row in each row
// block: 32 loads).
__device__ __forceinline__ void pair_last(PairState& st, const PairCtx& pc, int i, int e, int lane,
                                          u32x2 (&gv)[2][4][4]) {
  fbarrier();  // the partner's P^T of step i-1 is in
  const uint32_t pbuf_r = ((i - 1) & 1) * 16384u;
  u32x4 pf[4];
  {
    const uint32_t prd = pc.pxr + pbuf_r + (1 - e) * 4096;
    pf[0] = ds_b128<0>(prd);
    pf[1] = ds_b128<1024>(prd);
    pf[2] = ds_b128<2048>(prd);
    pf[3] = ds_b128<3072>(prd);
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const uint16_t* gp = pc.gate_row[rb] + 32 * (4 * e) + 4 * (lane >> 5);
    gv[rb][0][0] = g_b64<0>(gp);    gv[rb][0][1] = g_b64<16>(gp);
    gv[rb][0][2] = g_b64<32>(gp);   gv[rb][0][3] = g_b64<48>(gp);
    gv[rb][1][0] = g_b64<64>(gp);   gv[rb][1][1] = g_b64<80>(gp);
    gv[rb][1][2] = g_b64<96>(gp);   gv[rb][1][3] = g_b64<112>(gp);
    gv[rb][2][0] = g_b64<128>(gp);  gv[rb][2][1] = g_b64<144>(gp);
    gv[rb][2][2] = g_b64<160>(gp);  gv[rb][2][3] = g_b64<176>(gp);
    gv[rb][3][0] = g_b64<192>(gp);  gv[rb][3][1] = g_b64<208>(gp);
    gv[rb][3][2] = g_b64<224>(gp);  gv[rb][3][3] = g_b64<240>(gp);
  }
  // slots 4g .. 4g+3 of step i-1 landed: after slot 4g+3 came its 12 - 4g later
  // V loads, (g = 0) its 8 tile loads, and the 32 gate loads
#define PVP(k) pv_pos<k, false>(st, pc, pf, nullptr, nullptr, 0u, 0u, i, nullptr)
  vm_take<52>(st.v[0], st.v[1], st.v[2], st.v[3]);
  PVP(0); PVP(1); PVP(2); PVP(3);
  vm_take<40>(st.v[4], st.v[5], st.v[6], st.v[7]);
  PVP(4); PVP(5); PVP(6); PVP(7);
  vm_take<36>(st.v[8], st.v[9], st.v[10], st.v[11]);
  lgkm_take<0>(pf[0], pf[1], pf[2], pf[3]);
  PVP(8); PVP(9); PVP(10); PVP(11);
  vm_take<32>(st.v[12], st.v[13], st.v[14], st.v[15]);
  PVP(12); PVP(13); PVP(14); PVP(15);
#undef PVP
}

// Exact row max of S over the item's keys for this pair's rows (the QK-only pass
// for weights whose bound is too loose for a static shift). Step i reads K(2i),
// K(2i+1) from ring object i % 4 and loads K(2i+6), K(2i+7) into object (i+3) % 4.
template <bool CAUSAL, int J4>
__device__ __forceinline__ void max_step(PairState& st, const PairCtx& pc, const PairLds& L,
                                         const PairGeo& g, int i, int e, int lane, float (&m)[2]) {
  // K(2i), K(2i+1) landed: the loads after them are two steps' tile loads
  fwait_vmcnt<16>();
  fbarrier();
  uint32_t ka[8];
  u32x4 kf[16];
  uint32_t pw[2][8];
  k_addrs(pc, L.obj(J4), ka);
  PRK(0); PRK(1); PRK(2); PRK(3);
  issue_quarter(pc.c, 2 * i + 6, L.obj((J4 + 3) % 4));
  issue_quarter(pc.c, 2 * i + 7, L.obj((J4 + 3) % 4) + FT);
  qk_phase<false>(st, pc, ka, kf, st.s[0], st.s[1], pw);
  if (pair_needs_mask<CAUSAL>(g, 2 * i + e)) pair_mask<CAUSAL>(g, 2 * i + e, lane, st.s);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int j = 0; j < 16; ++j) m[rb] = fmaxf(m[rb], st.s[rb][j]);
}

template <bool CAUSAL>
__device__ __forceinline__ void prime_ring(const PairCtx& pc, const PairLds& L) {
  // K(0) .. K(5) into objects 0..2 (object 3 and the exchange area are free)
  issue_quarter(pc.c, 0, L.obj(0));
  issue_quarter(pc.c, 1, L.obj(0) + FT);
  issue_quarter(pc.c, 2, L.obj(1));
  issue_quarter(pc.c, 3, L.obj(1) + FT);
  issue_quarter(pc.c, 4, L.obj(2));
  issue_quarter(pc.c, 5, L.obj(2) + FT);
}

// One item (shift: the static softmax shift in log2 units, or < 0 for the
// exact-max pass).
template <bool CAUSAL>
__device__ __forceinline__ void pair_item(const PrefillArgs& a, const FItem& it, const PairLds& L,
                                          float shift) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h2 = lane >> 5;
  const int pr = wave >> 1, e = wave & 1;
  const ItemGeo ig = item_geo(a, it, CAUSAL);
  const int prow0 = ig.r0 + 64 * pr;
  const int row_own = prow0 + 32 * e + l32;  // this wave computes row block e's q
  QLoads ql;
  q_load_raw(a, ig.b, ig.h, row_own, h2, ql);
  if (ig.r0 >= ig.q_len) return;  // uniform over the workgroup
  PairGeo g;
  g.prow0 = prow0;
  g.row[0] = prow0 + l32;
  g.row[1] = prow0 + 32 + l32;
  g.off = ig.off;
  g.k_len = ig.k_len;
  PairCtx pc;
  init_fctx(pc.c, a, ig, wave, lane);
  pc.vt = reinterpret_cast<const char*>(pc.c.vtbase);
  pc.voff = (uint32_t)(e * 8192 + 16 * lane);
  {
    const int sk = fswz(l32);
#pragma unroll
    for (int q = 0; q < 8; ++q) pc.koffe[q] = e * (2 * FT) + l32 * 512 + 16 * ((2 * q + h2) ^ sk);
  }
  pc.pxr = lds_addr(L.PX) + (2 * pr) * 4096 + 16 * lane;
  pc.pxw = lds_addr(L.PX) + wave * 4096 + 16 * lane;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
    pc.gate_row[rb] = a.gate + (int64_t)ig.b * a.g_sb + (int64_t)ig.h * a.g_sh +
                      (int64_t)min(g.row[rb], a.L - 1) * a.g_st;
  q_load_rest(a, row_own, ig.prior, h2, ql);
  prime_ring<CAUSAL>(pc, L);

  PairState st;
  {
    uint4 qown[16];
    q_prologue(a, ql, qown);
    // exchange: wave w's 16 fragments (16 KB) in object 3 (waves 0, 1) or PX (2, 3)
    const uint32_t xbase = wave < 2 ? lds_addr(L.obj(3)) : lds_addr(L.PX);
    const uint32_t xw = xbase + e * (2 * FT) + 16 * lane;
    const uint32_t xr = xbase + (1 - e) * (2 * FT) + 16 * lane;
    ds_w128<0>(xw, qown[0]);         ds_w128<1024>(xw, qown[1]);
    ds_w128<2048>(xw, qown[2]);      ds_w128<3072>(xw, qown[3]);
    ds_w128<4096>(xw, qown[4]);      ds_w128<5120>(xw, qown[5]);
    ds_w128<6144>(xw, qown[6]);      ds_w128<7168>(xw, qown[7]);
    ds_w128<8192>(xw, qown[8]);      ds_w128<9216>(xw, qown[9]);
    ds_w128<10240>(xw, qown[10]);    ds_w128<11264>(xw, qown[11]);
    ds_w128<12288>(xw, qown[12]);    ds_w128<13312>(xw, qown[13]);
    ds_w128<14336>(xw, qown[14]);    ds_w128<15360>(xw, qown[15]);
    // K(0), K(1) landed (K(2) .. K(5) may be in flight); the exchange written
    fwait_vmcnt<16>();
    lgkm_wait<0>();
    fbarrier();
    // the partner's fragments: reads and their wait in one statement (the
    // outputs exist only once the data is in)
    u32x4 qx[16];
    asm volatile(
        "ds_read_b128 %0, %16 offset:0\n\tds_read_b128 %1, %16 offset:1024\n\t"
        "ds_read_b128 %2, %16 offset:2048\n\tds_read_b128 %3, %16 offset:3072\n\t"
        "ds_read_b128 %4, %16 offset:4096\n\tds_read_b128 %5, %16 offset:5120\n\t"
        "ds_read_b128 %6, %16 offset:6144\n\tds_read_b128 %7, %16 offset:7168\n\t"
        "ds_read_b128 %8, %16 offset:8192\n\tds_read_b128 %9, %16 offset:9216\n\t"
        "ds_read_b128 %10, %16 offset:10240\n\tds_read_b128 %11, %16 offset:11264\n\t"
        "ds_read_b128 %12, %16 offset:12288\n\tds_read_b128 %13, %16 offset:13312\n\t"
        "ds_read_b128 %14, %16 offset:14336\n\tds_read_b128 %15, %16 offset:15360\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(qx[0]), "=&v"(qx[1]), "=&v"(qx[2]), "=&v"(qx[3]), "=&v"(qx[4]), "=&v"(qx[5]),
          "=&v"(qx[6]), "=&v"(qx[7]), "=&v"(qx[8]), "=&v"(qx[9]), "=&v"(qx[10]), "=&v"(qx[11]),
          "=&v"(qx[12]), "=&v"(qx[13]), "=&v"(qx[14]), "=&v"(qx[15])
        : "v"(xr));
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const uint4 other = __builtin_bit_cast(uint4, qx[kk]);
      st.qop[0][kk] = e == 0 ? qown[kk] : other;
      st.qop[1][kk] = e == 0 ? other : qown[kk];
    }
  }
  // rows past the chunk hold finite junk q; their outputs are never stored
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) pin_acc(st.qop[rb][kk]);

  const int n_it = (pc.c.n_tiles + 1) >> 1;
  if (shift >= 0.f) {
    pc.negm[0] = -shift;
    pc.negm[1] = -shift;
  } else {
    // exact row max (QK only), combined over the pair through the exchange area
    float m[2] = {-INFINITY, -INFINITY};
    int i = 0;
    for (; i + 3 < n_it; i += 4) {
      max_step<CAUSAL, 0>(st, pc, L, g, i, e, lane, m);
      max_step<CAUSAL, 1>(st, pc, L, g, i + 1, e, lane, m);
      max_step<CAUSAL, 2>(st, pc, L, g, i + 2, e, lane, m);
      max_step<CAUSAL, 3>(st, pc, L, g, i + 3, e, lane, m);
    }
    if (i < n_it) max_step<CAUSAL, 0>(st, pc, L, g, i, e, lane, m);
    if (i + 1 < n_it) max_step<CAUSAL, 1>(st, pc, L, g, i + 1, e, lane, m);
    if (i + 2 < n_it) max_step<CAUSAL, 2>(st, pc, L, g, i + 2, e, lane, m);
    fwait_vmcnt<0>();
    fbarrier();  // ring and exchange area free again
    float* lx = reinterpret_cast<float*>(L.PX);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      m[rb] = xor32_max(m[rb]);
      if (h2 == 0) lx[wave * 64 + rb * 32 + l32] = m[rb];
    }
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const float mr = fmaxf(m[rb], lx[(wave ^ 1) * 64 + rb * 32 + l32]) * LOG2E;
      pc.negm[rb] = mr == -INFINITY ? 0.f : -mr;  // fully-masked row: P = 0
    }
    __syncthreads();
    prime_ring<CAUSAL>(pc, L);
    fwait_vmcnt<16>();  // K(0), K(1)
    fbarrier();
  }
#pragma unroll
  for (int dq = 0; dq < 4; ++dq)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int j = 0; j < 16; ++j) st.o[dq][rb][j] = 0.f;
  st.lsum[0] = 0.f;
  st.lsum[1] = 0.f;

  // S^T of tile e (object 0, half e)
  {
    uint32_t ka[8];
    u32x4 kf[16];
    uint32_t pw[2][8];
    k_addrs(pc, L.obj(0), ka);
    PRK(0); PRK(1); PRK(2); PRK(3);
    qk_phase<false>(st, pc, ka, kf, st.s[0], st.s[1], pw);
  }

  u32x2 gv[2][4][4];
  pair_first<CAUSAL>(st, pc, L, g, e, lane);
  for (int i = 1; i < n_it; ++i) pair_steady<CAUSAL>(st, pc, L, g, i, e, lane);
  pair_last(st, pc, n_it, e, lane, gv);

  // ---- epilogue: row sums of both waves of the pair through LDS, normalise,
  // gate (sigmoid, src/kernels/kernels.jl:34), store this wave's d-half in the Wo
  // input layout
  fbarrier();  // every wave is done with the P exchange area
  float* lx = reinterpret_cast<float*>(L.PX);
  float lrow[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    lrow[rb] = st.lsum[rb] + __shfl_xor(st.lsum[rb], 32, 64);
    if (h2 == 0) lx[wave * 64 + rb * 32 + l32] = lrow[rb];
  }
  __syncthreads();
  vm_take8<0>(gv[0], 0);
  vm_take8<0>(gv[0], 2);
  vm_take8<0>(gv[1], 0);
  vm_take8<0>(gv[1], 2);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float l_tot = lrow[rb] + lx[(wave ^ 1) * 64 + rb * 32 + l32];
    const float inv = l_tot > 0.f ? fast_rcp(l_tot) : 0.f;  // fully-masked row -> 0
    const int row = g.row[rb];
    if (row < ig.q_len) {
      uint16_t* op = a.o + (int64_t)ig.b * a.o_sb + (int64_t)ig.h * a.o_sh + (int64_t)row * a.o_st;
#pragma unroll
      for (int dq = 0; dq < 4; ++dq) {
        const f32x16& acc = st.o[dq][rb];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int d0 = 32 * (4 * e + dq) + 8 * jb + 4 * h2;
          const uint2 g2 = make_uint2(gv[rb][dq][jb].x, gv[rb][dq][jb].y);
          const float o0 = acc[4 * jb + 0] * inv * sigmoidf(__uint_as_float(g2.x << 16));
          const float o1 = acc[4 * jb + 1] * inv * sigmoidf(__uint_as_float(g2.x & 0xffff0000u));
          const float o2 = acc[4 * jb + 2] * inv * sigmoidf(__uint_as_float(g2.y << 16));
          const float o3 = acc[4 * jb + 3] * inv * sigmoidf(__uint_as_float(g2.y & 0xffff0000u));
          uint2 ov;
          ov.x = pack2(o0, o1);
          ov.y = pack2(o2, o3);
          *reinterpret_cast<uint2*>(op + d0) = ov;
        }
      }
    }
  }
}
#undef PRK

}  // namespace

template <bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_fused_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t RING[4 * 2 * FT], PX[2 * FT];
  const int lane = threadIdx.x & 63;
  // static bounds from the norm weights: |k~| <= sqrt(D) * max|kw + w_offset| for
  // every cached row, |q op| <= max|qw + w_offset| for every scaled query row
  // (RMS-normalised rows have norm <= sqrt(D)); 1% covers the bf16 roundings
  float kmax, qmax;
  {
    const uint2 kv = *reinterpret_cast<const uint2*>(a.kw + 4 * lane);
    const uint2 qv = *reinterpret_cast<const uint2*>(a.qw + 4 * lane);
    kmax = fmaxf(fmaxf(fabsf(__uint_as_float(kv.x << 16) + a.w_offset),
                       fabsf(__uint_as_float(kv.x & 0xffff0000u) + a.w_offset)),
                 fmaxf(fabsf(__uint_as_float(kv.y << 16) + a.w_offset),
                       fabsf(__uint_as_float(kv.y & 0xffff0000u) + a.w_offset)));
    qmax = fmaxf(fmaxf(fabsf(__uint_as_float(qv.x << 16) + a.w_offset),
                       fabsf(__uint_as_float(qv.x & 0xffff0000u) + a.w_offset)),
                 fmaxf(fabsf(__uint_as_float(qv.y << 16) + a.w_offset),
                       fabsf(__uint_as_float(qv.y & 0xffff0000u) + a.w_offset)));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      kmax = fmaxf(kmax, __shfl_xor(kmax, m, 64));
      qmax = fmaxf(qmax, __shfl_xor(qmax, m, 64));
    }
  }
  const float bound = qmax * 1.01f * 16.0f * kmax * 1.01f * LOG2E;  // >= every |logit|, log2 units
  PairLds L;
  L.ring = RING;
  L.PX = PX;
  pair_item<CAUSAL>(a, item_at(a, blockIdx.x), L, bound <= FSTATIC_LIMIT ? bound : -1.0f);
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
  // one item per workgroup, heaviest first (the hardware hands the next item to
  // the first CU that frees up)
  if (a.causal)
    hipLaunchKernelGGL((prefill_fused_kernel<true>), dim3((unsigned)n_items), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((prefill_fused_kernel<false>), dim3((unsigned)n_items), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace vm

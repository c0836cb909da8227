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
  c.krow_max = a.Lk - 1;  // rows up to here are readable (past k_len: masked)
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
  const float scale = QK_SCALE * LOG2E / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
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

// ============================ one wave per 32 rows ============================

constexpr int NSLOT = 16;  // slots per step: 4 MFMAs, 4 LDS reads, 1 softmax word each

// nothing is scheduled across this point (pins the VALU work between the MFMAs)
__device__ __forceinline__ void sfence() { __builtin_amdgcn_sched_barrier(0); }

struct SoloState {
  uint4 qop[16];     // Q^T operands of this wave's 32 rows (AGPRs)
  f32x16 o[8];       // O^T, d-blocks 0..7 (AGPRs)
  f32x16 s[2][2];    // shifted S^T in log2 units, by step parity and tile
  u32x4 p[2][4];     // packed P^T, by step parity and key step
  f32x16 c0;         // minus this lane's row shift in every element (first QK accumulator)
  float lsum;        // row sum of this lane's packed P^T
};

struct SoloCtx {
  FCtx c;             // K tile loads
  const char* vt;     // V^T tiles of (b, hk)
  uint32_t vsrc;      // this wave's first V^T piece of a tile, this lane's bytes: 4 KB wave + 16 lane
  uint32_t kaddr[8];  // LDS address of K fragment q (and q + 8 at +256) in tile 0 of K object 0
  uint32_t vaddr;     // LDS address of this lane's V^T bytes in tile 0 of V object 0
};

struct SoloGeo {
  int wrow0;  // first row of this wave
  int row;    // this lane's row
  int off, k_len;
};

// K objects (two tiles each, swizzled rows) and V^T objects (two tiles each,
// fragment-major); object j holds step block j's tiles
struct SoloLds {
  uint16_t* k;
  uint16_t* v;
};

template <bool CAUSAL>
__device__ __forceinline__ bool solo_needs_mask(const SoloGeo& g, int blk) {
  const int last = blk * (2 * FN) + 2 * FN - 1;
  return (last >= g.k_len) || (CAUSAL && last > g.off + g.wrow0);
}
template <bool CAUSAL>
__device__ __forceinline__ void solo_mask(const SoloGeo& g, int blk, int lane, f32x16 (&s)[2]) {
  const int lim = CAUSAL ? min(g.k_len - 1, g.row + g.off) : g.k_len - 1;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int key0 = blk * (2 * FN) + t * FN + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = key0 + 8 * (j >> 2) + (j & 3);
      s[t][j] = key <= lim ? s[t][j] : -INFINITY;
    }
  }
}

// S^T = K fragment . Q^T + c: the first d-step, the accumulator starts at the shift
__device__ __forceinline__ void mfma_qkc(f32x16& s, const u32x4& k, const uint4& q, const f32x16& c) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3"
               : "=&v"(s) : "v"(k), "a"(__builtin_bit_cast(u32x4, q)), "v"(c));
}
// O^T += V^T fragment . P^T, O in AGPRs
__device__ __forceinline__ void mfma_pv(f32x16& o, const u32x4& v, const u32x4& p) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(o) : "v"(v), "v"(p));
}

// K tile t (clamped to the last tile) piece p of this wave (rows 2g, 2g+1 with
// g = 4 wave + p) into the tile at dst; a tile reaching past the cache re-reads
// its last row (those keys are masked)
__device__ __forceinline__ void k_dma(const FCtx& c, int t, uint16_t* dst, int p) {
  t = min(t, c.n_tiles - 1);
  const int row0 = t * FN;
  const char* src = reinterpret_cast<const char*>(c.kbase + (int64_t)row0 * c.kv_st);
  const int g = 4 * c.wave + p;
  uint32_t off = c.dma_boff[p];
  if (row0 + FN - 1 > c.krow_max) {
    const int r = 2 * g + (c.lane >> 5);
    off -= (uint32_t)max(0, r - (c.krow_max - row0)) * c.row_bytes;
  }
  __builtin_amdgcn_global_load_lds((const void*)(src + off),
                                   (__attribute__((address_space(3))) void*)(dst + g * 512), 16, 0, 0);
}
// V^T tile t (clamped) piece 4 wave + p (1 KB) into the tile at dst
__device__ __forceinline__ void v_dma(const SoloCtx& sc, int t, uint16_t* dst, int p) {
  t = min(t, sc.c.n_tiles - 1);
  const char* src = sc.vt + (int64_t)t * (2 * FT) + sc.vsrc + p * 1024;
  __builtin_amdgcn_global_load_lds((const void*)src,
                                   (__attribute__((address_space(3))) void*)(dst + (4 * sc.c.wave + p) * 512),
                                   16, 0, 0);
}

// LDS reads of slot m: K fragments d-step m of both tiles (QK), V^T fragments
// d-blocks 2(m & 3), 2(m & 3) + 1 of key step m >> 2 (PV)
template <bool QK, bool PV, int J, int MM>
__device__ __forceinline__ void slot_reads(const SoloCtx& sc, u32x4 (&kf)[3][2], u32x4 (&vf)[3][2]) {
  constexpr int B = MM % 3;
  if constexpr (QK) {
    kf[B][0] = ds_b128<J * 32768 + 256 * (MM >> 3)>(sc.kaddr[MM & 7]);
    kf[B][1] = ds_b128<J * 32768 + 16384 + 256 * (MM >> 3)>(sc.kaddr[MM & 7]);
  }
  if constexpr (PV) {
    constexpr int KS = MM >> 2, D0 = 2 * (MM & 3);
    constexpr int base = J * 32768 + (KS >> 1) * 16384 + (KS & 1) * 1024;
    vf[B][0] = ds_b128<base + 2048 * D0>(sc.vaddr);
    vf[B][1] = ds_b128<base + 2048 * (D0 + 1)>(sc.vaddr);
  }
}

// Slot m of step i: QK d-step m of both tiles of block i + 2 (MFMAs 1, 3),
// PV d-blocks 2(m & 3), 2(m & 3) + 1 of key step m >> 2 of block i (MFMAs 2, 4),
// softmax word m of block i + 1 (its two exponentials and the pack between the
// MFMAs), the reads of slot m + 2, and (m < 8) two of this wave's 16 tile loads
// of the step: K of block i + 3 (m < 4), V^T of block i + 1.
template <bool QK, bool SM, bool PV, bool DV, int J, int M>
__device__ __forceinline__ void solo_slot(SoloState& st, const SoloCtx& sc, const SoloLds& L, int i,
                                          u32x4 (&kf)[3][2], u32x4 (&vf)[3][2]) {
  constexpr int B = M % 3, KS = M >> 2, D0 = 2 * (M & 3);
  constexpr int NR = (QK ? 2 : 0) + (PV ? 2 : 0);
  constexpr int W = M < NSLOT - 1 ? NR : 0;  // after slot m's reads: slot m + 1's
  if constexpr (QK && PV) lgkm_take<W>(kf[B][0], kf[B][1], vf[B][0], vf[B][1]);
  else if constexpr (QK) lgkm_take<W>(kf[B][0], kf[B][1]);
  else if constexpr (PV) lgkm_take<W>(vf[B][0], vf[B][1]);
  sfence();
  if constexpr (QK) {
    if constexpr (M == 0) mfma_qkc(st.s[J][0], kf[B][0], st.qop[0], st.c0);
    else mfma_qk(st.s[J][0], kf[B][0], st.qop[M]);
  }
  sfence();
  float e0 = 0.f, e1 = 0.f;
  if constexpr (SM) {
    e0 = fast_exp2(st.s[1 - J][M >> 3][2 * (M & 7)]);
    pin(e0);  // computed here (a pure value would otherwise sink to its use)
  }
  sfence();
  if constexpr (PV) mfma_pv(st.o[D0], vf[B][0], st.p[J][KS]);
  sfence();
  if constexpr (SM) {
    e1 = fast_exp2(st.s[1 - J][M >> 3][2 * (M & 7) + 1]);
    pin(e1);
  }
  sfence();
  if constexpr (QK) {
    if constexpr (M == 0) mfma_qkc(st.s[J][1], kf[B][1], st.qop[0], st.c0);
    else mfma_qk(st.s[J][1], kf[B][1], st.qop[M]);
  }
  sfence();
  if constexpr (SM) {
    uint32_t w = pack2(e0, e1);
    pin(w);
    st.p[1 - J][M >> 2][M & 3] = w;
    st.lsum = dot2_ones(w, st.lsum);
    pin(st.lsum);
  }
  sfence();
  if constexpr (PV) mfma_pv(st.o[D0 + 1], vf[B][1], st.p[J][KS]);
  sfence();
  if constexpr (M + 2 < NSLOT) slot_reads<QK, PV, J, M + 2>(sc, kf, vf);
  if constexpr (M < 4) {
    uint16_t* dst = L.k + (1 - J) * (2 * FT) + (M >> 1) * FT;
    const int t = 2 * (i + 3) + (M >> 1);
    k_dma(sc.c, t, dst, 2 * (M & 1));
    k_dma(sc.c, t, dst, 2 * (M & 1) + 1);
  } else if constexpr (M < 8 && DV) {
    uint16_t* dst = L.v + (1 - J) * (2 * FT) + ((M - 4) >> 1) * FT;
    const int t = 2 * (i + 1) + ((M - 4) >> 1);
    v_dma(sc, t, dst, 2 * (M & 1));
    v_dma(sc, t, dst, 2 * (M & 1) + 1);
  }
  sfence();
}

// Step i (parity J = i & 1): QK of block i + 2 (K object J) into s[J], the softmax
// of block i + 1 from s[1 - J] into p[1 - J], PV of block i from p[J] (V object J);
// this wave's loads of K block i + 3 and V^T block i + 1 into the objects of
// parity 1 - J (their last readers were in step i - 1). One barrier: every wave's
// loads of step i - 1 are in, and every wave is done with step i - 1's reads.
template <bool CAUSAL, int J, bool QK, bool SM, bool PV, bool DV>
__device__ __forceinline__ void solo_step(SoloState& st, const SoloCtx& sc, const SoloLds& L,
                                          const SoloGeo& g, int i, int lane) {
  fwait_vmcnt<0>();
  fbarrier();
  u32x4 kf[3][2], vf[3][2];
  slot_reads<QK, PV, J, 0>(sc, kf, vf);
  slot_reads<QK, PV, J, 1>(sc, kf, vf);
  if constexpr (SM) {
    if (solo_needs_mask<CAUSAL>(g, i + 1)) solo_mask<CAUSAL>(g, i + 1, lane, st.s[1 - J]);
  }
  sfence();
#define SS(m) solo_slot<QK, SM, PV, DV, J, m>(st, sc, L, i, kf, vf)
  SS(0); SS(1); SS(2); SS(3); SS(4); SS(5); SS(6); SS(7);
  SS(8); SS(9); SS(10); SS(11); SS(12); SS(13); SS(14); SS(15);
#undef SS
  if constexpr (QK) mfma_drain(st.s[J][0], st.s[J][1]);
}

// Exact row max of the shifted-free S over the item's keys (QK only, K object
// b & 1 for block b; block 0 primed by the caller). Returns the row max (log2
// units) of this lane's row.
template <bool CAUSAL>
__device__ __forceinline__ float solo_max(const SoloState& st, const SoloCtx& sc, const SoloLds& L,
                                       const SoloGeo& g, int nb, int lane) {
  float m = -INFINITY;
  for (int b = 0; b < nb; ++b) {
    fwait_vmcnt<0>();
    fbarrier();
    uint16_t* nxt = L.k + ((b + 1) & 1) * (2 * FT);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      k_dma(sc.c, 2 * (b + 1), nxt, p);
      k_dma(sc.c, 2 * (b + 1) + 1, nxt + FT, p);
    }
    const uint32_t ob = (b & 1) * 32768;
    f32x16 s[2];
    u32x4 kf[3][2];
    kf[0][0] = ds_b128<0>(sc.kaddr[0] + ob);
    kf[0][1] = ds_b128<16384>(sc.kaddr[0] + ob);
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      if (kk < 15) {
        kf[(kk + 1) % 3][0] = ds_b128<0>(sc.kaddr[(kk + 1) & 7] + ob + 256 * ((kk + 1) >> 3));
        kf[(kk + 1) % 3][1] = ds_b128<16384>(sc.kaddr[(kk + 1) & 7] + ob + 256 * ((kk + 1) >> 3));
        lgkm_take<2>(kf[kk % 3][0], kf[kk % 3][1]);
      } else {
        lgkm_take<0>(kf[kk % 3][0], kf[kk % 3][1]);
      }
      if (kk == 0) {
        mfma_qk0(s[0], kf[0][0], st.qop[0]);
        mfma_qk0(s[1], kf[0][1], st.qop[0]);
      } else {
        mfma_qk(s[0], kf[kk % 3][0], st.qop[kk]);
        mfma_qk(s[1], kf[kk % 3][1], st.qop[kk]);
      }
    }
    mfma_drain(s[0], s[1]);
    if (solo_needs_mask<CAUSAL>(g, b)) solo_mask<CAUSAL>(g, b, lane, s);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) m = fmaxf(m, s[t][j]);
  }
  return xor32_max(m);
}

// 8-byte loads into AGPRs (held across the item) and the wait that releases them
template <int IMM>
__device__ __forceinline__ void g_b64a(u32x2& r, const void* p) {
  asm volatile("global_load_dwordx2 %0, %1, off offset:%2" : "=a"(r) : "v"(p), "i"(IMM));
}
__device__ __forceinline__ void gate_loads(const uint16_t* gp, u32x2 (&g)[8][4]) {
#define GL(db, jb) g_b64a<64 * (db) + 16 * (jb)>(g[db][jb], gp)
  GL(0, 0); GL(0, 1); GL(0, 2); GL(0, 3); GL(1, 0); GL(1, 1); GL(1, 2); GL(1, 3);
  GL(2, 0); GL(2, 1); GL(2, 2); GL(2, 3); GL(3, 0); GL(3, 1); GL(3, 2); GL(3, 3);
  GL(4, 0); GL(4, 1); GL(4, 2); GL(4, 3); GL(5, 0); GL(5, 1); GL(5, 2); GL(5, 3);
  GL(6, 0); GL(6, 1); GL(6, 2); GL(6, 3); GL(7, 0); GL(7, 1); GL(7, 2); GL(7, 3);
#undef GL
}
__device__ __forceinline__ void gate_take(u32x2 (&g)[8][4]) {
#pragma unroll
  for (int db = 0; db < 8; db += 2)
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+a"(g[db][0]), "+a"(g[db][1]), "+a"(g[db][2]), "+a"(g[db][3]),
                   "+a"(g[db + 1][0]), "+a"(g[db + 1][1]), "+a"(g[db + 1][2]), "+a"(g[db + 1][3]));
}

// K block 0 (tiles 0, 1) into K object 0
__device__ __forceinline__ void solo_prime(const SoloCtx& sc, const SoloLds& L) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    k_dma(sc.c, 0, L.k, p);
    k_dma(sc.c, 1, L.k + FT, p);
  }
}

// One item (shift: the static softmax shift in log2 units, or < 0 for the
// exact-max pass).
template <bool CAUSAL>
__device__ __forceinline__ void solo_item(const PrefillArgs& a, const FItem& it, const SoloLds& L,
                                          float shift) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h2 = lane >> 5;
  const ItemGeo ig = item_geo(a, it, CAUSAL);
  SoloGeo g;
  g.wrow0 = ig.r0 + 32 * wave;
  g.row = g.wrow0 + l32;
  g.off = ig.off;
  g.k_len = ig.k_len;
  QLoads ql;
  q_load_raw(a, ig.b, ig.h, g.row, h2, ql);
  if (ig.r0 >= ig.q_len) return;  // uniform over the workgroup
  SoloCtx sc;
  init_fctx(sc.c, a, ig, wave, lane);
  sc.vt = reinterpret_cast<const char*>(sc.c.vtbase);
  sc.vsrc = (uint32_t)(wave * 4096 + 16 * lane);
  {
    const int sk = fswz(l32);
#pragma unroll
    for (int q = 0; q < 8; ++q) sc.kaddr[q] = lds_addr(L.k) + l32 * 512 + 16 * ((2 * q + h2) ^ sk);
  }
  sc.vaddr = lds_addr(L.v) + 16 * lane;
  // gate logits of this lane's row: 4 at d = 32 dblk + 8 jb + 4 h2, loaded into
  // AGPRs now (the first step's wait covers them), read in the epilogue
  u32x2 gv[8][4];
  {
    const uint16_t* gp = a.gate + (int64_t)ig.b * a.g_sb + (int64_t)ig.h * a.g_sh +
                         (int64_t)min(g.row, a.L - 1) * a.g_st + 4 * h2;
    gate_loads(gp, gv);
  }
  q_load_rest(a, g.row, ig.prior, h2, ql);
  solo_prime(sc, L);

  SoloState st;
  q_prologue(a, ql, st.qop);
  // rows past the chunk hold finite junk q; their outputs are never stored
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) pin_acc(st.qop[kk]);
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) st.o[db][j] = 0.f;
  st.lsum = 0.f;

  const int nb = (sc.c.n_tiles + 1) >> 1;  // step blocks of two tiles
  float negm;
  if (shift >= 0.f) {
    negm = -shift;
  } else {
    const float mr = solo_max<CAUSAL>(st, sc, L, g, nb, lane);
    negm = mr == -INFINITY ? 0.f : -mr;  // fully-masked row: P = 0
    fwait_vmcnt<0>();
    fbarrier();  // every wave is done with the K objects
    solo_prime(sc, L);
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) st.c0[j] = negm;

  solo_step<CAUSAL, 0, true, false, false, false>(st, sc, L, g, -2, lane);
  solo_step<CAUSAL, 1, true, true, false, true>(st, sc, L, g, -1, lane);
  int i = 0;
  for (; i + 1 < nb; i += 2) {
    solo_step<CAUSAL, 0, true, true, true, true>(st, sc, L, g, i, lane);
    solo_step<CAUSAL, 1, true, true, true, true>(st, sc, L, g, i + 1, lane);
  }
  if (i < nb) solo_step<CAUSAL, 0, true, true, true, true>(st, sc, L, g, i, lane);

  // ---- epilogue: normalise, gate (sigmoid, src/kernels/kernels.jl:34), store in
  // the Wo input layout
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
               : "+a"(st.o[0]), "+a"(st.o[1]), "+a"(st.o[2]), "+a"(st.o[3]),
                 "+a"(st.o[4]), "+a"(st.o[5]), "+a"(st.o[6]), "+a"(st.o[7]));
  gate_take(gv);
  const float l_tot = st.lsum + __shfl_xor(st.lsum, 32, 64);
  const float inv = l_tot > 0.f ? fast_rcp(l_tot) : 0.f;  // fully-masked row -> 0
  if (g.row < ig.q_len) {
    uint16_t* op = a.o + (int64_t)ig.b * a.o_sb + (int64_t)ig.h * a.o_sh + (int64_t)g.row * a.o_st;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const f32x16& acc = st.o[db];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int d0 = 32 * db + 8 * jb + 4 * h2;
        const u32x2 g2 = gv[db][jb];
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

}  // namespace

template <bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_fused_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t KO[2 * 2 * FT], VO[2 * 2 * FT];
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
  SoloLds L;
  L.k = KO;
  L.v = VO;
  solo_item<CAUSAL>(a, item_at(a, blockIdx.x), L, bound <= FSTATIC_LIMIT ? bound : -1.0f);
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

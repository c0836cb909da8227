// prefill_fused.hip — the fused gated-attention prefill of forward(::AttnLayer)
// (src/llm/qwen35.jl:292-318): q norm + RoPE prologue, causal GQA flash attention
// over the cache (src/kernels/attention.jl:12-91), sigmoid-gate epilogue written in
// the Wo input layout. Re-designed for CDNA4.
//
// One workgroup (4 waves, one per SIMD, the whole 160-KB LDS) per work item
// (b, h, 128-row q-block), heaviest causal q-blocks first (the hardware hands the
// next item to the first CU that frees up). Each wave owns 32 query rows. All
// products are 32x32x16 bf16 MFMAs with fp32 accumulation:
//     S^T[key][row] = K[key][:] . Q[row][:]       A = K fragment, B = Q^T (AGPRs)
//     O^T[d][row]  += V^T[d][key] . P^T[key][row] A = V^T fragment, B = P^T
// P^T is packed from the wave's own S^T accumulator, so P never leaves the wave.
//
// Steps of 64 keys (two 32-key tiles). K tiles and V^T tiles (fragment-major,
// written by the V^T transpose kernel) stream into LDS by direct global->LDS
// loads shared by the four waves: V^T one step ahead into two objects, K two
// steps ahead into three (160 KB). Step i is a three-stage software pipeline --
// QK of block i+2, the softmax of block i+1, PV of block i -- cut into 16 slots
// of four products; after each product the wave issues one LDS read for the slot
// two ahead and one piece of the softmax, and each slot issues one tile load.
// Scheduling fences keep the VALU work between the products. One barrier per step.
//
// LDS reads feeding the products are issued from inline asm and waited for by a
// counted s_waitcnt inside the product's own asm statement (the compiler would
// drain every load in flight, including the tile loads two steps ahead, before
// each use). Every read's register is consumed within its step.
//
// Softmax: the QK-norm weights bound every logit (|q op| <= max|qw + w_offset|,
// |k~| <= 16 max|kw + w_offset|). When the bound is at most 64 in log2 units,
// P = exp2(S) needs no shift (P stays within 2^+-64 and the final 1/l cancels any
// common scale). Otherwise an online row max, moved lazily (only when it grows
// by more than 8 in log2 units), shifts P = exp2(S - max); O and l are rescaled
// when it moves.
#include <hip/hip_ext.h>

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

// Batches (B > 1, at most 256 (sequence, q-block) pairs): the pairs are ranked
// by the keys their last row attends (prior + chunk rows, from the device-side
// lengths), heaviest first, ties by index, and rank r takes the H items
// r H .. r H + H - 1 (heads grouped per XCD as above). With ragged priors the
// q-block index alone says little about an item's work. All threads of the
// workgroup take part; `scratch` is 257 ints of LDS.
__device__ __forceinline__ FItem item_ranked(const PrefillArgs& a, int i, bool causal, int* scratch) {
  const int NB = a.B * a.n_qt;
  if (a.B == 1 || NB > 256) return item_at(a, i);
  const int r = i / a.H, rem = i % a.H;
  const int t = threadIdx.x;
  if (t < NB) {
    const int b = t / a.n_qt, qt = t % a.n_qt;
    const int q_len = a.q_lengths ? min(a.q_lengths[b], a.L) : a.L;
    const int prior = a.prior ? a.prior[b] : 0;
    const int r0 = qt * FM;
    scratch[t] = r0 >= q_len ? 0 : (causal ? prior + min(q_len, r0 + FM) : prior + q_len);
  }
  __syncthreads();
  if (t < NB) {
    const int w = scratch[t];
    int rank = 0;
    for (int u = 0; u < NB; ++u) {
      const int wu = scratch[u];
      rank += (wu > w) || (wu == w && u < t);
    }
    if (rank == r) scratch[256] = t;
  }
  __syncthreads();
  const int blk = scratch[256];
  __syncthreads();  // every thread has read it before the LDS is reused
  FItem it;
  it.b = blk / a.n_qt;
  it.qt = blk % a.n_qt;
  it.h = (a.H & 7) == 0 ? (rem & 7) * (a.H >> 3) + (rem >> 3) : rem;
  it.hk = it.h / (a.H / a.Hk);
  return it;
}

// ---- V^T tiles. Tile t of (b, hk) holds keys 32t .. 32t+31 as 16 MFMA
// A-operand fragments of 1 KB, fragment f = 2 * dblk + ks (d-block dblk of 32
// d-rows, key half ks): lane l's 16 bytes (at 1024 f + 16 l) are the 8 keys
// 16 ks + {4h .. 4h+3, 8+4h .. 8+4h+3} (h = l / 32) of d-row 32 dblk + l % 32 --
// the key order of the P^T operand that lane half h holds for key half ks (the
// S^T accumulator layout).
//
// Workgroup x of (kv head, sequence) stages tiles t0 + x, t0 + x + gridDim.x, ...
// below the attended length: the tile's 32 V rows into LDS (one 512-byte row per
// wave load), out as one V^T tile (coalesced). t0 = 0, or with vt_rows the tile
// holding row min(vt_rows[b], prior[b]): the rows below it are already in the
// workspace from earlier calls, so a chunk-by-chunk prefill stages each row once
// (plus the one partial tile at each chunk's start); the last workgroup of the
// sequence to finish sets vt_rows[b] = k_len, counting arrivals in vt_rows[B + b]. Keys past the attended
// length repeat the last one (they are masked; V stays finite).
// With the fused append (k_raw set), the chunk's keys prior .. k_len-1 come from
// the packed projection instead of the cache: their K rows are normed and
// rotated into the K cache and their V rows copied into the V cache, as
// knorm_rope_append does (src/kernels/qknorm_rope_append.jl:59-98; prefill
// src/llm/qwen35.jl:306-307), and the V^T tile is built from the same rows.
constexpr int VT_WAVES = 16;  // waves per V^T staging workgroup
constexpr int VT_TP = 1;      // tiles per pass: their loads are issued together
__global__ __launch_bounds__(64 * VT_WAVES) void vt_transpose_kernel(VtArgs a) {
  const int hk = blockIdx.y, b = blockIdx.z;
  const int q_len = a.q_lengths ? min(a.q_lengths[b], a.L) : a.L;
  const int64_t prior = a.prior ? a.prior[b] : 0;
  const int64_t k_len = min(prior + q_len, a.ctx);
  const int64_t held = a.vt_rows ? min((int64_t)max(a.vt_rows[b], 0), prior) : 0;
  const int t_end = (int)((k_len + FN - 1) / FN);
  __shared__ __attribute__((aligned(16))) uint16_t tile[VT_TP * FN][HEAD_DIM + 8];  // 16-B row pad
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t cache_off = (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
  const bool fused = a.k_raw != nullptr;
  // the K norm weights once, before any store (a load issued after this
  // workgroup's stores would wait for them: memory counts retire in order)
  const uint2 kwv = fused ? *reinterpret_cast<const uint2*>(a.kw + 4 * lane) : make_uint2(0u, 0u);
  constexpr int RW = VT_TP * FN / VT_WAVES;  // rows per wave: r = wave + VT_WAVES j
  for (int t = (int)(held / FN) + VT_TP * blockIdx.x; t < t_end; t += VT_TP * gridDim.x) {
    // every load of the wave's rows first (one memory latency, not RW of them)
    uint2 vv[RW], kv[RW];
    float4 cv[RW], sv[RW];
    bool app[RW];
    int64_t key_of[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      const int64_t key = (int64_t)t * FN + wave + VT_WAVES * j;
      const int64_t src = min(key, k_len - 1);
      const bool chunk = fused && src >= prior;  // a key of this chunk: not in the cache yet
      const int64_t raw_off = (int64_t)b * a.raw_sb + (int64_t)hk * a.raw_sh + (src - prior) * a.raw_st;
      const uint16_t* vp = chunk ? a.v_raw + raw_off : a.v + cache_off + src * a.v_st;
      vv[j] = *reinterpret_cast<const uint2*>(vp + 4 * lane);
      app[j] = chunk && key == src;  // append column `key` (position key, 0-based)
      key_of[j] = key;
      if (app[j]) {
        kv[j] = *reinterpret_cast<const uint2*>(a.k_raw + raw_off + 4 * lane);
        const int i0 = 4 * (lane & 7);
        cv[j] = *reinterpret_cast<const float4*>(a.cos_tab + key * HALF_ROT + i0);
        sv[j] = *reinterpret_cast<const float4*>(a.sin_tab + key * HALF_ROT + i0);
      }
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      const int r = wave + VT_WAVES * j;
      *reinterpret_cast<uint2*>(&tile[r][4 * lane]) = vv[j];
      if (app[j]) {
        const int64_t key = key_of[j];
        *reinterpret_cast<uint2*>(a.v + cache_off + key * a.v_st + 4 * lane) = vv[j];
        float x[4] = {__uint_as_float(kv[j].x << 16), __uint_as_float(kv[j].x & 0xffff0000u),
                      __uint_as_float(kv[j].y << 16), __uint_as_float(kv[j].y & 0xffff0000u)};
        norm_rope_row_wv(x, kwv, cv[j], sv[j], a.eps, a.w_offset, lane);
        store_row4(a.kc + cache_off + key * a.v_st, lane, x);
      }
    }
    __syncthreads();
    uint16_t* dst = a.vt + ((int64_t)b * a.Hk + hk) * a.vt_tiles * FT + (int64_t)t * FT;
#pragma unroll
    for (int o = tid; o < VT_TP * HEAD_DIM * 4; o += 64 * VT_WAVES) {
      if (t + (o >> 10) >= t_end) break;  // a pass's tiles past the attended ones
      const int f = (o >> 6) & 15, l = o & 63;
      const int tb = FN * (o >> 10);  // the pass tile's first row
      const int d = 32 * (f >> 1) + (l & 31);
      const int k0 = 16 * (f & 1) + 4 * (l >> 5);
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int u0 = 2 * e, u1 = 2 * e + 1;  // element u: key k0 + (u & 3) + 8 (u >> 2)
        const uint32_t lo = tile[tb + k0 + (u0 & 3) + 8 * (u0 >> 2)][d];
        const uint32_t hi = tile[tb + k0 + (u1 & 3) + 8 * (u1 >> 2)][d];
        w[e] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(dst + o * 8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    __syncthreads();  // the tile is read out before the next one is written
  }
  if (a.vt_rows) {
    // the last of the sequence's workgroups to finish records the rows the tiles
    // now hold: every workgroup has read vt_rows[b] by then (its loop bounds)
    __syncthreads();
    if (tid == 0) {
      int32_t* arrived = a.vt_rows + a.B + b;
      const int n = (int)(gridDim.x * gridDim.y);
      if (atomicAdd(arrived, 1) == n - 1) {
        a.vt_rows[b] = (int32_t)k_len;
        *arrived = 0;  // zero again for the next call
      }
    }
  }
}

struct FCtx {
  const uint16_t* kbase;
  const uint16_t* vtbase;  // V^T tiles of (b, hk): 16 KB each
  int64_t kv_st;
  int krow_max;   // last cache row that may be read
  int n_tiles;
  uint32_t row_bytes;   // cache row stride in bytes
  // per-lane byte offsets of this wave's 4 one-KB pieces of a tile, less 1 KB per
  // piece (the load's immediate offset adds it back, and moves the LDS side too)
  uint32_t dma_boff[4];
  uint32_t dma_clamp[4];  // the same for the tile that reaches past the cache
  int t_part;             // that tile, or -1
  int wave, lane;
};

template <int N>
__device__ __forceinline__ void fwait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
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
// ---- LDS reads into compiler registers and the waits that release them. A read
// defines its value; the wait takes it (tied, or inside the consuming asm) so
// every reader is placed after the wait; LDS reads complete in issue order.
template <int OFF>
__device__ __forceinline__ u32x4 ds_b128(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
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

// q_len_raw, prior: q_lengths[b] (or L) and prior[b] (or 0), loaded by the caller
__device__ __forceinline__ ItemGeo item_geo(const PrefillArgs& a, const FItem& it, bool causal,
                                            int q_len_raw, int prior) {
  ItemGeo ig;
  ig.b = it.b; ig.h = it.h; ig.hk = it.hk;
  ig.r0 = it.qt * FM;
  ig.q_len = min(q_len_raw, a.L);
  ig.prior = prior;
  // queries are the suffix of the attended keys: row t sits at position prior + t.
  // prior + q_len > Lk is out of contract (those keys were never appended): the
  // keys past the cache are masked rather than read
  ig.off = ig.prior;
  ig.k_len = min(ig.prior + ig.q_len, a.Lk);
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
  const int tl = c.n_tiles - 1;
  c.t_part = tl * FN + FN - 1 > c.krow_max ? tl : -1;
  const int last = c.krow_max - tl * FN;  // last readable row of that tile
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 2 * (4 * wave + i) + (lane >> 5);
    const uint32_t chunk = (uint32_t)(((lane & 31) ^ fswz(r)) * 16);
    c.dma_boff[i] = (uint32_t)r * c.row_bytes + chunk - 1024u * i;
    c.dma_clamp[i] = (uint32_t)min(r, max(last, 0)) * c.row_bytes + chunk - 1024u * i;
  }
}

// raw q row, norm weight, and RoPE table operands of this lane (row `row` of head h)
struct QLoads {
  uint4 qraw[16], qwv[16];
  float4 cv[4], sv[4];
};

// q rows of one 32-row block: qnorm_rope (src/kernels/qknorm_rope_append.jl:25-57)
// and the 1/16 scale. RoPE is linear, so the per-row 1/rms and the scale fold
// into the weight factor: x (w + offset) scale = x fma(w, scale, offset scale).
// Lane holds q[row][16kk + 8h2 + j]
__device__ __forceinline__ void q_prologue(const PrefillArgs& a, const QLoads& ql, uint4 (&qop)[16]) {
  // sum of squares straight from the packed pairs (bf16 products are exact in f32)
  float ss = 0.f;
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    const uint32_t w4[4] = {ql.qraw[kk].x, ql.qraw[kk].y, ql.qraw[kk].z, ql.qraw[kk].w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w4[j]), __builtin_bit_cast(bf16x2, w4[j]),
                                           ss, false);
  }
  ss += __shfl_xor(ss, 32, 64);
  const float scale = QK_SCALE * LOG2E / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
  const float wscale = a.w_offset * scale;  // x (w + offset) scale = x fma(w, scale, offset scale)
  const float* cs = reinterpret_cast<const float*>(ql.cv);
  const float* sn = reinterpret_cast<const float*>(ql.sv);
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    if (kk == 2 || kk == 3) continue;  // rotated with d-steps 0, 1
    float x1[8], wf[8];
    unpack8(ql.qraw[kk], x1);
    unpack8(ql.qwv[kk], wf);
#pragma unroll
    for (int j = 0; j < 8; ++j) x1[j] *= fmaf(wf[j], scale, wscale);
    if (kk < 2) {
      // d-steps 0..3 carry the rotary dims: pairs (d, d + 32) = d-steps (kk, kk + 2)
      float x2[8];
      unpack8(ql.qraw[kk + 2], x2);
      unpack8(ql.qwv[kk + 2], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x2[j] *= fmaf(wf[j], scale, wscale);
        const float cc = cs[8 * kk + j], si = sn[8 * kk + j];
        const float r1 = x1[j] * cc - x2[j] * si;
        const float r2 = x2[j] * cc + x1[j] * si;
        x1[j] = r1;
        x2[j] = r2;
      }
      qop[kk + 2] = pack8(x2);
    }
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
  f32x16 s[2][2];    // S^T in log2 units, by step parity and tile
  u32x4 p[2][4];     // packed P^T, by step parity and key step
  float negm;        // minus this lane's row shift (log2 units)
  float mrun;        // SHIFT: the running row max the shift follows (-inf before any key)
  uint32_t kb[8];    // LDS address of K fragment q (q + 8 at +256) in this step's K object
  u32x4 gv[16];      // gate logits of this wave's rows, coalesced (see gate_loads; AGPRs)
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

// K objects (three, two tiles each, swizzled rows; block j in object j % 3) and
// V^T objects (two, two tiles each, fragment-major; block j in object j % 2)
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

// Global->LDS tile loads. A tile is 16 one-KB pieces; wave w loads pieces 4w ..
// 4w+3 (K: rows 2g, 2g+1 of piece g, re-laid to the swizzled LDS rows through
// the per-lane source offsets; V^T: fragments g). Tile indices are clamped to the
// last tile of the item; a K tile reaching past the cache re-reads its last row
// there (those keys are masked).
struct TileSrc {
  const char* p;  // the tile's first byte
  bool part;      // K: the tile reaching past the cache
};
__device__ __forceinline__ TileSrc k_tile(const FCtx& c, int t) {
  t = min(t, c.n_tiles - 1);
  TileSrc r;
  r.p = reinterpret_cast<const char*>(c.kbase + (int64_t)(t * FN) * c.kv_st);
  r.part = t == c.t_part;
  return r;
}
// Tile sources of a stream advanced two tiles per step: tiles t, t + 1 clamped to
// the item's last tile (and, for K, the partial-tile flag)
struct TileStream {
  const char* p;     // tile t (unclamped)
  const char* last;  // the last tile
  int64_t stride;    // bytes per tile
  int t, tl, tpart;
  __device__ __forceinline__ TileSrc at(int k) const {
    TileSrc r;
    r.p = t + k <= tl ? p + k * stride : last;
    r.part = min(t + k, tl) == tpart;
    return r;
  }
  __device__ __forceinline__ void advance() {
    p += 2 * stride;
    t += 2;
  }
};
__device__ __forceinline__ TileStream k_stream(const FCtx& c, int t0) {
  TileStream s;
  s.stride = (int64_t)FN * c.kv_st * 2;
  s.tl = c.n_tiles - 1;
  s.t = t0;
  s.tpart = c.t_part;
  s.p = reinterpret_cast<const char*>(c.kbase) + t0 * s.stride;
  s.last = reinterpret_cast<const char*>(c.kbase) + s.tl * s.stride;
  return s;
}
template <int P>
__device__ __forceinline__ void k_piece(const FCtx& c, const TileSrc& src, uint16_t* dst) {
  const uint32_t off = src.part ? c.dma_clamp[P] : c.dma_boff[P];
  __builtin_amdgcn_global_load_lds((const void*)(src.p + off),
                                   (__attribute__((address_space(3))) void*)(dst + 4 * c.wave * 512),
                                   16, 1024 * P, 0);
}
template <int P>
__device__ __forceinline__ void v_piece(const SoloCtx& sc, const char* src, uint16_t* dst) {
  __builtin_amdgcn_global_load_lds((const void*)(src + sc.vsrc),
                                   (__attribute__((address_space(3))) void*)(dst + 4 * sc.c.wave * 512),
                                   16, 1024 * P, 0);
}

__device__ __forceinline__ TileStream v_stream(const SoloCtx& sc, int t0) {
  TileStream s;
  s.stride = 2 * FT;
  s.tl = sc.c.n_tiles - 1;
  s.t = t0;
  s.tpart = -1;
  s.p = sc.vt + t0 * s.stride;
  s.last = sc.vt + s.tl * s.stride;
  return s;
}

// Slot operands: QK reads K fragments d-step m of tiles 0, 1 (kb: the step's K
// object); PV reads V^T fragments d-blocks 2(m & 3), 2(m & 3) + 1 of key step
// m >> 2. Operand r of slot m lives in ops[m % 3][r] (QK's first).
template <bool QK, bool PV>
constexpr int slot_nops() { return (QK ? 2 : 0) + (PV ? 2 : 0); }
template <bool QK, bool PV, int J, int MM, int R>
__device__ __forceinline__ void slot_read(const SoloCtx& sc, const uint32_t (&kb)[8], u32x4 (&ops)[3][4]) {
  constexpr int B = MM % 3;
  if constexpr (QK && R < 2) {
    ops[B][R] = ds_b128<16384 * R + 256 * (MM >> 3)>(kb[MM & 7]);
  } else {
    constexpr int U = QK ? R - 2 : R;
    constexpr int KS = MM >> 2, DB = 2 * (MM & 3) + U;
    ops[B][R] = ds_b128<J * 32768 + (KS >> 1) * 16384 + (KS & 1) * 1024 + 2048 * DB>(sc.vaddr);
  }
}
// LDS ops issued after operand r of slot m when the slot's r-th MFMA issues: the
// rest of slot m's reads, slot m + 1's, and the r reads of slot m + 2 issued so far
template <int N, int M, int R>
constexpr int slot_wait() {
  return (N - 1 - R) + (M + 1 < NSLOT ? N : 0) + (M + 2 < NSLOT ? R : 0);
}

// the products with the wait for their LDS operand in front (one statement: no
// reader of the operand can be placed between the two)
template <int W>
__device__ __forceinline__ void qk_w0(f32x16& s, const u32x4& k, const uint4& q) {
  asm volatile("s_waitcnt lgkmcnt(%3)\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0"
               : "=&v"(s) : "v"(k), "a"(__builtin_bit_cast(u32x4, q)), "n"(W));
}
template <int W>
__device__ __forceinline__ void qk_w(f32x16& s, const u32x4& k, const uint4& q) {
  asm volatile("s_waitcnt lgkmcnt(%3)\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
               : "+v"(s) : "v"(k), "a"(__builtin_bit_cast(u32x4, q)), "n"(W));
}
template <int W>
__device__ __forceinline__ void pv_w0(f32x16& o, const u32x4& v, const u32x4& p) {
  asm volatile("s_waitcnt lgkmcnt(%3)\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0"
               : "=&a"(o) : "v"(v), "v"(p), "n"(W));
}
template <int W>
__device__ __forceinline__ void pv_w(f32x16& o, const u32x4& v, const u32x4& p) {
  asm volatile("s_waitcnt lgkmcnt(%3)\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
               : "+a"(o) : "v"(v), "v"(p), "n"(W));
}

// Slot m of step i: QK d-step m of both tiles of block i + 2, PV d-blocks
// 2(m & 3), 2(m & 3) + 1 of key step m >> 2 of block i, softmax word m of block
// i + 1, one LDS read of slot m + 2 after each product, and this wave's tile
// loads of the step: two pieces of V^T block i + 1 in each of slots 0-3 (needed
// next step, so issued first), one piece of K block i + 4 in each of slots 4-11
// (needed two steps on; kd: its object; ks, vs: the tiles' sources). The VALU
// work sits between the products (fences keep it there).
template <bool SHIFT, bool QK, bool SM, bool PV, bool DV, bool FIRST, int J, int M>
__device__ __forceinline__ void solo_slot(SoloState& st, const SoloCtx& sc, const SoloLds& L,
                                          const uint32_t (&kb)[8], uint16_t* kd, const TileSrc (&ks)[2],
                                          const TileSrc (&vs)[2], u32x4 (&ops)[3][4]) {
  constexpr int B = M % 3, KS = M >> 2, D0 = 2 * (M & 3);
  constexpr int N = slot_nops<QK, PV>();
  constexpr bool RD = M + 2 < NSLOT;
  float e0 = 0.f, e1 = 0.f;
  uint32_t w = 0;
  // product r, then read r of slot m + 2, then the VALU piece placed after it
#define SLOT_READ(r) \
  if constexpr (RD) slot_read<QK, PV, J, M + 2, r>(sc, kb, ops)
  if constexpr (QK) {
    if constexpr (M == 0) qk_w0<slot_wait<N, M, 0>()>(st.s[J][0], ops[B][0], st.qop[0]);
    else qk_w<slot_wait<N, M, 0>()>(st.s[J][0], ops[B][0], st.qop[M]);
    SLOT_READ(0);
    sfence();
    if constexpr (SM) {
      e0 = fast_exp2(SHIFT ? st.s[1 - J][M >> 3][2 * (M & 7)] + st.negm : st.s[1 - J][M >> 3][2 * (M & 7)]);
      pin(e0);  // computed here (a pure value would otherwise sink to its use)
    }
    sfence();
    if constexpr (M == 0) qk_w0<slot_wait<N, M, 1>()>(st.s[J][1], ops[B][1], st.qop[0]);
    else qk_w<slot_wait<N, M, 1>()>(st.s[J][1], ops[B][1], st.qop[M]);
    SLOT_READ(1);
    sfence();
    if constexpr (SM) {
      e1 = fast_exp2(SHIFT ? st.s[1 - J][M >> 3][2 * (M & 7) + 1] + st.negm
                           : st.s[1 - J][M >> 3][2 * (M & 7) + 1]);
      pin(e1);
      if constexpr (!PV) {
        w = pack2(e0, e1);
        pin(w);
        st.p[1 - J][M >> 2][M & 3] = w;
        st.lsum = dot2_ones(w, st.lsum);
        pin(st.lsum);
      }
    }
    sfence();
  }
  if constexpr (PV) {
    constexpr int R0 = QK ? 2 : 0;
    if constexpr (FIRST && KS == 0) pv_w0<slot_wait<N, M, R0>()>(st.o[D0], ops[B][R0], st.p[J][KS]);
    else pv_w<slot_wait<N, M, R0>()>(st.o[D0], ops[B][R0], st.p[J][KS]);
    SLOT_READ(R0);
    sfence();
    if constexpr (SM) {
      w = pack2(e0, e1);
      pin(w);
      st.p[1 - J][M >> 2][M & 3] = w;
    }
    sfence();
    if constexpr (FIRST && KS == 0) pv_w0<slot_wait<N, M, R0 + 1>()>(st.o[D0 + 1], ops[B][R0 + 1], st.p[J][KS]);
    else pv_w<slot_wait<N, M, R0 + 1>()>(st.o[D0 + 1], ops[B][R0 + 1], st.p[J][KS]);
    SLOT_READ(R0 + 1);
    sfence();
    if constexpr (SM) {
      st.lsum = dot2_ones(w, st.lsum);
      pin(st.lsum);
    }
  }
#undef SLOT_READ
  if constexpr (M < 4) {
    if constexpr (DV) {
      v_piece<(2 * M) & 3>(sc, vs[M >> 1].p, L.v + (1 - J) * (2 * FT) + (M >> 1) * FT);
      v_piece<(2 * M + 1) & 3>(sc, vs[M >> 1].p, L.v + (1 - J) * (2 * FT) + (M >> 1) * FT);
    }
  } else if constexpr (M < 12) {
    k_piece<(M - 4) & 3>(sc.c, ks[(M - 4) >> 2], kd + ((M - 4) >> 2) * FT);
  }
  sfence();
}

// SHIFT: the online row max, updated at the start of each softmax stage from the
// block's (masked) logits in s[1 - J], lazily: the shift moves only when a row's
// max grows by more than 8 (log2 units; P then stays below 2^8). The row sum is
// rescaled at once; the returned factor (1 for rows whose shift stays) is owed by
// O, whose products of this step still use the old shift (the caller applies it
// after them). A row with no valid key yet keeps shift 0 (its P are 0).
template <int J>
__device__ __forceinline__ float online_max(SoloState& st) {
  float mb = -INFINITY;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 16; ++j) mb = fmaxf(mb, st.s[1 - J][t][j]);
  mb = xor32_max(mb);
  const float m_new = fmaxf(st.mrun, mb);
  const bool need = m_new > st.mrun + 8.0f;  // false while both are -inf
  float resc = 1.0f;
  if (__ballot(need) != 0ull) {
    if (need) {
      resc = st.mrun == -INFINITY ? 1.0f : fast_exp2(st.mrun - m_new);
      st.lsum *= resc;
      st.mrun = m_new;
      st.negm = -m_new;
    }
  }
  return resc;
}

// Step i (parity J = i & 1): QK of block i + 2 (K object (i + 2) % 3) into s[J],
// the softmax of block i + 1 from s[1 - J] into p[1 - J], PV of block i from p[J]
// (V object J); this wave's loads of V^T block i + 1 (V object 1 - J) and then K
// block i + 4 (K object (i + 1) % 3), whose last readers were in step i - 1. One
// barrier: every wave's loads of V^T block i and K block i + 2 (issued one and two
// steps back; only the last step's K loads may still be in flight) are in, and
// every wave is done with step i - 1's reads.
template <bool CAUSAL, bool SHIFT, int J, bool QK, bool SM, bool PV, bool DV, bool FIRST = false,
          int WAITV = 8>
__device__ __forceinline__ void solo_step(SoloState& st, const SoloCtx& sc, const SoloLds& L,
                                          const SoloGeo& g, int i, int lane, TileStream& kst,
                                          TileStream& vst) {
  fwait_vmcnt<WAITV>();
  fbarrier();
  const uint32_t (&kb)[8] = st.kb;
  uint16_t* kd = L.k + ((i + 4) % 3) * (2 * FT);
  // kst: tiles 2(i + 4), 2(i + 4) + 1; vst: 2(i + 1), 2(i + 1) + 1
  const TileSrc ks[2] = {kst.at(0), kst.at(1)};
  const TileSrc vs[2] = {vst.at(0), vst.at(1)};
  kst.advance();
  if constexpr (DV) vst.advance();
  u32x4 ops[3][4];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    if (m == 0) {
      slot_read<QK, PV, J, 0, 0>(sc, kb, ops);
      slot_read<QK, PV, J, 0, 1>(sc, kb, ops);
      if constexpr (QK && PV) {
        slot_read<QK, PV, J, 0, 2>(sc, kb, ops);
        slot_read<QK, PV, J, 0, 3>(sc, kb, ops);
      }
    } else {
      slot_read<QK, PV, J, 1, 0>(sc, kb, ops);
      slot_read<QK, PV, J, 1, 1>(sc, kb, ops);
      if constexpr (QK && PV) {
        slot_read<QK, PV, J, 1, 2>(sc, kb, ops);
        slot_read<QK, PV, J, 1, 3>(sc, kb, ops);
      }
    }
  }
  if constexpr (SM) {
    if (solo_needs_mask<CAUSAL>(g, i + 1)) solo_mask<CAUSAL>(g, i + 1, lane, st.s[1 - J]);
  }
  float resc = 1.0f;  // SHIFT: O's rescale, owed after this step's products
  if constexpr (SHIFT && SM) resc = online_max<J>(st);
  sfence();
#define SS(m) solo_slot<SHIFT, QK, SM, PV, DV, FIRST, J, m>(st, sc, L, kb, kd, ks, vs, ops)
  SS(0); SS(1); SS(2); SS(3); SS(4); SS(5); SS(6); SS(7);
  SS(8); SS(9); SS(10); SS(11); SS(12); SS(13); SS(14); SS(15);
#undef SS
  if constexpr (QK) mfma_drain(st.s[J][0], st.s[J][1]);
  if constexpr (SHIFT && SM && PV) {
    if (__ballot(resc != 1.0f) != 0ull) {
      // O now holds blocks <= i at the old shift: move it to the new one before
      // the next step adds block i + 1 (rare: the max grows by > 8 a few times)
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                   : "+a"(st.o[0]), "+a"(st.o[1]), "+a"(st.o[2]), "+a"(st.o[3]),
                     "+a"(st.o[4]), "+a"(st.o[5]), "+a"(st.o[6]), "+a"(st.o[7]));
#pragma unroll
      for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) st.o[db][e] *= resc;
    }
  }
  {
    // next step's K object: (i + 3) % 3
    const int dk = (i + 2) % 3 == 2 ? -65536 : 32768;
#pragma unroll
    for (int q = 0; q < 8; ++q) st.kb[q] += dk;
  }
}

// Gate logits of this lane's row, loaded once into AGPRs after the prologue and
// held to the epilogue: load i holds bf16 16 i + 8 h .. +7 of the row (h = lane /
// 32; 32 contiguous bytes per row and load). Rows past the last valid one read
// that row (the epilogue stores no row past it). swap_halves() turns a pair of
// these chunks into the O^T accumulator's layout, and an output pair back.
__device__ __forceinline__ void gate_loads(const uint16_t* base, int64_t row_st, int row, int last_row, int h,
                                           u32x4 (&g)[16]) {
  const uint16_t* p = base + (int64_t)min(row, last_row) * row_st + 8 * h;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=a"(g[i]) : "v"(p), "i"(32 * i));
}
__device__ __forceinline__ void gate_take(u32x4 (&g)[16]) {
#pragma unroll
  for (int i = 0; i < 16; i += 4)
    asm volatile("s_waitcnt vmcnt(0)" : "+a"(g[i]), "+a"(g[i + 1]), "+a"(g[i + 2]), "+a"(g[i + 3]));
}
// Lane half h holds 8 bf16 of its row at 16 i + 8 h (words x..w). The O^T
// accumulator gives the lane 4 columns at 16 i + 4 h (j' = 2 (i & 1)) and 4 at
// 16 i + 8 + 4 h: words z, w of the low half trade places with words x, y of the
// high half. After it the lane's x, y are its first 4 columns and z, w its second
// 4 -- and the same swap applied to an output packed that way gives each lane 8
// contiguous columns at 16 i + 8 h again.
__device__ __forceinline__ void swap_halves(u32x4& v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
  v.x = a[0];
  v.z = a[1];
  v.y = b[0];
  v.w = b[1];
}

// lane (l32, h2): q[row l32][16kk + 8h2 .. +7] and the table floats 8h2 + 16kk + 4u.
// The reads are issued from asm (a compiler-visible LDS read after the staging
// loads would get a wait for every load in flight, the K tiles included) and
// released by counted waits tied to their registers.
__device__ __forceinline__ void q_read_lds(QLoads& ql, const SoloLds& L, int wave, int l32, int h2) {
  const uint32_t qs = lds_addr(L.v + wave * (32 * HEAD_DIM) + l32 * HEAD_DIM);
  const int sq = fswz(l32);
  u32x4 q[16], t[8];
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) q[kk] = ds_b128<0>(qs + 16 * ((2 * kk + h2) ^ sq));
  const uint32_t ts = lds_addr(reinterpret_cast<const float*>(L.k + 2 * (2 * FT)) +
                               wave * (2 * 32 * HALF_ROT) + l32 * HALF_ROT);
  const int st = l32 & 7;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t ch = (uint32_t)(16 * ((2 * h2 + 4 * kk + u) ^ st));
      t[2 * kk + u] = ds_b128<0>(ts + ch);
      t[4 + 2 * kk + u] = ds_b128<4 * 32 * HALF_ROT>(ts + ch);
    }
  asm volatile("s_waitcnt lgkmcnt(8)"
               : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]), "+v"(q[6]),
                 "+v"(q[7]), "+v"(q[8]), "+v"(q[9]), "+v"(q[10]), "+v"(q[11]), "+v"(q[12]),
                 "+v"(q[13]), "+v"(q[14]), "+v"(q[15]));
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]),
                 "+v"(t[7]));
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) ql.qraw[kk] = __builtin_bit_cast(uint4, q[kk]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ql.cv[i] = __builtin_bit_cast(float4, t[i]);
    ql.sv[i] = __builtin_bit_cast(float4, t[4 + i]);
  }
}

// The lane id recomputed from the hardware: values derived from it after a long
// loop are formed there rather than held in registers across the loop
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// One item's fixed context: geometry, tile sources and LDS read addresses.
struct SoloItem {
  ItemGeo ig;
  SoloGeo g;
  SoloCtx sc;
  bool live;  // the item has rows (uniform over the workgroup)
};

template <bool CAUSAL>
__device__ __forceinline__ void item_setup(SoloItem& I, const PrefillArgs& a, const FItem& it, const SoloLds& L,
                                           int q_len_raw, int prior, int wave, int lane) {
  const int l32 = lane & 31, h2 = lane >> 5;
  I.ig = item_geo(a, it, CAUSAL, q_len_raw, prior);
  I.g.wrow0 = I.ig.r0 + 32 * wave;
  I.g.row = I.g.wrow0 + l32;
  I.g.off = I.ig.off;
  I.g.k_len = I.ig.k_len;
  I.live = I.ig.r0 < I.ig.q_len;
  init_fctx(I.sc.c, a, I.ig, wave, lane);
  I.sc.vt = reinterpret_cast<const char*>(I.sc.c.vtbase);
  I.sc.vsrc = (uint32_t)(wave * 4096 + 16 * lane);
  const int sk = fswz(l32);
#pragma unroll
  for (int q = 0; q < 8; ++q) I.sc.kaddr[q] = lds_addr(L.k) + l32 * 512 + 16 * ((2 * q + h2) ^ sk);
  I.sc.vaddr = lds_addr(L.v) + 16 * lane;
}

// The item's 56 prologue loads, in issue order: 0..15 its q rows into LDS (the V
// objects; piece i = rows 2 i, 2 i + 1 of the wave, as q_stage), 16..23 their
// RoPE table rows (K object 2; cos, sin of rows 8 i .. 8 i + 7 in turn), 24..39
// the q norm weights into `qw` (as q_load_w), 40..55 K tiles 0..3 into K objects
// 0 and 1 (as solo_prime). Every LDS object must be free: no earlier load of the
// workgroup still writing LDS, every wave done reading it.
template <int N>
__device__ __forceinline__ void pro_load(const SoloItem& I, const PrefillArgs& a, const SoloLds& L, int wave,
                                         int lane, u32x4 (&qw)[16]) {
  if constexpr (N < 16) {
    const int hl = lane >> 5, c = lane & 31, r = 2 * N + hl;
    const char* qb = reinterpret_cast<const char*>(a.q + (int64_t)I.ig.b * a.q_sb + (int64_t)I.ig.h * a.q_sh);
    const int64_t row = min(I.g.wrow0 + r, a.L - 1);
    __builtin_amdgcn_global_load_lds((const void*)(qb + row * a.q_st * 2 + 16 * (c ^ fswz(r))),
                                     (__attribute__((address_space(3))) void*)(L.v + wave * (32 * HEAD_DIM) + N * 512),
                                     16, 0, 0);
  } else if constexpr (N < 24) {
    constexpr int i = (N - 16) >> 1;
    constexpr bool SN = ((N - 16) & 1) != 0;
    const int pr = lane >> 3, ck = lane & 7, r = 8 * i + pr;
    const int64_t pos = min((int64_t)I.ig.prior + min(I.g.wrow0 + r, a.L - 1), (int64_t)a.Lk - 1);
    const int64_t off = pos * HALF_ROT + 4 * (ck ^ (r & 7));
    float* td = reinterpret_cast<float*>(L.k + 2 * (2 * FT)) + wave * (2 * 32 * HALF_ROT) + (SN ? 32 * HALF_ROT : 0);
    __builtin_amdgcn_global_load_lds((const void*)((SN ? a.sin_tab : a.cos_tab) + off),
                                     (__attribute__((address_space(3))) void*)(td + i * 256), 16, 0, 0);
  } else if constexpr (N < 40) {
    constexpr int kk = N - 24;
    const uint16_t* p = a.qw + 8 * (lane >> 5);
    asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(qw[kk]) : "v"(p), "i"(32 * kk));
  } else {
    constexpr int t = (N - 40) >> 2, P = (N - 40) & 3;
    k_piece<P>(I.sc.c, k_tile(I.sc.c, t), L.k + t * FT);
  }
}
template <int N0, int N1>
__device__ __forceinline__ void pro_loads(const SoloItem& I, const PrefillArgs& a, const SoloLds& L, int wave,
                                          int lane, u32x4 (&qw)[16]) {
  if constexpr (N0 < N1) {
    pro_load<N0>(I, a, L, wave, lane, qw);
    sfence();  // each load's address is formed next to it (few live registers)
    pro_loads<N0 + 1, N1>(I, a, L, wave, lane, qw);
  }
}

// The rest of the item once q, its table rows and `qw` have landed (the caller's
// wait is tied to `qw`): q norm + RoPE into st.qop, the gate loads, the pipelined
// steps. Ends with every load of the workgroup landed
// (vmcnt(0), gates included) and a barrier after which no wave reads the tile
// objects: all of the LDS is free, and st.o, st.gv, st.lsum hold the result.
template <bool CAUSAL, bool SHIFT>
__device__ __forceinline__ void item_run(SoloItem& I, SoloState& st, const PrefillArgs& a, const SoloLds& L,
                                         u32x4 (&qw)[16], int wave, int lane) {
  const int l32 = lane & 31, h2 = lane >> 5;
  SoloCtx& sc = I.sc;
  const SoloGeo& g = I.g;
  QLoads ql;
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) ql.qwv[kk] = __builtin_bit_cast(uint4, qw[kk]);
  q_read_lds(ql, L, wave, l32, h2);
  q_prologue(a, ql, st.qop);
  // rows past the chunk hold finite junk q; their outputs are never stored
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) pin_acc(st.qop[kk]);
  // gate logits now (after q is in: the compiler's waits for q know nothing of
  // these); the two pipeline-filling steps leave them in flight
  gate_loads(a.gate + (int64_t)I.ig.b * a.g_sb + (int64_t)I.ig.h * a.g_sh, a.g_st, g.row, a.L - 1, h2, st.gv);
  st.lsum = 0.f;

  const int nb = (sc.c.n_tiles + 1) >> 1;  // step blocks of two tiles
  st.negm = 0.f;  // SHIFT: moved by online_max from the first block on
  st.mrun = -INFINITY;

  TileStream kst = k_stream(sc.c, 4), vst = v_stream(sc, 0);
#pragma unroll
  for (int q = 0; q < 8; ++q) st.kb[q] = sc.kaddr[q];  // step -2 reads K object 0
  // younger than K block 0 (-2) / 1 (-1): 8 tile loads and the 16 gate loads
  constexpr int WG = 24;
  solo_step<CAUSAL, SHIFT, 0, true, false, false, false, false, WG>(st, sc, L, g, -2, lane, kst, vst);
  solo_step<CAUSAL, SHIFT, 1, true, true, false, true, false, WG>(st, sc, L, g, -1, lane, kst, vst);
  // step 0 starts O (its first products take a zero accumulator)
  solo_step<CAUSAL, SHIFT, 0, true, true, true, true, true>(st, sc, L, g, 0, lane, kst, vst);
  int i = 1;
  for (; i + 1 < nb; i += 2) {
    solo_step<CAUSAL, SHIFT, 1, true, true, true, true>(st, sc, L, g, i, lane, kst, vst);
    solo_step<CAUSAL, SHIFT, 0, true, true, true, true>(st, sc, L, g, i + 1, lane, kst, vst);
  }
  if (i < nb) solo_step<CAUSAL, SHIFT, 1, true, true, true, true>(st, sc, L, g, i, lane, kst, vst);

  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
               : "+a"(st.o[0]), "+a"(st.o[1]), "+a"(st.o[2]), "+a"(st.o[3]),
                 "+a"(st.o[4]), "+a"(st.o[5]), "+a"(st.o[6]), "+a"(st.o[7]));
  // vmcnt(0) before the barrier: this wave's gate loads and its last tile loads
  // have landed, so after the barrier no tile load of any wave is still writing
  // LDS and no wave reads a tile object again
  gate_take(st.gv);
  fbarrier();
}

// Epilogue (no LDS): o sigma(g) / l for this lane's row (sigmoid:
// src/kernels/kernels.jl:34; the gate: src/llm/qwen35.jl:315), in 16 chunks:
// chunk i forms and stores the 8 contiguous bf16 at columns 16 i + 8 h .. +7.
// O^T d-block db = i / 2 holds the row at columns 32 db + 8 j' + 4 h + (0..3),
// j' = 0..3. With NEXT, chunks 0..7 first issue 7 each of the next item's 56
// prologue loads, so their address work overlaps this arithmetic.
struct EpiCtx {
  float lt;      // the row's l (or a finite stand-in for an empty row)
  uint16_t* op;  // this lane's first output column
  bool store;    // the row is inside the chunk
};
__device__ __forceinline__ EpiCtx epi_ctx(const SoloItem& I, const SoloState& st, const PrefillArgs& a, int lane) {
  const int l32 = lane & 31, h2 = lane >> 5;
  EpiCtx e;
  const float l_tot = st.lsum + __shfl_xor(st.lsum, 32, 64);
  // o sigma(g) / l = o / (l + l 2^(-g log2 e)); a fully-masked row (l = 0, o = 0)
  // takes a finite stand-in for l, so its output stays 0 for every gate
  e.lt = l_tot > 0.f ? l_tot : 3.0e38f;
  e.store = I.g.row < I.ig.q_len;
  e.op = a.o + (int64_t)I.ig.b * a.o_sb + (int64_t)I.ig.h * a.o_sh + (int64_t)(I.g.wrow0 + l32) * a.o_st + 8 * h2;
  return e;
}
template <int C>
__device__ __forceinline__ void epi_chunk(const SoloState& st, const EpiCtx& e) {
  u32x4 gq = st.gv[C];
  swap_halves(gq);  // x, y: columns of j' = 2 (C & 1); z, w: j' = 2 (C & 1) + 1
  const f32x16& acc = st.o[C >> 1];
  const uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w};
  uint32_t ow[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int j = 4 * (2 * (C & 1) + (u >> 1)) + 2 * (u & 1);  // acc index of the word's first column
    const float o0 = acc[j] * fast_rcp(fmaf(e.lt, fast_exp2(__uint_as_float(gw[u] << 16) * -LOG2E), e.lt));
    const float o1 = acc[j + 1] * fast_rcp(fmaf(e.lt, fast_exp2(__uint_as_float(gw[u] & 0xffff0000u) * -LOG2E), e.lt));
    ow[u] = pack2(o0, o1);
  }
  u32x4 out = u32x4{ow[0], ow[1], ow[2], ow[3]};
  swap_halves(out);  // 8 contiguous columns at 16 C + 8 h
  if (e.store) *reinterpret_cast<u32x4*>(e.op + 16 * C) = out;
}
template <int C, bool NEXT>
__device__ __forceinline__ void epi_chunks(const SoloState& st, const EpiCtx& e, const SoloItem& Bn,
                                           const PrefillArgs& a, const SoloLds& L, int wave, int lane,
                                           u32x4 (&qw)[16]) {
  if constexpr (C < 16) {
    if constexpr (NEXT && C < 8) pro_loads<7 * C, 7 * C + 7>(Bn, a, L, wave, lane, qw);
    sfence();
    epi_chunk<C>(st, e);
    sfence();
    epi_chunks<C + 1, NEXT>(st, e, Bn, a, L, wave, lane, qw);
  }
}

// q, its table rows and the weights (prologue loads 0..39) have landed: at most
// the 16 K tile loads, or younger operations, are in flight (vector-memory
// counts retire in issue order; more younger operations only make it stricter)
__device__ __forceinline__ void wait_q(u32x4 (&qw)[16]) {
  asm volatile("s_waitcnt vmcnt(16)"
               : "+v"(qw[0]), "+v"(qw[1]), "+v"(qw[2]), "+v"(qw[3]), "+v"(qw[4]), "+v"(qw[5]),
                 "+v"(qw[6]), "+v"(qw[7]), "+v"(qw[8]), "+v"(qw[9]), "+v"(qw[10]), "+v"(qw[11]),
                 "+v"(qw[12]), "+v"(qw[13]), "+v"(qw[14]), "+v"(qw[15])
               :
               : "memory");
}

// The workgroup's items (one, or a causal pair). SHIFT = false: every logit is
// within +-64 (log2 units), so P = exp2(S) needs no shift (the normalisation
// cancels any common scale); SHIFT = true: P = exp2(S - m) with m an online row
// max (online_max). A pair's second item issues its prologue loads as soon
// as the first item's loop has released the LDS, before the first item's
// epilogue, which then runs while they are in flight.
template <bool CAUSAL, bool SHIFT>
__device__ __forceinline__ void solo_items(const PrefillArgs& a, const FItem& it0, const FItem& it1, int n_it,
                                           const SoloLds& L, int q_len_raw, int prior) {
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  SoloState st;
  u32x4 qw[16];
  SoloItem A, B;
  item_setup<CAUSAL>(A, a, it0, L, q_len_raw, prior, wave, lane);
  if (A.live) {
    pro_loads<0, 56>(A, a, L, wave, lane, qw);
    wait_q(qw);
    item_run<CAUSAL, SHIFT>(A, st, a, L, qw, wave, lane);
  }
  B.live = false;
  // after A's loop every lane-derived value is formed afresh, not held across it
  const int lane2 = fresh_lane();
  if (n_it == 2) {
    // B's geometry is formed here, not hoisted above A's loop (its registers
    // would be held across the loop): its inputs become opaque at this point
    FItem ib = it1;
    asm volatile("" : "+s"(ib.b), "+s"(ib.h), "+s"(ib.hk), "+s"(ib.qt));
    item_setup<CAUSAL>(B, a, ib, L, q_len_raw, prior, wave, lane2);
  }
  // every path waits for B's q before the paths join: a register whose load is
  // still in flight must not reach a join (the allocator may copy it there)
  if (A.live) {
    const EpiCtx e = epi_ctx(A, st, a, lane2);
    if (B.live) {
      epi_chunks<0, true>(st, e, B, a, L, wave, lane2, qw);
      wait_q(qw);
    } else {
      epi_chunks<0, false>(st, e, B, a, L, wave, lane2, qw);
    }
  } else if (B.live) {
    pro_loads<0, 56>(B, a, L, wave, lane2, qw);
    wait_q(qw);
  }
  if (B.live) {
    item_run<CAUSAL, SHIFT>(B, st, a, L, qw, wave, lane2);
    const EpiCtx e = epi_ctx(B, st, a, lane2);
    epi_chunks<0, false>(st, e, B, a, L, wave, lane2, qw);
  }
}

}  // namespace

template <bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_fused_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(1024))) uint16_t KO[3 * 2 * FT], VO[2 * 2 * FT];
  const int lane = threadIdx.x & 63;
  // the items first, so that their sequence's lengths load beside the norm weights.
  // Pairs (causal, B = 1): workgroup g runs the q-blocks of rank r and n_qt - 1 - r
  // of one head, n_qt + 1 blocks of keys in all for every workgroup
  FItem it0, it1;
  int n_it = 1;
  if (CAUSAL && a.pairs) {
    const int HB = a.H * a.B, r = blockIdx.x / HB, rem = blockIdx.x % HB;
    it0 = item_at(a, r * HB + rem);
    it1 = item_at(a, (a.n_qt - 1 - r) * HB + rem);
    n_it = 2;
  } else {
    it0 = item_ranked(a, blockIdx.x, CAUSAL, reinterpret_cast<int*>(KO));
    it1 = it0;
  }
  const int q_len_raw = a.q_lengths ? a.q_lengths[it0.b] : a.L;
  const int prior = a.prior ? a.prior[it0.b] : 0;
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
  if (bound <= FSTATIC_LIMIT)
    solo_items<CAUSAL, false>(a, it0, it1, n_it, L, q_len_raw, prior);
  else
    solo_items<CAUSAL, true>(a, it0, it1, n_it, L, q_len_raw, prior);
  // No global->LDS load is in flight here: each item ends with vmcnt(0) before
  // its last barrier, and an item with no rows issued none. Only the output
  // stores may be outstanding, which need no wait.
}

hipError_t launch_vt_transpose(const VtArgs& a, hipStream_t st) {
  if (a.B == 0 || a.Hk == 0 || a.vt_tiles == 0) return hipSuccess;
  // with vt_rows, a chunk of at most L rows spans at most L / 32 + 1 new tiles;
  // rows between vt_rows and the prior (written since, e.g. by decode steps)
  // are staged by the same workgroups' later iterations. Without, two tiles per
  // workgroup: at config 2 (512 tiles over 256 CUs) 14.4 against 15.7 us for
  // one tile per workgroup, 18.6 us for four
  const int chunk_tiles = (a.L + FN - 1) / FN + 1;
  constexpr int PASSES = 2;  // passes per workgroup without vt_rows
  const int gx = a.vt_rows && chunk_tiles < a.vt_tiles ? (chunk_tiles + VT_TP - 1) / VT_TP
                                                         : (a.vt_tiles + PASSES * VT_TP - 1) / (PASSES * VT_TP);
  hipLaunchKernelGGL(vt_transpose_kernel, dim3(gx, a.Hk, a.B), dim3(64 * VT_WAVES), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_prefill_fused(const PrefillArgs& a0, hipStream_t st, hipEvent_t t0, hipEvent_t t1) {
  const int64_t n_items = (int64_t)a0.n_qt * a0.H * a0.B;
  if (n_items == 0) return hipSuccess;
  PrefillArgs a = a0;
  // causal, one sequence, an even number of q-blocks and at least two items per
  // CU: each workgroup runs a heavy and a light q-block of one head (all
  // workgroups equal work, one launch and length fetch per pair); otherwise one
  // item per workgroup, heaviest first (the hardware hands the next item to the
  // first CU that frees up)
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  a.pairs = a.causal && a.B == 1 && (a.n_qt & 1) == 0 && n_items >= 2 * (int64_t)cus;
  const dim3 grid((unsigned)(a.pairs ? n_items / 2 : n_items)), block(256);
  if (t0 && t1) {
    if (a.causal)
      hipExtLaunchKernelGGL((prefill_fused_kernel<true>), grid, block, 0, st, t0, t1, 0, a);
    else
      hipExtLaunchKernelGGL((prefill_fused_kernel<false>), grid, block, 0, st, t0, t1, 0, a);
  } else if (a.causal) {
    hipLaunchKernelGGL((prefill_fused_kernel<true>), grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL((prefill_fused_kernel<false>), grid, block, 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace vm

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
//   S^T[tok][head] = K[tok][:] . Q[head][:]    16x16x32; A = K fragment, B = Q
//                                                in registers
//   O^T[d][head]  += V^T[d][tok] . P^T[tok][head]   16x16x16
// S^T already sits in the lanes/slots of the P^T operand. V^T comes from the
// natural-layout V fragments through a 16x16x32 MFMA against a 0/1 selection
// matrix (bf16 * 1.0 plus exact zeros is exact in fp32).
// K/V rows stream through a per-wave LDS ring of two 16-token slots, filled by
// direct global->LDS loads (non-temporal, 1 KB contiguous per instruction, no
// VGPR staging): the issue side runs one slot ahead of the compute side, across
// segment boundaries, so a wave always has up to 32 KB of K/V in flight. Each
// landed slot is read into registers (b128, rows XOR-swizzled) and refilled at
// once. One wave per SIMD; the four waves of a workgroup share nothing.
//
// Softmax: with QK-norm the logits are bounded, |s| <= |q~| * sqrt(D) *
// max|kw + w_offset|, so when that bound is <= 64 (log2 units) the fused path
// takes p = exp2(s) unshifted (p within 2^+-64, the merge's 1/l cancels the
// common scale); otherwise, and for the unfused operator, a running max
// rescaled lazily (only when it grows by > 8).
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace vm {

// Workspace of the no-allocation decode entry point (vm_gated_attn_decode_noalloc):
// one copy per GPU, part of the code object, held until the process ends. Host
// code never passes `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address): decode_static_scratch() looks up this GPU's
// address once and every launch takes that pointer.
static __device__ __align__(256) unsigned char scratch[DECODE_STATIC_SCRATCH_BYTES];

hipError_t decode_static_scratch(void** ptr) {
  constexpr int MAX_DEV = 64;
  static std::mutex mu;
  static void* addr[MAX_DEV] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_DEV) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    // first call on this device, with it current: its own copy of the array
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return hipSuccess;
}

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

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// lengths[b] for a wave-uniform b through a scalar load: unlike a vector load it
// is not counted by vmcnt, so reading it does not drain the K/V loads in flight.
// (lengths is only read by this kernel.)
__device__ __forceinline__ int sload_len(const int32_t* lengths, int b) {
  const int32_t* p = lengths + uniform(b);
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

struct StepBuf {
  uint4 k[8], v[8];
};

// Per-wave LDS ring: two slots of one 16-token step, K then V, each 16 rows of
// 512 B with chunk c of row r at c ^ swz(r).
constexpr int STEP_ELEMS = DSTEP * HEAD_DIM;  // bf16 per K (or V) step: 8 KB

// Issue the direct global->LDS loads of tokens [t, t + 16) of one (b, hk):
// instruction u moves rows t+2u and t+2u+1 (1 KB contiguous per instruction,
// non-temporal), 8 for K and 8 for V. Rows past `last` re-read row `last`.
__device__ __forceinline__ void issue_step(uint16_t* lk, uint16_t* lv, const uint16_t* kb,
                                           const uint16_t* vb, int t, int64_t last,
                                           int64_t c_st, int lane) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int r = 2 * u + (lane >> 5);
    const int64_t row = min((int64_t)(t + r), last);
    const int64_t off = row * c_st + 8 * ((lane & 31) ^ swz(r));
    __builtin_amdgcn_global_load_lds(kb + off, (__attribute__((address_space(3))) void*)(lk + 512 * u),
                                     16, 0, 2);
    __builtin_amdgcn_global_load_lds(vb + off, (__attribute__((address_space(3))) void*)(lv + 512 * u),
                                     16, 0, 2);
  }
}

// MFMA operand layout from a landed slot: lane (n, g) chunk kk = row n, dims
// 32kk + 8g .. +7.
__device__ __forceinline__ void read_step(StepBuf& s, const uint16_t* lk, const uint16_t* lv,
                                          int n, int g) {
  const int sw = swz(n);
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const int off = n * HEAD_DIM + 8 * ((4 * kk + g) ^ sw);
    s.k[kk] = *reinterpret_cast<const uint4*>(lk + off);
    s.v[kk] = *reinterpret_cast<const uint4*>(lv + off);
  }
}

__device__ __forceinline__ void compute_step(StepBuf& s, int t, int hi, int n, int g,
                                             const uint4 (&qop)[8], const uint4 (&sel)[2],
                                             f32x4 (&acc)[16], float& m_run, float& l_part,
                                             bool dyn) {
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
  if (dyn) {
    // running max in log2 units, rescaled lazily: only when it grows by more
    // than D_RESCALE_SLACK (wave-uniform branch)
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
  }
  // static mode: m_run = 0 and every |logit| <= 64 (log2 units), so p stays in
  // [2^-64, 2^64] unshifted; the merge's 1/l cancels the common scale
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

// The new token's cache row (knorm_rope_append_fwd, src/kernels/qknorm_rope_append.jl:59-98),
// built in the StepBuf layout of one 16-token step (every lane n holds the same
// row: lane (n, g) chunk kk = dims 32kk + 8g .. +7) and written to cache row
// `row` of (b, hk) by the lanes n == 0.
__device__ __forceinline__ void append_row(StepBuf& s, const DecodeArgs& a, int b, int hk,
                                           int row, int n, int g) {
  const uint16_t* kr = a.k_new + (int64_t)b * a.new_sb + (int64_t)hk * a.new_sh + 8 * g;
  const uint16_t* vr = a.v_new + (int64_t)b * a.new_sb + (int64_t)hk * a.new_sh + 8 * g;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    s.k[kk] = load16(kr + 32 * kk);
    s.v[kk] = load16(vr + 32 * kk);
  }
  // transformed in place, a chunk at a time (few live floats)
  float ss = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    float x[8];
    unpack8(s.k[kk], x);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
  }
  ss = col_sum4(ss);
  const float r = 1.0f / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
  {
    // chunks 0 and 1 hold the rotate-half pairs (d, d + 32), d = 8g + j
    float x1[8], x2[8], w1[8], w2[8];
    unpack8(s.k[0], x1);
    unpack8(s.k[1], x2);
    unpack8(load16(a.kw + 8 * g), w1);
    unpack8(load16(a.kw + 32 + 8 * g), w2);
    const float* cs = a.cos_tab + (int64_t)row * HALF_ROT + 8 * g;
    const float* sn = a.sin_tab + (int64_t)row * HALF_ROT + 8 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float c = cs[j], si = sn[j];
      const float u1 = x1[j] * r * (w1[j] + a.w_offset), u2 = x2[j] * r * (w2[j] + a.w_offset);
      x1[j] = u1 * c - u2 * si;
      x2[j] = u2 * c + u1 * si;
    }
    s.k[0] = pack8(x1);
    s.k[1] = pack8(x2);
  }
#pragma unroll
  for (int kk = 2; kk < 8; ++kk) {
    float x[8], wf[8];
    unpack8(s.k[kk], x);
    unpack8(load16(a.kw + 32 * kk + 8 * g), wf);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = x[j] * r * (wf[j] + a.w_offset);
    s.k[kk] = pack8(x);
  }
  if (n == 0) {
    const int64_t off = (int64_t)b * a.c_sb + (int64_t)hk * a.c_sh + (int64_t)row * a.c_st + 8 * g;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      *reinterpret_cast<uint4*>(a.kc + off + 32 * kk) = s.k[kk];
      *reinterpret_cast<uint4*>(a.vc + off + 32 * kk) = s.v[kk];
    }
  }
}

// One (b, hk) segment of a wave's chunk: its tokens [lo, hi) (a suffix of the
// previous segment's end); hm = hi - 1 when the wave appends the new token.
struct Seg {
  int b, hk, len, seg_b_start;
  int raw;  // lengths[b] as passed (may exceed ctx)
  int lo, hi, hm;
  bool append;
};

__device__ __forceinline__ void seg_bounds(Seg& s, int pos, int gw1, const DecodeArgs& a,
                                           bool fused) {
  const int seg_start = s.seg_b_start + s.hk * s.len;
  s.lo = pos - seg_start;
  s.hi = min(gw1 - seg_start, s.len);
  // fused append: the one wave whose range ends the segment makes row len-1
  // from the raw projection (in contract only: lengths[b] <= ctx)
  s.append = fused && a.k_new != nullptr && s.hi == s.len && s.raw <= a.ctx;
  s.hm = s.append ? s.hi - 1 : s.hi;
}

// lengths[b] for a wave-uniform b: from the register copy of the first 64
// (lane b holds lengths[b]), else through a scalar load, which vmcnt does not
// count, so reading it does not drain the K/V loads in flight
__device__ __forceinline__ int seq_len_raw(const int32_t* lengths, int raw_l, int b) {
  return b < 64 ? __builtin_amdgcn_readlane(raw_l, b) : sload_len(lengths, b);
}

// Move to the next non-empty segment of the chunk; false when the chunk ends.
__device__ __forceinline__ bool seg_next(Seg& s, int gw1, const DecodeArgs& a, bool fused,
                                         int raw_l) {
  const int pos = s.seg_b_start + s.hk * s.len + s.hi;
  if (pos >= gw1) return false;
  if (++s.hk == a.Hk) {
    s.hk = 0;
    s.seg_b_start += a.Hk * s.len;
    do {
      ++s.b;
      s.raw = seq_len_raw(a.lengths, raw_l, s.b);
      s.len = s.raw < 0 ? 0 : (s.raw > a.ctx ? (int)a.ctx : s.raw);
    } while (s.len == 0 && s.b + 1 < a.B);
  }
  seg_bounds(s, pos, gw1, a, fused);
  return true;
}

// Issue side of the step pipeline: the next 16-token step of the chunk.
struct Issuer {
  Seg s;
  int t;
  __device__ __forceinline__ bool next(uint16_t* slot, const DecodeArgs& a, int gw1, int64_t last,
                                       int lane, bool fused, int raw_l) {
    while (t >= s.hm) {
      if (!seg_next(s, gw1, a, fused, raw_l)) return false;
      t = s.lo;
    }
    const int64_t base = (int64_t)s.b * a.c_sb + (int64_t)s.hk * a.c_sh;
    issue_step(slot, slot + STEP_ELEMS, a.kc + base, a.vc + base, t, last, a.c_st, lane);
    t += DSTEP;
    return true;
  }
};

template <bool FUSED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void decode_stream_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int G = a.G, Hk = a.Hk;
  // ---- first loads, independent of each other and all issued before any is
  // used: lengths[lane] (the first 64 sequences, kept in a register for the
  // partition, the segment search and the segment walk) and, fused, the norm
  // weights (the same for every segment)
  const int raw_l = lane < a.B ? a.lengths[lane] : 0;
  uint2 kwv = make_uint2(0, 0);
  uint4 qwv[8];
  if (FUSED) {
    kwv = *reinterpret_cast<const uint2*>(a.kw + 4 * lane);  // d = 4*lane .. +3
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qwv[kk] = load16(a.qw + 32 * kk + 8 * g);
  }
  const int len_l = raw_l < 0 ? 0 : (raw_l > a.ctx ? (int)a.ctx : raw_l);
  // clamped lengths of sequences b0 + lane, b0 a multiple of 64
  auto lens_at = [&](int b0) __attribute__((always_inline)) {
    return b0 == 0 ? len_l : ((b0 + lane < a.B) ? clamp_len(a.lengths, b0 + lane, a.ctx) : 0);
  };
  // ---- stream partition: total work and this wave's chunk [gw0, gw1).
  // incl_at(b0): inclusive prefix of len * Hk (token-heads) over sequences
  // b0 .. b0 + lane, relative to b0
  const int incl0 = wave_scan_add(len_l * Hk);
  auto incl_at = [&](int b0) __attribute__((always_inline)) {
    return b0 == 0 ? incl0 : wave_scan_add(lens_at(b0) * Hk);
  };
  int W = __builtin_amdgcn_readlane(incl0, 63);
  for (int b0 = 64; b0 < a.B; b0 += 64) W += __builtin_amdgcn_readlane(incl_at(b0), 63);
  W = uniform(W);
  const int chunk = stream_chunk(W, a.NW, a.min_chunk);
  if (w == 0) {
    // snapshot of the partition for the merge, which then never reads lengths
    // (so it may advance them): chunk, then per sequence its clamped length and
    // first token-head
    int pre = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
      const int l = lens_at(b0);
      const int incl = incl_at(b0) + pre;
      if (b0 + lane < a.B) {
        a.geom[1 + b0 + lane] = l;
        a.geom[1 + a.B + b0 + lane] = incl - l * Hk;
      }
      pre = __builtin_amdgcn_readlane(incl, 63);
    }
    if (lane == 0) a.geom[0] = chunk;
  }
  const int gw0 = w * chunk;
  if (gw0 >= W) return;
  const int gw1 = min(gw0 + chunk, W);

  // ---- locate the segment holding gw0: first b whose prefix (token-heads) passes it
  int b = 0, seg_b_start = 0;
  {
    int pre = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
      const int len = lens_at(b0);
      const int incl = incl_at(b0) + pre;
      const uint64_t m = __ballot(b0 + lane < a.B && incl > gw0);
      if (m != 0ull) {
        const int fl = uniform(__ffsll((unsigned long long)m) - 1);
        b = b0 + fl;
        seg_b_start = __builtin_amdgcn_readlane(incl - len * Hk, fl);
        break;
      }
      pre = __builtin_amdgcn_readlane(incl, 63);
    }
  }
  b = uniform(b);
  seg_b_start = uniform(seg_b_start);
  const int raw = seq_len_raw(a.lengths, raw_l, b);
  const int len = raw < 0 ? 0 : (raw > a.ctx ? (int)a.ctx : raw);
  const int hk = (gw0 - seg_b_start) / len;

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
    float wm = fmaxf(fmaxf(fabsf(__uint_as_float(kwv.x << 16) + a.w_offset),
                           fabsf(__uint_as_float(kwv.x & 0xffff0000u) + a.w_offset)),
                     fmaxf(fabsf(__uint_as_float(kwv.y << 16) + a.w_offset),
                           fabsf(__uint_as_float(kwv.y & 0xffff0000u) + a.w_offset)));
    kbound = 16.0f * wave_max_all(wm) * 1.01f;
  }

  // ---- one continuous 16-token step pipeline over the segments of the chunk:
  // the issue side runs two steps ahead of the compute side and crosses
  // segment boundaries on its own, so a new segment starts with its first
  // steps already in flight
  // one __shared__ object per ring slot: the compiler then sees that reads of one
  // slot do not alias the loads still landing in the other
  __shared__ __attribute__((aligned(16))) uint16_t ring0[4][2 * STEP_ELEMS];
  __shared__ __attribute__((aligned(16))) uint16_t ring1[4][2 * STEP_ELEMS];
  uint16_t* const r0 = ring0[threadIdx.x >> 6];
  uint16_t* const r1 = ring1[threadIdx.x >> 6];
  const int64_t last = a.ctx - 1;

  Seg cs;  // compute side
  cs.b = b; cs.hk = hk; cs.len = len; cs.seg_b_start = seg_b_start; cs.raw = raw;
  seg_bounds(cs, gw0, gw1, a, FUSED);
  Issuer is;  // issue side, two steps ahead
  is.s = cs;
  is.t = cs.lo;
  int ct = cs.lo, inflight = 0, cslot = 0;
  bool primed = false;

  while (true) {
    // ---- Q operand for (b, hk): lane (n, g) holds q[head n][32kk + 8g + j] / 16
    uint4 qop[8];
    float qn2 = 0.f;
    {
      const int nn = n < G ? n : 0;
      const uint16_t* qp =
          a.q + (int64_t)cs.b * a.q_sb + (int64_t)(cs.hk * G + nn) * a.q_sh + 8 * g;
      // every prologue load first; the first K/V steps go out right behind them
      // (loads return in order: the prologue math then runs under the K/V steps)
      uint4 qraw[8];
      float4 cv[2], sv[2];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) qraw[kk] = load16(qp + 32 * kk);
      if (FUSED) {
        const int64_t p = cs.len - 1;  // fused decode: lengths are the positions
        const float4* cp = reinterpret_cast<const float4*>(a.cos_tab + p * HALF_ROT + 8 * g);
        const float4* sp = reinterpret_cast<const float4*>(a.sin_tab + p * HALF_ROT + 8 * g);
        cv[0] = cp[0]; cv[1] = cp[1];
        sv[0] = sp[0]; sv[1] = sp[1];
      }
      if (!primed) {
        if (is.next(r0, a, gw1, last, lane, FUSED, raw_l)) ++inflight;
        if (is.next(r1, a, gw1, last, lane, FUSED, raw_l)) ++inflight;
        primed = true;
      }
      float x[8][8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) unpack8(qraw[kk], x[kk]);
      if (FUSED) {
        // qnorm_rope_fwd (src/kernels/qknorm_rope_append.jl:25-57) on the fly
        float ss = 0.f;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
          for (int j = 0; j < 8; ++j) ss += x[kk][j] * x[kk][j];
        ss = col_sum4(ss);
        const float r = 1.0f / sqrtf(ss * (1.0f / HEAD_DIM) + a.eps);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          float wf[8];
          unpack8(qwv[kk], wf);
#pragma unroll
          for (int j = 0; j < 8; ++j) x[kk][j] = x[kk][j] * r * (wf[j] + a.w_offset);
        }
        const float cf[8] = {cv[0].x, cv[0].y, cv[0].z, cv[0].w, cv[1].x, cv[1].y, cv[1].z, cv[1].w};
        const float sf[8] = {sv[0].x, sv[0].y, sv[0].z, sv[0].w, sv[1].x, sv[1].y, sv[1].z, sv[1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x1 = x[0][j], x2 = x[1][j];
          x[0][j] = x1 * cf[j] - x2 * sf[j];
          x[1][j] = x2 * cf[j] + x1 * sf[j];
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
      qn2 = col_sum4(qn2);
    }
    float m_run = -INFINITY;
    bool dyn = true;
    if (FUSED) {
      // |logit| <= |q op| * |k~| (log2 units): within +-64 the shift is static
      const float bound = sqrtf(qn2) * 1.01f * kbound * LOG2E;
      if (__ballot(n < G && !(bound <= D_STATIC_LIMIT)) == 0ull) {
        m_run = 0.f;
        dyn = false;
      }
    }

    // ---- stream tokens [lo, hm) of (b, hk)
    f32x4 acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float l_part = 0.f;
    if (cs.append) {
      // the new token as a one-row step (rows n >= 1 are masked), taken first so
      // that its loads overlap the K/V steps already in flight
      StepBuf sb;
      append_row(sb, a, cs.b, cs.hk, cs.hi - 1, n, g);
      compute_step(sb, cs.hi - 1, cs.hi, n, g, qop, sel, acc, m_run, l_part, dyn);
    }
    // one 16-token step from ring slot `slot` (inlined per slot: the two slots are
    // distinct LDS objects in the generated code)
    auto step = [&](uint16_t* slot) __attribute__((always_inline)) {
      // the oldest step in flight is this one; the 16 loads of a later step may stay out
      if (inflight >= 2) wait_vmcnt<16>(); else wait_vmcnt<0>();
      StepBuf sb;
      read_step(sb, slot, slot + STEP_ELEMS, n, g);
      --inflight;
      // the slot is free once its reads have returned; refill it
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (is.next(slot, a, gw1, last, lane, FUSED, raw_l)) ++inflight;
      compute_step(sb, ct, cs.hm, n, g, qop, sel, acc, m_run, l_part, dyn);
      ct += DSTEP;
    };
    if (cslot == 1 && ct < cs.hm) {
      step(r1);
      cslot = 0;
    }
    while (ct < cs.hm) {
      step(r0);
      cslot = 1;
      if (ct >= cs.hm) break;
      step(r1);
      cslot = 0;
    }

    // ---- partial for (w, segment): slot w + b*Hk + hk
    const float l_tot = col_sum4(l_part);
    const int64_t slot = (int64_t)w + (int64_t)cs.b * Hk + cs.hk;
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
    if (!seg_next(cs, gw1, a, FUSED, raw_l)) break;
    ct = cs.lo;
  }
  wait_vmcnt<0>();  // no LDS load may land after the wave is gone
}

// Log-sum-exp merge of a segment's partials (src/kernels/attention_decode.jl:91-132)
// and the sigmoid gate (src/llm/qwen35.jl:205). One workgroup per (DW-wide d
// range, head n of the group, hk, b); thread (sg, dq) merges slots w_first+sg,
// +NSG, ... of its float4 column, CM slots per batch with every load issued
// before the merge arithmetic; the NSG slot groups then merge through LDS.
// DW = 64 suits many short segments, DW = 16 a few long ones (more workgroups,
// more slot groups). With `advance`, workgroup 0 bumps positions[b]
// (src/llm/generate.jl:82-88).
constexpr int CM = 8;

template <int DW>
__global__ __launch_bounds__(256) void decode_combine_kernel(CombineArgs a) {
  constexpr int NDR = HEAD_DIM / DW;  // d ranges
  constexpr int NDQ = DW / 4;         // float4 columns per range
  constexpr int NSG = 256 / NDQ;      // slot groups
  const int dr = blockIdx.x % NDR, n = blockIdx.x / NDR, hk = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x;
  const int sg = t / NDQ, dq = t % NDQ;
  const int d = dr * DW + 4 * dq;
  if (a.advance && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0) {
    // the stream kernel has read every position and this kernel reads none
    // (it works from the partition snapshot): the clock can move right away
    for (int i = t; i < a.B; i += 256) a.advance[i] += 1;
  }
  // partition snapshot written by decode_stream_kernel
  const int chunk = a.geom[0];
  const int len = a.geom[1 + b];
  const int seg_start = a.geom[1 + a.B + b] + hk * len;
  const int h = hk * a.G + n;
  float gate = 0.f;  // fetched early: it does not depend on the partials
  if (a.gate && t < DW) gate = bf2f(a.gate[(int64_t)b * a.g_sb + (int64_t)h * a.g_sh + dr * DW + t]);
  float M = -INFINITY, L = 0.f;
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  if (len > 0) {
    const int w_first = seg_start / chunk, w_last = (seg_start + len - 1) / chunk;
    const int64_t base = (int64_t)b * a.Hk + hk;
    for (int w0 = w_first + sg; w0 <= w_last; w0 += NSG * CM) {
      float2 ml[CM];
      float4 o[CM];
#pragma unroll
      for (int u = 0; u < CM; ++u) {
        const int w = w0 + NSG * u;
        if (w <= w_last) {
          const int64_t r = (w + base) * a.G + n;
          ml[u] = *reinterpret_cast<const float2*>(a.part_ml + 2 * r);
          o[u] = *reinterpret_cast<const float4*>(a.part_o + r * HEAD_DIM + d);
        } else {
          ml[u] = make_float2(-INFINITY, 0.f);
          o[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < CM; ++u) {
        const float mn = fmaxf(M, ml[u].x);
        const float c1 = M == mn ? 1.0f : fast_exp2(M - mn);
        const float c2 = ml[u].x == mn ? 1.0f : fast_exp2(ml[u].x - mn);
        L = L * c1 + ml[u].y * c2;
        O.x = O.x * c1 + o[u].x * c2;
        O.y = O.y * c1 + o[u].y * c2;
        O.z = O.z * c1 + o[u].z * c2;
        O.w = O.w * c1 + o[u].w * c2;
        M = mn;
      }
    }
  }
  __shared__ float sM[NSG], sL[NSG];
  __shared__ float4 sO[NSG][NDQ];
  if (dq == 0) {
    sM[sg] = M;
    sL[sg] = L;
  }
  sO[sg][dq] = O;
  __syncthreads();
  if (t < DW) {
    // thread t finishes d = dr*DW + t
    float Mf = -INFINITY;
#pragma unroll 8
    for (int i = 0; i < NSG; ++i) Mf = fmaxf(Mf, sM[i]);
    float Lf = 0.f, Of = 0.f;
    if (Mf > -INFINITY) {
      const float* so = reinterpret_cast<const float*>(&sO[0][0]);
#pragma unroll 8
      for (int i = 0; i < NSG; ++i) {
        const float c = fast_exp2(sM[i] - Mf);
        Lf += sL[i] * c;
        Of += so[i * DW + t] * c;
      }
    }
    float out = Lf > 0.f ? Of / Lf : 0.f;  // no valid key: o = 0 (attention_decode.jl:126-128)
    const int dd = dr * DW + t;
    if (a.gate) out *= sigmoidf(gate);
    a.out[(int64_t)b * a.o_sb + (int64_t)h * a.o_sh + dd] = f2bf(out);
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
  // partials per segment on average: many -> narrow d ranges, more slot groups
  const bool wide = a.NW >= 32 * a.B * a.Hk;
  if (wide) {
    hipLaunchKernelGGL(decode_combine_kernel<16>, dim3(16 * a.G, a.Hk, a.B), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL(decode_combine_kernel<64>, dim3(4 * a.G, a.Hk, a.B), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace vm

// common.h — device-side building blocks shared by the gated-attention kernels
// (gfx950 / CDNA4 only: wave64, bf16 MFMA 16x16x32 and 32x32x16, LDS transpose
// reads). Host-side argument checking lives in vallmo_attn.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));

// Compile-time facts of the Qwen3.5 attention block (src/llm/qwen35.jl:15-23).
constexpr int HEAD_DIM = 256;
constexpr int HALF_ROT = 32;       // rotary dim 64, rotate-half pairs (i, i+32)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float QK_SCALE = 0.0625f;  // 1/sqrt(256), a power of two: folding it
                                     // into bf16 q is exact

__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
// f32 -> bf16 round-to-nearest-even (finite inputs), the rounding the oracle uses.
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// Two f32 -> packed bf16 pair with the hardware RNE conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// 8 bf16 held as 4 dwords; converts to the MFMA operand type by bit cast.
struct alignas(16) U4 { uint32_t x, y, z, w; };

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// Streaming 16-byte load with the non-temporal hint: data read exactly once
// (decode K/V) should not displace reused lines in L2 / MALL.
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xffff0000u);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack2(f[0], f[1]); v.y = pack2(f[2], f[3]);
  v.z = pack2(f[4], f[5]); v.w = pack2(f[6], f[7]);
  return v;
}

// D = A*B + C. 16x16x32: A lane l holds A[l%16][8*(l/16)+j], B lane l holds
// B[8*(l/16)+j][l%16], D lane l holds D[4*(l/16)+j][l%16].
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
// 32x32x16: A lane l holds A[l%32][8*(l/32)+j], B lane l holds B[8*(l/32)+j][l%32],
// D lane l holds D[8*(j/4)+4*(l/32)+j%4][l%32].
__device__ __forceinline__ f32x16 mfma32(const uint4& a, const uint4& b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, output lane i slot r is
// component i%4 of the 4 halves read by source lane 4r + i/4.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* lds_ptr) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(lds_ptr));
  return __builtin_bit_cast(uint2, r);
}

// LDS tiles of 512-byte rows (one D = 256 bf16 row each) keep 16-byte chunk c of
// row r at chunk c ^ swz(r): the 8 rows that one b128 read cycle touches then
// fall on distinct banks for the MFMA operand reads.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 1) | ((r >> 2) & 1); }

// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order); used to consume direct global->LDS loads.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// silu and sigmoid with the full-precision exp (the DeltaNet gates and norms)
__device__ __forceinline__ float accurate_silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float accurate_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}
__device__ __forceinline__ float wave_sum_all(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Cross-lane sums, maxima and scans without LDS, on DPP row moves and the
// gfx950 permlane swaps (a ds_bpermute shuffle costs an LDS round trip each).
// Inclusive prefix sum over the 64 lanes: Hillis-Steele within each 16-lane row
// (lanes shifted in from outside the row read 0), then lane 15 of each row added
// to the next row and lane 31 to the upper half.
__device__ __forceinline__ int wave_scan_add(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2, 3
  return v;
}
// Maximum over the 64 lanes (the same running form; lane 63 holds the result).
__device__ __forceinline__ float wave_max_all(float v) {
  const int ninf = (int)0xff800000u;
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x111, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x112, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x114, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x118, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x142, 0xa, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), 0x143, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// v[l] + v[l ^ 16] + v[l ^ 32] + v[l ^ 48]: the sum down a column of the four
// 16-lane rows, the same bits in all four lanes. permlane16_swap of v with
// itself gives rows (0, 0, 2, 2) and (1, 1, 3, 3), permlane32_swap halves
// (lo, lo) and (hi, hi).
__device__ __forceinline__ float col_sum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sigmoidf(float x) { return fast_rcp(1.0f + __expf(-x)); }

// ---------------------------------------------------------------------------
// One (head, token) row of D = 256 per wave64: lane l holds d = 4l .. 4l+3 (one
// 8-byte load). The rotate-half partner of d < 32 is d + 32, i.e. lane l ^ 8.
// Norm + RoPE of one row held as 4 floats per lane (d = 4*lane + c):
// qknorm_rope_append.jl:41-54 / :80-92.
// wv: this lane's 4 norm weights (w + 4 lane, loaded by the caller: a kernel
// that stages several rows loads them once, ahead of its stores, so no row's
// weight load waits behind an earlier row's stores)
__device__ __forceinline__ void norm_rope_row_wv(float x[4], uint2 wv, float4 cv, float4 sv, float eps,
                                                 float w_offset, int lane) {
  // Every rounding step is spelled out (fmaf / __fmul_rn / __fadd_rn): left to
  // contraction, the compiler would fuse differently in each kernel that
  // inlines this, and the cache rows that decode and prefill append must be
  // bit-identical.
  float ss = __fmul_rn(x[0], x[0]);
  ss = fmaf(x[1], x[1], ss);
  ss = fmaf(x[2], x[2], ss);
  ss = fmaf(x[3], x[3], ss);
  ss = wave_sum_all(ss);
  const float r = 1.0f / sqrtf(fmaf(ss, 1.0f / HEAD_DIM, eps));
  float wf[4] = {__uint_as_float(wv.x << 16), __uint_as_float(wv.x & 0xffff0000u),
                 __uint_as_float(wv.y << 16), __uint_as_float(wv.y & 0xffff0000u)};
#pragma unroll
  for (int c = 0; c < 4; ++c) x[c] = __fmul_rn(__fmul_rn(x[c], r), __fadd_rn(wf[c], w_offset));
  // rotate-half on d < 64: lanes 0..7 hold x1 (d < 32), lanes 8..15 hold x2.
  float other[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) other[c] = __shfl_xor(x[c], 8, 64);
  if (lane < 16) {
    const float cc[4] = {cv.x, cv.y, cv.z, cv.w}, ssn[4] = {sv.x, sv.y, sv.z, sv.w};
    if (lane < 8) {
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = fmaf(x[c], cc[c], -__fmul_rn(other[c], ssn[c]));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = fmaf(x[c], cc[c], __fmul_rn(other[c], ssn[c]));
    }
  }
}
__device__ __forceinline__ void norm_rope_row_cs(float x[4], const uint16_t* __restrict__ w,
                                                 float4 cv, float4 sv, float eps, float w_offset,
                                                 int lane) {
  norm_rope_row_wv(x, *reinterpret_cast<const uint2*>(w + 4 * lane), cv, sv, eps, w_offset, lane);
}
// cs, sn: the position's cos / sin table rows (lanes 0..15 read 4 each)
__device__ __forceinline__ void norm_rope_row(float x[4], const uint16_t* __restrict__ w,
                                              const float* __restrict__ cs,
                                              const float* __restrict__ sn, float eps,
                                              float w_offset, int lane) {
  float4 cv = make_float4(0.f, 0.f, 0.f, 0.f), sv = cv;
  if (lane < 16) {
    const int i0 = 4 * (lane & 7);
    cv = *reinterpret_cast<const float4*>(cs + i0);
    sv = *reinterpret_cast<const float4*>(sn + i0);
  }
  norm_rope_row_cs(x, w, cv, sv, eps, w_offset, lane);
}

__device__ __forceinline__ void load_row4(const uint16_t* p, int lane, float x[4]) {
  uint2 v = *reinterpret_cast<const uint2*>(p + 4 * lane);
  x[0] = __uint_as_float(v.x << 16); x[1] = __uint_as_float(v.x & 0xffff0000u);
  x[2] = __uint_as_float(v.y << 16); x[3] = __uint_as_float(v.y & 0xffff0000u);
}
__device__ __forceinline__ void store_row4(uint16_t* p, int lane, const float x[4]) {
  uint2 v; v.x = pack2(x[0], x[1]); v.y = pack2(x[2], x[3]);
  *reinterpret_cast<uint2*>(p + 4 * lane) = v;
}

// Rows m .. m + 3 (m % 4 == 0) of batch column n of a stream-K GEMV's result
// (step.hip, gemv_sk_kernel; G 64-k groups, chunk units per workgroup): the
// partials of row group m / 128, one 16 KB slot per workgroup that touched it
// ([4 tiles][32 columns][32 rows] fp32, slot = workgroup + row group), added
// in workgroup order.
// one row's sum (the same additions as gemv_sk_sum4's lane for it)
__device__ __forceinline__ float gemv_sk_sum1(const float* part, int G, int chunk, int m, int n) {
  const int rg = m >> 7, v = (m >> 5) & 3, r = m & 31;
  const int wf = (rg * G) / chunk, wl = ((rg + 1) * G - 1) / chunk;
  const float* src = part + ((int64_t)(wf + rg) * 4 + v) * 1024 + n * 32 + r;
  float s = *src;
  for (int w = wf + 1; w <= wl; ++w) {
    src += 4096;
    s += *src;
  }
  return s;
}
__device__ __forceinline__ float4 gemv_sk_sum4(const float* part, int G, int chunk, int m, int n) {
  const int rg = m >> 7, v = (m >> 5) & 3, r = m & 31;
  const int wf = (rg * G) / chunk, wl = ((rg + 1) * G - 1) / chunk;
  const float* src = part + ((int64_t)(wf + rg) * 4 + v) * 1024 + n * 32 + r;
  float4 s = *reinterpret_cast<const float4*>(src);
#pragma unroll 4
  for (int w = wf + 1; w <= wl; ++w) {
    src += 4096;  // the next workgroup's slot of the same row group
    const float4 t = *reinterpret_cast<const float4*>(src);
    s.x += t.x;
    s.y += t.y;
    s.z += t.z;
    s.w += t.w;
  }
  return s;
}

}  // namespace vm

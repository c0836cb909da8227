/*
 * oracle.c — CPU fp32 restatement of the reference's gated full-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped. The product path (libvallmo_attn.so)
 * does not link or call it.
 *
 * Every quantity is evaluated in fp32 from the bf16 inputs (taken as their
 * exact fp32 values); nothing is rounded back to bf16, so it is the "plain
 * fp32 evaluation of the same math" the parity tolerances are stated against.
 * Layouts are row-major with the reference's column-major dims reversed,
 * e.g. K_cache (D, Ctx, Hk, B) is [B][Hk][Ctx][D] here.
 *
 * Reference lines followed (relative to the reference checkout):
 *   rope tables ............ src/llm/qwen35.jl:115-119
 *   per-head RMSNorm ........ src/llm/qwen35.jl:276-278, src/kernels/qknorm_rope_append.jl:41,80
 *   partial rotate-half RoPE  src/llm/qwen35.jl:280-287, qknorm_rope_append.jl:49-54,87-92
 *   cache append ............ qknorm_rope_append.jl:82-95, src/llm/qwen35.jl:306-307
 *   attention (mask, GQA,
 *     suffix offset, l==0) .. src/kernels/attention.jl:28-88
 *   decode attention ........ src/kernels/attention_decode.jl:14-181 (unsplit here)
 *   sigmoid gate ............ src/kernels/kernels.jl:34, src/llm/qwen35.jl:205,315
 *   decode! / forward ....... src/llm/qwen35.jl:187-208, 292-318
 *   linear! (y = W^T x) ..... src/linear.jl:40-57 (fp32 accumulation, linear.jl:29)
 *   rms_norm! ............... src/kernels/rms_norm.jl:3-31
 *   fused_add_rms_norm! ..... src/kernels/residual_norm.jl:4-37 (the second pass
 *                             reloads the stored bf16 x': rounded here too)
 *   MLP silu(gate) .* up .... src/llm/qwen35.jl:234-243, src/kernels/kernels.jl:35
 *   lm_head_argmax! ......... src/kernels/lm_head_topk.jl:27-101 (ties -> smallest)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf(uint16_t h) {
  union { uint32_t u; float f; } c;
  c.u = (uint32_t)h << 16;
  return c.f;
}

/* f32 -> bf16 round-to-nearest-even (finite inputs). */
uint16_t orc_f2bf(float f) {
  union { uint32_t u; float f; } c;
  c.f = f;
  uint32_t u = c.u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* rope_tables (qwen35.jl:115-119): inv_freq = Float32(theta^-(i/half)) with the
 * power in Float64; angle = inv_freq * Float32(t) in Float32; cos/sin of the
 * Float32 angle (evaluated in f64 and rounded once). Tables are [ctx][half]. */
void orc_rope_tables(float* cos_tab, float* sin_tab, int half, int64_t ctx, double theta) {
  for (int64_t t = 0; t < ctx; ++t)
    for (int i = 0; i < half; ++i) {
      float inv = (float)pow(theta, -((double)i / (double)half));
      float ang = inv * (float)t;
      cos_tab[t * half + i] = (float)cos((double)ang);
      sin_tab[t * half + i] = (float)sin((double)ang);
    }
}

/* y = rope(x / sqrt(mean(x^2) + eps) * (w + w_off), pos); rotate-half on the
 * first 2*half dims (qwen35.jl:276-287). x, y may not alias. */
void orc_head_norm_rope(const float* x, const float* w, float eps, float w_off,
                        const float* cos_tab, const float* sin_tab, int64_t pos, int D,
                        int half, float* y) {
  float ss = 0.f;
  for (int d = 0; d < D; ++d) ss += x[d] * x[d];
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  for (int d = 0; d < D; ++d) y[d] = x[d] * r * (w[d] + w_off);
  const float* c = cos_tab + pos * half;
  const float* s = sin_tab + pos * half;
  for (int i = 0; i < half; ++i) {
    const float x1 = y[i], x2 = y[i + half];
    y[i] = x1 * c[i] - x2 * s[i];
    y[i + half] = x2 * c[i] + x1 * s[i];
  }
}

static inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

/* One query row against keys [0, nk): o = softmax(scale * q.k) v, o = 0 if nk == 0
 * (attention.jl:86). q, k rows of Dk, v, o rows of Dv. k_rows/v_rows are arrays
 * of row pointers (so the oracle can mix cache rows and freshly computed rows
 * without copying). */
static void attend_row(const float* q, const float* const* k_rows, const float* const* v_rows,
                       int64_t nk, int Dk, int D, float scale, float* s_buf, float* o) {
  for (int d = 0; d < D; ++d) o[d] = 0.f;
  if (nk <= 0) return;
  float m = -INFINITY;
  for (int64_t u = 0; u < nk; ++u) {
    const float* k = k_rows[u];
    float acc = 0.f;
#pragma omp simd reduction(+ : acc)
    for (int d = 0; d < Dk; ++d) acc += q[d] * k[d];
    s_buf[u] = acc * scale;
    if (s_buf[u] > m) m = s_buf[u];
  }
  float l = 0.f;
  for (int64_t u = 0; u < nk; ++u) {
    const float p = expf(s_buf[u] - m);
    l += p;
    const float* v = v_rows[u];
#pragma omp simd
    for (int d = 0; d < D; ++d) o[d] += p * v[d];
  }
  const float inv = 1.0f / l;
  for (int d = 0; d < D; ++d) o[d] *= inv;
}

static void set_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
}

/* attention! core (attention.jl:12-91): q [B][H][L][Dk], k [B][Hk][Lk][Dk], v
 * [B][Hk][Lk][Dv] (fp32), o [B][H][L][Dv], scale 1/sqrt(Dk) (attention.jl:114).
 * k_len = k_lengths ? k_lengths[b] : Lk, q_len likewise; the
 * causal offset is k_len - q_len (queries are the suffix of keys). Rows
 * t >= q_len are left untouched. row_step > 1 evaluates every row_step-th row
 * only (the others are left untouched) to bound the cost of large checks. */
void orc_attention(const float* q, const float* k, const float* v, float* o,
                   const int32_t* k_lengths, const int32_t* q_lengths, int B, int H, int Hk,
                   int L, int Lk, int Dk, int Dv, int causal, int row_step, int nthreads) {
  set_threads(nthreads);
  const int G = H / Hk;
  const float scale = 1.0f / sqrtf((float)Dk);
  if (row_step < 1) row_step = 1;
#pragma omp parallel
  {
    float* s_buf = (float*)malloc(sizeof(float) * (size_t)(Lk > 0 ? Lk : 1));
    const float** kr = (const float**)malloc(sizeof(float*) * (size_t)(Lk > 0 ? Lk : 1));
    const float** vr = (const float**)malloc(sizeof(float*) * (size_t)(Lk > 0 ? Lk : 1));
#pragma omp for collapse(3) schedule(dynamic, 1)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h)
        for (int t = 0; t < L; t += row_step) {
          const int k_len = k_lengths ? k_lengths[b] : Lk;
          const int q_len = q_lengths ? q_lengths[b] : L;
          if (t >= q_len) continue;
          const int off = k_len - q_len;
          const int hk = h / G;
          int64_t nk = causal ? (int64_t)t + off + 1 : k_len;
          if (nk > k_len) nk = k_len;
          if (nk < 0) nk = 0;
          const float* kb = k + ((size_t)b * Hk + hk) * (size_t)Lk * Dk;
          const float* vb = v + ((size_t)b * Hk + hk) * (size_t)Lk * Dv;
          for (int64_t u = 0; u < nk; ++u) {
            kr[u] = kb + u * Dk;
            vr[u] = vb + u * Dv;
          }
          attend_row(q + (((size_t)b * H + h) * L + t) * Dk, kr, vr, nk, Dk, Dv, scale, s_buf,
                     o + (((size_t)b * H + h) * L + t) * Dv);
        }
    free(s_buf);
    free(kr);
    free(vr);
  }
}

/* decode!(h, ::AttnLayer, ...) attention part (qwen35.jl:187-208) for one step.
 * qkv  [B][2Hq+2Hk][D] bf16 packed [q1 g1 .. qHq gHq | k1..kHk | v1..vHk]
 * kc/vc [B][Hk][ctx][D] bf16 prior cache; columns 0..pos-2 are attended from it
 * positions[b] = 1-based column of the new token = attended length
 * out  [B][Hq][D] fp32 = (attention over the cache + new row) * sigmoid(gate)
 * knew/vnew [B][Hk][D] fp32 = the rows the step appends at column positions[b]. */
void orc_gated_decode(const uint16_t* qkv, const uint16_t* kc, const uint16_t* vc, int64_t ctx,
                      const int32_t* positions, const uint16_t* qw, const uint16_t* kw,
                      const float* cos_tab, const float* sin_tab, int B, int Hq, int Hk, int D,
                      int half, float eps, float w_off, float* out, float* knew, float* vnew,
                      int nthreads) {
  set_threads(nthreads);
  const int S = 2 * Hq + 2 * Hk, G = Hq / Hk;
  const float scale = 1.0f / sqrtf((float)D);
  float* qwf = (float*)malloc(sizeof(float) * D);
  float* kwf = (float*)malloc(sizeof(float) * D);
  for (int d = 0; d < D; ++d) {
    qwf[d] = bf(qw[d]);
    kwf[d] = bf(kw[d]);
  }
  /* new K/V rows first (knorm_rope_append!) */
  for (int b = 0; b < B; ++b) {
    const int64_t pos = positions[b] - 1;
    if (pos < 0) { /* no new token: nothing is appended (rows returned as NaN) */
      for (size_t i = (size_t)b * Hk * D; i < (size_t)(b + 1) * Hk * D; ++i)
        knew[i] = vnew[i] = NAN;
      continue;
    }
    for (int j = 0; j < Hk; ++j) {
      float x[1024];
      const uint16_t* kr = qkv + ((size_t)b * S + 2 * Hq + j) * D;
      const uint16_t* vr = qkv + ((size_t)b * S + 2 * Hq + Hk + j) * D;
      for (int d = 0; d < D; ++d) x[d] = bf(kr[d]);
      orc_head_norm_rope(x, kwf, eps, w_off, cos_tab, sin_tab, pos, D, half,
                         knew + ((size_t)b * Hk + j) * D);
      for (int d = 0; d < D; ++d) vnew[((size_t)b * Hk + j) * D + d] = bf(vr[d]);
    }
  }
  /* attention per (b, kv head): the group's G query heads share the fp32 copy
   * of the attended rows; the token loops run in parallel (one sequence may
   * hold all the work) */
  float* qn = (float*)malloc(sizeof(float) * (size_t)G * D);
  float* o = (float*)malloc(sizeof(float) * (size_t)G * D);
  for (int b = 0; b < B; ++b)
    for (int hk = 0; hk < Hk; ++hk) {
      const int64_t len = positions[b];
      if (len <= 0) { /* no key: o = 0 (attention_decode.jl:126-128) */
        for (int g = 0; g < G; ++g)
          for (int d = 0; d < D; ++d) out[((size_t)b * Hq + hk * G + g) * D + d] = 0.f;
        continue;
      }
      float* krow = (float*)malloc(sizeof(float) * (size_t)len * D);
      float* vrow = (float*)malloc(sizeof(float) * (size_t)len * D);
      float* s_buf = (float*)malloc(sizeof(float) * (size_t)len * G);
      const uint16_t* kb = kc + ((size_t)b * Hk + hk) * (size_t)ctx * D;
      const uint16_t* vb = vc + ((size_t)b * Hk + hk) * (size_t)ctx * D;
#pragma omp parallel for schedule(static)
      for (int64_t u = 0; u < len; ++u) {
        const float* kn = knew + ((size_t)b * Hk + hk) * D;
        const float* vn = vnew + ((size_t)b * Hk + hk) * D;
        for (int d = 0; d < D; ++d) {
          krow[u * D + d] = u + 1 < len ? bf(kb[u * D + d]) : kn[d];
          vrow[u * D + d] = u + 1 < len ? bf(vb[u * D + d]) : vn[d];
        }
      }
      for (int g = 0; g < G; ++g) {
        float x[1024];
        const uint16_t* qr = qkv + ((size_t)b * S + 2 * (hk * G + g)) * D;
        for (int d = 0; d < D; ++d) x[d] = bf(qr[d]);
        orc_head_norm_rope(x, qwf, eps, w_off, cos_tab, sin_tab, len - 1, D, half, qn + g * D);
      }
      /* scores, then the softmax max, then p and o = sum_u p_u v_u / l */
#pragma omp parallel for schedule(static)
      for (int64_t u = 0; u < len; ++u)
        for (int g = 0; g < G; ++g) {
          float acc = 0.f;
          for (int d = 0; d < D; ++d) acc += qn[g * D + d] * krow[u * D + d];
          s_buf[u * G + g] = acc * scale;
        }
      for (int g = 0; g < G; ++g) {
        float m = -INFINITY, l = 0.f;
        for (int64_t u = 0; u < len; ++u) m = s_buf[u * G + g] > m ? s_buf[u * G + g] : m;
        for (int d = 0; d < D; ++d) o[g * D + d] = 0.f;
#pragma omp parallel
        {
          float* op = (float*)calloc((size_t)D, sizeof(float));
          float lp = 0.f;
#pragma omp for schedule(static)
          for (int64_t u = 0; u < len; ++u) {
            const float p = expf(s_buf[u * G + g] - m);
            lp += p;
            for (int d = 0; d < D; ++d) op[d] += p * vrow[u * D + d];
          }
#pragma omp critical
          {
            l += lp;
            for (int d = 0; d < D; ++d) o[g * D + d] += op[d];
          }
          free(op);
        }
        const float inv = 1.0f / l;
        const uint16_t* gr = qkv + ((size_t)b * S + 2 * (hk * G + g) + 1) * D;
        for (int d = 0; d < D; ++d)
          out[((size_t)b * Hq + hk * G + g) * D + d] = o[g * D + d] * inv * sigmoid_f(bf(gr[d]));
      }
      free(krow);
      free(vrow);
      free(s_buf);
    }
  free(qn);
  free(o);
  free(qwf);
  free(kwf);
}

/* forward(::AttnLayer, ...; offset) attention part (qwen35.jl:292-318), ragged.
 * qkv  [B][T][2Hq+2Hk][D] bf16; kc/vc [B][Hk][ctx][D] bf16 prior cache
 * prior[b] = tokens already cached (the chunk starts at 0-based position prior[b]);
 * q_len[b] <= T chunk length. Chunk token t attends cache columns
 * 0..prior[b]+t (causal, queries are the suffix of keys).
 * out [B][T][Hq][D] fp32 (rows t >= q_len untouched; with row_step > 1 only rows
 * t % row_step == 0 are evaluated); kout/vout [B][Hk][T][D] fp32 = appended rows. */
void orc_gated_prefill(const uint16_t* qkv, const uint16_t* kc, const uint16_t* vc, int64_t ctx,
                       const int32_t* prior, const int32_t* q_len, const uint16_t* qw,
                       const uint16_t* kw, const float* cos_tab, const float* sin_tab, int B,
                       int T, int Hq, int Hk, int D, int half, float eps, float w_off,
                       float* out, float* kout, float* vout, int row_step, int nthreads) {
  set_threads(nthreads);
  const int S = 2 * Hq + 2 * Hk, G = Hq / Hk;
  const float scale = 1.0f / sqrtf((float)D);
  if (row_step < 1) row_step = 1;
  float* qwf = (float*)malloc(sizeof(float) * D);
  float* kwf = (float*)malloc(sizeof(float) * D);
  for (int d = 0; d < D; ++d) {
    qwf[d] = bf(qw[d]);
    kwf[d] = bf(kw[d]);
  }
  /* appended rows (the prologue): norm+rope(k), v */
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      if (t >= q_len[b]) continue;
      for (int j = 0; j < Hk; ++j) {
        float x[1024];
        const uint16_t* kr = qkv + (((size_t)b * T + t) * S + 2 * Hq + j) * D;
        const uint16_t* vr = qkv + (((size_t)b * T + t) * S + 2 * Hq + Hk + j) * D;
        for (int d = 0; d < D; ++d) x[d] = bf(kr[d]);
        orc_head_norm_rope(x, kwf, eps, w_off, cos_tab, sin_tab, (int64_t)prior[b] + t, D, half,
                           kout + (((size_t)b * Hk + j) * T + t) * D);
        for (int d = 0; d < D; ++d) vout[(((size_t)b * Hk + j) * T + t) * D + d] = bf(vr[d]);
      }
    }
  /* prior cache rows as fp32 */
  int64_t maxp = 0;
  for (int b = 0; b < B; ++b)
    if (prior[b] > maxp) maxp = prior[b];
  float* kpf = (float*)malloc(sizeof(float) * (size_t)B * Hk * (size_t)(maxp > 0 ? maxp : 1) * D);
  float* vpf = (float*)malloc(sizeof(float) * (size_t)B * Hk * (size_t)(maxp > 0 ? maxp : 1) * D);
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int j = 0; j < Hk; ++j)
      for (int64_t u = 0; u < prior[b]; ++u)
        for (int d = 0; d < D; ++d) {
          kpf[(((size_t)b * Hk + j) * maxp + u) * D + d] = bf(kc[(((size_t)b * Hk + j) * ctx + u) * D + d]);
          vpf[(((size_t)b * Hk + j) * maxp + u) * D + d] = bf(vc[(((size_t)b * Hk + j) * ctx + u) * D + d]);
        }
#pragma omp parallel
  {
    const int64_t maxk = maxp + T;
    float* s_buf = (float*)malloc(sizeof(float) * (size_t)maxk);
    const float** kp = (const float**)malloc(sizeof(float*) * (size_t)maxk);
    const float** vp = (const float**)malloc(sizeof(float*) * (size_t)maxk);
#pragma omp for collapse(3) schedule(dynamic, 1)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < Hq; ++h)
        for (int t = 0; t < T; t += row_step) {
          if (t >= q_len[b]) continue;
          const int hk = h / G;
          const int64_t P = prior[b];
          float x[1024], qn[1024], o[1024];
          const uint16_t* qr = qkv + (((size_t)b * T + t) * S + 2 * h) * D;
          const uint16_t* gr = qkv + (((size_t)b * T + t) * S + 2 * h + 1) * D;
          for (int d = 0; d < D; ++d) x[d] = bf(qr[d]);
          orc_head_norm_rope(x, qwf, eps, w_off, cos_tab, sin_tab, P + t, D, half, qn);
          const int64_t nk = P + t + 1;
          for (int64_t u = 0; u < P; ++u) {
            kp[u] = kpf + (((size_t)b * Hk + hk) * maxp + u) * D;
            vp[u] = vpf + (((size_t)b * Hk + hk) * maxp + u) * D;
          }
          for (int64_t u = 0; u <= t; ++u) {
            kp[P + u] = kout + (((size_t)b * Hk + hk) * T + u) * D;
            vp[P + u] = vout + (((size_t)b * Hk + hk) * T + u) * D;
          }
          attend_row(qn, kp, vp, nk, D, D, scale, s_buf, o);
          float* orow = out + (((size_t)b * T + t) * Hq + h) * D;
          for (int d = 0; d < D; ++d) orow[d] = o[d] * sigmoid_f(bf(gr[d]));
        }
    free(s_buf);
    free(kp);
    free(vp);
  }
  free(kpf);
  free(vpf);
  free(qwf);
  free(kwf);
}

/* linear! (src/linear.jl:40-57): y = W^T x in fp32 from bf16 operands.
 * Row-major views of the reference's column-major arrays: x [N][K] (x :: (K, N)),
 * W [M][K] (W :: (K, M), K-major), y [N][M] (y :: (M, N)). */
void orc_linear(const uint16_t* x, const uint16_t* w, float* y, int M, int N, int K,
                int nthreads) {
  set_threads(nthreads);
  float* wf = (float*)malloc(sizeof(float) * (size_t)M * K);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)M * K; ++i) wf[i] = bf(w[i]);
#pragma omp parallel
  {
    float* xr = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int k = 0; k < K; ++k) xr[k] = bf(x[(size_t)n * K + k]);
      for (int m = 0; m < M; ++m) {
        const float* wr = wf + (size_t)m * K;
        float acc = 0.f;
#pragma omp simd reduction(+ : acc)
        for (int k = 0; k < K; ++k) acc += wr[k] * xr[k];
        y[(size_t)n * M + m] = acc;
      }
    }
    free(xr);
  }
  free(wf);
}

/* rms_norm! / fused_add_rms_norm! over N columns of M: x, dx [N][M] bf16 bits
 * (dx NULL: plain norm), w [M]. xo [N][M] fp32 = x + dx (fused; NULL allowed),
 * y [N][M] fp32 = x' * rstd * (w + off), rstd = 1/sqrt(sum x'^2 / M + eps) over
 * the fp32 x'; fused, y uses bf16(x'), the value the reference stores and
 * reloads (residual_norm.jl:26-36).                                          */
void orc_rms_norm(const uint16_t* x, const uint16_t* dx, const uint16_t* w, float* xo, float* y,
                  int M, int N, float eps, float off) {
  for (int n = 0; n < N; ++n) {
    const uint16_t* xr = x + (size_t)n * M;
    float ss = 0.f;
    for (int m = 0; m < M; ++m) {
      float v = bf(xr[m]);
      if (dx) v += bf(dx[(size_t)n * M + m]);
      if (xo) xo[(size_t)n * M + m] = v;
      ss += v * v;
    }
    const float rstd = 1.0f / sqrtf(ss / (float)M + eps);
    for (int m = 0; m < M; ++m) {
      float v = bf(xr[m]);
      if (dx) v = bf(orc_f2bf(v + bf(dx[(size_t)n * M + m])));
      y[(size_t)n * M + m] = v * rstd * (bf(w[m]) + off);
    }
  }
}

/* mid [N][I] = silu(gate) * up, gate / up = gu[n][0..I-1], gu[n][I..2I-1]. */
void orc_silu_mul(const uint16_t* gu, float* mid, int I, int N) {
  for (int n = 0; n < N; ++n)
    for (int i = 0; i < I; ++i) {
      const float g = bf(gu[(size_t)n * 2 * I + i]), u = bf(gu[(size_t)n * 2 * I + I + i]);
      mid[(size_t)n * I + i] = g / (1.0f + expf(-g)) * u;
    }
}

/* lm_head_argmax!: result[b] = 1 + argmax_v sum_k w[v][k] x[b][k] (fp32 sums in
 * k order, ties to the smallest v); gap[b] = best - second best logit (the
 * margin by which the choice is stable). x [B][K], w [N][K] bf16 bits.       */
void orc_lm_head_argmax(const uint16_t* x, const uint16_t* w, int K, int N, int B,
                        int32_t* result, float* gap, int nthreads) {
  set_threads(nthreads);
  for (int b = 0; b < B; ++b) {
    float* xr = (float*)malloc(sizeof(float) * (size_t)K);
    for (int k = 0; k < K; ++k) xr[k] = bf(x[(size_t)b * K + k]);
    float best = -INFINITY, second = -INFINITY;
    int besti = 0;
#pragma omp parallel
    {
      float lb = -INFINITY, ls = -INFINITY;
      int li = 0x7fffffff;
#pragma omp for schedule(static)
      for (int v = 0; v < N; ++v) {
        const uint16_t* wr = w + (size_t)v * K;
        float acc = 0.f;
        for (int k = 0; k < K; ++k) acc += bf(wr[k]) * xr[k];
        if (acc > lb || (acc == lb && v < li)) {
          ls = lb;
          lb = acc;
          li = v;
        } else if (acc > ls) {
          ls = acc;
        }
      }
#pragma omp critical
      {
        if (lb > best || (lb == best && li < besti)) {
          second = fmaxf(second, fmaxf(best, ls));
          best = lb;
          besti = li;
        } else {
          second = fmaxf(second, lb);
        }
      }
    }
    result[b] = besti + 1;
    gap[b] = best - second;
    free(xr);
  }
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

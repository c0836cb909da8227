/*
 * deltanet.c — CPU fp32 restatement of the reference's linear-attention layer
 * parts: the depthwise causal conv1d and the gated delta-rule recurrence.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker, like oracle.c): only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product path does not link or call it.
 *
 * Every quantity is fp32 from the bf16 inputs taken exactly; nothing is rounded
 * back to bf16 except where the reference stores a bf16 value (the conv ring
 * state holds raw bf16 inputs, copied exactly). Layouts are row-major with the
 * reference's column-major dims reversed: the state S (Dk, Dv, Hv, B) is
 * [B][Hv][Dv][Dk] here, the conv ring (D, K, B) is [B][K][D].
 *
 * Reference lines followed (relative to the reference checkout):
 *   causal_conv1d! (one step, ring shift) ...... src/kernels/causal_conv1d.jl:7-41
 *   causal_conv1d_sequence! (+ S' seed) ........ src/kernels/causal_conv1d.jl:73-128
 *   suffix prefill (ring as left context) ....... src/llm/qwen35.jl:325-345
 *   deltanet_recurrent_decode! .................. src/kernels/deltanet_recurrent.jl:15-70
 *   deltanet_sequence! .......................... src/kernels/deltanet_recurrent.jl:109-172
 *   fused_deltanet_decode! ...................... src/kernels/deltanet_fused.jl:27-107
 *   prefill prep (l2 norms, gate, beta) ......... src/llm/qwen35.jl:347-356
 *   gated RMSNorm + z gate (prefill) ............ src/llm/qwen35.jl:360-364
 *   silu / sigmoid / softplus ................... src/kernels/kernels.jl:34-35,
 *                                                 src/llm/qwen35.jl:30
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bfv(uint16_t h) {
  union { uint32_t u; float f; } c;
  c.u = (uint32_t)h << 16;
  return c.f;
}
static inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
static inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

/* One conv step (causal_conv1d.jl:7-41): the ring s_in [B][K][D] shifts left
 * by one column, the new input x [B][D] enters as column K (s_out, may alias
 * s_in: every channel's columns are read before they are written), and
 * y [B][D] = sum_i s'[i] w[i] (+ bias) (silu when act). w [K][D], bias [D]
 * or NULL. */
void orc_conv1d_update(const uint16_t* x, const uint16_t* s_in, uint16_t* s_out,
                       const uint16_t* w, const uint16_t* bias, float* y, int D, int K, int B,
                       int act) {
  uint16_t* col = (uint16_t*)malloc((size_t)K * sizeof(uint16_t));
  for (int b = 0; b < B; ++b)
    for (int d = 0; d < D; ++d) {
      const size_t base = (size_t)b * K * D + d;
      for (int i = 0; i < K; ++i)
        col[i] = i == K - 1 ? x[(size_t)b * D + d] : s_in[base + (size_t)(i + 1) * D];
      float acc = 0.f;
      for (int i = 0; i < K; ++i) {
        s_out[base + (size_t)i * D] = col[i];
        acc += bfv(col[i]) * bfv(w[(size_t)i * D + d]);
      }
      if (bias) acc += bfv(bias[d]);
      y[(size_t)b * D + d] = act ? silu_f(acc) : acc;
    }
  free(col);
}

/* The whole-sequence conv (causal_conv1d.jl:73-128): x [B][T][D] ->
 * y [B][T][D], y[t] = sum_k w[k] x[t - K + 1 + k] with the left context taken
 * from s_in (columns 1..K-1 of the ring [B][K][D], the last K-1 raw inputs of a
 * prefix: the reference's suffix path, qwen35.jl:333-344) or zeros when s_in is
 * NULL. s_out (NULL: none) gets the last K inputs of the extended sequence,
 * the ring a decode step continues from. */
void orc_conv1d_sequence(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                         const uint16_t* s_in, uint16_t* s_out, float* y, int D, int K, int T,
                         int B, int act) {
  /* ext[j], j = 0 .. T + K - 2: K - 1 context columns, then x[0 .. T-1] */
  for (int b = 0; b < B; ++b)
    for (int d = 0; d < D; ++d) {
      const int E = T + K - 1;
      uint16_t* ext = (uint16_t*)malloc((size_t)E * sizeof(uint16_t));
      for (int j = 0; j < K - 1; ++j)
        ext[j] = s_in ? s_in[(size_t)b * K * D + (size_t)(j + 1) * D + d] : 0;
      for (int t = 0; t < T; ++t) ext[K - 1 + t] = x[((size_t)b * T + t) * D + d];
      for (int t = 0; t < T; ++t) {
        float acc = 0.f;
        for (int k = 0; k < K; ++k) acc += bfv(ext[t + k]) * bfv(w[(size_t)k * D + d]);
        if (bias) acc += bfv(bias[d]);
        y[((size_t)b * T + t) * D + d] = act ? silu_f(acc) : acc;
      }
      if (s_out)
        for (int i = 0; i < K; ++i) s_out[(size_t)b * K * D + (size_t)i * D + d] = ext[T - 1 + i];
      free(ext);
    }
}

/* One delta-rule step of one (value head, sequence) on its state s [Dv][Dk]
 * (in place): s = decay s; delta = beta (v - s^T k); s += k delta^T; o = s^T q
 * (deltanet_recurrent.jl:32-67). Sums over dk in increasing order. */
static void delta_step(float* s, const float* q, const float* k, const float* v, float beta,
                       float decay, float* o, int Dk, int Dv) {
  for (int c = 0; c < Dv; ++c) {
    float* sc = s + (size_t)c * Dk;
    float acc = 0.f;
    for (int i = 0; i < Dk; ++i) {
      sc[i] *= decay;
      acc += sc[i] * k[i];
    }
    const float delta = beta * (v[c] - acc);
    float out = 0.f;
    for (int i = 0; i < Dk; ++i) {
      sc[i] += k[i] * delta;
      out += sc[i] * q[i];
    }
    o[c] = out;
  }
}

/* deltanet_recurrent_decode! (deltanet_recurrent.jl:15-95): q, k [B][Hk][Dk],
 * v [B][Hv][Dv], beta, gate [B][Hv] (decay = exp(gate)), state s_in ->
 * s_out [B][Hv][Dv][Dk] (may alias), o [B][Hv][Dv]; value head h reads qk head
 * h / (Hv / Hk). All fp32. */
void orc_deltanet_decode(const float* q, const float* k, const float* v, const float* beta,
                         const float* gate, const float* s_in, float* s_out, float* o, int Dk,
                         int Dv, int Hk, int Hv, int B) {
  const int vpk = Hv / Hk;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hv; ++h) {
      const size_t sb = ((size_t)b * Hv + h) * Dv * Dk;
      if (s_out != s_in) memcpy(s_out + sb, s_in + sb, (size_t)Dv * Dk * sizeof(float));
      const int hk = h / vpk;
      delta_step(s_out + sb, q + ((size_t)b * Hk + hk) * Dk, k + ((size_t)b * Hk + hk) * Dk,
                 v + ((size_t)b * Hv + h) * Dv, beta[(size_t)b * Hv + h],
                 expf(gate[(size_t)b * Hv + h]), o + ((size_t)b * Hv + h) * Dv, Dk, Dv);
    }
}

/* deltanet_sequence! (deltanet_recurrent.jl:109-198): T steps in order.
 * q, k [B][Hk][T][Dk], v [B][Hv][T][Dv], beta, gate [B][T][Hv], state s_in ->
 * s_out [B][Hv][Dv][Dk] (may alias), o [B][Hv][T][Dv]. */
void orc_deltanet_sequence(const float* q, const float* k, const float* v, const float* beta,
                           const float* gate, const float* s_in, float* s_out, float* o, int Dk,
                           int Dv, int T, int Hk, int Hv, int B) {
  const int vpk = Hv / Hk;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hv; ++h) {
      const size_t sb = ((size_t)b * Hv + h) * Dv * Dk;
      if (s_out != s_in) memcpy(s_out + sb, s_in + sb, (size_t)Dv * Dk * sizeof(float));
      const int hk = h / vpk;
      for (int t = 0; t < T; ++t) {
        const size_t qo = (((size_t)b * Hk + hk) * T + t) * Dk;
        const size_t vo = (((size_t)b * Hv + h) * T + t) * Dv;
        const size_t g = ((size_t)b * T + t) * Hv + h;
        delta_step(s_out + sb, q + qo, k + qo, v + vo, beta[g], expf(gate[g]), o + vo, Dk, Dv);
      }
    }
}

/* fused_deltanet_decode! (deltanet_fused.jl:27-141): q, k [B][Hk][Dk], v and
 * z [B][Hv][Dv], alpha, beta_raw [B][Hv] bf16 bits; a_log, dt_bias [Hv] fp32;
 * norm_w [Dv] bf16. decay = exp(-exp(a_log) softplus(alpha + dt_bias)) with the
 * reference's threshold (x > 20: x); beta = sigmoid(beta_raw); q, k l2-normed
 * (sum x^2 + 1e-6), q also by 1/sqrt(Dk); then the delta step and
 * o = out rstd norm_w silu(z), rstd = 1/sqrt(mean out^2 + eps). o fp32. */
void orc_fused_deltanet_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const uint16_t* alpha, const uint16_t* beta_raw,
                               const uint16_t* z, const float* a_log, const float* dt_bias,
                               const uint16_t* norm_w, const float* s_in, float* s_out, float* o,
                               int Dk, int Dv, int Hk, int Hv, int B, float eps) {
  const int vpk = Hv / Hk;
  float* qn = (float*)malloc((size_t)Dk * sizeof(float));
  float* kn = (float*)malloc((size_t)Dk * sizeof(float));
  float* vv = (float*)malloc((size_t)Dv * sizeof(float));
  float* out = (float*)malloc((size_t)Dv * sizeof(float));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hv; ++h) {
      const int hk = h / vpk;
      const uint16_t* qr = q + ((size_t)b * Hk + hk) * Dk;
      const uint16_t* kr = k + ((size_t)b * Hk + hk) * Dk;
      float qss = 0.f, kss = 0.f;
      for (int i = 0; i < Dk; ++i) {
        qss += bfv(qr[i]) * bfv(qr[i]);
        kss += bfv(kr[i]) * bfv(kr[i]);
      }
      const float qsc = 1.0f / sqrtf(qss + 1e-6f) / sqrtf((float)Dk);
      const float ksc = 1.0f / sqrtf(kss + 1e-6f);
      for (int i = 0; i < Dk; ++i) {
        qn[i] = bfv(qr[i]) * qsc;
        kn[i] = bfv(kr[i]) * ksc;
      }
      const size_t hb = (size_t)b * Hv + h;
      for (int c = 0; c < Dv; ++c) vv[c] = bfv(v[hb * Dv + c]);
      const float spi = bfv(alpha[hb]) + dt_bias[h];
      const float sp = spi > 20.0f ? spi : logf(1.0f + expf(spi));
      const float decay = expf(-expf(a_log[h]) * sp);
      const float beta = sigmoid_f(bfv(beta_raw[hb]));
      const size_t sb = hb * Dv * Dk;
      if (s_out != s_in) memcpy(s_out + sb, s_in + sb, (size_t)Dv * Dk * sizeof(float));
      delta_step(s_out + sb, qn, kn, vv, beta, decay, out, Dk, Dv);
      float ss = 0.f;
      for (int c = 0; c < Dv; ++c) ss += out[c] * out[c];
      const float rstd = 1.0f / sqrtf(ss / (float)Dv + eps);
      for (int c = 0; c < Dv; ++c)
        o[hb * Dv + c] = out[c] * rstd * bfv(norm_w[c]) * silu_f(bfv(z[hb * Dv + c]));
    }
  free(qn);
  free(kn);
  free(vv);
  free(out);
}

/* The prefill's inputs to deltanet_sequence! (qwen35.jl:347-356) from the conv
 * output cv [B][T][n] bf16 (n = 2 Hk Dk + Hv Dv: the q | k | v channels) and
 * ab [B][T][2 Hv] bf16 (alpha | beta_raw): qe, ke [B][Hk][T][Dk] =
 * l2n(q) / sqrt(Dk), l2n(k) (l2n(y) = y / sqrt(sum y^2 + 1e-6)), ve
 * [B][Hv][T][Dv], beta [B][T][Hv] = sigmoid(beta_raw), gate [B][T][Hv] =
 * -exp(a_log) log1p(exp(alpha + dt_bias)). All fp32. */
void orc_deltanet_prep(const uint16_t* cv, const uint16_t* ab, const float* a_log,
                       const float* dt_bias, float* qe, float* ke, float* ve, float* beta,
                       float* gate, int Dk, int Dv, int Hk, int Hv, int T, int B) {
  const int n = 2 * Hk * Dk + Hv * Dv;
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      const uint16_t* r = cv + ((size_t)b * T + t) * n;
      for (int h = 0; h < Hk; ++h) {
        float qss = 0.f, kss = 0.f;
        for (int i = 0; i < Dk; ++i) {
          const float qv = bfv(r[h * Dk + i]), kv = bfv(r[Hk * Dk + h * Dk + i]);
          qss += qv * qv;
          kss += kv * kv;
        }
        const float qd = sqrtf(qss + 1e-6f), kd = sqrtf(kss + 1e-6f);
        const float sc = 1.0f / sqrtf((float)Dk);
        float* qo = qe + (((size_t)b * Hk + h) * T + t) * Dk;
        float* ko = ke + (((size_t)b * Hk + h) * T + t) * Dk;
        for (int i = 0; i < Dk; ++i) {
          qo[i] = bfv(r[h * Dk + i]) / qd * sc;
          ko[i] = bfv(r[Hk * Dk + h * Dk + i]) / kd;
        }
      }
      for (int h = 0; h < Hv; ++h) {
        float* vo = ve + (((size_t)b * Hv + h) * T + t) * Dv;
        for (int c = 0; c < Dv; ++c) vo[c] = bfv(r[2 * Hk * Dk + h * Dv + c]);
        const uint16_t* a = ab + ((size_t)b * T + t) * 2 * Hv;
        const size_t g = ((size_t)b * T + t) * Hv + h;
        beta[g] = sigmoid_f(bfv(a[Hv + h]));
        gate[g] = -expf(a_log[h]) * log1pf(expf(bfv(a[h]) + dt_bias[h]));
      }
    }
}

/* The prefill's epilogue (qwen35.jl:360-364): o [B][Hv][T][Dv] fp32 and
 * z [B][T][Hv][Dv] bf16 (the z rows of the projection) -> y [B][T][Hv][Dv]
 * fp32 = o rstd norm_w silu(z), rstd = 1/sqrt(mean_c o^2 + eps): the Wout
 * input (Dv Hv, T B). z has per-token stride z_st elements. */
void orc_gated_rms_norm(const float* o, const uint16_t* z, int64_t z_st, const uint16_t* norm_w,
                        float* y, int Dv, int Hv, int T, int B, float eps) {
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t)
      for (int h = 0; h < Hv; ++h) {
        const float* or_ = o + (((size_t)b * Hv + h) * T + t) * Dv;
        float ss = 0.f;
        for (int c = 0; c < Dv; ++c) ss += or_[c] * or_[c];
        const float rstd = 1.0f / sqrtf(ss / (float)Dv + eps);
        const uint16_t* zr = z + ((size_t)b * T + t) * z_st + (size_t)h * Dv;
        float* yr = y + (((size_t)b * T + t) * Hv + h) * Dv;
        for (int c = 0; c < Dv; ++c) yr[c] = or_[c] * rstd * bfv(norm_w[c]) * silu_f(bfv(zr[c]));
      }
}

/*
 * gdn_oracle.c -- CPU restatement of qwen-mlx's batched GatedDeltaNet step.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for libgdn: only the
 * tests, the smoke check and the bench's CPU-baseline leg may load it. The
 * product path never calls into it.
 *
 * Every function names the reference lines it restates (paths relative to the
 * qwen-mlx source tree). The reference itself cannot run here (Rust crate
 * over MLX/Metal, no toolchain), so each function is pinned by the checks in
 * tests/test_oracle_*.py: closed forms, invariants, brute force on tiny
 * inputs and an independent restatement in another state layout.
 *
 * Rounding model. The reference computes in MLX on bf16 activations. Where MLX
 * rounds an intermediate to bf16 the restatement rounds too (round to nearest
 * even), as far as the reference source fixes it:
 *   - elementwise bf16 ops (multiply, sigmoid, silu) round their result;
 *   - reductions and fast::rms_norm accumulate in f32;
 *   - conv1d (prefill) accumulates in f32 and rounds once.
 * The exact MLX reduction orders and transcendental ULPs are not fixed by the
 * reference source; results that depend on them are tolerance-bounded.
 *
 * Built by oracle/Makefile into oracle/liboracle_gdn.so.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- bf16 ---- */

static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return bf2f(f2bf(f)); }

uint16_t orc_f32_to_bf16(float f) { return f2bf(f); }
float orc_bf16_to_f32(uint16_t h) { return bf2f(h); }

/* MLX's sigmoid on f32: 1/(1+exp(-|x|)), mirrored for x < 0. */
static inline float sigmoid_f32(float x) {
  float y = 1.0f / (1.0f + expf(-fabsf(x)));
  return x < 0.0f ? 1.0f - y : y;
}

/* nn::silu on a bf16 array: x * sigmoid(x), each op rounded to bf16. */
static inline float silu_bf16(float x) {
  float s = rbf(sigmoid_f32(x));
  return rbf(x * s);
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------ gates ----- */

/*
 * compiled_beta_g restated (src/models/compiled_ops.rs:30-43), fed with the
 * merged projection ab = [b | a] (src/models/qwen3_5.rs:580-583,1037-1040):
 *   beta = bf16(sigmoid(f32(b)))
 *   g    = exp(-exp(f32(A_log)) * log(exp(a + dt_bias) + 1))   (naive softplus)
 * g is the decay MULTIPLIER the kernel applies (metal_gdn.rs:41).
 * ab: [ntok, 2*Hv] bf16; beta_out [ntok,Hv] bf16; g_out [ntok,Hv] f32.
 */
void orc_beta_g(const uint16_t* ab, int64_t ntok, int Hv, const float* A_log,
                const float* dt_bias, uint16_t* beta_out, float* g_out) {
  for (int64_t t = 0; t < ntok; ++t) {
    for (int h = 0; h < Hv; ++h) {
      float b = bf2f(ab[t * 2 * Hv + h]);
      float a = bf2f(ab[t * 2 * Hv + Hv + h]);
      if (beta_out) beta_out[t * Hv + h] = f2bf(sigmoid_f32(b));
      if (g_out) {
        float sp = logf(expf(a + dt_bias[h]) + 1.0f);
        g_out[t * Hv + h] = expf(-(expf(A_log[h]) * sp));
      }
    }
  }
}

/* ------------------------------------------------------------- conv ----- */

/*
 * S=1 causal conv update (src/models/qwen3_5.rs:593-610), B sequences:
 *   padded = concat(conv_state[B,K-1,D], x[B,1,D])          (:602)
 *   new conv_state = padded[:, 1:, :]  (bit-exact shift)    (:604)
 *   out = silu( sum_k padded[:,k,:] * w_dec[0,k,:] )         (:608-610)
 * with w_dec[0,k,ch] = w[ch,k] (weight prep :1058-1066). The multiply is a
 * bf16 elementwise op (each product rounded), the sum over the K taps
 * accumulates in f32 and rounds once.
 * conv_state_in/out [B,K-1,D] (may alias), x [B,D], w [D,K], out [B,D].
 */
void orc_conv_update(const uint16_t* conv_state_in, const uint16_t* x, const uint16_t* w,
                     int B, int D, int K, uint16_t* conv_state_out, uint16_t* out) {
  for (int b = 0; b < B; ++b) {
    const uint16_t* cs = conv_state_in + (int64_t)b * (K - 1) * D;
    uint16_t* cso = conv_state_out + (int64_t)b * (K - 1) * D;
    for (int ch = 0; ch < D; ++ch) {
      float acc = 0.0f;
      uint16_t win[8];
      for (int k = 0; k < K - 1; ++k) win[k] = cs[(int64_t)k * D + ch];
      win[K - 1] = x[(int64_t)b * D + ch];
      for (int k = 0; k < K; ++k) acc += rbf(bf2f(win[k]) * bf2f(w[(int64_t)ch * K + k]));
      out[(int64_t)b * D + ch] = f2bf(silu_bf16(rbf(acc)));
      for (int k = 0; k < K - 1; ++k) cso[(int64_t)k * D + ch] = win[k + 1];
    }
  }
}

/*
 * Prefill conv for one sequence (src/models/qwen3_5.rs:611-624):
 *   padded = concat(conv_state[K-1,D], x[S,D])                (:617)
 *   new conv_state = last K-1 rows of padded                   (:618-619)
 *   out = silu(conv1d(padded, w[D,K,1], groups=D))             (:620-623)
 * conv1d is a cross-correlation, out[t,ch] = sum_k padded[t+k,ch]*w[ch,k],
 * accumulated in f32 and rounded once to bf16.
 * conv_state_in/out [K-1,D] (may alias), x [S,D], out [S,D].
 */
void orc_conv_prefill(const uint16_t* conv_state_in, const uint16_t* x, const uint16_t* w,
                      int S, int D, int K, uint16_t* conv_state_out, uint16_t* out) {
  const int P = S + K - 1;
  uint16_t* padded = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)P * D);
  memcpy(padded, conv_state_in, sizeof(uint16_t) * (size_t)(K - 1) * D);
  memcpy(padded + (size_t)(K - 1) * D, x, sizeof(uint16_t) * (size_t)S * D);
  for (int t = 0; t < S; ++t) {
    for (int ch = 0; ch < D; ++ch) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k)
        acc += bf2f(padded[(int64_t)(t + k) * D + ch]) * bf2f(w[(int64_t)ch * K + k]);
      out[(int64_t)t * D + ch] = f2bf(silu_bf16(rbf(acc)));
    }
  }
  memcpy(conv_state_out, padded + (size_t)(P - (K - 1)) * D, sizeof(uint16_t) * (size_t)(K - 1) * D);
  free(padded);
}

/* ------------------------------------------------------------- norm ----- */

/*
 * fast::rms_norm(x, w, eps) on bf16 rows of length dim (src/models/qwen3_5.rs:638-639):
 *   r = 1/sqrt(sum(x^2)/dim + eps)   (f32)
 *   y = bf16( w * bf16(x * r) )
 * with the weights baked at construction (qwen3_5.rs:551-552):
 *   q: w = bf16(1/Dk), k: w = bf16(Dk^-0.5) (= 0.08837890625 for Dk=128).
 * x, out: [rows, dim] bf16 (may alias).
 */
void orc_rms_norm(const uint16_t* x, int64_t rows, int dim, float w, float eps, uint16_t* out) {
  const float wb = rbf(w);
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * dim;
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) {
      float v = bf2f(xr[i]);
      ss += v * v;
    }
    float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i) out[r * dim + i] = f2bf(wb * rbf(bf2f(xr[i]) * inv));
  }
}

/*
 * RMSNormGated epilogue (src/models/qwen3_5.rs:660-665; the same math as
 * norm_gate_fn, src/models/compiled_ops.rs:247-263):
 *   out = silu(z) * rms_norm(y, w, eps) on rows of dim (= Dv) elements:
 *   r = 1/sqrt(sum(y^2)/dim + eps) (f32), normed_i = bf16(w_i * bf16(y_i * r)),
 *   silu on bf16 z with each op rounded, the product rounded to bf16.
 * y, z, out: [rows, dim] bf16 (out may alias y); w: [dim] bf16.
 */
void orc_norm_gate(const uint16_t* y, const uint16_t* z, const uint16_t* w, int64_t rows, int dim,
                   float eps, uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* yr = y + r * dim;
    const uint16_t* zr = z + r * dim;
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) {
      const float v = bf2f(yr[i]);
      ss += v * v;
    }
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i) {
      const float normed = rbf(bf2f(w[i]) * rbf(bf2f(yr[i]) * inv));
      out[r * dim + i] = f2bf(silu_bf16(bf2f(zr[i])) * normed);
    }
  }
}

float orc_q_norm_weight(int dk) { return rbf(1.0f / (float)dk); }
float orc_k_norm_weight(int dk) { return rbf(powf((float)dk, -0.5f)); }

/* ------------------------------------------------------- recurrence ----- */

/*
 * gated_delta_kernel restated (src/models/metal_gdn.rs:10-67, launch :144-155),
 * f32 arithmetic. For every (b, hv, dv) row, hk = hv / (Hv/Hk) (:14):
 *   for t: s *= g[b,t,hv]; kv = sum_dk s*k; d = (v[dv]-kv)*beta;
 *          s += k*d; y[b,t,hv,dv] = bf16(sum_dk s*q)
 * The two dk-sums are formed as the kernel forms them: 32 lanes each summing
 * Dk/32 consecutive products, then the lane partials (simd_sum; summed here
 * in lane order).
 * state_in -> state_out, [B,Hv,Dv,Dk] f32; they may alias (the reference
 * writes a new array, :63-66). Dk <= 512.
 */
void orc_recurrent_io(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                      const uint16_t* beta, const float* state_in, float* state_out, uint16_t* y,
                      int B, int T, int Hk, int Hv, int Dk, int Dv) {
  const int ratio = Hv / Hk;
  const int npt = Dk / 32;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b) {
    for (int hv = 0; hv < Hv; ++hv) {
      const int hk = hv / ratio;
      float lane_acc[32];
      float s[512];
      for (int dv = 0; dv < Dv; ++dv) {
        const int64_t row = (((int64_t)b * Hv + hv) * Dv + dv) * Dk;
        memcpy(s, state_in + row, sizeof(float) * Dk);
        for (int t = 0; t < T; ++t) {
          const uint16_t* qt = q + (((int64_t)b * T + t) * Hk + hk) * Dk;
          const uint16_t* kt = k + (((int64_t)b * T + t) * Hk + hk) * Dk;
          const float gt = g[((int64_t)b * T + t) * Hv + hv];
          const float bt = bf2f(beta[((int64_t)b * T + t) * Hv + hv]);
          const float vt = bf2f(v[(((int64_t)b * T + t) * Hv + hv) * Dv + dv]);
          for (int l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (int i = 0; i < npt; ++i) {
              int d = l * npt + i;
              s[d] = s[d] * gt;
              a += s[d] * bf2f(kt[d]);
            }
            lane_acc[l] = a;
          }
          float kv = 0.0f;
          for (int l = 0; l < 32; ++l) kv += lane_acc[l];
          const float delta = (vt - kv) * bt;
          for (int l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (int i = 0; i < npt; ++i) {
              int d = l * npt + i;
              s[d] = s[d] + bf2f(kt[d]) * delta;
              a += s[d] * bf2f(qt[d]);
            }
            lane_acc[l] = a;
          }
          float o = 0.0f;
          for (int l = 0; l < 32; ++l) o += lane_acc[l];
          y[(((int64_t)b * T + t) * Hv + hv) * Dv + dv] = f2bf(o);
        }
        memcpy(state_out + row, s, sizeof(float) * Dk);
      }
    }
  }
}

void orc_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                   const uint16_t* beta, float* state, uint16_t* y, int B, int T, int Hk,
                   int Hv, int Dk, int Dv) {
  orc_recurrent_io(q, k, v, g, beta, state, state, y, B, T, Hk, Hv, Dk, Dv);
}

/*
 * Same recurrence in f64 (state carried in double through the T loop, stored
 * back rounded to f32). Used to bound the f32 kernels' rounding drift.
 * y_f64 receives the unrounded outputs when non-NULL.
 */
void orc_recurrent_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                       const uint16_t* beta, float* state, uint16_t* y, double* y_f64, int B,
                       int T, int Hk, int Hv, int Dk, int Dv) {
  const int ratio = Hv / Hk;
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b) {
    for (int hv = 0; hv < Hv; ++hv) {
      const int hk = hv / ratio;
      double* s = (double*)malloc(sizeof(double) * (size_t)Dk);
      for (int dv = 0; dv < Dv; ++dv) {
        float* sf = state + (((int64_t)b * Hv + hv) * Dv + dv) * Dk;
        for (int d = 0; d < Dk; ++d) s[d] = sf[d];
        for (int t = 0; t < T; ++t) {
          const uint16_t* qt = q + (((int64_t)b * T + t) * Hk + hk) * Dk;
          const uint16_t* kt = k + (((int64_t)b * T + t) * Hk + hk) * Dk;
          const double gt = g[((int64_t)b * T + t) * Hv + hv];
          const double bt = bf2f(beta[((int64_t)b * T + t) * Hv + hv]);
          const double vt = bf2f(v[(((int64_t)b * T + t) * Hv + hv) * Dv + dv]);
          double kv = 0.0;
          for (int d = 0; d < Dk; ++d) {
            s[d] *= gt;
            kv += s[d] * (double)bf2f(kt[d]);
          }
          const double delta = (vt - kv) * bt;
          double o = 0.0;
          for (int d = 0; d < Dk; ++d) {
            s[d] += (double)bf2f(kt[d]) * delta;
            o += s[d] * (double)bf2f(qt[d]);
          }
          int64_t yi = (((int64_t)b * T + t) * Hv + hv) * Dv + dv;
          y[yi] = f2bf((float)o);
          if (y_f64) y_f64[yi] = o;
        }
        for (int d = 0; d < Dk; ++d) sf[d] = (float)s[d];
      }
      free(s);
    }
  }
}

/* ------------------------------------------------------ full layer ----- */

/*
 * One GDN layer after the input projections, S=1, B stacked sequences
 * (src/models/qwen3_5.rs:588-658): conv update (:593-610), split q|k|v
 * (:626-634), q/k rms-norm with baked weights (:636-639, :551-552), gates
 * (:641-642 -> compiled_ops.rs:30-43), recurrence (:650-658 -> metal_gdn.rs).
 * conv_in -> conv_out [B,K-1,D] and state_in -> state_out [B,Hv,Dv,Dk]
 * (either pair may alias; orc_decode is the in-place form).
 * mixed_qkv [B,D], ab [B,2Hv], conv_w [D,K], y [B,Hv,Dv].
 */
void orc_decode_io(const uint16_t* conv_in, uint16_t* conv_out, const float* state_in,
                   float* state_out, const uint16_t* mixed_qkv, const uint16_t* ab,
                   const float* A_log, const float* dt_bias, const uint16_t* conv_w, uint16_t* y,
                   int B, int Hk, int Hv, int Dk, int Dv, int K) {
  const int D = 2 * Hk * Dk + Hv * Dv;
  uint16_t* xc = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * D);
  uint16_t* q = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * Hk * Dk);
  uint16_t* k = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * Hk * Dk);
  uint16_t* v = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * Hv * Dv);
  uint16_t* beta = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)B * Hv);
  float* g = (float*)malloc(sizeof(float) * (size_t)B * Hv);
  orc_conv_update(conv_in, mixed_qkv, conv_w, B, D, K, conv_out, xc);
  for (int b = 0; b < B; ++b) {
    memcpy(q + (size_t)b * Hk * Dk, xc + (size_t)b * D, sizeof(uint16_t) * Hk * Dk);
    memcpy(k + (size_t)b * Hk * Dk, xc + (size_t)b * D + Hk * Dk, sizeof(uint16_t) * Hk * Dk);
    memcpy(v + (size_t)b * Hv * Dv, xc + (size_t)b * D + 2 * Hk * Dk, sizeof(uint16_t) * Hv * Dv);
  }
  orc_rms_norm(q, (int64_t)B * Hk, Dk, 1.0f / (float)Dk, 1e-6f, q);
  orc_rms_norm(k, (int64_t)B * Hk, Dk, powf((float)Dk, -0.5f), 1e-6f, k);
  orc_beta_g(ab, B, Hv, A_log, dt_bias, beta, g);
  orc_recurrent_io(q, k, v, g, beta, state_in, state_out, y, B, 1, Hk, Hv, Dk, Dv);
  free(xc); free(q); free(k); free(v); free(beta); free(g);
}

void orc_decode(uint16_t* conv_state, float* state, const uint16_t* mixed_qkv,
                const uint16_t* ab, const float* A_log, const float* dt_bias,
                const uint16_t* conv_w, uint16_t* y, int B, int Hk, int Hv, int Dk, int Dv,
                int K) {
  orc_decode_io(conv_state, conv_state, state, state, mixed_qkv, ab, A_log, dt_bias, conv_w, y,
                B, Hk, Hv, Dk, Dv, K);
}

/*
 * Prefill of one sequence of S tokens (src/models/qwen3_5.rs:611-658 with
 * b=1): prefill conv, split, norm, gates, then ONE recurrence launch with
 * T=S (metal_gdn.rs:37; the reference does not chunk).
 * conv_state [K-1,D], state [Hv,Dv,Dk] in/out; mixed_qkv [S,D], ab [S,2Hv],
 * y [S,Hv,Dv]. f64 != 0 runs the recurrence in f64.
 */
void orc_prefill(uint16_t* conv_state, float* state, const uint16_t* mixed_qkv,
                 const uint16_t* ab, const float* A_log, const float* dt_bias,
                 const uint16_t* conv_w, uint16_t* y, int S, int Hk, int Hv, int Dk, int Dv,
                 int K, int f64) {
  const int D = 2 * Hk * Dk + Hv * Dv;
  uint16_t* xc = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * D);
  uint16_t* q = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * Hk * Dk);
  uint16_t* k = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * Hk * Dk);
  uint16_t* v = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * Hv * Dv);
  uint16_t* beta = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)S * Hv);
  float* g = (float*)malloc(sizeof(float) * (size_t)S * Hv);
  orc_conv_prefill(conv_state, mixed_qkv, conv_w, S, D, K, conv_state, xc);
  for (int t = 0; t < S; ++t) {
    memcpy(q + (size_t)t * Hk * Dk, xc + (size_t)t * D, sizeof(uint16_t) * Hk * Dk);
    memcpy(k + (size_t)t * Hk * Dk, xc + (size_t)t * D + Hk * Dk, sizeof(uint16_t) * Hk * Dk);
    memcpy(v + (size_t)t * Hv * Dv, xc + (size_t)t * D + 2 * Hk * Dk, sizeof(uint16_t) * Hv * Dv);
  }
  orc_rms_norm(q, (int64_t)S * Hk, Dk, 1.0f / (float)Dk, 1e-6f, q);
  orc_rms_norm(k, (int64_t)S * Hk, Dk, powf((float)Dk, -0.5f), 1e-6f, k);
  orc_beta_g(ab, S, Hv, A_log, dt_bias, beta, g);
  if (f64)
    orc_recurrent_f64(q, k, v, g, beta, state, y, NULL, 1, S, Hk, Hv, Dk, Dv);
  else
    orc_recurrent(q, k, v, g, beta, state, y, 1, S, Hk, Hv, Dk, Dv);
  free(xc); free(q); free(k); free(v); free(beta); free(g);
}

/* ------------------------------------------------ quantized matmul ----- */

/*
 * mlx::core::quantized_matmul(x, w, scales, biases, transpose=true,
 * group_size=64, bits=4) as the reference calls it on the merged GDN input
 * projections (src/models/qwen3_5.rs:572-586, weights merged along the output
 * axis at :1037-1053) and the lm_head (:869-874). The operation lives in the
 * MLX dependency (mlx-rs 0.25.3 over mlx-sys 0.2.0, not vendored); its
 * published affine 4-bit format is restated here:
 *   w uint32 [N, K/8]: element k of row n is the nibble at bits 4*(k%8) of
 *   word k/8; scales, biases [N, K/64] (bf16 here); dequantized weight
 *   W[n,k] = scales[n,k/64] * q[n,k] + biases[n,k/64]   (mlx dequantize,
 *   used by the reference at qwen3_5.rs:852).
 * orc_dequant_w4 writes W in f64 (exact). orc_qmatmul_w4 forms
 *   y_exact[m,n] = sum_k x[m,k] W[n,k] in f64 (the dequantized weight is
 *   never rounded), y = y_exact correctly rounded to bf16 (round to odd to
 *   f32, then to nearest even: no double-rounding error), and
 *   mag[m,n] = sum_k |x[m,k]| (|s| (128 + q) + |b|), a scale for checkers'
 *   f32-accumulation bounds. MLX's own kernels accumulate in f32 (and its
 *   large-M path rounds the dequantized weight to bf16 first), so a result
 *   within f32 accumulation error of y_exact, rounded once, is as close as any
 *   implementation of this contract gets. Any pointer among y_exact, mag, y
 *   may be NULL.
 */
static inline uint16_t f64_to_bf16(double d) {
  float f = (float)d;
  if ((double)f != d && isfinite(f)) {  /* round to odd: truncate, set the sticky bit */
    if (fabs((double)f) > fabs(d)) f = nextafterf(f, 0.0f);
    uint32_t u;
    memcpy(&u, &f, 4);
    u |= 1u;
    memcpy(&f, &u, 4);
  }
  return f2bf(f);
}

uint16_t orc_f64_to_bf16(double d) { return f64_to_bf16(d); }

void orc_dequant_w4(const uint32_t* w, const uint16_t* s, const uint16_t* b, int N, int K,
                    double* out) {
  const int words = K / 8, G = K / 64;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      const uint32_t q = (w[(int64_t)n * words + k / 8] >> (4 * (k % 8))) & 0xFu;
      out[(int64_t)n * K + k] =
          (double)bf2f(s[(int64_t)n * G + k / 64]) * (double)q + (double)bf2f(b[(int64_t)n * G + k / 64]);
    }
}

void orc_qmatmul_w4(const uint16_t* x, int64_t xs, int M, int K, const uint32_t* w,
                    const uint16_t* s, const uint16_t* b, int N, double* y_exact, double* mag,
                    uint16_t* y) {
  const int words = K / 8, G = K / 64;
#pragma omp parallel
  {
    double* wr = (double*)malloc(sizeof(double) * K);
    double* wa = (double*)malloc(sizeof(double) * K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int k = 0; k < K; ++k) {
        const uint32_t q = (w[(int64_t)n * words + k / 8] >> (4 * (k % 8))) & 0xFu;
        const double sc = bf2f(s[(int64_t)n * G + k / 64]), bi = bf2f(b[(int64_t)n * G + k / 64]);
        wr[k] = sc * (double)q + bi;
        wa[k] = fabs(sc) * (128.0 + (double)q) + fabs(bi);
      }
      for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (int64_t)m * xs;
        double acc = 0.0, am = 0.0;
        for (int k = 0; k < K; ++k) {
          const double xv = bf2f(xr[k]);
          acc += xv * wr[k];
          am += fabs(xv) * wa[k];
        }
        const int64_t o = (int64_t)m * N + n;
        if (y_exact) y_exact[o] = acc;
        if (mag) mag[o] = am;
        if (y) y[o] = f64_to_bf16(acc);
      }
    }
    free(wr);
    free(wa);
  }
}

/* ---------------------------------------------------- stack/unstack ----- */

/*
 * stack_caches for the GDN layers (src/scheduler/mlx_executor.rs:42-55,92-115):
 * concatenate each sequence's [1,...] state along axis 0. The per-sequence
 * states live in a slot pool here, so the concat is a gather by slot id.
 * pool [num_slots, elems], out [n, elems] (element size esz bytes).
 */
void orc_stack(const void* pool, const int32_t* slot_ids, int n, int64_t elems, int esz,
               void* out) {
  for (int i = 0; i < n; ++i)
    memcpy((char*)out + (size_t)i * elems * esz, (const char*)pool + (size_t)slot_ids[i] * elems * esz,
           (size_t)elems * esz);
}

/*
 * unstack_caches (src/scheduler/mlx_executor.rs:118-130): sequence i takes row
 * i..i+1 of the batched result. With a slot pool that is a scatter.
 */
void orc_unstack(void* pool, const int32_t* slot_ids, int n, int64_t elems, int esz,
                 const void* in) {
  for (int i = 0; i < n; ++i)
    memcpy((char*)pool + (size_t)slot_ids[i] * elems * esz, (const char*)in + (size_t)i * elems * esz,
           (size_t)elems * esz);
}

/* ------------------------------------------------------ CPU baseline ----- */

/*
 * CPU baseline of one batched decode step over L layers, as the reference
 * executes it (src/scheduler/mlx_executor.rs:166-192 with the GDN layer of
 * qwen3_5.rs:588-658), OpenMP over (b, hv):
 *   per layer: stack = concat copy of the B per-sequence states into a batch
 *   buffer (mlx_executor.rs:54), the kernel writes a NEW state array
 *   (metal_gdn.rs:63-66), unstack = each sequence now refers to its row of that
 *   new array (mlx_executor.rs:126-127, views, no copy).
 * seq_state[l][b] / seq_conv[l][b] are the per-sequence state pointers; they
 * are re-pointed into out_state / out_conv (caller-owned [L][B*...] arrays).
 * in_state / in_conv are the stacked scratch buffers ([B*...] each, reused
 * across layers).
 */
void orc_baseline_step(int L, int B, float** seq_state, uint16_t** seq_conv,
                       float* in_state, uint16_t* in_conv, float** out_state,
                       uint16_t** out_conv, const uint16_t* mixed_qkv, const uint16_t* ab,
                       const float* A_log, const float* dt_bias, const uint16_t* conv_w,
                       uint16_t* y, int Hk, int Hv, int Dk, int Dv, int K) {
  const int D = 2 * Hk * Dk + Hv * Dv;
  const int64_t se = (int64_t)Hv * Dv * Dk;
  const int64_t ce = (int64_t)(K - 1) * D;
  for (int l = 0; l < L; ++l) {
    float** ss = seq_state + (size_t)l * B;
    uint16_t** sc = seq_conv + (size_t)l * B;
#pragma omp parallel for schedule(static)
    for (int b = 0; b < B; ++b) {
      memcpy(in_state + b * se, ss[b], sizeof(float) * se);
      memcpy(in_conv + b * ce, sc[b], sizeof(uint16_t) * ce);
    }
    /* kernel: reads the stacked buffers, writes new arrays */
    orc_decode_io(in_conv, out_conv[l], in_state, out_state[l], mixed_qkv + (size_t)l * B * D,
               ab + (size_t)l * B * 2 * Hv, A_log + (size_t)l * Hv, dt_bias + (size_t)l * Hv,
               conv_w + (size_t)l * D * K, y + (size_t)l * B * Hv * Dv, B, Hk, Hv, Dk, Dv, K);
    for (int b = 0; b < B; ++b) {
      ss[b] = out_state[l] + b * se;
      sc[b] = out_conv[l] + b * ce;
    }
  }
}

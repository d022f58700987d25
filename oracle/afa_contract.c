/*
 * C restatement of the reference AFA kernel's numeric contract.
 *
 * TEST INFRASTRUCTURE ONLY: linked by tests/ and by bench.py's cpu_baseline leg,
 * never by the product library.  Built by oracle/build_oracle.py into
 * oracle/_build/liboracle_afa.so.
 *
 * Forward contract (tasmaikeni13/algebraic-intelligence, src/kernels/pallas_afa.py):
 *   - per (b, h, query tile, key tile): S = (Q_tile K_tile^T) * scale with the products
 *     accumulated in fp32 (fp64 for fp64 inputs)                        (:104-110, :208)
 *   - P = rho(S)^8 with the two-branch cancellation-safe rho              (:32-49, :113)
 *   - key padding mask col >= valid_len and causal mask col <= row       (:115-124)
 *   - O += cast(P, v.dtype) @ V_tile (fp32 accumulation); D += rowsum(P) with the
 *     unrounded P                                                       (:126-139)
 *   - out = O / (D + Omega) cast to q.dtype; d = D + Omega in fp32       (:141-151)
 *   - causal key tiles at or beyond the query tile end are skipped       (:88-95, :388-392)
 * Optional AGO rotation of q and k (src/attention.py:142-152): this library's fused
 * contract rotates the input-dtype values in fp32 (fp64 for fp64) with fp32 tables and
 * rounds once to the input dtype.
 *
 * Backward contract (src/kernels/pallas_afa.py:409-522): E = rowsum(g * out) in fp32;
 * per tile s = (q k^T) * scale, r = rsqrt(1+s^2), w = rho(s)^8 masked, w /= d;
 * g_w = g v^T; ds = 8*scale*r*w*(g_w - E) masked; dq += ds k; dk += ds^T q; dv += w^T g,
 * with every matmul operand cast to the input dtype and fp32 accumulation.
 *
 * Accumulation order is fixed and sequential (in d for dot products, in keys for the P V
 * product), so the result is deterministic and independent of the thread count.
 * Build with -ffp-contract=off: every operation rounds separately, like the reference's
 * elementwise JAX ops.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_F64 = 3 };

/* ---------------------------------------------------------------- conversions */
static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16(float f) { /* round to nearest even */
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float f = (float)man * 5.9604644775390625e-08f;
      memcpy(&u, &f, 4);
      u |= sign;
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_f16(float f) { /* round to nearest even, overflow -> inf */
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                     /* below 2^-14: subnormal */
    float af;
    memcpy(&af, &a, 4);
    /* value / 2^-24, rounded to nearest even integer */
    float scaled = af * 16777216.0f;
    float r = nearbyintf(scaled);
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t exp = (a >> 23) - 112u;
  uint32_t man = a & 0x7fffffu;
  uint32_t h = (exp << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static inline float load_in(const void* p, int64_t i, int dt) {
  switch (dt) {
    case DT_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case DT_F16: return f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static inline float round_to(float x, int dt) {
  switch (dt) {
    case DT_BF16: return bf16_to_f32(f32_to_bf16(x));
    case DT_F16: return f16_to_f32(f32_to_f16(x));
    default: return x;
  }
}

static inline void store_out(void* p, int64_t i, float x, int dt) {
  switch (dt) {
    case DT_BF16: ((uint16_t*)p)[i] = f32_to_bf16(x); break;
    case DT_F16: ((uint16_t*)p)[i] = f32_to_f16(x); break;
    default: ((float*)p)[i] = x; break;
  }
}

/* ---------------------------------------------------------------- rho^8 */
/* Two-branch evaluation of src/kernels/pallas_afa.py:39-49 with each op rounded in fp32.
 * rsqrt is taken as the correctly rounded 1/sqrt. */
static inline float rho8_f32(float s) {
  float rad = 1.0f + s * s;
  float r = (float)(1.0 / sqrt((double)rad));
  float rho;
  if (s < 0.0f) {
    float u = s * r;
    rho = r / (1.0f - u);
  } else {
    rho = s + rad * r;
  }
  float k2 = rho * rho;
  float k4 = k2 * k2;
  return k4 * k4;
}

static inline double rho8_f64(double s) {
  double rad = 1.0 + s * s;
  double r = 1.0 / sqrt(rad);
  double rho;
  if (s < 0.0) {
    double u = s * r;
    rho = r / (1.0 - u);
  } else {
    rho = s + rad * r;
  }
  double k2 = rho * rho;
  double k4 = k2 * k2;
  return k4 * k4;
}

/* rsqrt factor used by the backward: r = 1/sqrt(1+s^2). */
static inline float rsq1p_f32(float s) { return (float)(1.0 / sqrt((double)(1.0f + s * s))); }

static int threads_for(int n) {
#ifdef _OPENMP
  return n > 0 ? n : omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

/* ---------------------------------------------------------------- forward (f32/bf16/f16) */
/* Rotated, input-dtype-rounded copy of rows [r0, r0+n) of one (b,h) slice into dst (fp32). */
static void load_rows(float* dst, const void* src, int dt, int64_t base, int64_t r0, int64_t n,
                      int64_t D, const float* rc, const float* rs) {
  for (int64_t r = 0; r < n; ++r) {
    int64_t row = r0 + r;
    for (int64_t d = 0; d < D; ++d) dst[r * D + d] = load_in(src, base + row * D + d, dt);
    if (rc) {
      const float* c = rc + row * (D / 2);
      const float* s = rs + row * (D / 2);
      for (int64_t p = 0; p < D / 2; ++p) {
        float x0 = dst[r * D + 2 * p], x1 = dst[r * D + 2 * p + 1];
        float y0 = c[p] * x0 - s[p] * x1;
        float y1 = s[p] * x0 + c[p] * x1;
        dst[r * D + 2 * p] = round_to(y0, dt);
        dst[r * D + 2 * p + 1] = round_to(y1, dt);
      }
    }
  }
}

int oracle_afa_fwd(int dtype, int64_t B, int64_t H, int64_t L, int64_t D, const void* q,
                   const void* k, const void* v, void* out, void* d_out, const void* rot_c,
                   const void* rot_s, double sink_omega, int causal, int64_t valid_len,
                   int64_t block_q, int64_t block_k, int nthreads) {
  if (B <= 0 || H <= 0 || L <= 0 || D <= 0 || block_q <= 0 || block_k <= 0) return 1;
  if (L % block_q || L % block_k) return 2;
  if (rot_c && (D % 2)) return 3;
  if (valid_len <= 0 || valid_len > L) valid_len = L;
  const int64_t nqb = L / block_q;
  const int64_t nkb = L / block_k;
  if (dtype == DT_F64) {
    const double scale = 1.0 / sqrt((double)D);
    const double* Q = (const double*)q;
    const double* K = (const double*)k;
    const double* V = (const double*)v;
    const double* rc = (const double*)rot_c;
    const double* rs = (const double*)rot_s;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_for(nthreads))
    for (int64_t task = 0; task < B * H * nqb; ++task) {
      const int64_t bh = task / nqb, qb = task % nqb;
      const int64_t base = bh * L * D;
      double* qt = malloc(sizeof(double) * block_q * D);
      double* kt = malloc(sizeof(double) * block_k * D);
      double* o = calloc(block_q * D, sizeof(double));
      double* dsum = calloc(block_q, sizeof(double));
      double* ot = malloc(sizeof(double) * D);
      for (int64_t r = 0; r < block_q; ++r) {
        int64_t row = qb * block_q + r;
        for (int64_t d = 0; d < D; ++d) qt[r * D + d] = Q[base + row * D + d];
        if (rc)
          for (int64_t p = 0; p < D / 2; ++p) {
            double c = rc[row * (D / 2) + p], s = rs[row * (D / 2) + p];
            double x0 = qt[r * D + 2 * p], x1 = qt[r * D + 2 * p + 1];
            qt[r * D + 2 * p] = c * x0 - s * x1;
            qt[r * D + 2 * p + 1] = s * x0 + c * x1;
          }
      }
      for (int64_t kb = 0; kb < nkb; ++kb) {
        if (causal && kb * block_k >= (qb + 1) * block_q) break;
        for (int64_t jj = 0; jj < block_k; ++jj) {
          int64_t col = kb * block_k + jj;
          for (int64_t d = 0; d < D; ++d) kt[jj * D + d] = K[base + col * D + d];
          if (rc)
            for (int64_t p = 0; p < D / 2; ++p) {
              double c = rc[col * (D / 2) + p], s = rs[col * (D / 2) + p];
              double x0 = kt[jj * D + 2 * p], x1 = kt[jj * D + 2 * p + 1];
              kt[jj * D + 2 * p] = c * x0 - s * x1;
              kt[jj * D + 2 * p + 1] = s * x0 + c * x1;
            }
        }
        for (int64_t r = 0; r < block_q; ++r) {
          int64_t row = qb * block_q + r;
          double tsum = 0.0;
          for (int64_t d = 0; d < D; ++d) ot[d] = 0.0;
          for (int64_t jj = 0; jj < block_k; ++jj) {
            int64_t col = kb * block_k + jj;
            if (col >= valid_len || (causal && col > row)) continue;
            double s = 0.0;
            for (int64_t d = 0; d < D; ++d) s += qt[r * D + d] * kt[jj * D + d];
            double p = rho8_f64(s * scale);
            tsum += p;
            for (int64_t d = 0; d < D; ++d) ot[d] += p * V[base + col * D + d];
          }
          for (int64_t d = 0; d < D; ++d) o[r * D + d] += ot[d];
          dsum[r] += tsum;
        }
      }
      for (int64_t r = 0; r < block_q; ++r) {
        int64_t row = qb * block_q + r;
        double tot = dsum[r] + sink_omega;
        for (int64_t d = 0; d < D; ++d) ((double*)out)[base + row * D + d] = o[r * D + d] / tot;
        if (d_out) ((double*)d_out)[bh * L + row] = tot;
      }
      free(qt); free(kt); free(o); free(dsum); free(ot);
    }
    return 0;
  }

  const float scale = (float)(1.0 / sqrt((double)D));
  const float omega = (float)sink_omega;
  const float* rc = (const float*)rot_c;
  const float* rs = (const float*)rot_s;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_for(nthreads))
  for (int64_t task = 0; task < B * H * nqb; ++task) {
    const int64_t bh = task / nqb, qb = task % nqb;
    const int64_t base = bh * L * D;
    float* qt = malloc(sizeof(float) * block_q * D);
    float* kt = malloc(sizeof(float) * block_k * D);   /* K tile, transposed: [d][jj] */
    float* krow = malloc(sizeof(float) * block_k * D); /* K tile rows (rotated) */
    float* vt = malloc(sizeof(float) * block_k * D);
    float* o = calloc(block_q * D, sizeof(float));
    float* dsum = calloc(block_q, sizeof(float));
    float* srow = malloc(sizeof(float) * block_k);
    float* ot = malloc(sizeof(float) * D);
    load_rows(qt, q, dtype, base, qb * block_q, block_q, D, rc, rs);
    for (int64_t kb = 0; kb < nkb; ++kb) {
      if (causal && kb * block_k >= (qb + 1) * block_q) break;
      load_rows(krow, k, dtype, base, kb * block_k, block_k, D, rc, rs);
      for (int64_t jj = 0; jj < block_k; ++jj)
        for (int64_t d = 0; d < D; ++d) kt[d * block_k + jj] = krow[jj * D + d];
      load_rows(vt, v, dtype, base, kb * block_k, block_k, D, NULL, NULL);
      for (int64_t r = 0; r < block_q; ++r) {
        const int64_t row = qb * block_q + r;
        /* scores for the whole key tile, summed sequentially in d for each key */
        for (int64_t jj = 0; jj < block_k; ++jj) srow[jj] = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
          const float qd = qt[r * D + d];
          const float* kd = kt + d * block_k;
          for (int64_t jj = 0; jj < block_k; ++jj) srow[jj] += qd * kd[jj];
        }
        float tsum = 0.0f;
        for (int64_t d = 0; d < D; ++d) ot[d] = 0.0f;
        for (int64_t jj = 0; jj < block_k; ++jj) {
          const int64_t col = kb * block_k + jj;
          if (col >= valid_len || (causal && col > row)) continue;
          const float p = rho8_f32(srow[jj] * scale);
          tsum += p;
          const float pv = round_to(p, dtype);
          const float* vr = vt + jj * D;
          for (int64_t d = 0; d < D; ++d) ot[d] += pv * vr[d];
        }
        for (int64_t d = 0; d < D; ++d) o[r * D + d] += ot[d];
        dsum[r] += tsum;
      }
    }
    for (int64_t r = 0; r < block_q; ++r) {
      const int64_t row = qb * block_q + r;
      const float tot = dsum[r] + omega;
      for (int64_t d = 0; d < D; ++d) store_out(out, base + row * D + d, o[r * D + d] / tot, dtype);
      if (d_out) ((float*)d_out)[bh * L + row] = tot;
    }
    free(qt); free(kt); free(krow); free(vt); free(o); free(dsum); free(srow); free(ot);
  }
  return 0;
}

/* ---------------------------------------------------------------- backward (f32/bf16/f16) */
int oracle_afa_bwd(int dtype, int64_t B, int64_t H, int64_t L, int64_t D, const void* q,
                   const void* k, const void* v, const void* out, const float* d_total,
                   const void* g, void* dq, void* dk, void* dv, int causal, int64_t valid_len,
                   int nthreads) {
  if (dtype == DT_F64 || B <= 0 || H <= 0 || L <= 0 || D <= 0) return 1;
  if (valid_len <= 0 || valid_len > L) valid_len = L;
  const float scale = (float)(1.0 / sqrt((double)D));
  const float c8 = 8.0f * scale;
  const int threads = threads_for(nthreads);
  float* Q = malloc(sizeof(float) * L * D);
  float* K = malloc(sizeof(float) * L * D);
  float* V = malloc(sizeof(float) * L * D);
  float* G = malloc(sizeof(float) * L * D);
  float* E = malloc(sizeof(float) * L);
  float* aq = malloc(sizeof(float) * L * D);
  float* ak = malloc(sizeof(float) * L * D);
  float* av = malloc(sizeof(float) * L * D);
  /* One head at a time; within a head the dq rows and the (dk, dv) rows are shared out over
   * the threads, each pair (i, j) evaluated once per side.  Every output row accumulates its
   * pairs in the same order as a single (i, j) sweep (dq_i over j, dk_j and dv_j over i), so
   * the result does not depend on the thread count. */
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t base = bh * L * D;
    load_rows(Q, q, dtype, base, 0, L, D, NULL, NULL);
    load_rows(K, k, dtype, base, 0, L, D, NULL, NULL);
    load_rows(V, v, dtype, base, 0, L, D, NULL, NULL);
    load_rows(G, g, dtype, base, 0, L, D, NULL, NULL);
    for (int64_t i = 0; i < L; ++i) {
      float e = 0.0f;
      for (int64_t d = 0; d < D; ++d) e += G[i * D + d] * load_in(out, base + i * D + d, dtype);
      E[i] = e;
    }
#pragma omp parallel num_threads(threads)
    {
      /* ds and w of pair (i, j), rounded to the operand dtype */
#define OAFA_PAIR(i, j, dsr, wr)                                                      \
  float sdot = 0.0f, gw = 0.0f;                                                       \
  for (int64_t d = 0; d < D; ++d) sdot += Q[(i) * D + d] * K[(j) * D + d];            \
  for (int64_t d = 0; d < D; ++d) gw += G[(i) * D + d] * V[(j) * D + d];              \
  const float s = sdot * scale;                                                       \
  const float r = rsq1p_f32(s);                                                       \
  const float w = rho8_f32(s) / d_total[bh * L + (i)];                                \
  const float ds = c8 * r * w * (gw - E[(i)]);                                        \
  const float dsr = round_to(ds, dtype), wr = round_to(w, dtype);
#pragma omp for schedule(dynamic, 16)
      for (int64_t i = 0; i < L; ++i) {
        for (int64_t d = 0; d < D; ++d) aq[i * D + d] = 0.0f;
        const int64_t jend = causal ? (i + 1 < valid_len ? i + 1 : valid_len) : valid_len;
        for (int64_t j = 0; j < jend; ++j) {
          OAFA_PAIR(i, j, dsr, wr)
          (void)wr;
          for (int64_t d = 0; d < D; ++d) aq[i * D + d] += dsr * K[j * D + d];
        }
      }
#pragma omp for schedule(dynamic, 16)
      for (int64_t j = 0; j < L; ++j) {
        for (int64_t d = 0; d < D; ++d) ak[j * D + d] = av[j * D + d] = 0.0f;
        if (j >= valid_len) continue;
        for (int64_t i = causal ? j : 0; i < L; ++i) {
          OAFA_PAIR(i, j, dsr, wr)
          for (int64_t d = 0; d < D; ++d) {
            ak[j * D + d] += dsr * Q[i * D + d];
            av[j * D + d] += wr * G[i * D + d];
          }
        }
      }
#undef OAFA_PAIR
    }
    for (int64_t x = 0; x < L * D; ++x) {
      store_out(dq, base + x, aq[x], dtype);
      store_out(dk, base + x, ak[x], dtype);
      store_out(dv, base + x, av[x], dtype);
    }
  }
  free(Q); free(K); free(V); free(G); free(E); free(aq); free(ak); free(av);
  return 0;
}

/* Elementwise helpers exposed for the checker tests. */
/* ---------------------------------------------------------------- exact_afa_reference */
/* The untiled reference of src/kernels/pallas_afa.py:267-327 for bf16 / fp16 inputs, as its JAX
 * program types every value: each jnp op on a bf16 (fp16) array returns bf16 (fp16), so each
 * result below is evaluated in fp32 and rounded to the input dtype:
 *   q_scaled = (q * scale).astype(q.dtype), the Python float scale taking q's dtype (:281-283);
 *   s = q_scaled @ k^T, accumulated in fp32 and rounded                          (:284);
 *   p = _vmu_octic_kernel(s), every elementwise op rounded                     (:32-49, :286);
 *   causal mask; p_v = p.astype(v.dtype) (already v's dtype)                     (:288-292);
 *   o = p_v @ v (fp32 accumulation, rounded); d = sum(p_v) (jnp.sum accumulates bf16 and fp16
 *   in fp32, then rounds)                                                        (:293-294);
 *   d_total = d + Omega; inv = reciprocal(d_total); out = o * inv, each rounded  (:296-297, :320-323).
 * XLA may keep some of these intermediates in fp32 (its excess-precision option) and sums in its
 * own order; neither is fixed by the program, so this restatement fixes them: the dot product
 * of a score is 8 fma chains over features d = sub + 8m (sub = 0..7, m ascending) added as
 * ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)), the products p_v v and the sums over keys run
 * as fma / add chains in key order.  rsqrt is 1 / sqrt, each rounded in fp32 (lax.rsqrt's
 * rounding on XLA-CPU is not fixed either). */
static inline float rho8_step(float s, int dt) {
  const float s_sq = round_to(s * s, dt);
  const float rad = round_to(1.0f + s_sq, dt);
  const float r = round_to(1.0f / sqrtf(rad), dt);
  const float u = round_to(s * r, dt);
  const float rho = s < 0.0f ? round_to(r / round_to(1.0f - u, dt), dt) : round_to(s + round_to(rad * r, dt), dt);
  const float k2 = round_to(rho * rho, dt);
  const float k4 = round_to(k2 * k2, dt);
  return round_to(k4 * k4, dt);
}

int oracle_afa_exact_ref(int dtype, int64_t B, int64_t H, int64_t L, int64_t D, const void* q, const void* k,
                         const void* v, void* out, float* d_out, double sink_omega, int causal, int nthreads) {
  if (dtype != DT_BF16 && dtype != DT_F16) return 4;
  if (B <= 0 || H <= 0 || L <= 0 || D <= 0) return 1;
  const float scale = round_to((float)(1.0 / sqrt((double)D)), dtype);
  const float omega = round_to((float)sink_omega, dtype);
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads_for(nthreads))
  for (int64_t task = 0; task < B * H * L; ++task) {
    const int64_t bh = task / L, row = task % L;
    const int64_t base = bh * L * D;
    float* qs = malloc(sizeof(float) * D);
    float* o = calloc(D, sizeof(float));
    for (int64_t d = 0; d < D; ++d) qs[d] = round_to(load_in(q, base + row * D + d, dtype) * scale, dtype);
    float dsum = 0.0f;
    const int64_t jend = causal ? row + 1 : L;
    for (int64_t j = 0; j < jend; ++j) {
      float c[8];
      for (int sub = 0; sub < 8; ++sub) {
        c[sub] = 0.0f;
        for (int64_t d = sub; d < D; d += 8) c[sub] = fmaf(qs[d], load_in(k, base + j * D + d, dtype), c[sub]);
      }
      const float sdot = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
      const float p = rho8_step(round_to(sdot, dtype), dtype);
      for (int64_t d = 0; d < D; ++d) o[d] = fmaf(p, load_in(v, base + j * D + d, dtype), o[d]);
      dsum += p;
    }
    const float tot = round_to(round_to(dsum, dtype) + omega, dtype);
    const float inv = round_to(1.0f / tot, dtype);
    for (int64_t d = 0; d < D; ++d) store_out(out, base + row * D + d, round_to(o[d], dtype) * inv, dtype);
    if (d_out) d_out[bh * L + row] = tot;
    free(qs);
    free(o);
  }
  return 0;
}

void oracle_rho8_step(const float* x, float* y, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) y[i] = rho8_step(x[i], dtype);
}

void oracle_rho8_f32(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = rho8_f32(x[i]);
}
void oracle_bf16_round(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}
void oracle_f16_round(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f32_to_f16(x[i]);
}
int oracle_max_threads(void) { return threads_for(0); }

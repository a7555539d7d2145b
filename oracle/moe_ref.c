/*
 * moe_ref.c — C restatement of nano-vllm-metal's MoE path on the CPU.
 *
 * TEST INFRASTRUCTURE ONLY: the CPU baseline timed by bench.py and a second,
 * independent oracle checked against oracle/moe_oracle.py by the CPU tests.
 * The product (libnvm_moe.so) never links or calls it.
 *
 * It follows the reference algorithm (paths relative to the reference's
 * src/nano_vllm_metal):
 *   1. router logits: x . dequant(Wr)^T (layers/moe.py:43 -> layers/linear.py:92-126),
 *      accumulated in double and rounded once to the activation dtype;
 *   2. softmax in double, rounded to act (layers/moe.py:44);
 *   3. top-k by (prob desc, index asc) and optional renormalisation
 *      rnd(s / rnd(sum s)) (layers/moe.py:45-48);
 *   4. a stable counting sort of the (token, slot) pairs by expert
 *      (layers/moe.py:16-17);
 *   5. per routed pair, the scalar dequant-dot loop of
 *      metal/src/quantized_matmul.cpp:117-145 (float accumulation,
 *      w = float(q)*float(scale) + float(bias)) for gate and up, rounded to
 *      act; h = rnd(silu(gate) * up) with silu's ops each rounded to act
 *      (layers/activation.py:21-24); the same loop for down, rounded to act
 *      (layers/moe.py:81-85, layers/activation.py:21-24);
 *   6. y = rnd(sum_j rnd(down_j * score_j)) in float (layers/moe.py:86).
 * Step 5 is parallelised over routed pairs with OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F16 = 0, DT_BF16 = 1 };

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  int exp = (h >> 10) & 0x1F;
  uint32_t man = h & 0x3FF;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: normalise */
      exp = 1;
      while (!(man & 0x400)) {
        man <<= 1;
        --exp;
      }
      man &= 0x3FF;
      u = sign | ((uint32_t)(exp + 112) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7F800000u | (man << 13);
  } else {
    u = sign | ((uint32_t)(exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float act_to_f32(uint16_t h, int dt) { return dt == DT_BF16 ? bf16_to_f32(h) : f16_to_f32(h); }

/* Round a double to `prec` significant bits with smallest normal exponent
 * `emin`, ties to even; exact scaling by powers of two, then rint(). */
static double round_to(double v, int prec, int emin) {
  if (v == 0.0) return v;
  int e = ilogb(v);
  if (e < emin) e = emin;
  const int sh = (prec - 1) - e;
  return ldexp(rint(ldexp(v, sh)), -sh);
}

static double round_act(double v, int dt) {
  return dt == DT_BF16 ? round_to(v, 8, -126) : round_to(v, 11, -14);
}

/* silu of layers/activation.py:21-24 on an act value g, each of its ops
 * (exp(-|g|), 1 + e, 1 / d, where(g < 0, 1 - s, s), g * sg) rounded to act. */
static double silu_act(double g, int dt) {
  const double e = round_act(exp(-fabs(g)), dt);
  const double d = round_act(1.0 + e, dt);
  const double s = round_act(1.0 / d, dt);
  const double sg = g < 0.0 ? round_act(1.0 - s, dt) : s;
  return round_act(g * sg, dt);
}

/* bit pattern of an act-representable value */
static uint16_t act_bits(double v, int dt) {
  float f = (float)v;
  uint32_t u;
  memcpy(&u, &f, 4);
  if (dt == DT_BF16) return (uint16_t)(u >> 16);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int exp = (int)((u >> 23) & 0xFF) - 127;
  const uint32_t man = u & 0x7FFFFF;
  if (f == 0.0f) return (uint16_t)sign;
  if (exp > 15) return (uint16_t)(sign | 0x7C00u);
  if (exp >= -14) return (uint16_t)(sign | ((uint32_t)(exp + 15) << 10) | (man >> 13));
  /* subnormal: value = m * 2^-24 with m integer (exact by construction) */
  return (uint16_t)(sign | (uint32_t)ldexp(fabs((double)f), 24));
}

/* One row of the reference's CPU loop (quantized_matmul.cpp:117-145):
 * sum over groups and packed words of float(q)*scale + bias times a. */
static float qdot_row(const uint16_t *a, const uint32_t *b_row, const uint16_t *s_row,
                      const uint16_t *bias_row, int64_t n, int gs, int dt) {
  float sum = 0.0f;
  const int64_t groups = n / gs;
  int64_t a_loc = 0, b_loc = 0;
  for (int64_t g = 0; g < groups; ++g) {
    const float scale = act_to_f32(s_row[g], dt);
    const float bias = act_to_f32(bias_row[g], dt);
    for (int item = 0; item < gs; item += 8) {
      const uint32_t word = b_row[b_loc++];
      for (int j = 0; j < 8; ++j) {
        const float w = (float)((word >> (4 * j)) & 0xFu) * scale + bias;
        sum += act_to_f32(a[a_loc++], dt) * w;
      }
    }
  }
  return sum;
}

static double qdot_row_f64(const uint16_t *a, const uint32_t *b_row, const uint16_t *s_row,
                           const uint16_t *bias_row, int64_t n, int gs, int dt) {
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t q = (b_row[i / 8] >> (4 * (i % 8))) & 0xFu;
    const double w = (double)q * act_to_f32(s_row[i / gs], dt) + act_to_f32(bias_row[i / gs], dt);
    sum += (double)act_to_f32(a[i], dt) * w;
  }
  return sum;
}

int moe_ref_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
  return omp_get_max_threads();
#else
  (void)nthreads;
  return 1;
#endif
}

/* Router + top-k: ids [T*k], scores [T*k] (act bits), probs [T*E] (act bits, may be NULL). */
int moe_ref_route(const uint16_t *x, int64_t T, int64_t H, const uint32_t *wr, const uint16_t *sr,
                  const uint16_t *br, int64_t E, int gs, int k, int norm, int dt, uint16_t *probs,
                  int32_t *ids, uint16_t *scores) {
  if (k < 1 || k > E || H % gs || H % 8) return -1;
  int rc = 0;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    double *lg = (double *)malloc(sizeof(double) * (size_t)E);
    double *p = (double *)malloc(sizeof(double) * (size_t)E);
    unsigned char *taken = (unsigned char *)calloc((size_t)E, 1);
    if (!lg || !p || !taken) {
      rc = -2;
    } else {
      double m = -INFINITY;
      for (int64_t e = 0; e < E; ++e) {
        lg[e] = round_act(qdot_row_f64(x + t * H, wr + e * (H / 8), sr + e * (H / gs),
                                       br + e * (H / gs), H, gs, dt), dt);
        if (lg[e] > m) m = lg[e];
      }
      double sum = 0.0;
      for (int64_t e = 0; e < E; ++e) {
        p[e] = exp(lg[e] - m);
        sum += p[e];
      }
      for (int64_t e = 0; e < E; ++e) {
        p[e] = round_act(p[e] / sum, dt);
        if (probs) probs[t * E + e] = act_bits(p[e], dt);
      }
      double psum = 0.0;
      for (int i = 0; i < k; ++i) {
        int64_t best = -1;
        for (int64_t e = 0; e < E; ++e)
          if (!taken[e] && (best < 0 || p[e] > p[best])) best = e; /* strict: lower index wins ties */
        taken[best] = 1;
        ids[t * k + i] = (int32_t)best;
        psum += p[best];
      }
      const double denom = round_act(psum, dt);
      for (int i = 0; i < k; ++i) {
        const double s = p[ids[t * k + i]];
        scores[t * k + i] = act_bits(norm ? round_act(s / denom, dt) : s, dt);
      }
    }
    free(lg);
    free(p);
    free(taken);
  }
  return rc;
}

/* Stable counting sort of n pair ids by expert: offsets [E+1], sorted [n]. */
int moe_ref_dispatch(const int32_t *ids, int64_t n, int64_t E, int32_t *offsets, int32_t *sorted) {
  memset(offsets, 0, sizeof(int32_t) * (size_t)(E + 1));
  for (int64_t p = 0; p < n; ++p) {
    if (ids[p] < 0 || ids[p] >= E) return -1;
    offsets[ids[p] + 1]++;
  }
  for (int64_t e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
  int32_t *fill = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
  if (!fill) return -2;
  memcpy(fill, offsets, sizeof(int32_t) * (size_t)E);
  for (int64_t p = 0; p < n; ++p) sorted[fill[ids[p]]++] = (int32_t)p;
  free(fill);
  return 0;
}

/* The whole block.  Weight layouts as in include/nvm_moe.h. */
int moe_ref_forward(const uint16_t *x, int64_t T, int64_t H, int64_t I, int64_t E, int k,
                    int norm, int gs, int dt, const uint32_t *wr, const uint16_t *sr,
                    const uint16_t *br, const uint32_t *wg, const uint16_t *sg,
                    const uint16_t *bg, const uint32_t *wu, const uint16_t *su,
                    const uint16_t *bu, const uint32_t *wd, const uint16_t *sd,
                    const uint16_t *bd, uint16_t *y, int32_t *ids_out, uint16_t *scores_out) {
  if (H % gs || I % gs || H % 8 || I % 8) return -1;
  const int64_t N = T * k;
  int32_t *ids = ids_out ? ids_out : (int32_t *)malloc(sizeof(int32_t) * (size_t)N);
  uint16_t *scores = scores_out ? scores_out : (uint16_t *)malloc(sizeof(uint16_t) * (size_t)N);
  int32_t *offsets = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
  int32_t *sorted = (int32_t *)malloc(sizeof(int32_t) * (size_t)N);
  uint16_t *down = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(N * H));
  int rc = (!ids || !scores || !offsets || !sorted || !down) ? -2 : 0;
  if (!rc) rc = moe_ref_route(x, T, H, wr, sr, br, E, gs, k, norm, dt, NULL, ids, scores);
  if (!rc) rc = moe_ref_dispatch(ids, N, E, offsets, sorted);
  if (!rc) {
    const int64_t hw = H / 8, hg = H / gs, iw = I / 8, ig = I / gs;
#pragma omp parallel
    {
      uint16_t *h = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)I);
#pragma omp for schedule(dynamic, 1)
      for (int64_t n = 0; n < N; ++n) {
        const int32_t p = sorted[n];
        const int64_t t = p / k;
        const int32_t e = ids[p];
        const uint16_t *xr = x + t * H;
        for (int64_t r = 0; r < I; ++r) {
          const int64_t row = (int64_t)e * I + r;
          const double g = round_act(qdot_row(xr, wg + row * hw, sg + row * hg, bg + row * hg, H, gs, dt), dt);
          const double u = round_act(qdot_row(xr, wu + row * hw, su + row * hg, bu + row * hg, H, gs, dt), dt);
          h[r] = act_bits(round_act(silu_act(g, dt) * u, dt), dt);
        }
        for (int64_t c = 0; c < H; ++c) {
          const int64_t row = (int64_t)e * H + c;
          down[(int64_t)p * H + c] =
              act_bits(round_act(qdot_row(h, wd + row * iw, sd + row * ig, bd + row * ig, I, gs, dt), dt), dt);
        }
      }
      free(h);
    }
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      for (int64_t c = 0; c < H; ++c) {
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) {
          const float d = act_to_f32(down[(t * k + j) * H + c], dt);
          const float s = act_to_f32(scores[t * k + j], dt);
          acc += (float)round_act((double)(d * s), dt);
        }
        y[t * H + c] = act_bits(round_act(acc, dt), dt);
      }
    }
  }
  if (!ids_out) free(ids);
  if (!scores_out) free(scores);
  free(offsets);
  free(sorted);
  free(down);
  return rc;
}

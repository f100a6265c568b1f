/*
 * CPU restatement of the Flash-Next Q4/g32 MoE decode layer (test
 * infrastructure: the timed CPU baseline and a cross-check of the numpy
 * oracle; never linked into the product library).
 *
 * Semantics restated from the reference:
 *   unpack q = (w[k>>3] >> 4(k&7)) & 15            models/flashnext/metal_runtime.py:980
 *   QMV  sum_g s*sum(x q) + b*sum(x), float accumulate, T-rounded output
 *                                                    models/flashnext/metal_runtime.py:955-987
 *   router softmax -> top-k (score desc, index asc) -> bf16 renorm
 *                                                    models/flashnext/compiled.py:61-71
 *   SwiGLU bf16 sequence                            models/flashnext/metal_runtime.py:278-284
 *   combine acc += float(T(d)) * score, then T(acc) + shared_y
 *                                                    models/flashnext/metal_runtime.py:299-333
 * Row loops are parallelised with OpenMP.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float rbf(float f) { return bf2f(f2bf(f)); }

/* float64 -> bf16, single rounding (round-to-odd to float32, then RNE). */
static uint16_t d2bf(double d) {
  float t = (float)d;
  uint32_t bits;
  memcpy(&bits, &t, 4);
  if (isfinite(d)) {
    if (fabs((double)t) > fabs(d)) bits -= 1u;
    float tt;
    memcpy(&tt, &bits, 4);
    if ((double)tt != d) bits |= 1u;
  }
  float r;
  memcpy(&r, &bits, 4);
  return f2bf(r);
}

/* y[o] = sum_g s*sum(x q) + b*sum(x) for one row, float accumulation. */
static float qmv_row(const float *x, const uint32_t *w, const uint16_t *s, const uint16_t *b,
                     uint32_t in_w, uint32_t group) {
  float acc = 0.0f;
  const uint32_t groups = in_w / group;
  for (uint32_t g = 0; g < groups; ++g) {
    float qs = 0.0f, xs = 0.0f;
    const uint32_t *wg = w + g * group / 8;
    const float *xg = x + g * group;
    for (uint32_t i = 0; i < group; ++i) {
      const float q = (float)((wg[i >> 3] >> (4 * (i & 7))) & 15u);
      qs += xg[i] * q;
      xs += xg[i];
    }
    acc += bf2f(s[g]) * qs + bf2f(b[g]) * xs;
  }
  return acc;
}

static float sigmoid_bf(float g) {
  const float m = fabsf(g);
  const float e = rbf((float)exp((double)m));
  const float d = rbf(1.0f + e);
  const float s = rbf(1.0f / d);
  const float om = rbf(1.0f - s);
  return g < 0.0f ? s : om;
}

static float swiglu_bf(float g, float u) {
  const float silu = rbf(g * sigmoid_bf(g));
  return rbf(silu * u);
}

typedef struct {
  const uint32_t *w;
  const uint16_t *s;
  const uint16_t *b;
} Bank;

/* One expert MLP on a bf16-valued input row -> bf16 down output [hidden]. */
static void expert_mlp(const float *x, Bank gate, Bank up, Bank down, uint32_t e, uint32_t hidden,
                       uint32_t inter, uint32_t group, float *act_scratch, float *down_out) {
  const uint64_t gw = (uint64_t)inter * (hidden / 8), gm = (uint64_t)inter * (hidden / group);
  const uint64_t dw = (uint64_t)hidden * (inter / 8), dm = (uint64_t)hidden * (inter / group);
#pragma omp parallel for schedule(static)
  for (uint32_t r = 0; r < inter; ++r) {
    const float g = rbf(qmv_row(x, gate.w + e * gw + (uint64_t)r * (hidden / 8),
                                gate.s + e * gm + (uint64_t)r * (hidden / group),
                                gate.b + e * gm + (uint64_t)r * (hidden / group), hidden, group));
    const float u = rbf(qmv_row(x, up.w + e * gw + (uint64_t)r * (hidden / 8),
                                up.s + e * gm + (uint64_t)r * (hidden / group),
                                up.b + e * gm + (uint64_t)r * (hidden / group), hidden, group));
    act_scratch[r] = swiglu_bf(g, u);
  }
#pragma omp parallel for schedule(static)
  for (uint32_t o = 0; o < hidden; ++o) {
    down_out[o] = rbf(qmv_row(act_scratch, down.w + e * dw + (uint64_t)o * (inter / 8),
                              down.s + e * dm + (uint64_t)o * (inter / group),
                              down.b + e * dm + (uint64_t)o * (inter / group), inter, group));
  }
}

/* Router for one token: bf16 logits (float64 dot), softmax (float64), top-k,
 * bf16 renorm.  inds/scores_bits are [k]; returns the shared gate bf16 bits
 * when shared_gate_w is given, else 0. */
static uint16_t route_token(const uint16_t *x, const uint16_t *wg, const uint16_t *shared_gate_w,
                            uint32_t hidden, uint32_t experts, uint32_t k, uint32_t *inds,
                            uint16_t *scores_bits, double *scratch) {
#pragma omp parallel for schedule(static)
  for (uint32_t e = 0; e < experts; ++e) {
    double acc = 0.0;
    const uint16_t *w = wg + (uint64_t)e * hidden;
    for (uint32_t i = 0; i < hidden; ++i) acc += (double)(bf2f(x[i]) * bf2f(w[i]));
    scratch[e] = (double)bf2f(d2bf(acc));
  }
  double m = -INFINITY, sum = 0.0;
  for (uint32_t e = 0; e < experts; ++e) m = scratch[e] > m ? scratch[e] : m;
  for (uint32_t e = 0; e < experts; ++e) {
    scratch[e] = exp(scratch[e] - m);
    sum += scratch[e];
  }
  uint16_t gates[512];
  for (uint32_t e = 0; e < experts; ++e) gates[e] = d2bf(scratch[e] / sum);
  uint8_t used[512] = {0};
  float mass = 0.0f;
  float raw[16];
  for (uint32_t j = 0; j < k; ++j) {
    int best = -1;
    for (uint32_t e = 0; e < experts; ++e)
      if (!used[e] && (best < 0 || gates[e] > gates[best])) best = (int)e;
    used[best] = 1;
    inds[j] = (uint32_t)best;
    raw[j] = bf2f(gates[best]);
    mass += raw[j];
  }
  const float mass_b = rbf(mass);
  /* selected == topk mass at threshold 1: normalizer = mass + 1*(sel - mass) */
  const float norm = rbf(mass_b + rbf(1.0f * rbf(mass_b - mass_b)));
  for (uint32_t j = 0; j < k; ++j) scores_bits[j] = f2bf(raw[j] / norm);
  if (!shared_gate_w) return 0;
  double acc = 0.0;
  for (uint32_t i = 0; i < hidden; ++i) acc += (double)(bf2f(x[i]) * bf2f(shared_gate_w[i]));
  return f2bf(sigmoid_bf(bf2f(d2bf(acc))));
}

/*
 * Full decode layer for `tokens` rows: router, routed experts, shared
 * expert (optional) and the fused combine.  Banks are dense
 * [experts, out, in/8] / [experts, out, in/group].  Shared banks are single
 * experts.  Writes bf16 out [tokens, hidden] and inds [tokens, k].
 */
int mqo_decode_layer(const uint16_t *x, uint32_t tokens, uint32_t hidden, uint32_t inter,
                     uint32_t experts, uint32_t k, uint32_t group, const uint16_t *router_w,
                     const uint16_t *shared_gate_w, const uint32_t *gw, const uint16_t *gs,
                     const uint16_t *gb, const uint32_t *uw, const uint16_t *us, const uint16_t *ub,
                     const uint32_t *dw, const uint16_t *ds, const uint16_t *db, const uint32_t *sgw,
                     const uint16_t *sgs, const uint16_t *sgb, const uint32_t *suw, const uint16_t *sus,
                     const uint16_t *sub, const uint32_t *sdw, const uint16_t *sds, const uint16_t *sdb,
                     uint16_t *out, uint32_t *inds_out, int threads) {
  if (k == 0 || k > 16 || experts > 512 || hidden % group || inter % group) return -1;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
  float *xf = (float *)malloc(sizeof(float) * hidden);
  float *act = (float *)malloc(sizeof(float) * inter);
  float *down = (float *)malloc(sizeof(float) * hidden);
  float *acc = (float *)malloc(sizeof(float) * hidden);
  double *scratch = (double *)malloc(sizeof(double) * 512);
  if (!xf || !act || !down || !acc || !scratch) return -2;
  Bank G = {gw, gs, gb}, U = {uw, us, ub}, D = {dw, ds, db};
  Bank SG = {sgw, sgs, sgb}, SU = {suw, sus, sub}, SD = {sdw, sds, sdb};
  for (uint32_t t = 0; t < tokens; ++t) {
    const uint16_t *xt = x + (uint64_t)t * hidden;
    for (uint32_t i = 0; i < hidden; ++i) xf[i] = bf2f(xt[i]);
    uint32_t inds[16];
    uint16_t sc[16];
    const uint16_t sgate = route_token(xt, router_w, sgw ? shared_gate_w : NULL, hidden, experts, k, inds, sc, scratch);
    for (uint32_t o = 0; o < hidden; ++o) acc[o] = 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
      expert_mlp(xf, G, U, D, inds[j], hidden, inter, group, act, down);
      const float s = bf2f(sc[j]);
      for (uint32_t o = 0; o < hidden; ++o) {
        const volatile float prod = down[o] * s; /* no contraction */
        acc[o] = acc[o] + prod;
      }
      if (inds_out) inds_out[(uint64_t)t * k + j] = inds[j];
    }
    if (sgw) {
      expert_mlp(xf, SG, SU, SD, 0, hidden, inter, group, act, down);
      const float gate = bf2f(sgate);
      for (uint32_t o = 0; o < hidden; ++o) {
        const float comp = rbf(down[o] * gate);
        out[(uint64_t)t * hidden + o] = f2bf(rbf(acc[o]) + comp);
      }
    } else {
      for (uint32_t o = 0; o < hidden; ++o) out[(uint64_t)t * hidden + o] = f2bf(acc[o]);
    }
  }
  free(xf);
  free(act);
  free(down);
  free(acc);
  free(scratch);
  return 0;
}

/* Dense quantized matvec y[r, n] = T(sum_k x[r,k] W[n,k]) for bf16 x (f32 out). */
int mqo_qmv(const uint16_t *x, const uint32_t *w, const uint16_t *s, const uint16_t *b, float *y,
            uint32_t rows, uint32_t n, uint32_t k, uint32_t group, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
  float *xf = (float *)malloc(sizeof(float) * k);
  if (!xf) return -2;
  for (uint32_t r = 0; r < rows; ++r) {
    for (uint32_t i = 0; i < k; ++i) xf[i] = bf2f(x[(uint64_t)r * k + i]);
#pragma omp parallel for schedule(static)
    for (uint32_t o = 0; o < n; ++o)
      y[(uint64_t)r * n + o] = qmv_row(xf, w + (uint64_t)o * (k / 8), s + (uint64_t)o * (k / group),
                                       b + (uint64_t)o * (k / group), k, group);
  }
  free(xf);
  return 0;
}

int mqo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

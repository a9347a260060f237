/*
 * CPU restatement of the batched sampler (TEST INFRASTRUCTURE ONLY).
 *
 * Follows xixi-vllm src/compute/sampler.py:27-119 (Sampler.forward,
 * _sample_ordered) and src/compute/layers/vocab_parallel.py:180-216 (greedy
 * argmax), with the draw made explicit: one uniform u per row, inverse CDF
 * over the kept candidates in ascending id order, masses in 2^-40 fixed point.
 * The logits are scaled by 1/T (one fp32 reciprocal per row), not divided.
 *
 * Written as the direct, sort-based formulation (the reference sorts the
 * scaled logits and takes a cumulative sum); the GPU kernel reaches the same
 * kept set through radix selection, so agreement checks one against the other.
 * Compile with -ffp-contract=off: every fused multiply-add is explicit.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define FLAG_ALL_GREEDY 1
#define FLAG_TOP_K 2
#define FLAG_TOP_P 4
#define FLAG_MIN_P 8

/* 2^x for x <= 0: x = n + f, f in [-1/2, 1/2]; 2^f by the degree-7 Taylor
 * polynomial of exp(f ln 2) in Horner form with fused multiply-adds;
 * 2^n applied exactly.  Results below 2^-125 flush to 0. */
float oracle_exp2(float x) {
  if (!(x > -125.0f)) return 0.0f;
  float n = rintf(x);
  float f = x - n;
  float p = 1.5252733646775596e-05f;
  p = fmaf(p, f, 1.5403529687318951e-04f);
  p = fmaf(p, f, 1.3333557872101665e-03f);
  p = fmaf(p, f, 9.6181286498904228e-03f);
  p = fmaf(p, f, 5.5504109710454941e-02f);
  p = fmaf(p, f, 2.4022650718688965e-01f);
  p = fmaf(p, f, 6.9314718246459961e-01f);
  p = fmaf(p, f, 1.0f);
  return ldexpf(p, (int)n);
}

static inline float bf16f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t order_key(uint16_t b) { return (b & 0x8000u) ? (uint16_t)~b : (uint16_t)(b | 0x8000u); }
static inline int is_nan16(uint16_t b) { return (b & 0x7fffu) > 0x7f80u; }

static const uint32_t *g_key;
static int cmp_rank(const void *pa, const void *pb) {
  int a = *(const int *)pa, b = *(const int *)pb;
  if (g_key[a] != g_key[b]) return g_key[a] > g_key[b] ? -1 : 1;
  return a < b ? -1 : 1;
}

int64_t oracle_sample_row(const uint16_t *logits, int V, float temperature, float top_p, int top_k, float min_p,
                          float u, int flags) {
  if ((flags & FLAG_ALL_GREEDY) || temperature <= 1e-5f) {
    /* torch.argmax (the reference's greedy, sampler.py:48,61,91 and
     * vocab_parallel.py:180-216): a NaN is the maximum, so the lowest NaN
     * index wins if there is one; otherwise the largest value, lowest index
     * on ties (-0 equals +0). */
    int best = -1;
    float bv = 0.f;
    for (int i = 0; i < V; ++i) {
      if (is_nan16(logits[i])) return i;
      float v = bf16f(logits[i]);
      if (best < 0 || v > bv) { best = i; bv = v; }
    }
    return best < 0 ? 0 : best;
  }
  uint32_t *key = malloc(sizeof(uint32_t) * V);
  int64_t *q = malloc(sizeof(int64_t) * V);
  int *order = malloc(sizeof(int) * V);
  int *rank = malloc(sizeof(int) * V);
  uint32_t kmax = 0;
  int n = 0;
  for (int i = 0; i < V; ++i) {
    key[i] = is_nan16(logits[i]) ? 0u : order_key(logits[i]);
    if (key[i] > kmax) kmax = key[i];
  }
  /* the max logit: inverse of order_key */
  uint16_t maxbits = (kmax & 0x8000u) ? (uint16_t)(kmax & 0x7fffu) : (uint16_t)~kmax;
  const float inv_t = 1.0f / temperature;
  const float zmax = bf16f(maxbits) * inv_t;
  float *e = malloc(sizeof(float) * V);
  for (int i = 0; i < V; ++i) {
    if (key[i] == 0u) { e[i] = 0.f; q[i] = 0; continue; }
    float z = bf16f(logits[i]) * inv_t;
    float d = z - zmax;
    d = d * 1.44269502162933349609375f; /* log2(e) in fp32 */
    e[i] = oracle_exp2(d);
    q[i] = (int64_t)(e[i] * 1099511627776.0f); /* 2^40 */
  }
  for (int i = 0; i < V; ++i) order[n++] = i;
  g_key = key;
  qsort(order, V, sizeof(int), cmp_rank);
  for (int r = 0; r < V; ++r) rank[order[r]] = r;

  int kk = V, kp = V, km = V;
  if ((flags & FLAG_TOP_K) && top_k > 0 && top_k < V) kk = top_k;
  int64_t total_k = 0;
  for (int r = 0; r < kk; ++r) total_k += q[order[r]];
  if ((flags & FLAG_TOP_P) && top_p < 1.0f) {
    int64_t thr = (int64_t)floor((double)top_p * (double)total_k);
    int64_t before = 0;
    kp = 0;
    for (int r = 0; r < kk; ++r) {
      if (before > thr) break;
      kp++;
      before += q[order[r]];
    }
  }
  if ((flags & FLAG_MIN_P) && min_p > 0.0f) {
    /* kept: every key >= the smallest key whose probability reaches min_p
       times the largest (e_max = 1) */
    uint32_t km_key = 0xffffffffu;
    for (int i = 0; i < V; ++i)
      if (key[i] != 0u && e[i] >= min_p && key[i] < km_key) km_key = key[i];
    km = 0;
    for (int i = 0; i < V; ++i) km += key[i] >= km_key;
  }
  int kstar = kk < kp ? kk : kp;
  if (km < kstar) kstar = km;
  if (kstar < 1) kstar = 1;
  int64_t M = 0;
  for (int r = 0; r < kstar; ++r) M += q[order[r]];
  int64_t rdraw = (int64_t)((double)u * (double)M);
  if (rdraw >= M) rdraw = M - 1;
  if (rdraw < 0) rdraw = 0;
  int64_t cum = 0, out = order[0];
  for (int i = 0; i < V; ++i) {
    if (rank[i] >= kstar) continue;
    cum += q[i];
    if (cum > rdraw) { out = i; break; }
  }
  free(key); free(q); free(order); free(rank); free(e);
  return out;
}

void oracle_sample(const uint16_t *logits, int64_t stride, int B, int V, const float *temps, const float *top_ps,
                   const int32_t *top_ks, const float *min_ps, const float *uniforms, int flags, int64_t *out) {
  for (int b = 0; b < B; ++b)
    out[b] = oracle_sample_row(logits + b * stride, V, temps ? temps[b] : 1.0f, top_ps ? top_ps[b] : 1.0f,
                               top_ks ? top_ks[b] : V, min_ps ? min_ps[b] : 0.0f, uniforms ? uniforms[b] : 0.5f,
                               flags);
}

/* Probability the explicit-draw sampler assigns to every id of one row
 * (mass / kept mass, 0 outside the kept set); for checks against the
 * reference's renormalised distributions. */
void oracle_probs_row(const uint16_t *logits, int V, float temperature, float top_p, int top_k, float min_p,
                      int flags, double *probs) {
  /* the kept set and masses are those of oracle_sample_row; recover them by
     drawing at every cut point would be quadratic, so recompute directly */
  uint32_t *key = malloc(sizeof(uint32_t) * V);
  int64_t *q = malloc(sizeof(int64_t) * V);
  float *e = malloc(sizeof(float) * V);
  int *order = malloc(sizeof(int) * V);
  int *rank = malloc(sizeof(int) * V);
  uint32_t kmax = 0;
  for (int i = 0; i < V; ++i) {
    key[i] = is_nan16(logits[i]) ? 0u : order_key(logits[i]);
    if (key[i] > kmax) kmax = key[i];
  }
  uint16_t maxbits = (kmax & 0x8000u) ? (uint16_t)(kmax & 0x7fffu) : (uint16_t)~kmax;
  const float inv_t = 1.0f / temperature;
  const float zmax = bf16f(maxbits) * inv_t;
  for (int i = 0; i < V; ++i) {
    if (key[i] == 0u) { e[i] = 0.f; q[i] = 0; continue; }
    float d = bf16f(logits[i]) * inv_t - zmax;
    d = d * 1.44269502162933349609375f;
    e[i] = oracle_exp2(d);
    q[i] = (int64_t)(e[i] * 1099511627776.0f);
  }
  for (int i = 0; i < V; ++i) order[i] = i;
  g_key = key;
  qsort(order, V, sizeof(int), cmp_rank);
  for (int r = 0; r < V; ++r) rank[order[r]] = r;
  int kk = V, kp = V, km = V;
  if ((flags & FLAG_TOP_K) && top_k > 0 && top_k < V) kk = top_k;
  int64_t total_k = 0;
  for (int r = 0; r < kk; ++r) total_k += q[order[r]];
  if ((flags & FLAG_TOP_P) && top_p < 1.0f) {
    int64_t thr = (int64_t)floor((double)top_p * (double)total_k);
    int64_t before = 0;
    kp = 0;
    for (int r = 0; r < kk; ++r) {
      if (before > thr) break;
      kp++;
      before += q[order[r]];
    }
  }
  if ((flags & FLAG_MIN_P) && min_p > 0.0f) {
    uint32_t km_key = 0xffffffffu;
    for (int i = 0; i < V; ++i)
      if (key[i] != 0u && e[i] >= min_p && key[i] < km_key) km_key = key[i];
    km = 0;
    for (int i = 0; i < V; ++i) km += key[i] >= km_key;
  }
  int kstar = kk < kp ? kk : kp;
  if (km < kstar) kstar = km;
  if (kstar < 1) kstar = 1;
  int64_t M = 0;
  for (int r = 0; r < kstar; ++r) M += q[order[r]];
  for (int i = 0; i < V; ++i) probs[i] = rank[i] < kstar ? (double)q[i] / (double)M : 0.0;
  free(key); free(q); free(e); free(order); free(rank);
}

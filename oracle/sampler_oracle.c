/*
 * sampler_oracle.c - CPU restatement of the reference sampling path.
 *
 * TEST INFRASTRUCTURE ONLY (see sampler_oracle.h).  Compiled with
 * -ffp-contract=off so every double operation rounds exactly as a JS
 * engine's does.
 *
 * Function -> reference it follows -> how it is pinned:
 *   orc_exp            V8 Math.exp, used by sample() (tokenizer.js:165); the
 *                      algorithm is fdlibm e_exp.c (Sun Microsystems 1993),
 *                      which V8's base::ieee754::exp implements.  Pinned by
 *                      tests/golden/v8_math_exp.json (outputs of Node's own
 *                      Math.exp) and closed forms (exp(0)=1, exp(-inf)=0).
 *   orc_sample_row     tokenizer.js:151-178 (penalty, stable sort, greedy,
 *                      softmax over top-k, top-p cut, draw), with the
 *                      per-element mask test of kernels.js:1422-1426 and the
 *                      tie order of kernels.js:1433,1439 (lowest id first).
 *                      Pinned by hand-derived known answers, brute-force
 *                      ordering (select_mode 1), exact-distribution tests and
 *                      bit-equality with the Node restatement sample_js.js
 *                      run on V8.
 *   orc_penalize       presence: tokenizer.js:157.  Repetition / frequency do
 *                      not exist in the reference ("parity unpinned" against
 *                      it); they follow the CTRL / OpenAI definitions and are
 *                      pinned by invariants (identity at r=1,f=0,p=0; ids
 *                      outside the history untouched; sign rule; monotone).
 *   orc_softcap        kernels.js:1393-1395 (cap*tanh(x/cap) in fp32), with
 *                      tanh defined by orc_tanhf so host and GPU agree bit for
 *                      bit.  Pinned against the correctly rounded tanh (from
 *                      double) and cap*tanh's closed form.  Against the
 *                      reference's WGSL tanh on Dawn the last ulp is parity
 *                      unpinned (no reference vectors exist).
 *   orc_pcg            kernels.js:91-95, uniform kernels.js:181, 320.
 *                      Pinned by a closed-form recomputation of the hash.
 *   orc_mask_from_ids  TokenMask (tool-constraint.ts:39-42) + isListed
 *                      (kernels.js:1401-1412); pinned by the reference test
 *                      tests/token-mask-state.test.ts:49-55 semantics and
 *                      brute force.
 *   orc_verify         no reference (acceptSpec is an exact-match cascade,
 *                      kernels.js:328-339): textbook rejection sampling;
 *                      pinned by distribution tests (empirical marginal = p,
 *                      q = p accepts always, one-hot q accepts w.p. p(d)).
 *   orc_spec_exact     acceptSpec kernels.js:211-369 on A.2 semantics: each
 *                      verify row sampled on its own with the uniform of
 *                      kernels.js:320, the cascade of kernels.js:328-339
 *                      (a stop id never extends it); drafts from
 *                      argmaxMerge kernels.js:373-401 (lowest id among equal
 *                      maxima).  Pinned by closed forms: drafts = first
 *                      np.argmax over the non-NaN values, planted picks with
 *                      hand-derived accept counts, and a stop-id draft.
 *   orc_q81_quantize   quantizeQ81 ggml/q8.js:27-42 (amax / 127 scale,
 *                      round-half-even, f16 d and d * sum).  Pinned by hand
 *                      blocks (tests/test_oracle.py): scale and rounding of
 *                      a planted block, ties to even, numpy's float16.
 *   orc_lm_head_q_logits  the GGUF heads (ggml/kernels.js:64-80 dequant
 *                      formulas; the Q8_1 GEMV terms of ggml/q8.js:202-240)
 *                      in this build's order.  Pinned by closed forms: a
 *                      block's weights recovered through one-hot hiddens
 *                      (scale 127 exactness), every block term against the
 *                      reference's per-element dequantization formula in
 *                      double, a planted order that separates the tree.
 *                      Against the reference's WGSL order: parity unpinned.
 *   orc_spec_commit    acceptSpec's commit kernels.js:340-367 (log entry,
 *                      position, ring appends without stop ids, stop freeze,
 *                      frozen rounds, round counter).  Pinned by hand-derived
 *                      chains (tests/test_oracle.py): planted picks whose
 *                      logs, positions, rings and freezes are worked out by
 *                      hand, a ring that wraps, a stop among the accepted
 *                      picks.
 */
#include "sampler_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ exp -- */

static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* fdlibm exp: x = k*ln2 + r, |r| <= ln2/2, exp(r) from a degree-5 Remez
 * rational form, scaled by 2^k.  Constants are fdlibm's published ones. */
double orc_exp(double x) {
  static const double ln2_hi[2] = {6.93147180369123816490e-01, -6.93147180369123816490e-01};
  static const double ln2_lo[2] = {1.90821492927058770002e-10, -1.90821492927058770002e-10};
  static const double half[2] = {0.5, -0.5};
  const double inv_ln2 = 1.44269504088896338700e+00;
  const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03,
               P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06,
               P5 = 4.13813679705723846039e-08;
  const double over = 7.09782712893383973096e+02, under = -7.45133219101941108420e+02;
  const double two_m1000 = 9.33263618503218878990e-302, big = 1.0e300;
  uint64_t bits = d2u(x);
  uint32_t hx = (uint32_t)(bits >> 32);
  int neg = (int)(hx >> 31);
  hx &= 0x7fffffffu;
  double hi = 0.0, lo = 0.0;
  int k = 0;
  if (hx >= 0x40862E42u) {                 /* |x| >= 709.78 */
    if (hx >= 0x7ff00000u) {
      if (((hx & 0xfffffu) | (uint32_t)bits) != 0) return x + x; /* NaN */
      return neg ? 0.0 : x;                /* exp(+-inf) */
    }
    if (x > over) return big * big;
    if (x < under) return two_m1000 * two_m1000;
  }
  if (hx > 0x3fd62e42u) {                  /* |x| > ln2/2 */
    if (hx < 0x3FF0A2B2u) {                /* |x| < 1.5 ln2 */
      if (x == 1.0) return 2.718281828459045;
      hi = x - ln2_hi[neg];
      lo = ln2_lo[neg];
      k = 1 - neg - neg;
    } else {
      k = (int)(inv_ln2 * x + half[neg]);
      double t = (double)k;
      hi = x - t * ln2_hi[0];
      lo = t * ln2_lo[0];
    }
    x = hi - lo;
  } else if (hx < 0x3e300000u) {           /* |x| < 2^-28 */
    if (big + x > 1.0) return 1.0 + x;
  } else {
    k = 0;
  }
  double t = x * x;
  double c = x - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) {
    if (k == 1024) return y * 2.0 * 8.988465674311579539e307;
    return y * u2d((uint64_t)(0x3ff00000 + (k << 20)) << 32);
  }
  return y * u2d((uint64_t)(0x3ff00000 + ((k + 1000) << 20)) << 32) * two_m1000;
}

/* ------------------------------------------------------------ pcg draw -- */

uint32_t orc_pcg(uint32_t x) {
  uint32_t h = x * 747796405u + 2891336453u;
  h = ((h >> ((h >> 28u) + 4u)) ^ h) * 277803737u;
  return (h >> 22u) ^ h;
}

double orc_pcg_uniform(uint32_t seed, uint32_t it, uint32_t row) {
  uint32_t h = orc_pcg(seed ^ (it * 0x9E3779B9u) ^ (row * 0x85EBCA6Bu));
  /* kernels.js:181 computes this in f32; 24-bit integer / 2^24 is exact. */
  return (double)(h & 0xFFFFFFu) / 16777216.0;
}

/* ------------------------------------------------------ value pipeline -- */

/* tanh of an fp32 value rounded once from a double evaluation: odd Taylor
 * polynomial below 2^-9, (e^2x - 1)/(e^2x + 1) with the fdlibm exp above,
 * 1 from 9.5 on.  The GPU evaluates the same expression, so both sides
 * produce the same bits; the result is the correctly rounded tanhf except
 * where the double result falls within its own error of a rounding
 * boundary. */
float orc_tanhf(float x) {
  double ax = fabs((double)x), r;
  if (ax != ax) return x;
  if (ax >= 9.5) {
    r = 1.0;
  } else if (ax < 0.001953125) {
    double x2 = ax * ax;
    r = ax * (1.0 - x2 * (1.0 / 3.0 - x2 * (2.0 / 15.0 - x2 * (17.0 / 315.0))));
  } else {
    double t = orc_exp(2.0 * ax);
    r = (t - 1.0) / (t + 1.0);
  }
  return copysignf((float)r, x);
}

float orc_softcap(float x, float cap) {
  float q = x / cap;
  float t = orc_tanhf(q);
  return cap * t;
}

double orc_penalize(double v, uint32_t count, const orc_params *p) {
  if (count == 0) return v;
  double r = p->repetition_penalty;
  v = v > 0.0 ? v / r : v * r;
  v = v - p->frequency_penalty * (double)count;
  v = v - p->presence_penalty;
  return v;
}

typedef struct cand { double v; uint32_t id; } cand;

/* (v desc, id asc): the order a stable descending sort of the reference's
 * id-ascending candidate list produces (tokenizer.js:160). */
static inline int better(const cand *a, const cand *b) {
  return a->v > b->v || (a->v == b->v && a->id < b->id);
}

static int cmp_cand(const void *pa, const void *pb) {
  const cand *a = (const cand *)pa, *b = (const cand *)pb;
  if (better(a, b)) return -1;
  if (better(b, a)) return 1;
  return 0;
}

/* min-heap on "worst first" of at most cap entries */
static void heap_push(cand *h, int *n, int cap, cand c) {
  if (*n < cap) {
    int i = (*n)++;
    h[i] = c;
    while (i > 0) {
      int par = (i - 1) >> 1;
      if (!better(&h[par], &h[i])) break;
      cand t = h[par]; h[par] = h[i]; h[i] = t;
      i = par;
    }
    return;
  }
  if (!better(&c, &h[0])) return;
  h[0] = c;
  int i = 0;
  for (;;) {
    int l = 2 * i + 1, r = l + 1, w = i;
    if (l < *n && better(&h[w], &h[l])) w = l;
    if (r < *n && better(&h[w], &h[r])) w = r;
    if (w == i) break;
    cand t = h[w]; h[w] = h[i]; h[i] = t;
    i = w;
  }
}

static int clamp_top_k(int32_t k) {
  if (k < 1) return 1;
  if (k > ORC_MAX_TOP_K) return ORC_MAX_TOP_K;
  return k;
}

void orc_sample_row(const float *logits, int32_t vocab, const uint32_t *mask,
                    const uint32_t *hist, int32_t hist_len,
                    const orc_params *p, double uniform, int select_mode,
                    orc_result *out) {
  memset(out, 0, sizeof(*out));
  out->id = ORC_NO_TOKEN;
  /* history counts */
  uint32_t *counts = NULL;
  if (hist && hist_len > 0) {
    counts = (uint32_t *)calloc((size_t)vocab, sizeof(uint32_t));
    for (int32_t i = 0; i < hist_len; i++)
      if (hist[i] < (uint32_t)vocab) counts[hist[i]]++;
  }
  int greedy = !(p->temperature > 0.0);
  int kreq = greedy ? 1 : clamp_top_k(p->top_k);
  cand *sel;
  int nsel = 0;
  int64_t nvalid = 0;
  cand *all = NULL;
  if (select_mode == 1) all = (cand *)malloc(sizeof(cand) * (size_t)vocab);
  cand heap[ORC_MAX_TOP_K];
  for (int32_t i = 0; i < vocab; i++) {
    if (mask && !((mask[i >> 5] >> (i & 31)) & 1u)) continue;
    float x = logits[i];
    if (p->softcap > 0.0f) x = orc_softcap(x, p->softcap);
    if (x != x) continue; /* NaN never becomes a candidate */
    double v = (double)x;
    if (counts) v = orc_penalize(v, counts[i], p);
    if (v != v) continue;
    cand c = {v, (uint32_t)i};
    nvalid++;
    if (select_mode == 1) all[nsel++] = c;
    else heap_push(heap, &nsel, kreq, c);
  }
  free(counts);
  if (nvalid == 0) {
    out->flags |= ORC_FLAG_EMPTY_ROW;
    free(all);
    return;
  }
  if (select_mode == 1) {
    qsort(all, (size_t)nsel, sizeof(cand), cmp_cand);
    sel = all;
    if (nsel > kreq) nsel = kreq;
  } else {
    qsort(heap, (size_t)nsel, sizeof(cand), cmp_cand);
    sel = heap;
  }
  /* tokenizer.js:161-162 */
  int k = nsel < kreq ? nsel : kreq;
  if (greedy) {
    out->id = sel[0].id;
    free(all);
    return;
  }
  /* tokenizer.js:163-168: p_i = exp((v_i - v_0) / T), sum in order */
  double probs[ORC_MAX_TOP_K], prefix[ORC_MAX_TOP_K];
  double mx = sel[0].v, sum = 0.0;
  for (int i = 0; i < k; i++) {
    probs[i] = orc_exp((sel[i].v - mx) / p->temperature);
    sum += probs[i];
    prefix[i] = sum;
  }
  /* tokenizer.js:169-174: top-p cut */
  double cum = 0.0;
  int cut = k;
  for (int i = 0; i < k; i++) {
    cum += probs[i] / sum;
    if (fabs(cum - p->top_p) < 1e-6) out->flags |= ORC_FLAG_TOPP_EDGE;
    if (cum >= p->top_p) { cut = i + 1; break; }
  }
  /* tokenizer.js:175-177: r = U * sum(probs[0..cut)) with reduce from 0,
   * which equals the running sum prefix[cut-1] bit for bit. */
  double sub = prefix[cut - 1];
  double r = uniform * sub;
  uint32_t id = sel[cut - 1].id;
  for (int i = 0; i < cut; i++) {
    r -= probs[i];
    if (fabs(r) <= 1e-12 * sub) out->flags |= ORC_FLAG_DRAW_EDGE;
    if (r <= 0.0) { id = sel[i].id; break; }
  }
  out->id = id;
  out->k = k;
  out->cut = cut;
  for (int i = 0; i < k; i++) {
    out->cand_ids[i] = sel[i].id;
    out->probs[i] = probs[i] / sum;
  }
  free(all);
}

/* ----------------------------------------------------------------- batch -- */

typedef struct batch_job {
  const float *logits; int64_t logits_stride; int32_t vocab; int32_t rows;
  const uint32_t *mask; int64_t mask_stride;
  const uint32_t *hist_ids; const int32_t *hist_offsets;
  const double *uniforms; const orc_params *params; const orc_params *row_params;
  uint32_t *out_ids; double *out_probs; uint32_t *out_cand_ids;
  int32_t *out_counts; uint32_t *out_flags;
  int32_t r0, r1;
} batch_job;

static void *batch_worker(void *arg) {
  batch_job *j = (batch_job *)arg;
  orc_result res;
  for (int32_t r = j->r0; r < j->r1; r++) {
    const orc_params *p = j->row_params ? &j->row_params[r] : j->params;
    const uint32_t *h = NULL;
    int32_t hl = 0;
    if (j->hist_ids && j->hist_offsets) {
      h = j->hist_ids + j->hist_offsets[r];
      hl = j->hist_offsets[r + 1] - j->hist_offsets[r];
    }
    double u = j->uniforms ? j->uniforms[r] : 0.0;
    orc_sample_row(j->logits + (int64_t)r * j->logits_stride, j->vocab,
                   j->mask ? j->mask + (int64_t)r * j->mask_stride : NULL, h, hl,
                   p, u, 0, &res);
    j->out_ids[r] = res.id;
    if (j->out_counts) { j->out_counts[2 * r] = res.k; j->out_counts[2 * r + 1] = res.cut; }
    if (j->out_flags) j->out_flags[r] = res.flags;
    if (j->out_probs)
      for (int i = 0; i < ORC_MAX_TOP_K; i++)
        j->out_probs[(int64_t)r * ORC_MAX_TOP_K + i] = i < res.k ? res.probs[i] : 0.0;
    if (j->out_cand_ids)
      for (int i = 0; i < ORC_MAX_TOP_K; i++)
        j->out_cand_ids[(int64_t)r * ORC_MAX_TOP_K + i] = i < res.k ? res.cand_ids[i] : ORC_NO_TOKEN;
  }
  return NULL;
}

void orc_sample_rows(const float *logits, int64_t logits_stride, int32_t vocab,
                     int32_t rows, const uint32_t *mask, int64_t mask_stride,
                     const uint32_t *hist_ids, const int32_t *hist_offsets,
                     const double *uniforms, const orc_params *params,
                     const orc_params *row_params, uint32_t *out_ids,
                     double *out_probs, uint32_t *out_cand_ids,
                     int32_t *out_counts, uint32_t *out_flags, int threads) {
  if (threads < 1) threads = 1;
  if (threads > rows) threads = rows > 0 ? rows : 1;
  batch_job base = {logits, logits_stride, vocab, rows, mask, mask_stride,
                    hist_ids, hist_offsets, uniforms, params, row_params,
                    out_ids, out_probs, out_cand_ids, out_counts, out_flags, 0, rows};
  if (threads == 1) { batch_worker(&base); return; }
  pthread_t tid[64];
  batch_job jobs[64];
  if (threads > 64) threads = 64;
  for (int t = 0; t < threads; t++) {
    jobs[t] = base;
    jobs[t].r0 = (int32_t)((int64_t)rows * t / threads);
    jobs[t].r1 = (int32_t)((int64_t)rows * (t + 1) / threads);
    pthread_create(&tid[t], NULL, batch_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------------ mask -- */

int64_t orc_mask_from_ids(int32_t kind, const uint32_t *ids, size_t count,
                          int32_t vocab, uint32_t *words, int64_t nwords) {
  int64_t need = ((int64_t)vocab + 31) / 32;
  if (nwords < need || kind < 0 || kind > 2) return -1;
  memset(words, 0, sizeof(uint32_t) * (size_t)nwords);
  if (kind == 1) {
    for (size_t i = 0; i < count; i++)
      if (ids[i] < (uint32_t)vocab) words[ids[i] >> 5] |= 1u << (ids[i] & 31);
  } else {
    for (int32_t i = 0; i < vocab; i++) words[i >> 5] |= 1u << (i & 31);
    if (kind == 2)
      for (size_t i = 0; i < count; i++)
        if (ids[i] < (uint32_t)vocab) words[ids[i] >> 5] &= ~(1u << (ids[i] & 31));
  }
  int64_t n = 0;
  for (int64_t w = 0; w < need; w++) n += __builtin_popcount(words[w]);
  return n;
}

/* ---------------------------------------------------------------- verify -- */

/* Masked softmax weights of one row: w_i = exp((x_i - M) / T) for allowed
 * non-NaN ids (0 otherwise); returns Z = sum in ascending id order. */
static double soft_weights(const float *x, int32_t vocab, const uint32_t *mask,
                           double T, double *w) {
  double m = -INFINITY;
  for (int32_t i = 0; i < vocab; i++) {
    if (mask && !((mask[i >> 5] >> (i & 31)) & 1u)) continue;
    if (x[i] != x[i]) continue;
    if ((double)x[i] > m) m = (double)x[i];
  }
  double z = 0.0;
  for (int32_t i = 0; i < vocab; i++) {
    w[i] = 0.0;
    if (mask && !((mask[i >> 5] >> (i & 31)) & 1u)) continue;
    if (x[i] != x[i]) continue;
    w[i] = orc_exp(((double)x[i] - m) / T);
    z += w[i];
  }
  return z;
}

/* smallest id with w > 0 whose running sum exceeds u * total */
static uint32_t draw_cdf(const double *w, int32_t vocab, double total, double u) {
  double target = u * total, cum = 0.0;
  uint32_t last = ORC_NO_TOKEN;
  for (int32_t i = 0; i < vocab; i++) {
    if (w[i] <= 0.0) continue;
    cum += w[i];
    last = (uint32_t)i;
    if (cum > target) return (uint32_t)i;
  }
  return last;
}

void orc_verify(const float *target, const float *draft, int64_t stride,
                int32_t vocab, int32_t seqs, int32_t draft_len,
                const uint32_t *draft_ids, const uint32_t *mask,
                int64_t mask_stride, const double *uniforms,
                double temperature, uint32_t *out_tokens,
                int32_t *out_accepted, double *out_ratio) {
  double *wp = (double *)malloc(sizeof(double) * (size_t)vocab);
  double *wq = (double *)malloc(sizeof(double) * (size_t)vocab);
  int32_t L = draft_len;
  for (int32_t s = 0; s < seqs; s++) {
    uint32_t *out = out_tokens + (int64_t)s * (L + 1);
    for (int32_t j = 0; j <= L; j++) out[j] = ORC_NO_TOKEN;
    int32_t acc = 0;
    int done = 0;
    for (int32_t j = 0; j < L && !done; j++) {
      const uint32_t *m = mask ? mask + ((int64_t)s * (L + 1) + j) * mask_stride : NULL;
      const float *tx = target + ((int64_t)s * (L + 1) + j) * stride;
      const float *dx = draft + ((int64_t)s * L + j) * stride;
      double zp = soft_weights(tx, vocab, m, temperature, wp);
      double zq = soft_weights(dx, vocab, m, temperature, wq);
      uint32_t d = draft_ids[(int64_t)s * L + j];
      double pd = d < (uint32_t)vocab ? wp[d] / zp : 0.0;
      double qd = d < (uint32_t)vocab ? wq[d] / zq : 0.0;
      const double *u = uniforms + ((int64_t)s * (L + 1) + j) * 2;
      if (out_ratio) out_ratio[(int64_t)s * (L + 1) + j] = qd > 0.0 ? pd / qd : INFINITY;
      if (d < (uint32_t)vocab && pd > 0.0 && u[0] * qd <= pd) {
        out[j] = d;
        acc++;
        continue;
      }
      /* residual max(0, p - q), drawn in ascending id order */
      double tot = 0.0;
      for (int32_t i = 0; i < vocab; i++) {
        double r = wp[i] / zp - wq[i] / zq;
        wp[i] = r > 0.0 ? r : 0.0;
        tot += wp[i];
      }
      if (tot > 0.0) {
        out[j] = draw_cdf(wp, vocab, tot, u[1]);
      } else {
        soft_weights(tx, vocab, m, temperature, wp);
        out[j] = draw_cdf(wp, vocab, zp, u[1]);
      }
      done = 1;
    }
    if (!done) {
      const uint32_t *m = mask ? mask + ((int64_t)s * (L + 1) + L) * mask_stride : NULL;
      const float *tx = target + ((int64_t)s * (L + 1) + L) * stride;
      double zp = soft_weights(tx, vocab, m, temperature, wp);
      const double *u = uniforms + ((int64_t)s * (L + 1) + L) * 2;
      out[L] = draw_cdf(wp, vocab, zp, u[1]);
    }
    out_accepted[s] = acc;
  }
  free(wp);
  free(wq);
}

/* ------------------------------------------------ exact-match spec round -- */

void orc_spec_exact(const float *target, const float *draft, int64_t stride,
                    int32_t vocab, int32_t seqs, int32_t draft_len,
                    uint32_t *draft_ids, const uint32_t *mask,
                    int64_t mask_stride, const uint32_t *hist_ids,
                    const int32_t *hist_offsets, const orc_params *params,
                    const orc_params *seq_params, const uint32_t *seeds,
                    uint32_t round, const uint32_t *stop_ids,
                    uint32_t *out_picks, int32_t *out_accepted,
                    uint32_t *out_next) {
  const int32_t L = draft_len;
  orc_params greedy;
  memset(&greedy, 0, sizeof greedy);
  greedy.top_p = 1.0;
  greedy.repetition_penalty = 1.0;
  greedy.top_k = 1;
  orc_result res;
  for (int32_t s = 0; s < seqs; s++) {
    /* drafts: the top-1 of each draft row (argmaxMerge, kernels.js:373-401) */
    if (draft) {
      for (int32_t j = 0; j < L; j++) {
        orc_sample_row(draft + ((int64_t)s * L + j) * stride, vocab, NULL, NULL, 0, &greedy, 0.0, 0, &res);
        draft_ids[(int64_t)s * L + j] = res.id;
      }
    }
    const orc_params *p = seq_params ? &seq_params[s] : params;
    const uint32_t *h = NULL;
    int32_t hn = 0;
    if (hist_ids) {
      h = hist_ids + hist_offsets[s];
      hn = hist_offsets[s + 1] - hist_offsets[s];
    }
    /* every verify row on its own, history as of the round's start
     * (kernels.js:255-327) */
    uint32_t *pk = out_picks + (int64_t)s * (L + 1);
    for (int32_t j = 0; j <= L; j++) {
      const int64_t row = (int64_t)s * (L + 1) + j;
      const uint32_t *m = mask ? mask + (mask_stride ? row * mask_stride : 0) : NULL;
      orc_sample_row(target + row * stride, vocab, m, h, hn, p, orc_pcg_uniform(seeds[s], round, (uint32_t)j), 0,
                     &res);
      pk[j] = res.id;
    }
    /* the cascade (kernels.js:328-339) */
    int32_t a = 1;
    while (a <= L) {
      const uint32_t t = pk[a - 1];
      int stop = 0;
      if (stop_ids)
        for (int i = 0; i < 4; i++) stop |= t == stop_ids[4 * s + i];
      if (t != draft_ids[(int64_t)s * L + a - 1] || stop) break;
      a++;
    }
    out_accepted[s] = a;
    if (out_next) out_next[s] = pk[a - 1];
  }
}

/* ---- the LM head (sas_lm_head_sample) ----------------------------------
 * The reference's BF16 head (lib/webgpu-llm/ggml/kernels.js:31-33 widens
 * the weight as bits << 16; gemvGGML, ggml/kernels.js:84-110, sums f32
 * products) in the build's fixed order: eight partial fmaf chains over
 * interleaved slices of k, then a fixed pairwise tree.  fmaf is the
 * correctly rounded fused multiply-add, the GPU's v_fma_f32. */
void orc_lm_head_logits(const float *hidden, int64_t hidden_stride, const uint16_t *weight,
                        int64_t weight_stride, int32_t dim, int32_t rows, int32_t vocab,
                        float *logits) {
  for (int32_t r = 0; r < rows; ++r) {
    const float *h = hidden + (int64_t)r * hidden_stride;
    for (int32_t id = 0; id < vocab; ++id) {
      const uint16_t *w = weight + (int64_t)id * weight_stride;
      float p[8];
      for (int g = 0; g < 8; ++g) {
        float acc = 0.0f;
        for (int32_t c = 0; 64 * c + 8 * g < dim; ++c) {
          for (int j = 0; j < 8; ++j) {
            const int32_t k = 64 * c + 8 * g + j;
            if (k >= dim) break;
            const uint32_t bits = (uint32_t)w[k] << 16;
            float wf;
            memcpy(&wf, &bits, sizeof wf);
            acc = fmaf(wf, h[k], acc);
          }
        }
        p[g] = acc;
      }
      logits[(int64_t)r * vocab + id] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
  }
}

/* ------------------------------------------------- chained round commit -- */

void orc_spec_commit(int32_t seqs, int32_t draft_len, const uint32_t *picks, const uint32_t *draft_ids,
                     const int32_t *accepted, const uint32_t *stop_ids, uint32_t *state, uint32_t *ring,
                     int32_t ring_len, uint32_t *log, int32_t max_rounds, uint32_t *next_tokens,
                     int32_t *accepted_out) {
  const int32_t L = draft_len;
  for (int32_t s = 0; s < seqs; s++) {
    const uint32_t *sp = stop_ids ? stop_ids + 4 * (int64_t)s : NULL;
    const uint32_t stop0 = sp ? sp[0] : 0xFFFFFFFFu;
    uint32_t *st = state + 4 * (int64_t)s;
    const uint32_t frozen = st[0], rnd = st[1];
    const uint32_t *pk = picks + (int64_t)s * (L + 1);
    int32_t a = 0;
    uint32_t next = stop0;
    if (!frozen) {
      a = accepted[s];
      next = pk[a - 1];
    }
    if (log && rnd < (uint32_t)max_rounds) {
      uint32_t *lg = log + ((int64_t)s * max_rounds + rnd) * (L + 2);
      lg[0] = (uint32_t)a;
      lg[1] = next;
      for (int32_t j = 0; j < L; j++) lg[2 + j] = frozen ? 0u : draft_ids[(int64_t)s * L + j];
    }
    if (!frozen) {
      st[2] += (uint32_t)a;   /* posBuf[0] += a */
      st[3] = (uint32_t)a;    /* posBuf[1] = a */
      for (int32_t i = 0; i < a; i++) {
        const uint32_t t = pk[i];
        int stop = 0;
        for (int q = 0; q < 4 && sp; q++) stop |= t == sp[q];
        if (!stop && ring) {
          uint32_t *rg = ring + (int64_t)s * (ring_len + 1);
          const uint32_t c = rg[0];
          rg[1 + c % (uint32_t)ring_len] = t;
          rg[0] = c + 1u;
        }
      }
      int stop = 0;
      for (int q = 0; q < 4 && sp; q++) stop |= next == sp[q];
      if (stop) st[0] = 1u;
    }
    if (next_tokens) next_tokens[s] = next;
    if (accepted_out) accepted_out[s] = a;
    st[1] = rnd + 1u;
  }
}

/* ------------------------------------------------ quantized LM head ---- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static uint16_t f32_to_f16_bits(float f) {
  const uint32_t x = f2u(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t e = (x >> 23) & 0xFFu;
  uint32_t m = x & 0x7FFFFFu;
  if (e == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u | (m >> 13) : 0u));
  const int32_t ee = (int32_t)e - 127 + 15;
  if (ee >= 31) return (uint16_t)(sign | 0x7C00u);
  if (ee <= 0) {
    if (ee < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - ee);
    const uint32_t half = 1u << (shift - 1), rest = m & ((1u << shift) - 1u);
    uint32_t r = m >> shift;
    if (rest > half || (rest == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((uint32_t)ee << 10) | (m >> 13);
  const uint32_t rest = m & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (r & 1u))) r++;
  return (uint16_t)(sign | r);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
  if (e == 0) {
    /* subnormal: m * 2^-24, exact in f32 */
    const float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

float orc_f16_round(float x) { return orc_f16_to_f32(f32_to_f16_bits(x)); }

void orc_q81_quantize(const float *x, int32_t dim, int8_t *q, float *d8, float *s8) {
  for (int32_t b = 0; b < dim / 32; b++) {
    const float *v = x + 32 * b;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
      const float a = fabsf(v[i]);
      if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    int32_t sum = 0;
    for (int i = 0; i < 32; i++) {
      const float t = v[i] * inv;
      float r = t != t ? 0.0f : rintf(t);
      if (r > 127.0f) r = 127.0f;
      if (r < -128.0f) r = -128.0f;
      q[32 * b + i] = (int8_t)r;
      sum += (int32_t)r;
    }
    d8[b] = orc_f16_round(d);
    s8[b] = orc_f16_round(d * (float)sum);
  }
}

static inline float head_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* The term of weight block / piece `it` of one row (see the header). */
static float q_term(int32_t format, const uint8_t *w, int32_t it, int32_t piece, const int8_t *q, const float *d8,
                    const float *s8) {
  if (format == ORC_HEAD_Q8_0) {
    const uint8_t *blk = w + 34 * (int64_t)it;
    int32_t dot = 0;
    for (int i = 0; i < 32; i++) dot += (int32_t)(int8_t)blk[2 + i] * q[32 * it + i];
    const float d = head_f16(blk);
    return ((float)dot * d) * d8[it];
  }
  if (format == ORC_HEAD_Q4_0) {
    const uint8_t *blk = w + 18 * (int64_t)it;
    int32_t dot = 0;
    for (int i = 0; i < 32; i++) {
      const int32_t nib = i < 16 ? (blk[2 + i] & 15) : (blk[2 + i - 16] >> 4);
      dot += nib * q[32 * it + i];
    }
    const float d = head_f16(blk);
    return ((float)dot * d) * d8[it] - (8.0f * d) * s8[it];
  }
  /* Q6_K: unit it, piece (quarter) 0..3 */
  const int32_t sb = it / 4, un = it % 4, h = un >> 1, lh = un & 1, quarter = piece;
  const uint8_t *blk = w + 210 * (int64_t)sb;
  int32_t dot = 0;
  const int32_t qblk = sb * 8 + h * 4 + quarter;  /* the Q8_1 block of the 16 values */
  for (int e = 0; e < 16; e++) {
    const int32_t l = lh * 16 + e;
    const uint8_t packed = blk[h * 64 + ((quarter & 1) ? 32 : 0) + l];
    const int32_t nib = quarter >= 2 ? packed >> 4 : packed & 15;
    const int32_t hi = (blk[128 + h * 32 + l] >> (quarter * 2)) & 3;
    dot += ((nib | (hi << 4)) - 32) * q[32 * qblk + lh * 16 + e];
  }
  const float d = head_f16(blk + 208);
  const float sc = (float)(int8_t)blk[192 + h * 8 + lh + quarter * 2];
  return ((d * sc) * d8[qblk]) * (float)dot;
}

void orc_lm_head_q_logits(int32_t format, const float *hidden, int64_t hidden_stride, const uint8_t *weight,
                          int64_t row_bytes, int32_t dim, int32_t rows, int32_t vocab, float *logits) {
  int8_t *q = (int8_t *)malloc((size_t)dim);
  float *d8 = (float *)malloc(sizeof(float) * (size_t)(dim / 32));
  float *s8 = (float *)malloc(sizeof(float) * (size_t)(dim / 32));
  const int32_t items = format == ORC_HEAD_Q6_K ? dim / 64 : dim / 32;
  const int32_t pieces = format == ORC_HEAD_Q6_K ? 4 : 1;
  for (int32_t r = 0; r < rows; r++) {
    orc_q81_quantize(hidden + (int64_t)r * hidden_stride, dim, q, d8, s8);
    for (int32_t id = 0; id < vocab; id++) {
      const uint8_t *w = weight + (int64_t)id * row_bytes;
      float p[8];
      for (int g = 0; g < 8; g++) {
        float acc = 0.0f;
        for (int32_t it = g; it < items; it += 8)
          for (int32_t pc = 0; pc < pieces; pc++) acc = acc + q_term(format, w, it, pc, q, d8, s8);
        p[g] = acc;
      }
      logits[(int64_t)r * vocab + id] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
  }
  free(q);
  free(d8);
  free(s8);
}

// sample_kernel.hip - logit processing + top-k/top-p sampling for gfx950.
//
// Two launches per decode step, stream-ordered.
//
// The parts kernel: grid = rows x parts blocks of 256 threads.  Block
// (row, q) owns ids [q * span, (q + 1) * span) of its row (one pass of 8192
// ids unless the vocabulary is huge):
//   1. loads: the pass's fp32 logits as 16-byte nontemporal loads (8 per
//      thread, all in flight at once) and the mask word of each float4; the
//      row's history ids are counted into an LDS bitmap over the part's ids
//      and an (id, count) hash while the logits are in flight;
//   2. per value: masked ids and history ids become NaN (never selected
//      here; ids past the row too); Gemma's softcap when the row has one;
//   3. the bound: every wave finds the j-th largest of its 64 lane maxima
//      (j = ceil(k / 4)) by a ballot search on order-preserving keys, and the
//      part's bound is the smallest of the four: at least 4 j >= k values of
//      the part reach it, so no value below it is in the row's top k;
//   4. values at or above the bound go to per-wave LDS lists (one ballot per
//      value slot); the part's history ids are handled one by one with their
//      exact penalized double values (with long, bucketed histories and
//      penalties that only lower values, members ride in the lists with
//      their raw values and only those reaching the bound are penalized);
//   5. the lists are written as records to the part's own slots: plain
//      values as {fp32 value, id}, history members as {round-down key, id,
//      exact double}.
// The merge kernel: one block per row.
//   6. one round of loads brings every part's counts, bound and records;
//   7. the bound again, over the records: the largest part bound, and the
//      j-th largest of each wave's lane maxima, the smallest over the waves;
//   8. the records at or above it are ranked exactly by (value desc, id asc)
//      through 64-bit (key, inexact, ~id) composites;
//   9. the reference's sample() tail in double precision: a parallel scan
//      of the weights decides the top-p cut and the draw whenever rounding
//      cannot change them, else the reference's sequential chains run.
//
// A part list that overflows (heavy ties) or a merge with too many survivors
// takes an exact radix select over (value, id) keys (SAS_FLAG_SLOW_SELECT).
//
// Logits cross HBM once.  Replaces the topk + sampler WGSL pair
// (lib/webgpu-llm/kernels.js:1389-1449, 65-201) and the CPU sample()
// (lib/webgpu-llm/tokenizer.js:151-178).
#include "sas_device.h"
#include "sas_launch.h"

namespace sas {

constexpr int kSlots = kSpanPass / (4 * kThreads);  // float4 per thread per pass
static_assert(kSlots == 8, "a thread holds 32 values of a pass");
constexpr int kHashSlots = 512;
constexpr int kHistPre = 2;                          // history ids per thread loaded before the logits
constexpr int kQuadCap = 128;                        // float4 entries of one wave's candidate list: two per lane
static_assert(kQuadCap == 128, "a wave's list is at most two entries per lane at the end");
constexpr uint32_t kEmpty = 0xFFFFFFFFu;



// Lane i's double on every lane (i wave-uniform).
__device__ __forceinline__ double bcast(double x, int i) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, i);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), i);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}


// (va, ia) ranks before (vb, ib): value desc, then id asc (tokenizer.js:160
// stable sort of an id-ascending list; kernels.js:1433, 1439 tie rule).
__device__ __forceinline__ bool before(double va, uint32_t ia, double vb, uint32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// ----------------------------------------------------------------- merge --
//
// One block per row merges the row after the parts kernel: it loads every
// part's records, bounds the row's k-th largest key by the j-th largest of
// each wave's lane maxima, ranks the records at or above the bound exactly
// by (value desc, id asc) and runs the reference's sample() tail.

// The merge kernel loads kMR plain record slots per thread before the
// counts are known (between them a part's first kThreads * kMR / parts
// slots, as whole 128-byte lines); a part's records past them are loaded
// where they are used.  launch_merge picks kMR from the expected count per
// part (about 2 k plus a few).
constexpr int kMRMax = 16;
constexpr int kSurvCap = 1024;    // survivors the merge ranks
constexpr uint32_t kInexact = 0x80000000u;  // composite bit: the exact value lies above the key

struct MergeLds {
  uint32_t wred[kWaves][4];          // per-wave partial results
  uint64_t s_c[kSurvCap + 8];        // survivors: rank composites (zero padded to a multiple of 8)
  double s_v[kSurvCap];              // and exact values
  uint32_t s_rank[kSurvCap];
  double t_val[SAS_MAX_TOP_K + 1];   // the ranked top k (and the one after)
  uint32_t t_id[SAS_MAX_TOP_K + 1];
  uint64_t t_c[SAS_MAX_TOP_K + 1];
  double t_p[SAS_MAX_TOP_K + 8];     // weights exp((v_i - v_0) / T), zero past k
  double t_q[SAS_MAX_TOP_K + 8];     // weights / their sum, zero past k
  double t_pre[SAS_MAX_TOP_K + 8];   // running weight sums
  double t_cum[SAS_MAX_TOP_K + 8];   // running top-p masses
  double t_r[SAS_MAX_TOP_K + 8];     // running draw residuals
  uint32_t m;
  uint32_t p_np[kMaxParts];          // the parts' plain record counts
  double g_v[kWaves];                // greedy rows: each wave's best (value, id), has-any | slow bits
  uint32_t g_id[kWaves];
  uint32_t g_f[kWaves];
};

struct MergeOut {
  uint32_t *ids;
  double *probs;
  uint32_t *cand_ids;
  int32_t *counts;
  uint32_t *flags;
};

// A member record: {fp32 key bits of the penalized value (rounded toward
// -inf), id, the penalized double (low word, high word)}.
__device__ __forceinline__ double member_value(const uint4 &mr) {
  return __longlong_as_double((long long)(((uint64_t)mr.w << 32) | mr.z));
}

// Rank composite, larger = ranks first: the key, then whether the exact
// value lies above it (strictly between the key and the next float, so it
// ranks after every larger key and before the exact values of its own
// key), then the id reversed.  Only two inexact values of one key need
// their doubles to be ordered.
__device__ __forceinline__ uint64_t composite(uint32_t key, bool inexact, uint32_t id) {
  return ((uint64_t)key << 32) | (inexact ? kInexact : 0u) | (0x7FFFFFFFu - id);
}
__device__ __forceinline__ uint32_t comp_id(uint64_t c) { return 0x7FFFFFFFu - ((uint32_t)c & 0x7FFFFFFFu); }

// One running chain in the reference's left-to-right order, run by the
// calling lane alone: dst[i] = init (+ or -) src[0] ... (+ or -) src[i] for
// every i < n (and a few past it, over the zero padding).  Each step is one
// add and one LDS store; the operands arrive 8 at a time, the next batch in
// flight.
template <bool kSub>
__device__ __forceinline__ void chain(const double *src, double *dst, int n, double init) {
  double run = init;
  double x[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) x[u] = src[u];
  for (int i = 0; i < n; i += 8) {
    const int in = i + 8 < n ? i + 8 : i;
    double y[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) y[u] = src[in + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      run = kSub ? run - x[u] : run + x[u];
      dst[i + u] = run;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = y[u];
  }
}

// The first index (lanes 0..63 of `lo`, then 64..127 of `hi`) below n whose
// condition holds, or n.
__device__ __forceinline__ int first_true(bool c_lo, bool c_hi, int n) {
  const int lane = threadIdx.x & 63;
  const uint64_t a = __ballot(c_lo && lane < n), b = __ballot(c_hi && lane + 64 < n);
  if (a) return __builtin_ctzll(a);
  if (b) return 64 + __builtin_ctzll(b);
  return n;
}

// A double moved between lanes by DPP (both halves); lanes without a
// source read +0.0.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ double dpp0_d(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = dpp0<kCtrl, kRowMask>((uint32_t)b), hi = dpp0<kCtrl, kRowMask>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Inclusive prefix sum of a double over the wave (a tree of depth 6):
// Hillis-Steele within each row of 16 lanes, then the rows' totals carried
// forward.  Adding the +0.0 of a lane without a source leaves x unchanged
// (the weights are >= +0.0).
__device__ __forceinline__ double wave_scan_d(double x) {
  x = x + dpp0_d<kDppRowShr1>(x);
  x = x + dpp0_d<kDppRowShr2>(x);
  x = x + dpp0_d<kDppRowShr4>(x);
  x = x + dpp0_d<kDppRowShr8>(x);
  x = x + dpp0_d<kDppRowBcast15, 0xA>(x);
  x = x + dpp0_d<kDppRowBcast31, 0xC>(x);
  return x;
}

// The reference's sample() tail (tokenizer.js:161-177) in double precision
// over the ranked top kk in ml.t_val / ml.t_id, by wave 0 (lane i holds
// candidate i and i + 64).
//
// The reference runs three sequential chains: the weight sum s_i (each
// addition rounded), the top-p mass cum_i = sum of fl(p_j / s_{k-1}), and
// the draw residual r_i = fl(U * s_{cut-1}) - p_0 - ... - p_i.  The token
// depends only on the signs of cum_i - top_p (up to the cut) and of r_i
// (up to the draw).  A parallel scan t_i of the same weights decides those
// signs wherever they are clear by a margin, with rounding-error bounds
// (n <= 128 terms, u = 2^-53, S_i = exact sum p_0..p_i >= 1 = p_0):
//   |s_i - S_i| <= 128u/(1-128u) S_i <= 1.43e-14 S_i   (sequential, any order)
//   |t_i - S_i| <= 8u S_i <= 1e-15 S_i                  (scan: depth <= 8)
//   cum_i = (S_i / S_{k-1})(1 + e), |e| <= 2.9e-14, so with
//   D_i = t_i - fl(top_p t_{k-1}):  |S_{k-1}(cum_i - top_p) - D_i| <= 3.3e-14 S_{k-1}
//   |r_i - (fl(U t_{cut-1}) - t_i)| <= 3.2e-14 S_{cut-1}
// A row is taken from the scan when every D_i up to the cut is clear of 0
// by 1e-13 t_{k-1} and also of the top-p edge test (|cum_i - top_p| < 1e-6),
// and every residual up to the draw is clear of 0 and of the draw edge test
// (|r_i| <= 1e-12 s_{cut-1}) by 1e-13 t_{cut-1}: then the sequential chains
// give the same cut, draw and flags.  Other rows run the chains.
__device__ __forceinline__ uint32_t sample_tail(MergeLds &ml, int kk, int row, double T, double top_p,
                                                double u_row, uint32_t flags, const MergeOut &o) {
  const int lane = threadIdx.x & 63;
  const bool greedy = !(T > 0.0);
  const bool draw = !greedy && kk > 0;
  uint32_t out_id = SAS_NO_TOKEN;
  int cut = 0;
  double q_a = 0.0, q_b = 0.0;
  if (kk == 0) {
    flags |= SAS_FLAG_EMPTY_ROW;
  } else if (greedy) {
    out_id = ml.t_id[0];
  } else {
    const double v0 = ml.t_val[0];
    // p_i = exp((v_i - v_0) / T), zero past kk (x / 1 is x)
    double d_a = lane < kk ? ml.t_val[lane] - v0 : 0.0;
    double d_b = lane + 64 < kk ? ml.t_val[lane + 64] - v0 : 0.0;
    if (T != 1.0) {  // uniform: no division at T = 1
      d_a = d_a / T;
      if (kk > 64) d_b = d_b / T;
    }
    double p_a = 0.0, p_b = 0.0;
    if (lane < kk) p_a = fd_exp(d_a);
    if (lane + 64 < kk) p_b = fd_exp(d_b);
    ml.t_p[lane] = p_a;
    ml.t_p[lane + 64] = p_b;
    if (lane < 8) ml.t_p[128 + lane] = 0.0;
    // ---- the scan ----
    const double ta = wave_scan_d(p_a);
    const double tot_a = bcast(ta, 63);
    const double tb = kk > 64 ? tot_a + wave_scan_d(p_b) : tot_a;
    const double tk = kk > 64 ? bcast(tb, 63) : tot_a;  // t_{k-1}: the weights past kk are zero
    const double tp = top_p * tk;
    const double da = ta - tp, db = tb - tp;
    int c = min(first_true(da >= 0.0, db >= 0.0, kk) + 1, kk);
    const double mc = (1e-6 + 1e-13) * tk;
    bool fast = __ballot((lane < c && fabs(da) < mc) || (lane + 64 < c && fabs(db) < mc)) == 0ull;
    int pk = 0;
    if (fast) {
      const double sub = c - 1 < 64 ? bcast(ta, c - 1) : bcast(tb, c - 65);
      const double us = u_row * sub;
      const double ra = us - ta, rb = us - tb;
      pk = min(first_true(ra <= 0.0, rb <= 0.0, c), c - 1);
      const double md = (1e-12 + 1e-13) * sub;
      fast = __ballot((lane <= pk && fabs(ra) <= md) || (lane + 64 <= pk && fabs(rb) <= md)) == 0ull;
    }
    if (fast && !o.probs) {
      cut = c;
      out_id = ml.t_id[pk];
    } else {
      wave_lds_sync();  // the weights in t_p
      // the weight sum and its prefixes (tokenizer.js:164-167)
      if (lane == 0) chain<false>(ml.t_p, ml.t_pre, kk, 0.0);
      wave_lds_sync();
      const double sum = ml.t_pre[kk - 1];
      q_a = p_a / sum;
      q_b = p_b / sum;
      if (fast) {
        cut = c;
        out_id = ml.t_id[pk];
      } else {
        ml.t_q[lane] = q_a;
        ml.t_q[lane + 64] = q_b;
        if (lane < 8) ml.t_q[128 + lane] = 0.0;
        wave_lds_sync();
        // top-p (tokenizer.js:169-174): the first i with q_0 + ... + q_i >= top_p
        if (lane == 0) chain<false>(ml.t_q, ml.t_cum, kk, 0.0);
        wave_lds_sync();
        const double c_a = ml.t_cum[lane], c_b = ml.t_cum[lane + 64];
        cut = min(first_true(c_a >= top_p, c_b >= top_p, kk) + 1, kk);
        const bool te = __ballot((lane < cut && fabs(c_a - top_p) < 1e-6) ||
                                 (lane + 64 < cut && fabs(c_b - top_p) < 1e-6)) != 0ull;
        // the draw (tokenizer.js:175-177): r = U * (p_0 + ... + p_{cut-1}),
        // minus p_0, p_1, ... until it reaches 0; else the last of the cut
        const double sub = ml.t_pre[cut - 1];
        if (lane == 0) chain<true>(ml.t_p, ml.t_r, cut, u_row * sub);
        wave_lds_sync();
        const double r_a = ml.t_r[lane], r_b = ml.t_r[lane + 64];
        const int pick = min(first_true(r_a <= 0.0, r_b <= 0.0, cut), cut - 1);
        const double eps = 1e-12 * sub;
        const bool de = __ballot((lane <= pick && fabs(r_a) <= eps) || (lane + 64 <= pick && fabs(r_b) <= eps)) != 0ull;
        if (te) flags |= SAS_FLAG_TOPP_EDGE;
        if (de) flags |= SAS_FLAG_DRAW_EDGE;
        out_id = ml.t_id[pick];
      }
    }
  }
  if (lane == 0) {
    o.ids[row] = out_id;
    if (o.counts) {
      o.counts[2 * row] = draw ? kk : 0;
      o.counts[2 * row + 1] = draw ? cut : 0;
    }
    if (o.flags) o.flags[row] = flags;
  }
  const int np = draw ? kk : 0;
  if (o.probs) {
    double *op = o.probs + (int64_t)row * SAS_MAX_TOP_K;
    op[lane] = lane < np ? q_a : 0.0;
    op[lane + 64] = lane + 64 < np ? q_b : 0.0;
  }
  if (o.cand_ids) {
    uint32_t *oc = o.cand_ids + (int64_t)row * SAS_MAX_TOP_K;
    oc[lane] = lane < np ? ml.t_id[lane] : SAS_NO_TOKEN;
    oc[lane + 64] = lane + 64 < np ? ml.t_id[lane + 64] : SAS_NO_TOKEN;
  }
  return out_id;
}

// The reference GPU samplers' uniform (kernels.js:91-95, 181, 320): the
// in-graph step draws with j = 0, verify row j of a speculative round with j.
__device__ __forceinline__ double pcg_uniform(uint32_t seed, uint32_t it, uint32_t j) {
  uint32_t h = (seed ^ (it * 0x9E3779B9u) ^ (j * 0x85EBCA6Bu)) * 747796405u + 2891336453u;
  h = ((h >> ((h >> 28u) + 4u)) ^ h) * 277803737u;
  h = (h >> 22u) ^ h;
  return (double)(h & 0xFFFFFFu) / 16777216.0;
}

// The step's bookkeeping after a row's token is known (kernels.js:189-199):
// record it, hand it to the next step, advance the iteration; a stop id or
// no token freezes the row, any other token joins the row's penalty ring.
// One thread.
__device__ __forceinline__ void step_feedback(const SampleArgs &a, int row, uint32_t tok, bool frozen) {
  uint32_t *st = a.st_state + 2 * row;
  const uint32_t it = st[1];
  if (a.st_sampled && it < (uint32_t)a.st_max_steps) a.st_sampled[(int64_t)row * a.st_max_steps + it] = tok;
  if (a.st_next) a.st_next[row] = tok;
  st[1] = it + 1u;
  bool stop = tok == SAS_NO_TOKEN;
  if (a.stop_ids) {
    const uint32_t *sp = a.stop_ids + 4 * row;
    stop = stop || tok == sp[0] || tok == sp[1] || tok == sp[2] || tok == sp[3];
  }
  if (stop) {
    st[0] = 1u;
  } else if (!frozen && a.ring) {
    uint32_t *rg = a.ring + (int64_t)row * (a.ring_len + 1);
    const uint32_t c = rg[0];
    rg[1 + c % (uint32_t)a.ring_len] = tok;
    rg[0] = c + 1u;
  }
}

// Loads of the records the row's parts published.  A record line is written
// only by its part (whole lines per part and per row of part counts) and read
// once, by the row's merge block in the next launch: nontemporal, since no
// other block reads it again.
__device__ __forceinline__ uint64_t load_rec(const uint64_t *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint4 load_rec4(const uint4 *p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Merge of row `row`: one block.
template <int kMR>
__device__ __forceinline__ void merge_row(const SampleArgs &a, MergeLds &ml, int row, const sas_params &p,
                                          uint32_t *s_hist, uint32_t *s_sel) {
  static_assert(kMR >= 1 && kMR <= kMRMax, "record slots per thread");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int P = a.parts;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  // Thread (q, sub) = (tid / G, tid % G), G threads per part, reads part
  // q's counts and bound and member record sub of part q.
  const int G = kThreads / P;
  const int q = tid / G, sub = tid - q * G;
  const bool qok = q < P;
  const int64_t pq = (int64_t)row * P + (qok ? q : 0);
  const uint64_t *rq = a.rec + pq * kListCap;
  const uint4 *mq = a.mrec + pq * kMemSlots;

  // ---- loads, all in flight at once, none behind a branch ----
  // The part's counts first: they go to LDS while the records still arrive.
  const uint64_t i4 = load_rec(a.pinfo + (int64_t)row * pinfo_stride(P) + min(q, P - 1));
  const uint4 m4 = load_rec4(mq + min(sub, kMemSlots - 1));
  // Plain records: the first 16 Lc slots of every part as whole 128-byte
  // lines.  Lanes 8 g .. 8 g + 7 of a wave read one line, 16 bytes (two
  // records) each; load i of reader R = 4 g + wave is chunk z = R +
  // (kThreads / 8) i, line z / P of part z % P.  Readers alternate over the
  // waves, so that every wave holds a fair share of every part's lines (the
  // bound below takes the weakest wave).  A chunk past the part's Lc lines
  // reads line 0 again, and it is dropped with the slots past the part's
  // count.  (Lanes reading 16-byte pieces of 64 different lines per load
  // took the step longer: each load then asks the cache for 64 lines.)
  constexpr int kReaders = kThreads / 8, kChunks = kMR / 2;
  static_assert(kMR % 2 == 0, "records in pairs");
  static_assert(kReaders * kChunks >= kMaxParts, "at least one line of every part");
  const int R = (lane >> 3) * kWaves + wave, l8 = tid & 7;
  const int Lc = min(kReaders * kChunks / P, kListCap / 16);
  const int zdiv = kReaders / P, zmod = kReaders - zdiv * P;  // chunk z + kReaders: part + zmod, line + zdiv
  const uint4 *rb = reinterpret_cast<const uint4 *>(a.rec);
  const uint32_t rrow = (uint32_t)row * (uint32_t)P;
  uint64_t rec[kMR];
  {
    int zq = R % P, zc = R / P;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const uint32_t at = (rrow + (uint32_t)zq) * (uint32_t)(kListCap / 2) + 8u * (uint32_t)(zc < Lc ? zc : 0) + (uint32_t)l8;
      const uint4 x = load_rec4(rb + at);
      rec[2 * i] = ((uint64_t)x.y << 32) | x.x;
      rec[2 * i + 1] = ((uint64_t)x.w << 32) | x.z;
      zq += zmod;
      zc += zdiv;
      if (zq >= P) {
        zq -= P;
        ++zc;
      }
    }
  }
  const uint4 mr = qok ? m4 : make_uint4(0u, 0u, 0u, 0u);
  const uint64_t info = qok ? i4 : 0ull;
  const int srow = a.group > 1 ? row / a.group : row;
  const double u_row = greedy        ? 0.0
                       : a.spec_seeds ? pcg_uniform(a.spec_seeds[srow], a.sp_state ? a.sp_state[4 * srow + 1] : a.spec_round,
                                                    (uint32_t)(row - srow * a.group))
                       : a.seeds      ? pcg_uniform(a.seeds[row], a.st_state[2 * row + 1], 0u)
                                      : a.uniforms[row];
  // padding: ranks after everything (past more survivors, cleared once their count is known)
  for (int i = tid; i < kSurvCap / 2 + 8; i += kThreads) ml.s_c[i] = 0ull;
  ml.s_rank[tid] = 0u;
  ml.s_rank[tid + kThreads] = 0u;
  if (tid == 0) ml.m = 0u;
  // plain and member records of part q (within its slots whatever the word holds)
  const uint32_t np = min((uint32_t)info & 0x7FFFu, (uint32_t)kListCap);
  const uint32_t nm = min(((uint32_t)info >> 16) & 0x7FFFu, (uint32_t)kMemSlots);
  const bool pslow = ((uint32_t)info & kPinfoSlow) != 0u;
  const uint32_t bq = (uint32_t)(info >> 32);                       // the part's bound key
  if (qok && sub == 0) ml.p_np[q] = np;
  lds_barrier();  // every part's count (the records stay in flight)
  // records past a part's first 16 Lc plain or G member ones (rarely any)
  // are read again where they are used: f(key, composite, exact value)
  auto for_extra = [&](auto f) __attribute__((always_inline)) {
    for (int j = 16 * Lc + sub; j < (int)np; j += G) {
      const uint64_t rc = load_rec(rq + j);
      const float x = __uint_as_float((uint32_t)rc);
      const uint32_t kx = okey(x);
      f(kx, composite(kx, false, (uint32_t)(rc >> 32)), (double)x);
    }
    for (int j = sub + G; j < (int)nm; j += G) {
      const uint4 m4 = load_rec4(mq + j);
      const uint32_t kx = okey(__uint_as_float(m4.x));
      const double v = member_value(m4);
      f(kx, composite(kx, (double)__uint_as_float(m4.x) != v, m4.y), v);
    }
  };
  // a plain record's value is fkey(key): keep (key, id) pairs
  uint32_t key[kMR], rid[kMR];
  uint32_t kmax = 0u;
  {
    int zq = R % P, zc = R / P;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      // slots 16 zc + 2 l8 and the next, kept below the part's count
      const uint32_t j0 = 16u * (uint32_t)zc + 2u * (uint32_t)l8;
      const uint32_t n = zc < Lc ? ml.p_np[zq] : 0u;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 2 * i + h;
        // okey of every slot, kept where the slot holds a record (no
        // branch); the opaque copy lets the raw record's register go
        const uint32_t kx = okey(__uint_as_float((uint32_t)rec[r]));
        key[r] = kx & (0u - (uint32_t)(j0 + (uint32_t)h < n));
        rid[r] = (uint32_t)(rec[r] >> 32);
        asm volatile("" : "+v"(key[r]));
        kmax = max(kmax, key[r]);
      }
      zq += zmod;
      zc += zdiv;
      if (zq >= P) {
        zq -= P;
        ++zc;
      }
    }
  }
  const uint32_t mkey = (uint32_t)sub < nm ? okey(__uint_as_float(mr.x)) : 0u;
  kmax = max(kmax, mkey);
  for_extra([&](uint32_t kx, uint64_t, double) { kmax = max(kmax, kx); });
  if (greedy) {
    // ---- a greedy row's token is its best record by (value desc, id asc)
    // (the exact doubles: members by their penalized value), the first
    // candidate sample() would rank (tokenizer.js:162); one barrier ----
    bool have = false;
    double bv = 0.0;
    uint32_t bid = 0u;
    auto offer = [&](double v, uint32_t id) __attribute__((always_inline)) {
      if (!have || ranks_before(v, id, bv, bid)) {
        have = true;
        bv = v;
        bid = id;
      }
    };
#pragma unroll
    for (int r = 0; r < kMR; ++r)
      if (key[r] != 0u) offer((double)fkey(key[r]), rid[r]);
    if (mkey != 0u) offer(member_value(mr), mr.y);
    for_extra([&](uint32_t, uint64_t c, double v) { offer(v, comp_id(c)); });
    wave_best(have, bv, bid);
    const bool wslow = __ballot(pslow) != 0ull;
    if (lane == 0) {
      ml.g_v[wave] = bv;
      ml.g_id[wave] = bid;
      ml.g_f[wave] = (have ? 1u : 0u) | (wslow ? 2u : 0u);
    }
    __syncthreads();
    if (wave != 0) return;
    bool h = false, sl = false;
    double v = 0.0;
    uint32_t id = 0u;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const uint32_t f = ml.g_f[w];
      sl = sl || (f & 2u) != 0u;
      if ((f & 1u) && (!h || ranks_before(ml.g_v[w], ml.g_id[w], v, id))) {
        h = true;
        v = ml.g_v[w];
        id = ml.g_id[w];
      }
    }
    const uint32_t tok = h ? id : SAS_NO_TOKEN;
    // the outputs of sample()'s greedy return: no draw, so no candidates
    if (lane == 0) {
      a.out_ids[row] = tok;
      if (a.out_counts) {
        a.out_counts[2 * row] = 0;
        a.out_counts[2 * row + 1] = 0;
      }
      if (a.out_flags) a.out_flags[row] = (sl ? SAS_FLAG_SLOW_SELECT : 0u) | (h ? 0u : SAS_FLAG_EMPTY_ROW);
      if (a.st_state) step_feedback(a, row, tok, false);
    }
    if (a.out_probs) {
      double *op = a.out_probs + (int64_t)row * SAS_MAX_TOP_K;
      op[lane] = 0.0;
      op[lane + 64] = 0.0;
    }
    if (a.out_cand_ids) {
      uint32_t *oc = a.out_cand_ids + (int64_t)row * SAS_MAX_TOP_K;
      oc[lane] = SAS_NO_TOKEN;
      oc[lane + 64] = SAS_NO_TOKEN;
    }
    return;
  }
  // ---- the bound: at least jw lanes of every wave hold a key at or above
  // the wave's result, so k keys reach the smallest; and every part's bound
  // certifies k values of its own ----
  const int jw = (k + kWaves - 1) / kWaves;
  {
    const uint32_t tw = wave_jth_largest_key16(kmax, jw), wb = wave_max_u32(bq);
    const uint32_t ws = __ballot(pslow) ? 1u : 0u;
    if (lane == 0) {
      ml.wred[wave][0] = tw;
      ml.wred[wave][1] = wb;
      ml.wred[wave][2] = ws;
    }
  }
  __syncthreads();
  uint32_t lo = 0xFFFFFFFFu, pb = 0u;
  bool slow = false;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    lo = min(lo, ml.wred[w][0]);
    pb = max(pb, ml.wred[w][1]);
    slow = slow || ml.wred[w][2] != 0u;
  }
  lo = max(max(lo, pb), 1u);  // key 0: no value
  // ---- survivors: composites and exact values of the keys at or above lo,
  // one LDS atomic per wave ----
  {
    uint32_t mine = (mkey >= lo) ? 1u : 0u;
#pragma unroll
    for (int r = 0; r < kMR; ++r) mine += key[r] >= lo ? 1u : 0u;
    static_assert(kMR + 1 < 32, "a lane's survivor count fits 5 bits");
    uint32_t pre = 0u, tot = 0u;
#pragma unroll
    for (int bit = 0; bit < 5; ++bit) {
      const uint64_t bb = __ballot((mine >> bit) & 1u);
      pre += lanes_below(bb) << bit;
      tot += (uint32_t)__popcll(bb) << bit;
    }
    uint32_t base = 0u;
    if (lane == 0 && tot) base = atomicAdd(&ml.m, tot);
    uint32_t d = uni(base) + pre;
#pragma unroll
    for (int r = 0; r < kMR; ++r) {
      const bool kp = key[r] >= lo;
      if (kp && d < (uint32_t)kSurvCap) {
        ml.s_c[d] = composite(key[r], false, rid[r]);
        ml.s_v[d] = (double)fkey(key[r]);
      }
      d += kp ? 1u : 0u;
    }
    if (mkey >= lo && d < (uint32_t)kSurvCap) {
      const double v = member_value(mr);
      ml.s_c[d] = composite(mkey, (double)__uint_as_float(mr.x) != v, mr.y);
      ml.s_v[d] = v;
    }
    for_extra([&](uint32_t kx, uint64_t c, double v) {
      if (kx >= lo) {
        const uint32_t e = atomicAdd(&ml.m, 1u);
        if (e < (uint32_t)kSurvCap) {
          ml.s_c[e] = c;
          ml.s_v[e] = v;
        }
      }
    });
  }
  __syncthreads();
  uint32_t m = ml.m;
  uint32_t flags = slow ? SAS_FLAG_SLOW_SELECT : 0u;
  bool exact = false;  // rank by exact doubles (ties of inexact keys, or the slow path)
  if (m > (uint32_t)kSurvCap) {
    // too many survivors (ties): the exact k-th largest (value, id) over
    // every record, then the records at or above it
    flags |= SAS_FLAG_SLOW_SELECT;
    exact = true;
    auto for_recs = [&](auto f) {
      const int rounds = (kListCap + G - 1) / G;
      for (int i = 0; i < rounds; ++i) {
        const int j = sub + G * i;
        const bool ok = j < (int)np;
        double v = 0.0;
        uint32_t id = 0u;
        if (ok) {
          const uint64_t rc = load_rec(rq + j);
          v = (double)__uint_as_float((uint32_t)rc);
          id = (uint32_t)(rc >> 32);
        }
        f(key96(v, id), ok, v, id);
      }
      const int mrounds = (kMemSlots + G - 1) / G;
      for (int i = 0; i < mrounds; ++i) {
        const int j = sub + G * i;
        const bool ok = j < (int)nm;
        double v = 0.0;
        uint32_t id = 0u;
        if (ok) {
          const uint4 m4 = load_rec4(mq + j);
          v = member_value(m4);
          id = m4.y;
        }
        f(key96(v, id), ok, v, id);
      }
    };
    uint32_t tot = 0u;
    for_recs([&](const Key96 &, bool ok, double, uint32_t) { tot += ok ? 1u : 0u; });
    if (tid == 0) ml.m = 0u;
    __syncthreads();
    atomicAdd(&ml.m, tot);
    __syncthreads();
    const uint32_t need = min(ml.m, (uint32_t)k);
    __syncthreads();
    const Key96 kth = block_select96(
        [&](auto f) { for_recs([&](const Key96 &kx, bool ok, double, uint32_t) { f(kx, ok); }); }, need, s_hist,
        s_sel);
    if (tid == 0) ml.m = 0u;
    __syncthreads();
    for_recs([&](const Key96 &kx, bool ok, double v, uint32_t id) {
      if (ok && key_ge(kx, kth)) {
        const uint32_t e = atomicAdd(&ml.m, 1u);
        if (e < (uint32_t)kSurvCap) {
          ml.s_c[e] = composite(0u, false, id);  // the id; the value is s_v
          ml.s_v[e] = v;
        }
      }
    });
    __syncthreads();
    m = min(ml.m, (uint32_t)kSurvCap);
  }
  if (m > (uint32_t)(kSurvCap / 2)) {  // m is uniform over the block
    if ((uint32_t)tid < 8u && m + (uint32_t)tid < (uint32_t)kSurvCap + 8u) ml.s_c[m + (uint32_t)tid] = 0ull;
    __syncthreads();
  }
  const uint32_t m8 = (m + 7u) & ~7u;
  const uint32_t m64 = (m + 63u) & ~63u;
  const uint32_t groups = m64 >= (uint32_t)kThreads ? 1u : (uint32_t)kThreads / max(m64, 64u);
  const uint32_t per = (uint32_t)kThreads / groups;
  const uint32_t share = ((m8 + groups - 1u) / groups + 7u) & ~7u;
  if (!exact) {
    // ---- rank by composites; the first k + 1 ranks are kept ----
    for (uint32_t i0 = 0; i0 < m; i0 += per) {
      const uint32_t i = i0 + (uint32_t)tid % per;
      const uint32_t g = (uint32_t)tid / per;
      if (i < m) {
        const uint64_t c = ml.s_c[i];
        uint32_t rank = 0u;
        const uint32_t j0 = g * share, j1 = min(j0 + share, m8);
        for (uint32_t j = j0; j < j1; j += 8) {
          uint64_t o8[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) o8[u] = ml.s_c[j + u];
#pragma unroll
          for (int u = 0; u < 8; ++u) rank += o8[u] > c ? 1u : 0u;
        }
        if (groups == 1u) ml.s_rank[i] = rank;
        else atomicAdd(&ml.s_rank[i], rank);
      }
    }
    __syncthreads();
    for (uint32_t i = (uint32_t)tid; i < m; i += kThreads) {
      const uint32_t rank = ml.s_rank[i];
      if (rank <= (uint32_t)k) {
        const uint64_t c = ml.s_c[i];
        ml.t_c[rank] = c;
        ml.t_val[rank] = ml.s_v[i];
        ml.t_id[rank] = comp_id(c);
      }
    }
    __syncthreads();
    // two inexact values of one key within the first k + 1 ranks: their
    // order needs the doubles (every wave reads the same ranks, so the
    // waves agree without another barrier)
    const uint32_t nt = min(m, (uint32_t)k + 1u);
    bool cl = false;
    for (uint32_t t = (uint32_t)lane; t + 1u < nt; t += 64u) {
      const uint64_t x = ml.t_c[t], y = ml.t_c[t + 1u];
      cl = cl || ((x & kInexact) && (y & kInexact) && (x >> 32) == (y >> 32));
    }
    if (__ballot(cl) != 0ull) {
      exact = true;
      flags |= SAS_FLAG_SLOW_SELECT;
      for (uint32_t i = (uint32_t)tid; i < kSurvCap; i += kThreads) ml.s_rank[i] = 0u;
      __syncthreads();
    }
  }
  if (exact) {
    // ---- rank by exact (value, id) ----
    for (uint32_t i0 = 0; i0 < m; i0 += per) {
      const uint32_t i = i0 + (uint32_t)tid % per;
      const uint32_t g = (uint32_t)tid / per;
      if (i < m) {
        const double v = ml.s_v[i];
        const uint32_t id = comp_id(ml.s_c[i]);
        uint32_t rank = 0u;
        const uint32_t j0 = g * share, j1 = min(j0 + share, m);
        for (uint32_t j = j0; j < j1; ++j) rank += before(ml.s_v[j], comp_id(ml.s_c[j]), v, id) ? 1u : 0u;
        if (groups == 1u) ml.s_rank[i] = rank;
        else atomicAdd(&ml.s_rank[i], rank);
      }
    }
    __syncthreads();
    for (uint32_t i = (uint32_t)tid; i < m; i += kThreads) {
      const uint32_t rank = ml.s_rank[i];
      if (rank < (uint32_t)k) {
        ml.t_val[rank] = ml.s_v[i];
        ml.t_id[rank] = comp_id(ml.s_c[i]);
      }
    }
    __syncthreads();
  }
  if (wave != 0) return;
  const int kk = (int)min(m, (uint32_t)k);
  const MergeOut o{a.out_ids, a.out_probs, a.out_cand_ids, a.out_counts, a.out_flags};
  const uint32_t tok = sample_tail(ml, kk, row, p.temperature, p.top_p, u_row, flags, o);
  if (a.st_state && lane == 0) step_feedback(a, row, tok, false);
}

// One block per row, after the parts kernel (stream order makes every record
// visible).  Block b takes the row whose parts ran on its XCD (the parts
// kernel gives each XCD a contiguous run of rows), so the records come from
// that XCD's L2.
template <int kMR>
__global__ __launch_bounds__(kThreads) void sample_merge_kernel(const SampleArgs a) {
  __shared__ MergeLds ml;
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[4];
  int row = blockIdx.x;
  if ((a.rows & 7) == 0 && ((a.rows * a.parts) & 7) == 0) row = (row & 7) * (a.rows >> 3) + (row >> 3);
  const bool stopped = a.st_state && a.st_state[2 * row] != 0u;
  const bool frozen = a.sp_state && a.sp_state[4 * (a.group > 1 ? row / a.group : row)] != 0u;
  if (stopped || frozen) {
    // a stopped row emits its first stop id (kernels.js:184-185), a frozen
    // sequence's verify row no pick; neither has candidates
    const int tid = threadIdx.x;
    const uint32_t tok = stopped && a.stop_ids ? a.stop_ids[4 * row] : SAS_STOP_PAD;
    if (tid == 0) {
      a.out_ids[row] = tok;
      if (a.out_counts) {
        a.out_counts[2 * row] = 0;
        a.out_counts[2 * row + 1] = 0;
      }
      if (a.out_flags) a.out_flags[row] = 0u;
      if (stopped) step_feedback(a, row, tok, true);
    }
    if (tid < SAS_MAX_TOP_K) {
      if (a.out_probs) a.out_probs[(int64_t)row * SAS_MAX_TOP_K + tid] = 0.0;
      if (a.out_cand_ids) a.out_cand_ids[(int64_t)row * SAS_MAX_TOP_K + tid] = SAS_NO_TOKEN;
    }
    return;
  }
  sas_params p = a.params;
  if (a.row_params) p = load_row_params(a.row_params + (a.group > 1 ? row / a.group : row));
  merge_row<kMR>(a, ml, row, p, s_hist, s_sel);
}

// The exact-match cascade (kernels.js:328-339): a = 1, next = pick[0];
// each draft equal to the pick before it that is not a stop id accepts one
// more pick.  With a chained round's state, the commit of acceptSpec
// (kernels.js:340-367) follows, by the same thread.
__global__ __launch_bounds__(kThreads) void spec_cascade_kernel(const uint32_t *picks, const uint32_t *drafts,
                                                                const uint32_t *stop_ids, int seqs, int L,
                                                                int32_t *accepted, uint32_t *next,
                                                                const SpecCommit c) {
  const int s = (int)(blockIdx.x * kThreads + threadIdx.x);
  if (s >= seqs) return;
  const uint32_t *pk = picks + (int64_t)s * (L + 1);
  const uint32_t *dr = drafts + (int64_t)s * L;
  uint32_t st[4] = {SAS_STOP_PAD, SAS_STOP_PAD, SAS_STOP_PAD, SAS_STOP_PAD};
  if (stop_ids)
    for (int i = 0; i < 4; ++i) st[i] = stop_ids[4 * s + i];
  auto is_stop = [&](uint32_t t) { return t == st[0] || t == st[1] || t == st[2] || t == st[3]; };
  uint32_t *sq = c.state ? c.state + 4 * (int64_t)s : nullptr;
  const uint32_t frozen = sq ? sq[0] : 0u;
  int n = 0;
  uint32_t tok = st[0];
  if (!frozen) {
    n = 1;
    while (n <= L) {
      const uint32_t t = pk[n - 1];
      if (t != dr[n - 1] || is_stop(t)) break;
      ++n;
    }
    tok = pk[n - 1];
  }
  accepted[s] = n;
  if (next) next[s] = tok;
  if (!sq) return;
  // ---- the commit: log, position, ring, stop freeze, round ----
  const uint32_t rnd = sq[1];
  if (c.log && rnd < (uint32_t)c.max_rounds) {
    uint32_t *lg = c.log + ((int64_t)s * c.max_rounds + rnd) * (L + 2);
    lg[0] = (uint32_t)n;
    lg[1] = tok;
    for (int j = 0; j < L; ++j) lg[2 + j] = frozen ? 0u : dr[j];
  }
  if (!frozen) {
    sq[2] += (uint32_t)n;
    sq[3] = (uint32_t)n;
    if (c.ring) {
      uint32_t *rg = c.ring + (int64_t)s * (c.ring_len + 1);
      uint32_t cnt = rg[0];
      for (int i = 0; i < n; ++i) {
        const uint32_t t = pk[i];
        if (!is_stop(t)) {
          rg[1 + cnt % (uint32_t)c.ring_len] = t;
          ++cnt;
        }
      }
      rg[0] = cnt;
    }
    if (is_stop(tok)) sq[0] = 1u;
  }
  if (c.next_tokens) c.next_tokens[s] = tok;
  sq[1] = rnd + 1u;
}

hipError_t launch_spec_cascade(const uint32_t *picks, const uint32_t *drafts, const uint32_t *stop_ids, int seqs,
                               int L, int32_t *accepted, uint32_t *next, const SpecCommit &c, hipStream_t stream) {
  if (seqs <= 0) return hipSuccess;
  hipLaunchKernelGGL(spec_cascade_kernel, dim3((unsigned)((seqs + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     stream, picks, drafts, stop_ids, seqs, L, accepted, next, c);
  return hipGetLastError();
}

// ------------------------------------------------------------------ parts --

constexpr int kPassWords = kSpanPass / 32;  // mask / history words of one pass: one per thread
static_assert(kPassWords == kThreads, "one word of 32 ids per thread");
constexpr int kXCap = 256;                  // exact-valued entries of a part: history members, or an exact selection
static_assert(kXCap == kThreads, "one exact entry per thread");
static_assert(kXCap >= SAS_MAX_TOP_K, "an exact part selection fits the exact list");

// x_id bit of an exact-selection entry that is a history member
constexpr uint32_t kXMem = 0x80000000u;

struct PartLds {
  uint2 hent[kHashSlots];       // (id, count) open-addressing hash of the part's history ids
  uint32_t hbits[kPassWords];   // history membership of the pass's ids
  uint32_t comb[kPassWords];    // the pass's ids to select from: allowed, not history, inside the part
  uint32_t hmem[kPassWords];    // the pass's allowed history members
  float4 q_val[kWaves * kQuadCap];     // per-wave candidate lists: float4s with a value at the bound
  uint32_t q_base[kWaves * kQuadCap];  // and the id of their first value
  double x_val[kXCap];          // exact-valued entries: value, id (| kXMem for a member)
  uint32_t x_id[kXCap];
  uint32_t hover;               // some history id did not fit in the hash
};

__device__ __forceinline__ uint32_t hash_slot(uint32_t id) { return (id * 2654435761u) >> 23; }
static_assert(kHashSlots == 512, "hash_slot yields 9 bits");

// A record store: the merge kernel reads it after the launch boundary, on
// the same XCD (rows stay on one XCD), so from L2.
__device__ __forceinline__ void put_rec(uint64_t *p, uint64_t v) { *p = v; }

// kList: the history is bucketed (long histories, kHist only): members may
// ride in the lists (see `lower`).
template <bool kMask, bool kHist, bool kSoftcap, bool kList>
__global__ __launch_bounds__(kThreads, kSoftcap ? 4 : (kMask && !kHist) ? 5 : 6) void sample_parts_kernel(const SampleArgs a) {
  __shared__ PartLds L;
  __shared__ uint32_t s_nw[kWaves];   // records of each wave's list
  __shared__ uint32_t s_qover;        // a wave's list overflowed
  __shared__ uint32_t s_thr[kWaves];
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[4];
  __shared__ uint32_t s_nx;           // exact-valued entries (may pass kXCap: overflow)
  __shared__ uint32_t s_nxk;          // exact-valued entries kept at the end
  __shared__ uint32_t s_nxw;          // exact-valued plain records written
  __shared__ uint32_t s_nmw;          // member records written
  __shared__ uint32_t s_nxm;          // members among an exact selection's entries
  __shared__ uint32_t s_flags;

  const int tid = threadIdx.x, lane = tid & 63, wave = kList ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;  // a scalar where registers are short
  const int P = a.parts;
  int lb = blockIdx.x;
  // XCD-aware order: consecutive dispatches rotate over the 8 XCDs, so give
  // each XCD a contiguous run of rows; a row's parts then share one L2 for
  // the history, the mask words and the records.
  const int nblocks = a.rows * P;
  if ((nblocks & 7) == 0) lb = (lb & 7) * (nblocks >> 3) + (lb >> 3);
  const int row = lb / P;
  const int part = lb - row * P;
  const int vocab = a.vocab;
  const int lo = part * a.span;
  const int nids = min(a.span, vocab - lo);  // > 0

  const int srow = a.group > 1 ? row / a.group : row;  // the row's sequence
  // a row that already sampled a stop id (sas_sample_step), or a row of a
  // frozen sequence (sas_spec_step), reads nothing
  if (a.st_state && a.st_state[2 * row] != 0u) return;
  if (a.sp_state && a.sp_state[4 * srow] != 0u) return;
  sas_params p = a.params;
  if (a.row_params) p = load_row_params(a.row_params + srow);
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const float softcap = kSoftcap ? p.softcap : 0.0f;
  const float *lrow = a.logits + (int64_t)row * a.logits_stride;
  const uint32_t *mrow = kMask ? a.mask + (int64_t)row * a.mask_stride : nullptr;

  // ---- history ids (loaded first: the tables fill while the logits load) ----
  const uint32_t *hid = a.hist_ids;
  int h0 = 0, h1 = 0;
  if (kHist) {
    if (a.hb_offs) {
      // this part's own ids, bucketed by hist_bucket_kernel
      const int32_t *bo = a.hb_offs + (int64_t)srow * (P + 1) + part;
      hid = a.hb_ids;
      h0 = bo[0];
      h1 = bo[1];
    } else if (a.ring) {
      // the row's (or its sequence's) penalty ring: its first
      // min(count, ring_len) slots
      const uint32_t *rg = a.ring + (int64_t)srow * (a.ring_len + 1);
      hid = rg + 1;
      h1 = (int)min(rg[0], (uint32_t)a.ring_len);
    } else {
      // the row's range, clamped into the ids the caller holds and to the
      // largest window
      const int64_t o0 = min(max((int64_t)a.hist_offsets[srow], (int64_t)0), a.hist_count);
      const int64_t o1 = min(max((int64_t)a.hist_offsets[srow + 1], o0), min(a.hist_count, o0 + SAS_MAX_HISTORY));
      h0 = (int)o0;
      h1 = (int)o1;
    }
  }
  const bool has_hist = kHist && h1 > h0;
  uint32_t hpre[kHistPre];
#pragma unroll
  for (int j = 0; j < kHistPre; ++j) {
    const int i = h0 + j * kThreads + tid;
    hpre[j] = has_hist && i < h1 ? hid[i] : kEmpty;
  }

  // ---- loads of one pass --------------------------------------------------------
  // Slot f of thread t holds ids base + 1024 f + 4 t .. + 3.  A float4 is
  // loaded from element max(min(e, vocab - 4), 0): 16 bytes inside the row
  // (rows hold at least 4 floats; the loads need 4-byte alignment only); the
  // float4 that straddles the end of the row is shifted into place later.
  // Slots past the part read the row's first line (never used).  Thread t
  // also loads the mask word of ids base + 32 t .. + 31.
  const int last_word = ((vocab + 31) >> 5) - 1;
  const int npass = (nids + kSpanPass - 1) / kSpanPass;
  // the row's last float4 is partial: in the part that ends the row
  const bool straddle = lo + nids == vocab && (vocab & 3) != 0;
  float4 v[kSlots];
  uint32_t mword = ~0u;
  auto load_pass = [&](int base) __attribute__((always_inline)) {
    const int nrem = lo + nids - base;
    // the mask word first: the pass's id words are built from it while the
    // logits still arrive, and the slots are then taken in load order
    if (kMask) mword = mrow[min((base >> 5) + tid, last_word)];
#pragma unroll
    for (int f = 0; f < kSlots; ++f) {
      const int e = base + 1024 * f + 4 * tid;
      const bool in = 1024 * f < nrem;
      const int ec = in ? max(min(e, vocab - 4), 0) : 0;
      const f32x4u t = __builtin_nontemporal_load(reinterpret_cast<const f32x4u *>(lrow + ec));
      v[f] = make_float4(t.x, t.y, t.z, t.w);
    }
  };
  load_pass(lo);

  // ---- the part's history: (id, count) hash, the first pass's bitmap -----------
  if (tid < kWaves) s_nw[tid] = 0u;
  if (tid == 0) s_qover = 0u;
  if (tid == 0) {
    s_nx = 0u;
    s_nxk = 0u;
    s_nxw = 0u;
    s_nmw = 0u;
    s_nxm = 0u;
    s_flags = 0u;
  }
  auto set_bit = [&](uint32_t id, int base) __attribute__((always_inline)) {
    const uint32_t off = id - (uint32_t)base;
    if (off < (uint32_t)min(kSpanPass, lo + nids - base)) atomicOr(&L.hbits[off >> 5], 1u << (off & 31u));
  };
  if (has_hist) {
    for (int s = tid; s < kHashSlots; s += kThreads) {
      L.hent[s] = make_uint2(kEmpty, 0u);
    }
    L.hbits[tid] = 0u;
    if (tid == 0) L.hover = 0u;
    lds_barrier();
    auto insert = [&](uint32_t id) __attribute__((always_inline)) {
      const uint32_t off = id - (uint32_t)lo;
      if (off >= (uint32_t)nids) return;
      set_bit(id, lo);
      uint32_t sl = hash_slot(id);
      int probe = 0;
      for (; probe < kHashSlots; ++probe) {
        const uint32_t old = atomicCAS(&L.hent[sl].x, kEmpty, id);
        if (old == kEmpty || old == id) {
          atomicAdd(&L.hent[sl].y, 1u);
          break;
        }
        sl = (sl + 1u) & (uint32_t)(kHashSlots - 1);
      }
      if (probe == kHashSlots) L.hover = 1u;
    };
#pragma unroll
    for (int j = 0; j < kHistPre; ++j) insert(hpre[j]);
    // longer histories: rounds of 8 ids per thread, all 8 loads in flight
    for (int i0 = h0 + kHistPre * kThreads + tid; i0 < h1; i0 += 8 * kThreads) {
      uint32_t hb8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * kThreads;
        hb8[j] = i < h1 ? hid[i] : kEmpty;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) insert(hb8[j]);
    }
    lds_barrier();
  }
  // occurrences of a history member of the part
  auto hcount = [&](uint32_t id) __attribute__((always_inline)) -> uint32_t {
    uint32_t sl = hash_slot(id);
    for (int probe = 0; probe < kHashSlots; ++probe) {
      const uint2 e = L.hent[sl];
      const uint32_t kk = e.x;
      if (kk == id) return e.y;
      if (kk == kEmpty) break;
      sl = (sl + 1u) & (uint32_t)(kHashSlots - 1);
    }
    uint32_t c = 0u;
    if (L.hover)
      for (int i = h0; i < h1; ++i) c += hid[i] == id ? 1u : 0u;
    return c;
  };
  // ---- passes: values, the bound, the lists ---------------------------------
  // Long (bucketed) histories, whose members are many, with penalties that
  // only lower values (repetition >= 1, frequency >= 0, presence >= 0;
  // rounding keeps this): a member whose raw value is below the bound stays
  // below it, so members ride in the lists with their raw values and only
  // those that reach the bound are penalized.  Otherwise every allowed
  // member goes to the exact list from the slot loop.
  const bool lower = kList && p.repetition_penalty >= 1.0 && p.frequency_penalty >= 0.0 && p.presence_penalty >= 0.0;
  const uint32_t sh = 4u * (uint32_t)(tid & 7);
  uint32_t tkey = 0u;  // the part's bound (okey image; 0 = none)
  uint32_t n_q = 0u;   // float4 entries of this wave's list (may pass kQuadCap: overflow)
  // Softcap rows of one pass, members in the exact list: the values stay raw
  // until the cut.  The cap is non-decreasing, so the raw bound certifies k
  // capped values at or above its cap, and a capped value can reach that only
  // within a margin below the raw bound (the margin spans the cap's f32
  // plateaus there): the lists take the values down to the margin, and only
  // they are capped.  Where the cap flattens (a bound beyond 5 cap) the part
  // caps every value and bounds the capped values instead.
  const bool raw_cap = kSoftcap && !kList && softcap > 0.0f && npass == 1;
  bool capped = !raw_cap;  // the registers and lists hold capped values (or the row has no cap)
  auto run_pass = [&](int base) __attribute__((always_inline)) {
    // the history members of this thread's word
    const uint32_t hb = has_hist ? L.hbits[tid] : 0u;
    // ids to select from, 32 per word: allowed, not history, inside the part
    {
      const int rem = lo + nids - (base + 32 * tid);
      uint32_t cw = rem >= 32 ? ~0u : rem > 0 ? (1u << rem) - 1u : 0u;
      L.comb[tid] = cw & mword & ~hb;
      L.hmem[tid] = cw & mword & hb;
    }
    lds_barrier();
    float m = qnan();
#pragma unroll
    for (int f = 0; f < kSlots; ++f) {
      const uint32_t nib = L.comb[32 * f + (tid >> 3)] >> sh;
      if (straddle) {
        // loaded from vocab - 4: shift the values into place (slots past
        // the row hold no allowed bit; rows of fewer than 4 ids are padded)
        const int e = base + 1024 * f + 4 * tid;
        const int s2 = e - max(min(e, vocab - 4), 0);
        if (s2 > 0 && e < vocab) {
          const float ty = v[f].y, tz = v[f].z, tw = v[f].w;
          v[f].x = s2 == 1 ? ty : s2 == 2 ? tz : tw;
          v[f].y = s2 == 1 ? tz : tw;
          v[f].z = tw;
        }
      }
      if (kSoftcap && softcap > 0.0f && !raw_cap) {
        v[f].x = softcap_f32(v[f].x, softcap);
        v[f].y = softcap_f32(v[f].y, softcap);
        v[f].z = softcap_f32(v[f].z, softcap);
        v[f].w = softcap_f32(v[f].w, softcap);
      }
      uint32_t hn = 0u;
      if (has_hist) {
        // allowed history members of this float4: their values (in the
        // registers now) and ids go to the exact list, penalized after the
        // passes (unless penalties only lower values)
        hn = (L.hmem[32 * f + (tid >> 3)] >> sh) & 0xFu;
        if (!(kList && lower) && __ballot(hn != 0u)) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if ((hn >> j) & 1u) {
              const uint32_t d = atomicAdd(&s_nx, 1u);
              if (d < (uint32_t)kXCap) {
                L.x_val[d] = (double)(j == 0 ? v[f].x : j == 1 ? v[f].y : j == 2 ? v[f].z : v[f].w);
                L.x_id[d] = (uint32_t)(base + 1024 * f + 4 * tid + j);
              }
            }
          }
        }
      }
      // bit j of the nibble -> all ones or zero, then one bit-field insert
      // keeps the value or puts a quiet NaN in its place
      auto keep = [&](float x, uint32_t nb, uint32_t bit) {
        const uint32_t msk = (uint32_t)__builtin_amdgcn_sbfe((int)nb, bit, 1u);  // 0 or ~0
        return __uint_as_float((msk & __float_as_uint(x)) | (~msk & 0x7FC00000u));
      };
      // the bound from the plain values; the lists also take the members'
      // raw values when penalties only lower them
      if constexpr (kList) {
        m = fmaxf(m, fmaxf(fmaxf(keep(v[f].x, nib, 0u), keep(v[f].y, nib, 1u)),
                           fmaxf(keep(v[f].z, nib, 2u), keep(v[f].w, nib, 3u))));
        const uint32_t an = lower ? nib | hn : nib;
        v[f].x = keep(v[f].x, an, 0u);
        v[f].y = keep(v[f].y, an, 1u);
        v[f].z = keep(v[f].z, an, 2u);
        v[f].w = keep(v[f].w, an, 3u);
      } else {
        v[f].x = keep(v[f].x, nib, 0u);
        v[f].y = keep(v[f].y, nib, 1u);
        v[f].z = keep(v[f].z, nib, 2u);
        v[f].w = keep(v[f].w, nib, 3u);
        m = fmaxf(m, fmaxf(fmaxf(v[f].x, v[f].y), fmaxf(v[f].z, v[f].w)));
      }
    }
    // the bound: at least j lane maxima of each of the first nw waves reach
    // its own result, so at least nw j >= k values of the part reach the
    // smallest.  A pass of 1,024 ids or more puts ids in every lane (four
    // waves at rank ceil(k / 4)); a shorter one (the row's last part) leaves
    // the last waves' lanes without ids, and those waves take no part (their
    // results are left out of the minimum, which spills no register).
    const int rem = lo + nids - base;
    const BoundRank br = rem >= 4 * 64 * kWaves ? BoundRank{kWaves, (k + kWaves - 1) / kWaves} : bound_rank(rem, 4, k);
    const uint32_t tw = wave_rank_key(okey(m), br.j);
    if (lane == 0) s_thr[wave] = tw;
    lds_barrier();
    {
      uint32_t t = s_thr[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w)
        if (w < br.nw) t = min(t, s_thr[w]);
      tkey = max(tkey, t);
    }
    // keys at or below okey(-inf) (0 or truncated) admit every valid value
    float tf = tkey > 0x007FFFFFu ? fkey(tkey) : -__builtin_inff();
    if (kSoftcap && !capped) {
      if (tf > -__builtin_inff() && !(fabsf(tf) <= 5.0f * softcap)) {
        // the cap flattens at the bound: cap every value, bound the capped ones
        float m2 = qnan();
#pragma unroll
        for (int f = 0; f < kSlots; ++f) {
          v[f].x = softcap_f32(v[f].x, softcap);
          v[f].y = softcap_f32(v[f].y, softcap);
          v[f].z = softcap_f32(v[f].z, softcap);
          v[f].w = softcap_f32(v[f].w, softcap);
          m2 = fmaxf(m2, fmaxf(fmaxf(v[f].x, v[f].y), fmaxf(v[f].z, v[f].w)));
        }
        const uint32_t tw2 = wave_rank_key(okey(m2), br.j);
        lds_barrier();  // every wave has read the raw results
        if (lane == 0) s_thr[wave] = tw2;
        lds_barrier();
        uint32_t t = s_thr[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w)
          if (w < br.nw) t = min(t, s_thr[w]);
        tkey = t;
        tf = tkey > 0x007FFFFFu ? fkey(tkey) : -__builtin_inff();
        capped = true;
      } else if (tf > -__builtin_inff()) {
        // values whose cap can equal the bound's: the cap rises by 3 ulp of
        // tanh (near 1) over cap 2^-24 / sech^2(b / cap), plus the rounding
        // of x / cap; the margin is five times that
        const float ch = coshf(tf / softcap);
        tf -= softcap * 0x1p-20f * ch * ch + 1e-5f * (1.0f + fabsf(tf));
      }
    }
    // whole float4s with a value at or above the bound go to the list (one
    // ballot per float4); their values are cut to the final bound at the end
#pragma unroll
    for (int f = 0; f < kSlots; ++f) {
      const float m4 = fmaxf(fmaxf(v[f].x, v[f].y), fmaxf(v[f].z, v[f].w));
      const bool pass = m4 >= tf;
      const uint64_t bb = __ballot(pass);
      if (bb) {
        const uint32_t cnt = (uint32_t)__popcll(bb);
        if (n_q + cnt <= (uint32_t)kQuadCap && pass) {
          const uint32_t d = (uint32_t)wave * kQuadCap + n_q + lanes_below(bb);
          L.q_val[d] = v[f];
          L.q_base[d] = (uint32_t)(base + 1024 * f + 4 * tid);
        }
        n_q += cnt;
      }
    }
  };
  run_pass(lo);
  for (int c = 1; c < npass; ++c) {
    // parts of more than one pass (vocabularies beyond kMaxParts passes):
    // the next pass's loads, then its history bitmap from the row's history
    const int base = lo + c * kSpanPass;
    __syncthreads();
    load_pass(base);
    if (has_hist) {
      L.hbits[tid] = 0u;
      lds_barrier();
      for (int i = h0 + tid; i < h1; i += kThreads) set_bit(hid[i], base);
    }
    lds_barrier();
    run_pass(base);
  }
  // this wave's list, cut to the final bound: entries lane and lane + 64 of
  // each lane (the second only in a wave whose list passed 64 entries,
  // which takes top-k above 64), each lane's values at or above the bound,
  // and their places among the wave's records
  // (raw values: the listed ones capped here, the bound's cap the final bound)
  const float tfr = tkey > 0x007FFFFFu ? fkey(tkey) : -__builtin_inff();
  const float tff = kSoftcap && !capped ? softcap_f32(tfr, softcap) : tfr;
  const uint32_t qat = (uint32_t)wave * kQuadCap + (uint32_t)lane;
  auto cut = [&](uint32_t e, float4 &q, uint32_t &qid) __attribute__((always_inline)) -> uint32_t {
    const bool qin = (uint32_t)lane + e < n_q && n_q <= (uint32_t)kQuadCap;
    q = qin ? L.q_val[qat + e] : make_float4(qnan(), qnan(), qnan(), qnan());
    if (kSoftcap && !capped)
      q = make_float4(softcap_f32(q.x, softcap), softcap_f32(q.y, softcap), softcap_f32(q.z, softcap),
                      softcap_f32(q.w, softcap));
    qid = L.q_base[qat + e];
    uint32_t pm = (q.x >= tff ? 1u : 0u) | (q.y >= tff ? 2u : 0u) | (q.z >= tff ? 4u : 0u) | (q.w >= tff ? 8u : 0u);
    if (kList && has_hist && lower) {
      // members that reached the bound with their raw values: penalized here,
      // and written as member records when they still reach it
      uint4 *mrow4 = a.mrec + ((int64_t)row * P + part) * kMemSlots;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if ((pm >> c) & 1u) {
          const uint32_t id = qid + (uint32_t)c;
          // one pass: the part's history bitmap is still in LDS
          const uint32_t off = id - (uint32_t)lo;
          const bool member = npass == 1 ? ((L.hbits[off >> 5] >> (off & 31u)) & 1u) != 0u : hcount(id) != 0u;
          if (member) {
            pm &= ~(1u << c);
            const double pen = penalize((double)(c == 0 ? q.x : c == 1 ? q.y : c == 2 ? q.z : q.w), hcount(id), p);
            if (pen >= (double)tff) {
              atomicAdd(&s_nxk, 1u);
              const uint32_t d = atomicAdd(&s_nmw, 1u);
              if (d < (uint32_t)kMemSlots) {
                uint64_t *w = reinterpret_cast<uint64_t *>(mrow4 + d);
                put_rec(w, (uint64_t)__float_as_uint(rd_f32(pen)) | ((uint64_t)id << 32));
                put_rec(w + 1, (uint64_t)__double_as_longlong(pen));
              } else {
                s_qover = 1u;  // more than the part's member slots: the exact selection
              }
            }
          }
        }
      }
    }
    return pm;
  };
  float4 q, q1 = make_float4(qnan(), qnan(), qnan(), qnan());
  uint32_t qid, qid1 = 0u;
  uint32_t pm = cut(0u, q, qid);
  if (n_q > 64u) pm |= cut(64u, q1, qid1) << 4;  // uniform over the wave
  const uint32_t qcnt = (uint32_t)__popc(pm);  // at most 4, or 8 with a second entry
  uint32_t qpre = 0u, qtot = 0u;
#pragma unroll
  for (int bit = 0; bit < 3; ++bit) {
    const uint64_t bb = __ballot((qcnt >> bit) & 1u);
    qpre += lanes_below(bb) << bit;
    qtot += (uint32_t)__popcll(bb) << bit;
  }
  if (n_q > 64u) {
    const uint64_t bb = __ballot((qcnt >> 3) & 1u);
    qpre += lanes_below(bb) << 3;
    qtot += (uint32_t)__popcll(bb) << 3;
  }
  if (lane == 0) {
    s_nw[wave] = qtot;
    if (n_q > (uint32_t)kQuadCap) s_qover = 1u;
  }
  // the history members' exact values, kept at or above the final bound
  // (NaN ones never are).  The list is complete: every wave recorded its
  // members before the last pass's bound barrier.  A member's record holds
  // the round-down key of its penalized value and the double itself.
  bool xw = false;   // this thread writes exact entry tid
  bool xmem = true;  // ... as a member record
  uint32_t xid = 0u;
  double xv = 0.0;
  if (has_hist && (uint32_t)tid < min(s_nx, (uint32_t)kXCap)) {
    xid = L.x_id[tid];
    // members recorded raw are capped first
    const double xr = L.x_val[tid];
    xv = penalize(kSoftcap && raw_cap ? (double)softcap_f32((float)xr, softcap) : xr, hcount(xid), p);
    xw = xv >= (double)tff;
    if (xw) atomicAdd(&s_nxk, 1u);
  }
  __syncthreads();
  uint32_t nw[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) nw[w] = s_nw[w];
  uint32_t nx = s_nxk;
  uint32_t nxm = nx;  // exact entries that are members (all of them unless the slow selection ran)
  const bool overflow = s_qover != 0u || s_nx > (uint32_t)kXCap || nw[0] + nw[1] + nw[2] + nw[3] + nx > (uint32_t)kListCap;
  if (overflow) {
    // more values at or above the bound than the lists hold (ties): the
    // part's exact top k by a radix select over (value, id) keys, every
    // value read again from memory
    const int rounds = (nids + kThreads - 1) / kThreads;
    auto for_elems = [&](auto f) {
      for (int i = 0; i < rounds; ++i) {
        const uint32_t off = (uint32_t)(i * kThreads + tid);
        const uint32_t id = (uint32_t)lo + off;
        bool ok = off < (uint32_t)nids;
        uint32_t cnt = 0u;
        float x = 0.0f;
        double val = 0.0;
        if (ok) {
          const uint32_t mw = kMask ? mrow[id >> 5] : ~0u;
          x = lrow[id];
          cnt = has_hist ? hcount(id) : 0u;
          ok = !kMask || ((mw >> (id & 31u)) & 1u);
          if (kSoftcap && softcap > 0.0f) x = softcap_f32(x, softcap);
          ok = ok && x == x;
          val = cnt ? penalize((double)x, cnt, p) : (double)x;
          ok = ok && val == val;
        }
        f(key96(val, id), ok, val, id | (cnt ? kXMem : 0u), x, cnt);
      }
    };
    uint32_t nval = 0u;
    for_elems([&](const Key96 &, bool ok, double, uint32_t, float, uint32_t) { nval += ok ? 1u : 0u; });
    if (tid == 0) s_sel[3] = 0u;
    __syncthreads();
    atomicAdd(&s_sel[3], nval);
    __syncthreads();
    const uint32_t need = min(s_sel[3], (uint32_t)k);
    __syncthreads();
    if (tid < kWaves) s_nw[tid] = 0u;
    if (tid == 0) {
      s_nx = 0u;
      s_nmw = 0u;  // member records the cut may have written are rewritten
      s_flags = SAS_FLAG_SLOW_SELECT;
    }
    if (need > 0u) {
      const Key96 kth = block_select96(
          [&](auto f) {
            for_elems([&](const Key96 &kx, bool ok, double, uint32_t, float, uint32_t) { f(kx, ok); });
          },
          need, s_hist, s_sel);
      // exactly need <= kXCap entries
      for_elems([&](const Key96 &kx, bool ok, double val, uint32_t idm, float x, uint32_t cnt) {
        if (ok && key_ge(kx, kth)) {
          const uint32_t d = atomicAdd(&s_nx, 1u);
          L.x_val[d] = val;
          L.x_id[d] = idm;
          if (cnt) atomicAdd(&s_nxm, 1u);
        }
      });
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) nw[w] = s_nw[w];
    nx = s_nx;
    xw = (uint32_t)tid < nx;
    pm = 0u;
    nxm = s_nxm;
    if (xw) {
      // an exact entry: a plain value, or a member with its penalized double
      xv = L.x_val[tid];
      const uint32_t xi = L.x_id[tid];
      xmem = (xi & kXMem) != 0u;
      xid = xi & ~kXMem;
    }
  }

  // ---- records: each wave's values after those of the waves before it, then
  // the exact plain values, in the part's own kListCap slots; the members in
  // the part's own member slots.  The plain records are staged in LDS (over
  // the lists, read above) and then stored as whole lines, 16 bytes per
  // thread: stored where they were made, each store instruction touched
  // many partly written lines.
  uint32_t off = 0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) off += w < wave ? nw[w] : 0u;
  const uint32_t nplain = nw[0] + nw[1] + nw[2] + nw[3];
  uint64_t *rrow = a.rec + ((int64_t)row * P + part) * kListCap;
  uint4 *mrow4 = a.mrec + ((int64_t)row * P + part) * kMemSlots;
  uint64_t *stg = reinterpret_cast<uint64_t *>(L.q_val);
  static_assert(sizeof(L.q_val) + sizeof(L.q_base) >= kListCap * sizeof(uint64_t), "the lists hold a part's records");
  {
    uint32_t j = off + qpre;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if ((pm >> c) & 1u) {
        const float x = c == 0 ? q.x : c == 1 ? q.y : c == 2 ? q.z : q.w;
        stg[j] = (uint64_t)__float_as_uint(x) | ((uint64_t)(qid + (uint32_t)c) << 32);
        ++j;
      }
    }
    if (n_q > 64u) {  // the second entries, uniform over the wave
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if ((pm >> (c + 4)) & 1u) {
          const float x = c == 0 ? q1.x : c == 1 ? q1.y : c == 2 ? q1.z : q1.w;
          stg[j] = (uint64_t)__float_as_uint(x) | ((uint64_t)(qid1 + (uint32_t)c) << 32);
          ++j;
        }
      }
    }
  }
  if (xw) {
    if (xmem) {
      const uint32_t j = atomicAdd(&s_nmw, 1u);
      uint64_t *d = reinterpret_cast<uint64_t *>(mrow4 + j);
      put_rec(d, (uint64_t)__float_as_uint(rd_f32(xv)) | ((uint64_t)xid << 32));
      put_rec(d + 1, (uint64_t)__double_as_longlong(xv));
    } else {
      const uint32_t j = nplain + atomicAdd(&s_nxw, 1u);
      stg[j] = (uint64_t)__float_as_uint((float)xv) | ((uint64_t)xid << 32);
    }
  }
  lds_barrier();
  {
    // nplain + the exact plain values <= kListCap (else the exact
    // selection ran); the slot past an odd count is written too (unread)
    const uint32_t ntot = nplain + nx - nxm;
    for (uint32_t e = 2u * (uint32_t)tid; e < ntot; e += 2u * (uint32_t)kThreads)
      *reinterpret_cast<uint4 *>(rrow + e) = *reinterpret_cast<const uint4 *>(stg + e);
  }
  // the part's counts, bound and slow-selection flag
  if (tid == 0)
    put_rec(a.pinfo + (int64_t)row * pinfo_stride(P) + part,
            (uint64_t)((nplain + nx - nxm) | (nxm << 16) | (s_flags ? kPinfoSlow : 0u)) |
                ((uint64_t)(kSoftcap && !capped ? (tkey > 0x007FFFFFu ? okey(tff) : 0u) : tkey) << 32));
}

// Parts per row and ids per part: one pass per part (8192 ids), more
// passes only when the vocabulary needs more than kMaxParts parts; shorter
// parts (multiples of 1024 ids) when the grid would hold fewer than
// min_blocks blocks.
void choose_parts(int rows, int vocab, int min_blocks, int *parts, int *span) {
  long long s = kSpanPass;
  if ((long long)vocab > (long long)kMaxParts * kSpanPass) {
    const long long per = ((long long)vocab + kMaxParts - 1) / kMaxParts;
    s = (per + kSpanPass - 1) / kSpanPass * kSpanPass;
  }
  long long pc = ((long long)vocab + s - 1) / s;
  if (s == kSpanPass && rows > 0 && (long long)rows * pc < min_blocks) {
    long long want = ((long long)min_blocks + rows - 1) / rows;
    if (want > kMaxParts) want = kMaxParts;
    long long s2 = ((long long)vocab + want - 1) / want;
    s2 = (s2 + 1023) / 1024 * 1024;
    if (s2 < 1024) s2 = 1024;
    if (s2 < s) s = s2;
    pc = ((long long)vocab + s - 1) / s;
  }
  *span = (int)s;
  *parts = (int)pc;
}

size_t sample_rec_bytes(int rows, int parts) {
  return (size_t)rows * parts * kListCap * 16 + (size_t)rows * pinfo_stride(parts) * 8;
}

__global__ __launch_bounds__(kThreads) void pad_rows_kernel(const float *src, int64_t stride, int vocab, int rows,
                                                           float *dst) {
  const int i = (int)(blockIdx.x * kThreads + threadIdx.x);
  if (i >= rows * 4) return;
  const int r = i >> 2, j = i & 3;
  dst[i] = j < vocab ? src[(int64_t)r * stride + j] : __builtin_nanf("");
}

hipError_t launch_pad_rows(const float *src, int64_t stride, int vocab, int rows, float *dst, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((rows * 4 + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(pad_rows_kernel, dim3(blocks), dim3(kThreads), 0, stream, src, stride, vocab, rows, dst);
  return hipGetLastError();
}

// Buckets each history row's ids by part (one block per history row): a
// counting sort over the row's parts, ids past the vocabulary dropped.  The
// buckets take the row's own index range of hb_ids (its CSR range, or
// ring_len slots of a ring row).  Each round holds kBucketPer ids per
// thread, all loaded before any is counted.
constexpr int kBucketPer = 4;
constexpr int kBucketThreads = 1024;

__global__ __launch_bounds__(kBucketThreads) void hist_bucket_kernel(const SampleArgs a) {
  __shared__ uint32_t s_cnt[kMaxParts + 1];
  __shared__ uint32_t s_cur[kMaxParts + 1];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int P = a.parts;
  const uint32_t *ids;
  int64_t o0, o1, base;
  if (a.ring) {
    const uint32_t *rg = a.ring + (int64_t)h * (a.ring_len + 1);
    ids = rg + 1;
    o0 = 0;
    o1 = min(rg[0], (uint32_t)a.ring_len);
    base = (int64_t)h * a.ring_len;
  } else {
    ids = a.hist_ids;
    o0 = min(max((int64_t)a.hist_offsets[h], (int64_t)0), a.hist_count);
    o1 = min(max((int64_t)a.hist_offsets[h + 1], o0), min(a.hist_count, o0 + SAS_MAX_HISTORY));
    base = o0;
  }
  // spans are multiples of 1024, in practice powers of two: a shift
  const uint32_t span = (uint32_t)a.span, vocab = (uint32_t)a.vocab;
  const bool pow2 = (span & (span - 1u)) == 0u;
  const uint32_t shift = (uint32_t)__builtin_ctz(span);
  auto part_of = [&](uint32_t id) -> uint32_t {
    return id < vocab ? (pow2 ? id >> shift : id / span) : (uint32_t)P;
  };
  // one round of kBucketPer ids per thread (the first round's ids stay in
  // registers for the scatter)
  uint32_t v[kBucketPer];
  auto load_round = [&](int64_t r0) {
#pragma unroll
    for (int j = 0; j < kBucketPer; ++j) {
      const int64_t i = r0 + (int64_t)j * kBucketThreads + tid;
      v[j] = i < o1 ? ids[i] : 0xFFFFFFFFu;
    }
  };
  constexpr int64_t kRound = (int64_t)kBucketPer * kBucketThreads;
  for (int q = tid; q <= P; q += kBucketThreads) s_cnt[q] = 0u;
  load_round(o0);
  __syncthreads();
  for (int64_t r0 = o0; r0 < o1; r0 += kRound) {
    if (r0 != o0) load_round(r0);
#pragma unroll
    for (int j = 0; j < kBucketPer; ++j)
      if (r0 + (int64_t)j * kBucketThreads + tid < o1) atomicAdd(&s_cnt[part_of(v[j])], 1u);
  }
  __syncthreads();
  // offsets: an exclusive scan of the counts by the first wave
  if (tid < 64) {
    const int lane = tid;
    uint32_t c0 = lane < P ? s_cnt[lane] : 0u;
    uint32_t c1 = lane + 64 < P ? s_cnt[lane + 64] : 0u;
    uint32_t x0 = c0, x1 = c1;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t y0 = __shfl_up(x0, d), y1 = __shfl_up(x1, d);
      if (lane >= d) {
        x0 += y0;
        x1 += y1;
      }
    }
    const uint32_t tot0 = __shfl(x0, 63);
    x1 += tot0;
    // exclusive: inclusive minus own count
    const uint32_t e0 = x0 - c0, e1 = x1 - c1;
    int32_t *bo = a.hb_offs + (int64_t)h * (P + 1);
    if (lane <= P) {
      s_cur[lane] = e0;
      bo[lane] = (int32_t)(base + e0);
    }
    if (lane + 64 <= P) {
      s_cur[lane + 64] = e1;
      bo[lane + 64] = (int32_t)(base + e1);
    }
  }
  __syncthreads();
  // v still holds the first round when there was only one
  const bool reload = o1 - o0 > kRound;
  for (int64_t r0 = o0; r0 < o1; r0 += kRound) {
    if (reload) load_round(r0);
#pragma unroll
    for (int j = 0; j < kBucketPer; ++j) {
      const uint32_t q = part_of(v[j]);
      if (r0 + (int64_t)j * kBucketThreads + tid < o1 && q < (uint32_t)P) a.hb_ids[base + atomicAdd(&s_cur[q], 1u)] = v[j];
    }
  }
}

template <bool kMask, bool kHist, bool kSoftcap>
static void launch_kernel(const SampleArgs &a, hipStream_t stream) {
  // the list mode pays only with the many members of long (bucketed)
  // histories; short ones keep collecting members in the slot loop
  if (kHist && a.hb_offs)
    hipLaunchKernelGGL((sample_parts_kernel<kMask, kHist, kSoftcap, kHist>), dim3((unsigned)(a.rows * a.parts)),
                       dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((sample_parts_kernel<kMask, kHist, kSoftcap, false>), dim3((unsigned)(a.rows * a.parts)),
                       dim3(kThreads), 0, stream, a);
}

hipError_t launch_sample(const SampleArgs &a, bool softcap, hipStream_t stream) {
  if (a.hb_offs) {
    const int hrows = a.group > 1 ? a.rows / a.group : a.rows;
    hipLaunchKernelGGL(hist_bucket_kernel, dim3((unsigned)hrows), dim3(kBucketThreads), 0, stream, a);
  }
  switch ((a.mask ? 4 : 0) | (a.hist_ids || a.ring ? 2 : 0) | (softcap ? 1 : 0)) {
    case 0: launch_kernel<false, false, false>(a, stream); break;
    case 1: launch_kernel<false, false, true>(a, stream); break;
    case 2: launch_kernel<false, true, false>(a, stream); break;
    case 3: launch_kernel<false, true, true>(a, stream); break;
    case 4: launch_kernel<true, false, false>(a, stream); break;
    case 5: launch_kernel<true, false, true>(a, stream); break;
    case 6: launch_kernel<true, true, false>(a, stream); break;
    default: launch_kernel<true, true, true>(a, stream); break;
  }
  return launch_merge(a, stream);
}

// Record slots per thread for the merge: a part emits about k to 2 k
// records (its bound certifies k of its own values; ties and the bound's
// slack add more), so the first 2 k + 8 slots hold nearly every part's
// records.  Per-row parameters are unknown here: the most slots.
int merge_slots(const SampleArgs &a) {
  if (a.row_params) return kMRMax;
  const bool greedy = !(a.params.temperature > 0.0);
  const int k = greedy ? 1 : std::min(std::max(a.params.top_k, 1), SAS_MAX_TOP_K);
  const int G = kThreads / std::max(a.parts, 1);
  const int want = (2 * k + 8 + G - 1) / G;
  return want <= 4 ? 4 : want <= 8 ? 8 : kMRMax;
}

hipError_t launch_merge(const SampleArgs &a, hipStream_t stream) {
  if (a.parts < 1 || a.parts > kMaxParts) return hipErrorInvalidValue;  // the merge's count table
  switch (merge_slots(a)) {
    case 4: hipLaunchKernelGGL(sample_merge_kernel<4>, dim3((unsigned)a.rows), dim3(kThreads), 0, stream, a); break;
    case 8: hipLaunchKernelGGL(sample_merge_kernel<8>, dim3((unsigned)a.rows), dim3(kThreads), 0, stream, a); break;
    default:
      hipLaunchKernelGGL(sample_merge_kernel<kMRMax>, dim3((unsigned)a.rows), dim3(kThreads), 0, stream, a);
      break;
  }
  return hipGetLastError();
}

}  // namespace sas

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
//      exact penalized double values;
//   5. the lists are written as records, unordered: {fp32 key, id}, where
//      the key of a penalized value is its double rounded toward -inf and a
//      flag marks keys below their exact value (kept beside the record).
// The merge kernel: one block per row.
//   6. one round of loads brings the parts' counts and bounds and the
//      records (slot-major: record j of every part back to back, so every
//      lane holds records of its own part);
//   7. the bound again, over the records: the largest part bound, and the
//      j-th largest of each wave's lane maxima, the smallest over the waves;
//   8. the records at or above it (about k + 20) are ranked exactly by
//      (value desc, id asc) through 64-bit (key, flag, ~id) composites;
//   9. the reference's sample() tail in double precision.
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
constexpr int kQuadCap = 64;                         // float4 entries of one wave's candidate list
static_assert(kQuadCap == 64, "a wave's list is one entry per lane at the end");
constexpr int kSurvCap = 512;                        // survivors the merge ranks
constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr uint32_t kXFlag = 0x80000000u;             // record id flag: the exact value lies above the key
constexpr uint32_t kIdBits = 0x7FFFFFFFu;

// The value of the wave's first active lane (wave-uniform values).
__device__ __forceinline__ uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// One row's parameters from the per-row array: read as 32-bit words by
// nontemporal loads, so that the compiler never forms a pointer that may
// point into the kernel's by-value arguments (which would copy them to
// scratch memory).
__device__ __forceinline__ sas_params load_row_params(const sas_params *q) {
  static_assert(sizeof(sas_params) % 4 == 0, "whole words");
  union {
    sas_params p;
    uint32_t w[sizeof(sas_params) / 4];
  } u;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(q);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(sas_params) / 4); ++i) u.w[i] = __builtin_nontemporal_load(src + i);
  return u.p;
}

// Lane i's double on every lane (i wave-uniform).
__device__ __forceinline__ double bcast(double x, int i) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, i);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), i);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Barrier over the block's LDS accesses alone: it waits for this wave's LDS
// operations but not for its global loads, so loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// (va, ia) ranks before (vb, ib): value desc, then id asc (tokenizer.js:160
// stable sort of an id-ascending list; kernels.js:1433, 1439 tie rule).
__device__ __forceinline__ bool before(double va, uint32_t ia, double vb, uint32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// Record composite: larger = ranks first.  An unflagged value equals its key;
// a flagged one lies strictly between its key and the next float, so it
// ranks after every larger key and before the unflagged values of its own
// key.  Only two flagged records of one key need their exact values.
__device__ __forceinline__ uint64_t composite(uint32_t keybits, uint32_t idf) {
  return ((uint64_t)okey(__uint_as_float(keybits)) << 32) | (idf & kXFlag) | (kIdBits - (idf & kIdBits));
}
__device__ __forceinline__ uint32_t comp_id(uint64_t c) { return kIdBits - ((uint32_t)c & kIdBits); }

// 96-bit key of (value, id), larger = ranks first: an order-preserving
// image of the double (-0 and +0 one value), then the id reversed.
struct Key96 {
  uint32_t w[3];
};
__device__ __forceinline__ Key96 key96(double v, uint32_t id) {
  v = v + 0.0;  // -0 -> +0
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint64_t d = (b >> 63) ? ~b : (b | 0x8000000000000000ull);
  return Key96{{(uint32_t)(d >> 32), (uint32_t)d, ~id}};
}
__device__ __forceinline__ bool key_ge(const Key96 &a, const Key96 &b) {
  if (a.w[0] != b.w[0]) return a.w[0] > b.w[0];
  if (a.w[1] != b.w[1]) return a.w[1] > b.w[1];
  return a.w[2] >= b.w[2];
}

// The need-th largest (1-based) of the block's 96-bit keys; need must not
// exceed their number.  for_keys(f) calls f(key, valid) the same number of
// times on every lane of a wave.  Radix passes of 8 bits from the top, each
// an LDS histogram; ends early once the bin holding the need-th key is
// taken whole (the bits below stay zero: exactly `need` keys reach the
// result).  LDS: hist[256], sel[3].  Block-wide; every thread returns it.
template <typename ForKeys>
__device__ __forceinline__ Key96 block_select96(ForKeys for_keys, uint32_t need, uint32_t *hist, uint32_t *sel) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  Key96 res{{0u, 0u, 0u}};
  for (int pass = 0; pass < 12; ++pass) {
    const int w = pass >> 2;
    const int sh = 24 - 8 * (pass & 3);
    const uint32_t hm = sh == 24 ? 0u : ~0u << (sh + 8);
    for (int i = tid; i < 256; i += (int)blockDim.x) hist[i] = 0u;
    __syncthreads();
    // word w of a key by selects (no indexed registers)
    auto word = [&](const Key96 &x) { return w == 0 ? x.w[0] : w == 1 ? x.w[1] : x.w[2]; };
    const uint32_t rw = word(res);
    for_keys([&](const Key96 &key, bool valid) {
      const uint32_t kw = word(key);
      bool match = valid && (kw & hm) == (rw & hm);
      if (w > 0) match = match && key.w[0] == res.w[0];
      if (w > 1) match = match && key.w[1] == res.w[1];
      const uint32_t d = (kw >> sh) & 0xFFu;
      const uint64_t act = __ballot(match);
      if (act) {
        // one atomic per wave when every matching lane has the same digit
        const int first = __builtin_ctzll(act);
        const uint32_t d0 = (uint32_t)__builtin_amdgcn_readlane((int)d, first);
        if (__ballot(match && d != d0) == 0) {
          if (lane == first) atomicAdd(&hist[d0], (uint32_t)__popcll(act));
        } else if (match) {
          atomicAdd(&hist[d], 1u);
        }
      }
    });
    __syncthreads();
    if (wave == 0) {
      const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1], c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
      const uint32_t s4 = c0 + c1 + c2 + c3;
      uint32_t suf = s4;  // keys in the bins of this lane and above
#pragma unroll
      for (int s = 1; s < 64; s <<= 1) {
        const uint32_t y = (uint32_t)__shfl_down((int)suf, s, 64);
        if (lane + s < 64) suf += y;
      }
      const uint32_t above = suf - s4;
      if (above < need && need <= suf) {
        uint32_t acc = above, d, cb;
        if (acc + c3 >= need) {
          d = 3; cb = c3;
        } else if ((acc += c3) + c2 >= need) {
          d = 2; cb = c2;
        } else if ((acc += c2) + c1 >= need) {
          d = 1; cb = c1;
        } else {
          acc += c1; d = 0; cb = c0;
        }
        sel[0] = 4u * (uint32_t)lane + d;
        sel[1] = need - acc;
        sel[2] = cb;
      }
    }
    __syncthreads();
    const uint32_t d = sel[0], cb = sel[2];
    need = sel[1];
    if (w == 0) res.w[0] |= d << sh;
    else if (w == 1) res.w[1] |= d << sh;
    else res.w[2] |= d << sh;
    __syncthreads();
    if (cb == need) break;
  }
  return res;
}

// ----------------------------------------------------------------- merge --

constexpr int kMThreads = 256;   // threads of a merge block (more measured no faster)
constexpr int kMWaves = kMThreads / 64;

struct MergeLds {
  uint32_t cnt[kMaxParts];          // records of each part
  uint32_t thr[kMWaves];
  uint64_t m_c[kSurvCap + 8];       // survivors: composites (zero-padded to a multiple of 8)
  uint32_t m_g[kSurvCap];           // their record index in the row
  double m_v[kSurvCap + 8];         // exact values (exact ranking only; sentinel padded)
  uint32_t m_id[kSurvCap + 8];
  double t_val[SAS_MAX_TOP_K + 1];  // the ranked top k and the one after
  uint32_t t_id[SAS_MAX_TOP_K + 1];
  uint64_t t_c[SAS_MAX_TOP_K + 1];
  double t_p[SAS_MAX_TOP_K];        // exp weights (zero past k)
  double t_q[SAS_MAX_TOP_K];        // weights / sum
  uint32_t m, clash, rflags;
};

struct MergeOut {
  uint32_t *ids;
  double *probs;
  uint32_t *cand_ids;
  int32_t *counts;
  uint32_t *flags;
};

// The reference's sample() tail (tokenizer.js:161-177) in double precision
// over the ranked top kk in ml.t_val / ml.t_id, by wave 0.  The weights and
// divisions run across lanes (lane i holds candidates i and i + 64) and are
// staged in LDS; each running sum is one chain in the reference's
// left-to-right order, run alike by every lane on operands read 8 at a time
// (broadcast reads), its 8 partial values kept in registers for the tests.
__device__ void sample_tail(MergeLds &ml, int kk, int row, double temperature, double top_p, double u_row,
                            uint32_t flags, MergeOut o) {
  const int lane = threadIdx.x & 63;
  const bool greedy = !(temperature > 0.0);
  const bool draw = !greedy && kk > 0;
  uint32_t out_id = SAS_NO_TOKEN;
  int cut = 0;
  double q_a = 0.0, q_b = 0.0;
  if (kk == 0) {
    flags |= SAS_FLAG_EMPTY_ROW;
  } else if (greedy) {
    out_id = ml.t_id[0];
  } else {
    const double T = temperature;
    const double v0 = ml.t_val[0];
    const bool two = kk > 64;
    // p_i = exp((v_i - v_0) / T); x / 1 is x, so the division only runs
    // for other temperatures.  Weights past kk are zero.
    double p_a = 0.0, p_b = 0.0;
    if (lane < kk) {
      double d = ml.t_val[lane] - v0;
      if (T != 1.0) d = d / T;
      p_a = fd_exp(d);
    }
    if (two && lane + 64 < kk) {
      double d = ml.t_val[lane + 64] - v0;
      if (T != 1.0) d = d / T;
      p_b = fd_exp(d);
    }
    ml.t_p[lane] = p_a;
    ml.t_p[lane + 64] = p_b;
    __builtin_amdgcn_wave_barrier();
    const int nb = (kk + 7) >> 3;  // batches of 8 (zeros past kk leave every sum as it is)
    // the sum of the weights, left to right
    // (each chain reads the next batch of 8 while it adds the current one)
    double run = 0.0;
    double x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = ml.t_p[u];
    for (int b = 0; b < nb; ++b) {
      const int bn = b + 1 < nb ? b + 1 : b;
      double y[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) y[u] = ml.t_p[8 * bn + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) run = run + x[u];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = y[u];
    }
    const double sum = run;
    q_a = p_a / sum;
    if (two) q_b = p_b / sum;
    ml.t_q[lane] = q_a;
    ml.t_q[lane + 64] = q_b;
    __builtin_amdgcn_wave_barrier();
    // top-p cut: the first i with p_0/sum + ... + p_i/sum >= top_p, with
    // the running weight sum beside it (the draw's mass at the cut)
    double cum = 0.0, pre = 0.0, sub = 0.0;
    bool te = false;
    cut = kk;
    double xp[8], xq[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      xp[u] = ml.t_p[u];
      xq[u] = ml.t_q[u];
    }
    for (int b = 0; b < nb; ++b) {
      const int bn = b + 1 < nb ? b + 1 : b;
      double yp[8], yq[8], pr[8];
      uint32_t hit = 0u, edge = 0u;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        yp[u] = ml.t_p[8 * bn + u];
        yq[u] = ml.t_q[8 * bn + u];
      }
      double cv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        pre = pre + xp[u];
        cum = cum + xq[u];
        pr[u] = pre;
        cv[u] = cum;
      }
      // the running mass never decreases (zero weights past kk leave it as
      // it is): a batch whose last value lies 1e-6 or more below top_p holds
      // neither the cut nor an edge
      if (cum - top_p > -1e-6) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          hit |= (cv[u] >= top_p ? 1u : 0u) << u;
          edge |= (fabs(cv[u] - top_p) < 1e-6 ? 1u : 0u) << u;
        }
      }
      const int left = kk - 8 * b;  // candidates of this batch
      const uint32_t live = left >= 8 ? 0xFFu : (1u << left) - 1u;
      hit = uni(hit) & live;
      edge = uni(edge) & live;
      if (hit) {
        const int f = __builtin_ctz(hit);
        cut = 8 * b + f + 1;
        te |= (edge & ((2u << f) - 1u)) != 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (u == f) sub = pr[u];
        break;
      }
      te |= edge != 0u;
      sub = pre;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        xp[u] = yp[u];
        xq[u] = yq[u];
      }
    }
    // r = U * (p_0 + ... + p_{cut-1}); the first i at which
    // r - p_0 - ... - p_i <= 0 is drawn, else the last of the cut
    double r = u_row * sub;
    int pick = cut - 1;
    bool de = false;
    const int nc = (cut + 7) >> 3;
#pragma unroll
    for (int u = 0; u < 8; ++u) xp[u] = ml.t_p[u];
    for (int b = 0; b < nc; ++b) {
      const int bn = b + 1 < nc ? b + 1 : b;
      double yp[8];
      uint32_t hit = 0u, edge = 0u;
#pragma unroll
      for (int u = 0; u < 8; ++u) yp[u] = ml.t_p[8 * bn + u];
      double rv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        r = r - xp[u];
        rv[u] = r;
      }
      // the residual never increases: a batch whose last value lies above
      // 1e-12 * sub holds neither the draw nor an edge
      if (r <= 1e-12 * sub) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          hit |= (rv[u] <= 0.0 ? 1u : 0u) << u;
          edge |= (fabs(rv[u]) <= 1e-12 * sub ? 1u : 0u) << u;
        }
      }
      const int left = cut - 8 * b;
      const uint32_t live = left >= 8 ? 0xFFu : (1u << left) - 1u;
      hit = uni(hit) & live;
      edge = uni(edge) & live;
      if (hit) {
        const int f = __builtin_ctz(hit);
        pick = 8 * b + f;
        de |= (edge & ((2u << f) - 1u)) != 0u;
        break;
      }
      de |= edge != 0u;
#pragma unroll
      for (int u = 0; u < 8; ++u) xp[u] = yp[u];
    }
    if (te) flags |= SAS_FLAG_TOPP_EDGE;
    if (de) flags |= SAS_FLAG_DRAW_EDGE;
    out_id = ml.t_id[pick];
  }
  const uint32_t id_a = lane < kk ? ml.t_id[lane] : SAS_NO_TOKEN;
  const uint32_t id_b = lane + 64 < kk ? ml.t_id[lane + 64] : SAS_NO_TOKEN;
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
    oc[lane] = lane < np ? id_a : SAS_NO_TOKEN;
    oc[lane + 64] = lane + 64 < np ? id_b : SAS_NO_TOKEN;
  }
}

// Rank of (v, id) among n entries of LDS arrays (value desc, id asc); the
// arrays hold sentinels (-inf, kEmpty) up to a multiple of 8 past n.
__device__ __forceinline__ uint32_t rank_exact(const double *vals, const uint32_t *ids, uint32_t n8, double v,
                                               uint32_t id) {
  uint32_t rank = 0u;
  for (uint32_t j = 0; j < n8; j += 8) {
    double vv[8];
    uint32_t ii[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      vv[u] = vals[j + u];
      ii[u] = ids[j + u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) rank += before(vv[u], ii[u], v, id) ? 1u : 0u;
  }
  return rank;
}

constexpr int kMergeR = 20;  // record slots per thread in the first round

template <bool kRowParams>
__global__ __launch_bounds__(kMThreads) void sample_merge_kernel(const SampleArgs a) {
  __shared__ MergeLds ml;
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the XCD that ran the row's parts (the parts kernel gives each XCD a
  // contiguous run of rows): the row's records may still be in its L2
  int row = blockIdx.x;
  if ((a.rows & 7) == 0 && ((a.rows * a.parts) & 7) == 0) row = (row & 7) * (a.rows >> 3) + (row >> 3);
  const int P = a.parts;
  const uint64_t *pin = a.pinfo + (int64_t)row * P;
  // record j of part q: index j * P + q of the row
  const uint64_t *rrow = a.rec + (int64_t)row * kListCap * P;
  const int NS = kListCap * P;

  // ---- round 1: records and counts first, every load in flight, then the ---
  // row's parameters, uniform and flags (their scalar loads are not waited
  // for before the records are requested)
  uint64_t rec[kMergeR];
#pragma unroll
  for (int r = 0; r < kMergeR; ++r) {
    const int g = tid + kMThreads * r;
    rec[r] = g < NS ? __builtin_nontemporal_load(rrow + g) : 0ull;
  }
  const uint64_t my_info = lane < P ? pin[lane] : 0ull;
  sas_params p;
  if constexpr (kRowParams) p = load_row_params(a.row_params + row);
  else p = a.params;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const double u_row = greedy ? 0.0 : a.uniforms[row];
  uint32_t *ctl = a.ctl + (int64_t)row * kCtlStride;
  const double *xrow = a.xval + (int64_t)row * kListCap * P;
  // the parts' flags: read and then reset by thread 0 alone
  const uint32_t rflags_v = tid == 0 ? ctl[kCtlFlags] : 0u;
  const uint32_t my_cnt = (uint32_t)my_info;
  if (wave == 0 && lane < P) ml.cnt[lane] = my_cnt;
  const uint32_t total = wave_sum_u32(my_cnt);
  const uint32_t maxc = wave_max_u32(my_cnt);
  const uint32_t pbound = wave_max_u32((uint32_t)(my_info >> 32));
  if (tid == 0) {
    ml.m = 0u;
    ml.clash = 0u;
    ml.rflags = rflags_v;
  }
  __syncthreads();
  const uint32_t rflags = ml.rflags;
  if (tid == 0) {
    // read by every part of this launch: reset for the next one
    ctl[kCtlFlags] = 0u;
  }
  // slot g = tid + kMThreads r is record s of part q: (s, q) stepped without division
  const int s0 = tid / P, q0 = tid - s0 * P;
  const int ds = kMThreads / P, dq = kMThreads - ds * P;
  // ---- the bound ----------------------------------------------------------------
  uint32_t key[kMergeR];
  uint32_t kmax = 0u;
  {
    // every slot's part count read at once (no branch, one LDS wait), then
    // the keys of the slots that hold a record
    uint32_t cq[kMergeR];
    int ss[kMergeR];
    if (dq == 0) {
      // the part count divides the block: every slot of a thread is its one
      // part's, at records s0, s0 + ds, ...
      const uint32_t c0 = ml.cnt[q0];
#pragma unroll
      for (int r = 0; r < kMergeR; ++r) {
        ss[r] = s0 + r * ds;
        cq[r] = c0;
      }
    } else {
      int s = s0, q = q0;
#pragma unroll
      for (int r = 0; r < kMergeR; ++r) {
        ss[r] = s;
        cq[r] = ml.cnt[q];
        s += ds;
        q += dq;
        const bool wrap = q >= P;
        q = wrap ? q - P : q;
        s = wrap ? s + 1 : s;
      }
    }
#pragma unroll
    for (int r = 0; r < kMergeR; ++r) {
      const bool ok = (tid + kMThreads * r < NS) & ((uint32_t)ss[r] < cq[r]);
      const uint32_t kx = okey(__uint_as_float((uint32_t)rec[r]));
      key[r] = ok ? kx : 0u;
      kmax = max(kmax, key[r]);
    }
  }
  const int jw = (k + kMWaves - 1) / kMWaves;
  const uint32_t tw = wave_jth_largest_key16(kmax, jw);
  if (lane == 0) ml.thr[wave] = tw;
  __syncthreads();
  uint32_t tmin = 0xFFFFFFFFu;
#pragma unroll
  for (int w = 0; w < kMWaves; ++w) tmin = min(tmin, ml.thr[w]);
  const uint32_t bnd = max(pbound, max(tmin, 1u));
  // ---- survivors: composites and record indices ----------------------------------
  auto keep_one = [&](uint32_t kk, uint64_t rc, int g) {
    const bool keep = kk >= bnd;
    const uint64_t bb = __ballot(keep);
    if (bb) {
      uint32_t base = 0u;
      if (lane == 0) base = atomicAdd(&ml.m, (uint32_t)__popcll(bb));
      base = uni(base);
      if (keep) {
        const uint32_t d = base + lanes_below(bb);
        if (d < (uint32_t)kSurvCap) {
          ml.m_c[d] = composite((uint32_t)rc, (uint32_t)(rc >> 32));
          ml.m_g[d] = (uint32_t)g;
        }
      }
    }
  };
  {
    // first round: each lane's count, a ballot prefix over the count bits,
    // one LDS atomic per wave, then the lane's own records
    uint32_t mine = 0u;
#pragma unroll
    for (int r = 0; r < kMergeR; ++r) mine += key[r] >= bnd ? 1u : 0u;
    static_assert(kMergeR < 32, "a lane's survivor count fits 5 bits");
    uint32_t pre = 0u, tot = 0u;
#pragma unroll
    for (int bit = 0; bit < 5; ++bit) {
      const uint64_t bb = __ballot((mine >> bit) & 1u);
      pre += lanes_below(bb) << bit;
      tot += (uint32_t)__popcll(bb) << bit;
    }
    if (tot) {
      uint32_t base = 0u;
      if (lane == 0) base = atomicAdd(&ml.m, tot);
      uint32_t d = uni(base) + pre;
#pragma unroll
      for (int r = 0; r < kMergeR; ++r) {
        if (key[r] >= bnd) {
          if (d < (uint32_t)kSurvCap) {
            ml.m_c[d] = composite((uint32_t)rec[r], (uint32_t)(rec[r] >> 32));
            ml.m_g[d] = (uint32_t)(tid + kMThreads * r);
          }
          ++d;
        }
      }
    }
  }
  // records past the first round (parts with many candidates)
  const int gend = min(NS, (int)maxc * P);
  for (int g0 = kMThreads * kMergeR; g0 < gend; g0 += kMThreads) {
    const int g = g0 + tid;
    const int s = g / P;
    const bool ok = g < gend && (uint32_t)s < ml.cnt[g - s * P];
    const uint64_t rc = ok ? rrow[g] : 0ull;
    keep_one(ok ? okey(__uint_as_float((uint32_t)rc)) : 0u, rc, g);
  }
  __syncthreads();
  uint32_t m = ml.m;
  uint32_t flags = rflags;
  bool exact = false;  // rank by exact doubles (m_v, m_id) instead of composites
  if (m > (uint32_t)kSurvCap) {
    // too many survivors (ties): exact select over every record
    flags |= SAS_FLAG_SLOW_SELECT;
    exact = true;
    const int rounds = (gend + kMThreads - 1) / kMThreads;
    auto for_recs = [&](auto f) {
      for (int i = 0; i < rounds; ++i) {
        const int g = i * kMThreads + tid;
        const int s = g / P;
        const bool ok = g < gend && (uint32_t)s < ml.cnt[g - s * P];
        double v = 0.0;
        uint32_t id = 0u;
        if (ok) {
          const uint64_t rc = rrow[g];
          id = (uint32_t)(rc >> 32) & kIdBits;
          v = ((uint32_t)(rc >> 32) & kXFlag) ? xrow[g] : (double)__uint_as_float((uint32_t)rc);
        }
        f(key96(v, id), ok, v, id);
      }
    };
    const uint32_t need = min(total, (uint32_t)k);
    const Key96 kth = block_select96(
        [&](auto f) { for_recs([&](const Key96 &kx, bool ok, double, uint32_t) { f(kx, ok); }); }, need, s_hist,
        s_sel);
    if (tid == 0) ml.m = 0u;
    __syncthreads();
    for_recs([&](const Key96 &kx, bool ok, double v, uint32_t id) {
      if (ok && key_ge(kx, kth)) {
        const uint32_t d = atomicAdd(&ml.m, 1u);
        ml.m_v[d] = v;
        ml.m_id[d] = id;
      }
    });
    __syncthreads();
    m = ml.m;
  }
  const uint32_t m8 = (m + 7u) & ~7u;
  if (!exact) {
    // ---- rank by composites; the first k + 1 ranks are kept ----------------------
    if ((uint32_t)tid < m8 - m) ml.m_c[m + tid] = 0ull;
    __syncthreads();
    // up to 8 threads per survivor (as m allows), each counting a share of
    // the others; the shares are summed across the group's lanes
    int lg = 0;
    while (lg < 3 && (uint32_t)(kMThreads >> (lg + 1)) >= m) ++lg;
    const uint32_t gsz = 1u << lg;
    const uint32_t share = ((m8 >> lg) + 7u) & ~7u;  // entries per thread, a multiple of 8
    for (uint32_t i0 = 0; i0 < m; i0 += (uint32_t)(kMThreads >> lg)) {
      const uint32_t i = i0 + ((uint32_t)tid >> lg);
      const uint32_t part = (uint32_t)tid & (gsz - 1u);
      const uint64_t c = i < m ? ml.m_c[i] : ~0ull;
      // a flagged record's exact value: loaded while the rank is counted
      const bool lead = i < m && part == 0u;
      const double xv = lead && (c & kXFlag) ? xrow[ml.m_g[i]] : (double)fkey((uint32_t)(c >> 32));
      uint32_t rank = 0u;
      const uint32_t j0 = part * share, j1 = min(j0 + share, m8);
#pragma unroll 4
      for (uint32_t j = j0; j < j1; j += 8) {
        uint64_t o[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) o[u] = ml.m_c[j + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) rank += o[u] > c ? 1u : 0u;
      }
      if (lg >= 1) rank += (uint32_t)__shfl_xor((int)rank, 1, 64);
      if (lg >= 2) rank += (uint32_t)__shfl_xor((int)rank, 2, 64);
      if (lg >= 3) rank += (uint32_t)__shfl_xor((int)rank, 4, 64);
      if (lead && rank <= (uint32_t)k) {
        ml.t_c[rank] = c;
        ml.t_id[rank] = comp_id(c);
        ml.t_val[rank] = xv;
      }
    }
    __syncthreads();
    // Two flagged records of one key rank next to each other, by id: if
    // such a pair lies within the first k + 1 ranks, rank by exact values.
    const uint32_t nt = min(m, (uint32_t)k + 1u);
    if ((uint32_t)tid + 1u < nt) {
      const uint64_t x = ml.t_c[tid], y = ml.t_c[tid + 1];
      if ((x & kXFlag) && (y & kXFlag) && (x >> 32) == (y >> 32)) ml.clash = 1u;
    }
    __syncthreads();
    if (ml.clash) {
      exact = true;
      flags |= SAS_FLAG_SLOW_SELECT;
      for (uint32_t i = (uint32_t)tid; i < m; i += kMThreads) {
        const uint64_t c = ml.m_c[i];
        ml.m_id[i] = comp_id(c);
        ml.m_v[i] = (c & kXFlag) ? xrow[ml.m_g[i]] : (double)fkey((uint32_t)(c >> 32));
      }
    }
  }
  if (exact) {
    if ((uint32_t)tid < m8 - m) {
      ml.m_v[m + tid] = -__builtin_inf();
      ml.m_id[m + tid] = kEmpty;
    }
    __syncthreads();
    for (uint32_t i = (uint32_t)tid; i < m; i += kMThreads) {
      const double v = ml.m_v[i];
      const uint32_t id = ml.m_id[i];
      const uint32_t rank = rank_exact(ml.m_v, ml.m_id, m8, v, id);
      if (rank < (uint32_t)k) {
        ml.t_val[rank] = v;
        ml.t_id[rank] = id;
      }
    }
    __syncthreads();
  }
  if (wave != 0) return;
  const int kk = (int)min(m, (uint32_t)k);
  const MergeOut o{a.out_ids, a.out_probs, a.out_cand_ids, a.out_counts, a.out_flags};
  sample_tail(ml, kk, row, p.temperature, p.top_p, u_row, flags, o);
}

// ------------------------------------------------------------------ parts --

constexpr int kPassWords = kSpanPass / 32;  // mask / history words of one pass: one per thread
static_assert(kPassWords == kThreads, "one word of 32 ids per thread");
constexpr int kXCap = 256;                  // exact-valued entries of a part: history members, or an exact selection
static_assert(kXCap == kThreads, "one exact entry per thread");
static_assert(kXCap >= SAS_MAX_TOP_K, "an exact part selection fits the exact list");

struct PartLds {
  uint32_t hkey[kHashSlots];    // (id, count) open-addressing hash of the part's history ids
  uint32_t hcnt[kHashSlots];
  uint32_t hbits[kPassWords];   // history membership of the pass's ids
  uint32_t comb[kPassWords];    // the pass's ids to select from: allowed, not history, inside the part
  uint32_t hmem[kPassWords];    // the pass's allowed history members
  float4 q_val[kWaves * kQuadCap];     // per-wave candidate lists: float4s with a value at the bound
  uint32_t q_base[kWaves * kQuadCap];  // and the id of their first value
  double x_val[kXCap];          // exact-valued entries: value, id
  uint32_t x_id[kXCap];
  uint32_t hover;               // some history id did not fit in the hash
};

__device__ __forceinline__ uint32_t hash_slot(uint32_t id) { return (id * 2654435761u) >> 23; }
static_assert(kHashSlots == 512, "hash_slot yields 9 bits");

template <bool kMask, bool kHist, bool kSoftcap>
__global__ __launch_bounds__(kThreads, kSoftcap ? 4 : (kMask && !kHist) ? 5 : 6) void sample_parts_kernel(const SampleArgs a) {
  __shared__ PartLds L;
  __shared__ uint32_t s_nw[kWaves];   // records of each wave's list
  __shared__ uint32_t s_qover;        // a wave's list overflowed
  __shared__ uint32_t s_thr[kWaves];
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[4];
  __shared__ uint32_t s_nx;           // exact-valued entries (may pass kXCap: overflow)
  __shared__ uint32_t s_nxk;          // exact-valued entries kept at the end
  __shared__ uint32_t s_nxw;          // exact-valued records written
  __shared__ uint32_t s_flags;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  sas_params p = a.params;
  if (a.row_params) p = load_row_params(a.row_params + row);
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const float softcap = kSoftcap ? p.softcap : 0.0f;
  const float *lrow = a.logits + (int64_t)row * a.logits_stride;
  const uint32_t *mrow = kMask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
  uint32_t *ctl = a.ctl + (int64_t)row * kCtlStride;

  // ---- history ids (loaded first: the tables fill while the logits load) ----
  int h0 = 0, h1 = 0;
  if (kHist) {
    // the row's range, clamped into the ids the caller holds and to the
    // largest window
    const int64_t o0 = min(max((int64_t)a.hist_offsets[row], (int64_t)0), a.hist_count);
    const int64_t o1 = min(max((int64_t)a.hist_offsets[row + 1], o0), min(a.hist_count, o0 + SAS_MAX_HISTORY));
    h0 = (int)o0;
    h1 = (int)o1;
  }
  const bool has_hist = kHist && h1 > h0;
  uint32_t hpre[kHistPre];
#pragma unroll
  for (int j = 0; j < kHistPre; ++j) {
    const int i = h0 + j * kThreads + tid;
    hpre[j] = has_hist && i < h1 ? a.hist_ids[i] : kEmpty;
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
#pragma unroll
    for (int f = 0; f < kSlots; ++f) {
      const int e = base + 1024 * f + 4 * tid;
      const bool in = 1024 * f < nrem;
      const int ec = in ? max(min(e, vocab - 4), 0) : 0;
      const f32x4u t = __builtin_nontemporal_load(reinterpret_cast<const f32x4u *>(lrow + ec));
      v[f] = make_float4(t.x, t.y, t.z, t.w);
    }
    if (kMask) mword = mrow[min((base >> 5) + tid, last_word)];
  };
  load_pass(lo);

  // ---- the part's history: (id, count) hash, the first pass's bitmap -----------
  if (tid < kWaves) s_nw[tid] = 0u;
  if (tid == 0) s_qover = 0u;
  if (tid == 0) {
    s_nx = 0u;
    s_nxk = 0u;
    s_nxw = 0u;
    s_flags = 0u;
  }
  auto set_bit = [&](uint32_t id, int base) __attribute__((always_inline)) {
    const uint32_t off = id - (uint32_t)base;
    if (off < (uint32_t)min(kSpanPass, lo + nids - base)) atomicOr(&L.hbits[off >> 5], 1u << (off & 31u));
  };
  if (has_hist) {
    for (int s = tid; s < kHashSlots; s += kThreads) {
      L.hkey[s] = kEmpty;
      L.hcnt[s] = 0u;
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
        const uint32_t old = atomicCAS(&L.hkey[sl], kEmpty, id);
        if (old == kEmpty || old == id) {
          atomicAdd(&L.hcnt[sl], 1u);
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
        hb8[j] = i < h1 ? a.hist_ids[i] : kEmpty;
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
      const uint32_t kk = L.hkey[sl];
      if (kk == id) return L.hcnt[sl];
      if (kk == kEmpty) break;
      sl = (sl + 1u) & (uint32_t)(kHashSlots - 1);
    }
    uint32_t c = 0u;
    if (L.hover)
      for (int i = h0; i < h1; ++i) c += a.hist_ids[i] == id ? 1u : 0u;
    return c;
  };
  // exact value of a history member: CTRL repetition, then OpenAI frequency
  // and presence (presence alone is tokenizer.js:157)
  auto hist_value = [&](uint32_t id, float x, uint32_t mw, double &val) __attribute__((always_inline)) -> bool {
    if (kMask && !((mw >> (id & 31u)) & 1u)) return false;
    if (kSoftcap && softcap > 0.0f) x = softcap_f32(x, softcap);
    if (x != x) return false;
    val = penalize((double)x, hcount(id), p);
    return val == val;
  };

  // ---- passes: values, the bound, the lists ---------------------------------
  const int jw = (k + kWaves - 1) / kWaves;  // per-wave rank of the bound
  const uint32_t sh = 4u * (uint32_t)(tid & 7);
  uint32_t tkey = 0u;  // the part's bound (okey image; 0 = none)
  uint32_t n_q = 0u;   // float4 entries of this wave's list (may pass kQuadCap: overflow)
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
      if (kSoftcap && softcap > 0.0f) {
        v[f].x = softcap_f32(v[f].x, softcap);
        v[f].y = softcap_f32(v[f].y, softcap);
        v[f].z = softcap_f32(v[f].z, softcap);
        v[f].w = softcap_f32(v[f].w, softcap);
      }
      if (has_hist) {
        // allowed history members of this float4: their values (in the
        // registers now) and ids go to the exact list, penalized after the
        // passes
        const uint32_t hn = (L.hmem[32 * f + (tid >> 3)] >> sh) & 0xFu;
        if (__ballot(hn != 0u)) {
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
      auto keep = [&](float x, uint32_t bit) {
        const uint32_t msk = (uint32_t)__builtin_amdgcn_sbfe((int)nib, bit, 1u);  // 0 or ~0
        return __uint_as_float((msk & __float_as_uint(x)) | (~msk & 0x7FC00000u));
      };
      v[f].x = keep(v[f].x, 0u);
      v[f].y = keep(v[f].y, 1u);
      v[f].z = keep(v[f].z, 2u);
      v[f].w = keep(v[f].w, 3u);
      m = fmaxf(m, fmaxf(fmaxf(v[f].x, v[f].y), fmaxf(v[f].z, v[f].w)));
    }
    // the bound: at least jw lane maxima of every wave reach its own
    // result, so at least 4 jw >= k values of the part reach the smallest
    const uint32_t tw = wave_jth_largest_key16(okey(m), jw);
    if (lane == 0) s_thr[wave] = tw;
    lds_barrier();
    tkey = max(tkey, min(min(s_thr[0], s_thr[1]), min(s_thr[2], s_thr[3])));
    // keys at or below okey(-inf) (0 or truncated) admit every valid value
    const float tf = tkey > 0x007FFFFFu ? fkey(tkey) : -__builtin_inff();
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
      for (int i = h0 + tid; i < h1; i += kThreads) set_bit(a.hist_ids[i], base);
    }
    lds_barrier();
    run_pass(base);
  }
  // this wave's list, one float4 per lane, cut to the final bound: each
  // lane's values at or above it, and their places among the wave's records
  const float tff = tkey > 0x007FFFFFu ? fkey(tkey) : -__builtin_inff();
  const uint32_t qat = (uint32_t)wave * kQuadCap + (uint32_t)lane;
  const bool qin = (uint32_t)lane < n_q && n_q <= (uint32_t)kQuadCap;
  const float4 q = qin ? L.q_val[qat] : make_float4(qnan(), qnan(), qnan(), qnan());
  const uint32_t qid = L.q_base[qat];
  uint32_t pm = (q.x >= tff ? 1u : 0u) | (q.y >= tff ? 2u : 0u) | (q.z >= tff ? 4u : 0u) | (q.w >= tff ? 8u : 0u);
  const uint32_t qcnt = (uint32_t)__popc(pm);
  uint32_t qpre = 0u, qtot = 0u;
#pragma unroll
  for (int bit = 0; bit < 3; ++bit) {
    const uint64_t bb = __ballot((qcnt >> bit) & 1u);
    qpre += lanes_below(bb) << bit;
    qtot += (uint32_t)__popcll(bb) << bit;
  }
  if (lane == 0) {
    s_nw[wave] = qtot;
    if (n_q > (uint32_t)kQuadCap) s_qover = 1u;
  }
  // the history members' exact values, kept at or above the final bound
  // (NaN ones never are).  The list is complete: every wave recorded its
  // members before the last pass's bound barrier.
  bool xw = false;  // this thread writes exact entry tid
  if (has_hist && (uint32_t)tid < min(s_nx, (uint32_t)kXCap)) {
    const double val = penalize(L.x_val[tid], hcount(L.x_id[tid]), p);
    L.x_val[tid] = val;
    xw = val >= (double)tff;
    if (xw) atomicAdd(&s_nxk, 1u);
  }
  __syncthreads();
  uint32_t nw[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) nw[w] = s_nw[w];
  uint32_t nx = s_nxk;
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
        double val = 0.0;
        if (ok) {
          const uint32_t mw = kMask ? mrow[id >> 5] : ~0u;
          float x = lrow[id];
          const uint32_t cnt = has_hist ? hcount(id) : 0u;
          if (cnt) {
            ok = hist_value(id, x, mw, val);
          } else {
            ok = !kMask || ((mw >> (id & 31u)) & 1u);
            if (kSoftcap && softcap > 0.0f) x = softcap_f32(x, softcap);
            ok = ok && x == x;
            val = (double)x;
          }
        }
        f(key96(val, id), ok, val, id);
      }
    };
    uint32_t nval = 0u;
    for_elems([&](const Key96 &, bool ok, double, uint32_t) { nval += ok ? 1u : 0u; });
    if (tid == 0) s_sel[3] = 0u;
    __syncthreads();
    atomicAdd(&s_sel[3], nval);
    __syncthreads();
    const uint32_t need = min(s_sel[3], (uint32_t)k);
    __syncthreads();
    if (tid < kWaves) s_nw[tid] = 0u;
    if (tid == 0) {
      s_nx = 0u;
      s_flags = SAS_FLAG_SLOW_SELECT;
    }
    if (need > 0u) {
      const Key96 kth = block_select96(
          [&](auto f) { for_elems([&](const Key96 &kx, bool ok, double, uint32_t) { f(kx, ok); }); }, need, s_hist,
          s_sel);
      // exactly need <= kXCap entries
      for_elems([&](const Key96 &kx, bool ok, double val, uint32_t id) {
        if (ok && key_ge(kx, kth)) {
          const uint32_t d = atomicAdd(&s_nx, 1u);
          L.x_val[d] = val;
          L.x_id[d] = id;
        }
      });
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) nw[w] = s_nw[w];
    nx = s_nx;
    xw = (uint32_t)tid < nx;
    pm = 0u;
  }

  // ---- records: each wave's values after those of the waves before it, then
  // the exact-valued entries (record j of this part at row index j * P + part)
  uint32_t off = 0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) off += w < wave ? nw[w] : 0u;
  const uint32_t nplain = nw[0] + nw[1] + nw[2] + nw[3];
  uint64_t *rrow = a.rec + (int64_t)row * kListCap * P + part;
  double *xrow = a.xval + (int64_t)row * kListCap * P + part;
  {
    uint32_t j = off + qpre;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if ((pm >> c) & 1u) {
        const float x = c == 0 ? q.x : c == 1 ? q.y : c == 2 ? q.z : q.w;
        rrow[(int64_t)j * P] = (uint64_t)__float_as_uint(x) | ((uint64_t)(qid + (uint32_t)c) << 32);
        ++j;
      }
    }
  }
  if (xw) {
    // an exact value's round-down key, flagged when the value lies above it
    const double val = L.x_val[tid];
    const float kf = rd_f32(val);
    const uint32_t idf = L.x_id[tid] | ((double)kf != val ? kXFlag : 0u);
    const int64_t j = (int64_t)(nplain + atomicAdd(&s_nxw, 1u)) * P;
    rrow[j] = (uint64_t)__float_as_uint(kf) | ((uint64_t)idf << 32);
    if (idf & kXFlag) xrow[j] = val;
  }
  if (tid == 0) {
    a.pinfo[(int64_t)row * P + part] = (uint64_t)(nplain + nx) | ((uint64_t)tkey << 32);
    if (s_flags) __hip_atomic_fetch_or(ctl + kCtlFlags, s_flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
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

size_t sample_rec_bytes(int rows, int parts) { return (size_t)rows * parts * (kListCap * 16 + 8); }

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

template <bool kMask, bool kHist, bool kSoftcap>
static void launch_parts(const SampleArgs &a, hipStream_t stream) {
  hipLaunchKernelGGL((sample_parts_kernel<kMask, kHist, kSoftcap>), dim3((unsigned)(a.rows * a.parts)), dim3(kThreads),
                     0, stream, a);
}

hipError_t launch_sample(const SampleArgs &a, bool softcap, hipStream_t stream) {
  switch ((a.mask ? 4 : 0) | (a.hist_ids ? 2 : 0) | (softcap ? 1 : 0)) {
    case 0: launch_parts<false, false, false>(a, stream); break;
    case 1: launch_parts<false, false, true>(a, stream); break;
    case 2: launch_parts<false, true, false>(a, stream); break;
    case 3: launch_parts<false, true, true>(a, stream); break;
    case 4: launch_parts<true, false, false>(a, stream); break;
    case 5: launch_parts<true, false, true>(a, stream); break;
    case 6: launch_parts<true, true, false>(a, stream); break;
    default: launch_parts<true, true, true>(a, stream); break;
  }
  if (a.row_params)
    hipLaunchKernelGGL(sample_merge_kernel<true>, dim3((unsigned)a.rows), dim3(kMThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(sample_merge_kernel<false>, dim3((unsigned)a.rows), dim3(kMThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sas

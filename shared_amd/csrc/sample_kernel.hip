// sample_kernel.hip - fused logit processing + top-k/top-p sampling for gfx950.
//
// One launch per decode step.  Grid = rows x splits blocks; block (row, s)
// owns vocabulary chunk [s*CHUNK, (s+1)*CHUNK) of one row:
//
//   1. 128-bit loads of the chunk's fp32 logits straight into registers
//      (CHUNK/256 values per thread), the chunk's mask words and the row's
//      history ids (counted into a packed u16 LDS table) into LDS;
//   2. per value: softcap, mask (masked -> NaN, never selected), history
//      penalties for the few ids with a count (double precision, kept as a
//      round-down fp32 key; the exact double is recomputed when emitted),
//      running lane max;
//   3. block threshold: the j-th largest lane max of each wave via a lane
//      bitonic network, combined so that >= top_k values are >= it;
//   4. values >= threshold (typically ~top_k of them) are appended to an LDS
//      list with wave-aggregated atomics and written out as records;
//   5. the last block of the row to finish (atomic counter) merges the
//      records of all splits: global threshold, exact rank by (value desc,
//      id asc), then the reference's sample() tail in double precision.
//
// Logits cross HBM once; everything else is O(top_k) per block.  Replaces
// the topk + sampler WGSL pair (lib/webgpu-llm/kernels.js:1389-1449, 65-201)
// and the CPU sample() (lib/webgpu-llm/tokenizer.js:151-178).
#include "sas_device.h"
#include "sas_launch.h"

namespace sas {

template <int F4>
struct Lds {
  static constexpr int kChunk = F4 * 1024;
  static constexpr int kMaskWords = kChunk / 32;
  static constexpr int kCountWords = kChunk / 2;  // two u16 counts per word
  // merge scratch, overlaid on the count table
  static constexpr int kMergeBytes = kCapMerge * 8 + kCapMerge * 4 + SAS_MAX_TOP_K * (8 + 4 + 8 + 8) +
                                     (kMaxSplits + 1) * 4;
  static constexpr int kCountBytes = kCountWords * 4;
  static constexpr int kRawBytes = kCountBytes > kMergeBytes ? kCountBytes : kMergeBytes;
};

// LDS used by block-wide reductions.
struct Red {
  int have[kWaves];
  double v[kWaves];
  uint32_t id[kWaves];
  float f[kWaves];
};

// Recomputes one chunk element from global memory and the LDS tables; used
// by the rare paths so the hot loop keeps only fp32 keys in registers.
struct ElemCtx {
  const float *lrow;
  const uint32_t *s_mask;  // NULL: every id allowed
  const uint32_t *s_cnt;   // NULL: no history
  int lo;
  int vocab;
  sas_params p;

  __device__ double penalized(uint32_t id, float x) const {
    const uint32_t off = id - (uint32_t)lo;
    const uint32_t c = (s_cnt[off >> 1] >> ((off & 1u) * 16u)) & 0xFFFFu;
    return c ? penalize((double)x, c, p) : (double)x;
  }
  // Element `slot` (0 .. 4*F4-1) of this thread; false if masked or NaN.
  __device__ bool value(int slot, double &val, uint32_t &id) const {
    const int f = slot >> 2, j = slot & 3;
    const int q = f * kThreads + (int)threadIdx.x;
    const int e = lo + 4 * q + j;
    if (e >= vocab) return false;
    if (s_mask && !((s_mask[q >> 3] >> ((q & 7) * 4 + j)) & 1u)) return false;
    float x = lrow[e];
    if (p.softcap > 0.0f) x = softcap_f32(x, p.softcap);
    if (x != x) return false;
    val = s_cnt ? penalized((uint32_t)e, x) : (double)x;
    id = (uint32_t)e;
    return val == val;
  }
  // Exact value of an emitted record.
  __device__ double exact(uint32_t idf, float key) const {
    if (!(idf & kPenFlag)) return (double)key;
    const uint32_t id = idf & ~kPenFlag;
    float x = lrow[id];
    if (p.softcap > 0.0f) x = softcap_f32(x, p.softcap);
    return penalized(id, x);
  }
};

// Block-wide best (value, id); every thread returns the winner.  Barriers.
__device__ __forceinline__ bool block_best(bool have, double v, uint32_t id, Red *red, double &ov,
                                           uint32_t &oid) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  wave_best(have, v, id);
  if (lane == 0) {
    red->have[wave] = have;
    red->v[wave] = v;
    red->id[wave] = id;
  }
  __syncthreads();
  bool h = false;
  double bv = 0.0;
  uint32_t bi = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (red->have[w] && (!h || ranks_before(red->v[w], red->id[w], bv, bi))) {
      h = true;
      bv = red->v[w];
      bi = red->id[w];
    }
  }
  __syncthreads();
  ov = bv;
  oid = bi;
  return h;
}

// Exact top-k of one block by repeated block argmax, each round taking the
// best element strictly after the previous pick in (value desc, id asc)
// order.  Runs when more than kCapBlock values tie at or above the block
// threshold.  Writes records to s_rec_*; returns the count and the block
// threshold (round-down key of the k-th value, or -inf if fewer than k).
__device__ __forceinline__ int block_topk_slow(const ElemCtx &c, int E, int k, uint32_t *s_rec_id,
                                               float *s_rec_key, Red *red, float *thr) {
  double pv = 0.0;
  uint32_t pid = 0;
  int got = 0;
  for (int r = 0; r < k; ++r) {
    bool have = false;
    double bv = 0.0;
    uint32_t bi = 0;
#pragma unroll 1
    for (int s = 0; s < E; ++s) {
      double val;
      uint32_t id;
      if (!c.value(s, val, id)) continue;
      if (r > 0 && !ranks_before(pv, pid, val, id)) continue;
      if (!have || ranks_before(val, id, bv, bi)) {
        have = true;
        bv = val;
        bi = id;
      }
    }
    double wv;
    uint32_t wi;
    if (!block_best(have, bv, bi, red, wv, wi)) break;
    if (threadIdx.x == 0) {
      // Only a penalized value can differ from its fp32 key; flag it so the
      // record writer recomputes the double.
      const float key = rd_f32(wv);
      s_rec_id[r] = wi | ((double)key != wv ? kPenFlag : 0u);
      s_rec_key[r] = key;
    }
    pv = wv;
    pid = wi;
    ++got;
  }
  __syncthreads();
  *thr = got == k ? rd_f32(pv) : -__builtin_inff();
  return got;
}

// Exact top-k over all records of a row when more than kCapMerge of them
// reach the global threshold (degenerate ties); repeated block argmax.
__device__ __forceinline__ int merge_topk_slow(const Rec *rrow, const uint32_t *pre, int S, uint32_t total,
                                               float tstar, int k, double *t_val, uint32_t *t_id, Red *red) {
  double pv = 0.0;
  uint32_t pid = 0;
  int got = 0;
  for (int r = 0; r < k; ++r) {
    bool have = false;
    double bv = 0.0;
    uint32_t bi = 0;
    for (uint32_t g = threadIdx.x; g < total; g += kThreads) {
      int lo_b = 0, hi_b = S - 1;
      while (lo_b < hi_b) {
        const int mid = (lo_b + hi_b + 1) >> 1;
        if (pre[mid] <= g) lo_b = mid;
        else hi_b = mid - 1;
      }
      const Rec rc = rrow[(int64_t)lo_b * kCapBlock + (g - pre[lo_b])];
      if (!(rc.key >= tstar)) continue;
      if (r > 0 && !ranks_before(pv, pid, rc.val, rc.id)) continue;
      if (!have || ranks_before(rc.val, rc.id, bv, bi)) {
        have = true;
        bv = rc.val;
        bi = rc.id;
      }
    }
    double wv;
    uint32_t wi;
    if (!block_best(have, bv, bi, red, wv, wi)) break;
    if (threadIdx.x == 0) {
      t_val[r] = wv;
      t_id[r] = wi;
    }
    pv = wv;
    pid = wi;
    ++got;
  }
  return got;
}

template <int F4, bool kAligned>
__global__ __launch_bounds__(kThreads) void sample_rows_kernel(const SampleArgs a) {
  using L = Lds<F4>;
  constexpr int kChunk = L::kChunk;
  constexpr int E = F4 * 4;

  __shared__ __align__(16) unsigned char s_raw[L::kRawBytes];
  __shared__ uint32_t s_mask[L::kMaskWords];
  __shared__ uint32_t s_rec_id[kCapBlock];
  __shared__ float s_rec_key[kCapBlock];
  __shared__ float s_wthr[kWaves];
  __shared__ uint32_t s_n;
  __shared__ int s_last;
  __shared__ Red s_red;

  uint32_t *s_cnt = reinterpret_cast<uint32_t *>(s_raw);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nblocks = a.rows * a.splits;
  int lb = blockIdx.x;
  // XCD-aware order: consecutive dispatches rotate over the 8 XCDs, so give
  // each XCD a contiguous run of rows; a row's splits then share one L2 for
  // the history reads and the merge.
  if ((nblocks & 7) == 0) lb = (lb & 7) * (nblocks >> 3) + (lb >> 3);
  const int row = lb / a.splits;
  const int split = lb - row * a.splits;
  const int lo = split * kChunk;
  const int vocab = a.vocab;

  const sas_params p = a.row_params ? a.row_params[row] : a.params;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const float *lrow = a.logits + (int64_t)row * a.logits_stride;

  // ---- 1. loads --------------------------------------------------------
  float4 v[F4];
#pragma unroll
  for (int f = 0; f < F4; ++f) {
    const int e = lo + 4 * (f * kThreads + tid);
    if (kAligned && e + 3 < vocab) {
      const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(lrow + e));
      v[f] = make_float4(t.x, t.y, t.z, t.w);
    } else {
      v[f].x = e + 0 < vocab ? lrow[e + 0] : qnan();
      v[f].y = e + 1 < vocab ? lrow[e + 1] : qnan();
      v[f].z = e + 2 < vocab ? lrow[e + 2] : qnan();
      v[f].w = e + 3 < vocab ? lrow[e + 3] : qnan();
    }
  }
  const bool has_mask = a.mask != nullptr;
  if (has_mask && tid < L::kMaskWords) {
    const int gw = (lo >> 5) + tid;
    const int nw = (vocab + 31) >> 5;
    s_mask[tid] = gw < nw ? a.mask[(int64_t)row * a.mask_stride + gw] : 0u;
  }
  int h0 = 0, h1 = 0;
  if (a.hist_ids) {
    h0 = a.hist_offsets[row];
    h1 = a.hist_offsets[row + 1];
  }
  const bool has_hist = h1 > h0;
  if (has_hist) {
    uint4 *c4 = reinterpret_cast<uint4 *>(s_cnt);
    for (int w = tid; w < L::kCountWords / 4; w += kThreads) c4[w] = make_uint4(0u, 0u, 0u, 0u);
  }
  if (tid == 0) s_n = 0u;
  __syncthreads();
  if (has_hist) {
    for (int i = h0 + tid; i < h1; i += kThreads) {
      const uint32_t id = a.hist_ids[i];
      const uint32_t off = id - (uint32_t)lo;
      if (off < (uint32_t)kChunk && id < (uint32_t)vocab)
        atomicAdd(&s_cnt[off >> 1], 1u << ((off & 1u) * 16u));
    }
    __syncthreads();
  }
  const ElemCtx ec{lrow, has_mask ? s_mask : nullptr, has_hist ? s_cnt : nullptr, lo, vocab, p};

  // ---- 2. values (in place in v) -----------------------------------------
  uint32_t penbits = 0;
  float tmax = -__builtin_inff();
#pragma unroll
  for (int f = 0; f < F4; ++f) {
    const int q = f * kThreads + tid;
    if (p.softcap > 0.0f) {
      v[f].x = softcap_f32(v[f].x, p.softcap);
      v[f].y = softcap_f32(v[f].y, p.softcap);
      v[f].z = softcap_f32(v[f].z, p.softcap);
      v[f].w = softcap_f32(v[f].w, p.softcap);
    }
    if (has_mask) {
      const uint32_t nib = s_mask[q >> 3] >> ((q & 7) * 4);
      v[f].x = (nib & 1u) ? v[f].x : qnan();
      v[f].y = (nib & 2u) ? v[f].y : qnan();
      v[f].z = (nib & 4u) ? v[f].z : qnan();
      v[f].w = (nib & 8u) ? v[f].w : qnan();
    }
    if (has_hist) {
      const uint2 c = *reinterpret_cast<const uint2 *>(&s_cnt[2 * q]);
      if ((c.x | c.y) != 0u) {
        float x[4] = {v[f].x, v[f].y, v[f].z, v[f].w};
        for (int j = 0; j < 4; ++j) {
          const uint32_t w = j < 2 ? c.x : c.y;
          const uint32_t cnt = (w >> ((j & 1) * 16)) & 0xFFFFu;
          if (cnt != 0u && x[j] == x[j]) {
            x[j] = rd_f32(penalize((double)x[j], cnt, p));
            penbits |= 1u << (4 * f + j);
          }
        }
        v[f] = make_float4(x[0], x[1], x[2], x[3]);
      }
    }
    tmax = fmaxf(tmax, fmaxf(fmaxf(v[f].x, v[f].y), fmaxf(v[f].z, v[f].w)));
  }

  // ---- 3. block threshold ----------------------------------------------
  // Wave w guarantees jth lanes with a value >= its jth-largest lane max;
  // the mth largest of the wave thresholds then has >= mth*jth >= k values
  // at or above it.  -inf means "no guarantee": every valid value passes.
  const int jth = (k + kWaves - 1) / kWaves;
  const int mth = (k + jth - 1) / jth;
  const float tw = wave_jth_largest(tmax, jth);
  if (lane == 0) s_wthr[wave] = tw;
  __syncthreads();
  float t4[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t4[w] = s_wthr[w];
#pragma unroll
  for (int i = 0; i < kWaves; ++i)
#pragma unroll
    for (int j = 0; j < kWaves - 1 - i; ++j)
      if (t4[j] < t4[j + 1]) {
        const float t = t4[j];
        t4[j] = t4[j + 1];
        t4[j + 1] = t;
      }
  float thr = t4[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w)
    if (w == mth - 1) thr = t4[w];

  // ---- 4. emission -----------------------------------------------------
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int f = i >> 2, j = i & 3;
    const float x = j == 0 ? v[f].x : j == 1 ? v[f].y : j == 2 ? v[f].z : v[f].w;
    const bool pred = x >= thr;
    const uint64_t bal = __ballot(pred);
    if (bal) {
      const int leader = __ffsll((unsigned long long)bal) - 1;
      uint32_t base = 0;
      if (lane == leader) base = atomicAdd(&s_n, (uint32_t)__popcll(bal));
      base = __builtin_amdgcn_readlane(base, leader);
      if (pred) {
        const uint32_t slot = base + lanes_below(bal);
        if (slot < (uint32_t)kCapBlock) {
          const uint32_t id = (uint32_t)(lo + 4 * (f * kThreads + tid) + j);
          s_rec_id[slot] = id | (((penbits >> i) & 1u) ? kPenFlag : 0u);
          s_rec_key[slot] = x;
        }
      }
    }
  }
  __syncthreads();
  uint32_t n = s_n;
  if (n > (uint32_t)kCapBlock) n = (uint32_t)block_topk_slow(ec, E, k, s_rec_id, s_rec_key, &s_red, &thr);

  // ---- records out -----------------------------------------------------
  Rec *recs = a.recs + ((int64_t)row * a.splits + split) * kCapBlock;
  for (int i = tid; i < (int)n; i += kThreads) {
    const uint32_t idf = s_rec_id[i];
    const float kk = s_rec_key[i];
    Rec r;
    r.val = ec.exact(idf, kk);
    r.id = idf & ~kPenFlag;
    r.key = kk;
    recs[i] = r;
  }
  if (tid == 0) {
    BlockHdr h;
    h.n = n;
    h.thr = thr;
    a.hdrs[(int64_t)row * a.splits + split] = h;
  }

  // ---- 5. last block of the row merges -----------------------------------
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&a.counters[row], 1u) == (uint32_t)(a.splits - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid == 0) a.counters[row] = 0u;  // ready for the next launch

  double *m_val = reinterpret_cast<double *>(s_raw);
  uint32_t *m_id = reinterpret_cast<uint32_t *>(m_val + kCapMerge);
  double *t_val = reinterpret_cast<double *>(m_id + kCapMerge);   // ranked top-k
  double *t_p = t_val + SAS_MAX_TOP_K;                             // exp weights
  double *t_pre = t_p + SAS_MAX_TOP_K;                             // running sums
  uint32_t *t_id = reinterpret_cast<uint32_t *>(t_pre + SAS_MAX_TOP_K);
  uint32_t *pre = t_id + SAS_MAX_TOP_K;                            // [splits + 1]

  const int S = a.splits;
  const BlockHdr *hdrs = a.hdrs + (int64_t)row * S;
  const Rec *rrow = a.recs + (int64_t)row * S * kCapBlock;

  // global threshold and record offsets
  float tl = -__builtin_inff();
  for (int b = tid; b < S; b += kThreads) tl = fmaxf(tl, hdrs[b].thr);
  tl = wave_max(tl);
  if (lane == 0) s_red.f[wave] = tl;
  if (wave == 0) {
    uint32_t carry = 0;
    for (int b0 = 0; b0 < S; b0 += 64) {
      const int b = b0 + lane;
      const uint32_t nb = b < S ? hdrs[b].n : 0u;
      const uint32_t inc = wave_incl_scan(nb);
      if (b < S) pre[b] = carry + inc - nb;
      carry += __shfl(inc, 63, 64);
    }
    if (lane == 0) {
      pre[S] = carry;
      s_n = 0u;
    }
  }
  __syncthreads();
  float tstar = s_red.f[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) tstar = fmaxf(tstar, s_red.f[w]);
  const uint32_t total = pre[S];

  // gather records at or above the global threshold
  for (uint32_t g = tid; g < total; g += kThreads) {
    int lo_b = 0, hi_b = S - 1;  // last b with pre[b] <= g
    while (lo_b < hi_b) {
      const int mid = (lo_b + hi_b + 1) >> 1;
      if (pre[mid] <= g) lo_b = mid;
      else hi_b = mid - 1;
    }
    const Rec r = rrow[(int64_t)lo_b * kCapBlock + (g - pre[lo_b])];
    if (r.key >= tstar) {
      const uint32_t slot = atomicAdd(&s_n, 1u);
      if (slot < (uint32_t)kCapMerge) {
        m_val[slot] = r.val;
        m_id[slot] = r.id;
      }
    }
  }
  __syncthreads();
  const uint32_t m = s_n;
  int kk = 0;  // candidates ranked into t_val/t_id
  uint32_t flags = 0;
  if (m <= (uint32_t)kCapMerge) {
    for (uint32_t c = tid; c < m; c += kThreads) {
      const double vc0 = m_val[c];
      const uint32_t ic = m_id[c];
      uint32_t rank = 0;
      for (uint32_t j = 0; j < m; ++j) rank += ranks_before(m_val[j], m_id[j], vc0, ic) ? 1u : 0u;
      if (rank < (uint32_t)k) {
        t_val[rank] = vc0;
        t_id[rank] = ic;
      }
    }
    kk = (int)min(m, (uint32_t)k);
  } else {
    flags |= SAS_FLAG_SLOW_SELECT;
    kk = merge_topk_slow(rrow, pre, S, total, tstar, k, t_val, t_id, &s_red);
  }
  __syncthreads();

  // ---- sample() tail (tokenizer.js:161-177), double precision -----------
  const double T = p.temperature;
  if (!greedy && kk > 0) {
    const double v0 = t_val[0];
    for (int i = tid; i < kk; i += kThreads) t_p[i] = fd_exp((t_val[i] - v0) / T);
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t out_id = SAS_NO_TOKEN;
    int cut = 0;
    if (kk == 0) {
      flags |= SAS_FLAG_EMPTY_ROW;
    } else if (greedy) {
      out_id = t_id[0];
    } else {
      double sum = 0.0;
      for (int i = 0; i < kk; ++i) {
        sum += t_p[i];
        t_pre[i] = sum;
      }
      double cum = 0.0;
      cut = kk;
      for (int i = 0; i < kk; ++i) {
        cum += t_p[i] / sum;
        if (fabs(cum - p.top_p) < 1e-6) flags |= SAS_FLAG_TOPP_EDGE;
        if (cum >= p.top_p) {
          cut = i + 1;
          break;
        }
      }
      const double sub = t_pre[cut - 1];
      double r = a.uniforms[row] * sub;
      out_id = t_id[cut - 1];
      for (int i = 0; i < cut; ++i) {
        r -= t_p[i];
        if (fabs(r) <= 1e-12 * sub) flags |= SAS_FLAG_DRAW_EDGE;
        if (r <= 0.0) {
          out_id = t_id[i];
          break;
        }
      }
      t_pre[0] = sum;  // normaliser for the probability output
    }
    a.out_ids[row] = out_id;
    if (a.out_counts) {
      a.out_counts[2 * row] = greedy ? 0 : kk;
      a.out_counts[2 * row + 1] = greedy ? 0 : cut;
    }
    if (a.out_flags) a.out_flags[row] = flags;
  }
  if (a.out_probs || a.out_cand_ids) {
    __syncthreads();
    const int np = greedy ? 0 : kk;
    const double sum = np > 0 ? t_pre[0] : 1.0;
    for (int i = tid; i < SAS_MAX_TOP_K; i += kThreads) {
      if (a.out_probs) a.out_probs[(int64_t)row * SAS_MAX_TOP_K + i] = i < np ? t_p[i] / sum : 0.0;
      if (a.out_cand_ids) a.out_cand_ids[(int64_t)row * SAS_MAX_TOP_K + i] = i < np ? t_id[i] : SAS_NO_TOKEN;
    }
  }
}

// Splits per row: the largest chunk that still gives every CU several
// blocks, bounded so that a row never has more than kMaxSplits splits.
int choose_f4(int rows, int vocab) {
  const int f4s[3] = {8, 4, 2};
  int pick = 2;
  for (int i = 0; i < 3; ++i) {
    const int chunk = f4s[i] * 1024;
    const long long blocks = (long long)rows * ((vocab + chunk - 1) / chunk);
    if (blocks >= 2048) {
      pick = f4s[i];
      break;
    }
  }
  while (pick < 8 && (vocab + pick * 1024 - 1) / (pick * 1024) > kMaxSplits) pick *= 2;
  return pick;
}

template <int F4>
static hipError_t launch_f4(const SampleArgs &a, bool aligned, hipStream_t stream) {
  const dim3 grid((unsigned)(a.rows * a.splits)), block(kThreads);
  if (aligned) hipLaunchKernelGGL((sample_rows_kernel<F4, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((sample_rows_kernel<F4, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_sample(const SampleArgs &a, int f4, bool aligned, hipStream_t stream) {
  switch (f4) {
    case 8: return launch_f4<8>(a, aligned, stream);
    case 4: return launch_f4<4>(a, aligned, stream);
    default: return launch_f4<2>(a, aligned, stream);
  }
}

}  // namespace sas

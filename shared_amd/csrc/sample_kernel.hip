// sample_kernel.hip - fused logit processing + top-k/top-p sampling for gfx950.
//
// Two launches per decode step, stream-ordered:
//
// split_kernel   grid = rows x splits blocks; block (row, s) owns vocabulary
//                chunk [s*CHUNK, (s+1)*CHUNK) of one row:
//   1. the row's history ids, then the chunk's fp32 logits (128-bit loads
//      straight into registers, CHUNK/256 values per thread) and the mask
//      words (one 32-bit load per float4: the 8 threads of a word share it);
//      history ids falling in the chunk are counted into a packed u16 LDS
//      table while the logits are in flight;
//   2. per value: softcap, mask (masked -> NaN, never selected), history
//      penalties for the few ids with a count (double precision, kept as a
//      round-down fp32 key; the exact double is recomputed when emitted);
//   3. block threshold: the j-th largest lane max of each wave by a ballot
//      bit search over order-preserving keys, combined so that >= top_k
//      values are >= it;
//   4. values >= threshold (typically a little over top_k of them) are
//      appended to an LDS list with wave-aggregated atomics; if more than
//      kCapBlock pass, a radix search over the chunk's keys finds a tighter
//      bound; then a relaxed atomic reserves space in the row's record area
//      and 16-byte records are written.  No fence: nothing in this launch
//      reads them.
//
// merge_kernel   one block per row, after the split kernel has completed:
//   5. the row's records are loaded into registers in one round and a radix
//      search (8-bit digits from the top, LDS histograms) finds a key bound
//      that keeps at least top_k and at most top_k + kMergeSlack records;
//   6. exact rank of the survivors by (value desc, id asc) in double;
//   7. the reference's sample() tail in double precision: exp weights and
//      divisions in parallel, the running sums sequentially in JS order.
//
// Logits cross HBM once.  Replaces the topk + sampler WGSL pair
// (lib/webgpu-llm/kernels.js:1389-1449, 65-201) and the CPU sample()
// (lib/webgpu-llm/tokenizer.js:151-178).
#include "sas_device.h"
#include "sas_launch.h"

namespace sas {

template <int F4>
struct SplitLds {
  static constexpr int kChunk = F4 * 1024;
  static constexpr int kCountWords = kChunk / 2;  // two u16 counts per word
};

constexpr int kHistRegs = 4;     // history ids per thread held in registers
constexpr int kMergeRecs = 16;   // records per merge thread held in registers
constexpr int kMergeSlack = 32;  // survivors beyond top_k the merge may rank

// LDS used by block-wide reductions.
struct Red {
  int have[kWaves];
  double v[kWaves];
  uint32_t id[kWaves];
};

// Block-wide search, 8-bit digits from the most significant, for a bound L
// on the keys key(0..N-1) of all threads (0 = no key): at least `need` keys
// are >= L, and at most `cap` are unless more than that tie at the need-th
// largest key (then L is that key exactly).  `need` must not exceed the
// number of keys.  LDS: hist[256], sel[3].
// U bounds the unrolling of the key loop (and with it the keys in flight).
template <int N, int U = N, typename KeyFn>
__device__ uint32_t radix_bound(KeyFn key, uint32_t need, uint32_t cap, uint32_t *hist, uint32_t *sel) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = 0u, kr = need, taken = 0u;
  for (int shift = 24;; shift -= 8) {
    for (int i = tid; i < 256; i += kThreads) hist[i] = 0u;
    __syncthreads();
#pragma unroll U
    for (int j = 0; j < N; ++j) {
      const uint32_t x = key(j);
      if (x != 0u && (shift == 24 || (x >> (shift + 8)) == prefix)) atomicAdd(&hist[(x >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      // lane l holds bins 255-4l .. 252-4l (largest digits first)
      uint32_t c[4], sum = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = hist[255 - 4 * lane - j];
        sum += c[j];
      }
      const uint32_t incl = wave_incl_scan(sum);
      const uint64_t hit = __ballot(incl >= kr);
      const int first = __ffsll((unsigned long long)hit) - 1;
      if (lane == first) {
        uint32_t acc = incl - sum;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= kr) {
            sel[0] = (uint32_t)(255 - 4 * lane - j);
            sel[1] = acc;
            sel[2] = c[j];
            break;
          }
          acc += c[j];
        }
      }
    }
    __syncthreads();
    const uint32_t bin = sel[0], above = sel[1], cnt = sel[2];
    __syncthreads();  // hist and sel are reused
    prefix = (prefix << 8) | bin;
    if (taken + above + cnt <= cap || shift == 0) return prefix << shift;
    taken += above;
    kr -= above;
  }
}

// Appends the ids whose predicate holds to the LDS candidate list with one
// LDS atomic per wave per element slot.  pred(i) / key(i) for slot i; U
// bounds the unrolling.
template <int E, int U = E, typename Pred, typename Key>
__device__ __forceinline__ void emit_candidates(int lo, uint32_t penbits, Pred pred_of, Key key_of,
                                                uint32_t *s_n, uint32_t *s_rec_id, float *s_rec_key) {
  const int tid = threadIdx.x, lane = tid & 63;
#pragma unroll U
  for (int i = 0; i < E; ++i) {
    const int f = i >> 2, j = i & 3;
    const bool pred = pred_of(i);
    const uint64_t bal = __ballot(pred);
    if (bal) {
      const int leader = __ffsll((unsigned long long)bal) - 1;
      uint32_t base = 0;
      if (lane == leader) base = atomicAdd(s_n, (uint32_t)__popcll(bal));
      base = __builtin_amdgcn_readlane(base, leader);
      if (pred) {
        const uint32_t slot = base + lanes_below(bal);
        if (slot < (uint32_t)kCapBlock) {
          const uint32_t id = (uint32_t)(lo + 4 * (f * kThreads + tid) + j);
          s_rec_id[slot] = id | (((penbits >> i) & 1u) ? kPenFlag : 0u);
          s_rec_key[slot] = key_of(i);
        }
      }
    }
  }
}

// Recomputes one chunk element from global memory and the LDS count table;
// used by the rare paths so the hot loop keeps only fp32 keys in registers.
struct ElemCtx {
  const float *lrow;
  const uint32_t *mrow;    // the row's mask words, NULL: every id allowed
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
    if (mrow && !((mrow[e >> 5] >> (e & 31)) & 1u)) return false;
    float x = lrow[e];
    if (p.softcap > 0.0f) x = softcap_f32(x, p.softcap);
    if (x != x) return false;
    val = s_cnt ? penalized((uint32_t)e, x) : (double)x;
    id = (uint32_t)e;
    return val == val;
  }
  // Exact value of an emitted candidate.
  __device__ double exact(uint32_t idf, float key) const {
    if (!(idf & kPenFlag)) return (double)key;
    const uint32_t id = idf & ~kPenFlag;
    float x = lrow[id];
    if (p.softcap > 0.0f) x = softcap_f32(x, p.softcap);
    return s_cnt ? penalized(id, x) : (double)x;
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
// order.  Runs only when more than kCapBlock values tie exactly at the
// k-th largest key of the block.  Writes candidates to s_rec_*; returns the
// count.
__device__ __forceinline__ int block_topk_slow(const ElemCtx &c, int E, int k, uint32_t *s_rec_id,
                                               float *s_rec_key, Red *red) {
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
  return got;
}

template <int F4, bool kAligned>
__global__ __launch_bounds__(kThreads) void split_kernel(const SampleArgs a) {
  using L = SplitLds<F4>;
  constexpr int kChunk = L::kChunk;
  constexpr int E = F4 * 4;

  __shared__ __align__(16) uint32_t s_cnt[L::kCountWords];
  __shared__ uint32_t s_rec_id[kCapBlock];
  __shared__ float s_rec_key[kCapBlock];
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[3];
  __shared__ uint32_t s_wkey[2 * kWaves];
  __shared__ uint32_t s_n;
  __shared__ uint32_t s_base;
  __shared__ Red s_red;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nblocks = a.rows * a.splits;
  int lb = blockIdx.x;
  // XCD-aware order: consecutive dispatches rotate over the 8 XCDs, so give
  // each XCD a contiguous run of rows; a row's splits then share one L2 for
  // the history reads.
  if ((nblocks & 7) == 0) lb = (lb & 7) * (nblocks >> 3) + (lb >> 3);
  const int row = lb / a.splits;
  const int split = lb - row * a.splits;
  const int lo = split * kChunk;
  const int vocab = a.vocab;

  const sas_params p = a.row_params ? a.row_params[row] : a.params;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const float *lrow = a.logits + (int64_t)row * a.logits_stride;
  const uint32_t *mrow = a.mask ? a.mask + (int64_t)row * a.mask_stride : nullptr;

  // ---- 1. loads: history first, so its atomics overlap the logits' flight --
  int h0 = 0, h1 = 0;
  if (a.hist_ids) {
    h0 = a.hist_offsets[row];
    h1 = a.hist_offsets[row + 1];
  }
  const bool has_hist = h1 > h0;
  uint32_t hreg[kHistRegs];
#pragma unroll
  for (int j = 0; j < kHistRegs; ++j) {
    const int i = h0 + j * kThreads + tid;
    hreg[j] = i < h1 ? a.hist_ids[i] : 0xFFFFFFFFu;
  }
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
  // mask word of float4 f: word (lo + 4q) / 32 with q = f*256 + tid
  uint32_t mw[F4];
  if (mrow) {
    const int nw = (vocab + 31) >> 5;
#pragma unroll
    for (int f = 0; f < F4; ++f) {
      const int w = (lo >> 5) + f * (kThreads / 8) + (tid >> 3);
      mw[f] = w < nw ? mrow[w] : 0u;
    }
  }
  if (has_hist) {
    uint4 *c4 = reinterpret_cast<uint4 *>(s_cnt);
    for (int w = tid; w < L::kCountWords / 4; w += kThreads) c4[w] = make_uint4(0u, 0u, 0u, 0u);
  }
  if (tid == 0) s_n = 0u;
  __syncthreads();
  if (has_hist) {
    auto count = [&](uint32_t id) {
      const uint32_t off = id - (uint32_t)lo;
      if (off < (uint32_t)kChunk && id < (uint32_t)vocab) atomicAdd(&s_cnt[off >> 1], 1u << ((off & 1u) * 16u));
    };
#pragma unroll
    for (int j = 0; j < kHistRegs; ++j) count(hreg[j]);
    for (int i = h0 + kHistRegs * kThreads + tid; i < h1; i += kThreads) count(a.hist_ids[i]);
    __syncthreads();
  }
  const ElemCtx ec{lrow, mrow, has_hist ? s_cnt : nullptr, lo, vocab, p};

  // ---- 2. values (in place in v) -----------------------------------------
  uint32_t penbits = 0;
  float tmax = qnan();  // stays NaN in a lane without a valid value
  const int nshift = 4 * (tid & 7);
#pragma unroll
  for (int f = 0; f < F4; ++f) {
    const int q = f * kThreads + tid;
    if (p.softcap > 0.0f) {
      v[f].x = softcap_f32(v[f].x, p.softcap);
      v[f].y = softcap_f32(v[f].y, p.softcap);
      v[f].z = softcap_f32(v[f].z, p.softcap);
      v[f].w = softcap_f32(v[f].w, p.softcap);
    }
    if (mrow) {
      const uint32_t nib = mw[f] >> nshift;
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
  auto elem = [&](int i) -> float {
    const int f = i >> 2, j = i & 3;
    return j == 0 ? v[f].x : j == 1 ? v[f].y : j == 2 ? v[f].z : v[f].w;
  };

  // ---- 3. block threshold ----------------------------------------------
  // Wave w guarantees jth lanes with a value >= its jth-largest lane max;
  // the mth largest of the wave thresholds then has >= mth*jth >= k values
  // at or above it.  If some wave cannot (too few valid lanes: a sparse
  // mask, a partial chunk), a wave that alone has k valid lanes can; with
  // neither, every valid value passes.
  const int jth = (k + kWaves - 1) / kWaves;
  const int mth = (k + jth - 1) / jth;
  const uint32_t lkey = okey(tmax);
  const uint32_t tw = wave_jth_largest_key(lkey, jth);
  if (lane == 0) s_wkey[wave] = tw;
  __syncthreads();
  uint32_t t4[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t4[w] = s_wkey[w];
#pragma unroll
  for (int i = 0; i < kWaves; ++i)
#pragma unroll
    for (int j = 0; j < kWaves - 1 - i; ++j)
      if (t4[j] < t4[j + 1]) {
        const uint32_t t = t4[j];
        t4[j] = t4[j + 1];
        t4[j + 1] = t;
      }
  uint32_t tkey = t4[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w)
    if (w == mth - 1) tkey = t4[w];
  if (tkey == 0u && k <= 64) {
    // block-uniform: the combination failed; try one wave alone
    const uint32_t tk = wave_jth_largest_key(lkey, k);
    if (lane == 0) s_wkey[kWaves + wave] = tk;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tkey = max(tkey, s_wkey[kWaves + w]);
  }
  const float thr = tkey ? fkey(tkey) : -__builtin_inff();

  // ---- 4. emission -----------------------------------------------------
  emit_candidates<E>(lo, penbits, [&](int i) { return elem(i) >= thr; }, elem, &s_n, s_rec_id, s_rec_key);
  __syncthreads();
  uint32_t n = s_n;
  if (n > (uint32_t)kCapBlock) {
    // The wave thresholds were too weak (few valid lanes or heavy ties):
    // bound the keys exactly and emit again.  The keys are recomputed from
    // memory so the register-resident values are dead here and this rare
    // path costs the hot one no registers.
    auto key = [&](int i) {
      double val;
      uint32_t id;
      return ec.value(i, val, id) ? okey(rd_f32(val)) : 0u;
    };
    const uint32_t bound = radix_bound<E, 8>(key, (uint32_t)k, (uint32_t)kCapBlock, s_hist, s_sel);
    if (tid == 0) s_n = 0u;
    __syncthreads();
    // every record of this path recomputes its exact value when written
    emit_candidates<E, 8>(
        lo, ~0u,
        [&](int i) {
          const uint32_t x = key(i);
          return x != 0u && x >= bound;
        },
        [&](int i) { return fkey(key(i)); }, &s_n, s_rec_id, s_rec_key);
    __syncthreads();
    n = s_n;
    if (n > (uint32_t)kCapBlock) n = (uint32_t)block_topk_slow(ec, E, k, s_rec_id, s_rec_key, &s_red);
  }

  // ---- records out -----------------------------------------------------
  // Reservation only: the merge kernel reads the records after this launch
  // has completed, so no ordering beyond the atomic itself is needed.
  if (tid == 0) s_base = n ? atomicAdd(&a.counters[row], n) : 0u;
  __syncthreads();
  Rec *out = a.recs + (int64_t)row * a.rec_cap + s_base;
  for (int i = tid; i < (int)n; i += kThreads) {
    const uint32_t idf = s_rec_id[i];
    const float kk = s_rec_key[i];
    Rec r;
    r.val = ec.exact(idf, kk);
    r.id = idf & ~kPenFlag;
    r.key = kk;
    out[i] = r;
  }
}

// ------------------------------------------------------------------ merge --

// Radix bound over record keys read from global memory on every pass; used
// when a row has more records than the merge holds in registers.
__device__ uint32_t radix_bound_global(const Rec *recs, uint32_t total, uint32_t need, uint32_t cap,
                                       uint32_t *hist, uint32_t *sel) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = 0u, kr = need, taken = 0u;
  for (int shift = 24;; shift -= 8) {
    for (int i = tid; i < 256; i += kThreads) hist[i] = 0u;
    __syncthreads();
    for (uint32_t g = tid; g < total; g += kThreads) {
      const uint32_t x = okey(recs[g].key);
      if (x != 0u && (shift == 24 || (x >> (shift + 8)) == prefix)) atomicAdd(&hist[(x >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wave == 0) {
      uint32_t c[4], sum = 0u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = hist[255 - 4 * lane - j];
        sum += c[j];
      }
      const uint32_t incl = wave_incl_scan(sum);
      const uint64_t hit = __ballot(incl >= kr);
      const int first = __ffsll((unsigned long long)hit) - 1;
      if (lane == first) {
        uint32_t acc = incl - sum;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (acc + c[j] >= kr) {
            sel[0] = (uint32_t)(255 - 4 * lane - j);
            sel[1] = acc;
            sel[2] = c[j];
            break;
          }
          acc += c[j];
        }
      }
    }
    __syncthreads();
    const uint32_t bin = sel[0], above = sel[1], cnt = sel[2];
    __syncthreads();
    prefix = (prefix << 8) | bin;
    if (taken + above + cnt <= cap || shift == 0) return prefix << shift;
    taken += above;
    kr -= above;
  }
}

// Exact top-k over the records whose key maps to >= lower when more than
// kCapMerge of them survive (degenerate ties); repeated block argmax.
__device__ __forceinline__ int merge_topk_slow(const Rec *recs, uint32_t total, uint32_t lower, int k,
                                               double *t_val, uint32_t *t_id, Red *red) {
  double pv = 0.0;
  uint32_t pid = 0;
  int got = 0;
  for (int r = 0; r < k; ++r) {
    bool have = false;
    double bv = 0.0;
    uint32_t bi = 0;
    for (uint32_t g = threadIdx.x; g < total; g += kThreads) {
      const Rec rc = recs[g];
      const uint32_t x = okey(rc.key);
      if (x == 0u || x < lower) continue;
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

__global__ __launch_bounds__(kThreads) void merge_kernel(const SampleArgs a) {
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[3];
  __shared__ double m_val[kCapMerge];
  __shared__ uint32_t m_id[kCapMerge];
  __shared__ double t_val[SAS_MAX_TOP_K];  // ranked top-k values
  __shared__ double t_p[SAS_MAX_TOP_K];    // exp weights
  __shared__ double t_q[SAS_MAX_TOP_K];    // weights / sum
  __shared__ double t_pre[SAS_MAX_TOP_K];  // running sums
  __shared__ uint32_t t_id[SAS_MAX_TOP_K];
  __shared__ uint32_t s_n;
  __shared__ Red s_red;

  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const sas_params p = a.row_params ? a.row_params[row] : a.params;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const Rec *recs = a.recs + (int64_t)row * a.rec_cap;

  const uint32_t total = a.counters[row];
  if (tid == 0) s_n = 0u;
  __syncthreads();
  if (tid == 0) a.counters[row] = 0u;  // every wave has read it; ready for the next launch
  const uint32_t need = min((uint32_t)k, total);
  const uint32_t cap = min((uint32_t)kCapMerge, (uint32_t)k + (uint32_t)kMergeSlack);

  // ---- 5/6. bound the keys, gather the survivors -------------------------
  uint32_t lower = 1u;
  if (total <= (uint32_t)(kThreads * kMergeRecs)) {
    Rec r[kMergeRecs];
#pragma unroll
    for (int j = 0; j < kMergeRecs; ++j) {
      const uint32_t g = (uint32_t)(tid + j * kThreads);
      if (g < total) {
        r[j] = recs[g];
      } else {
        r[j].key = qnan();
        r[j].id = 0u;
        r[j].val = 0.0;
      }
    }
    if (total > cap)
      lower = radix_bound<kMergeRecs>([&](int j) { return okey(r[j].key); }, need, cap, s_hist, s_sel);
#pragma unroll
    for (int j = 0; j < kMergeRecs; ++j) {
      const uint32_t x = okey(r[j].key);
      if (x != 0u && x >= lower) {
        const uint32_t slot = atomicAdd(&s_n, 1u);
        if (slot < (uint32_t)kCapMerge) {
          m_val[slot] = r[j].val;
          m_id[slot] = r[j].id;
        }
      }
    }
  } else {
    lower = radix_bound_global(recs, total, need, cap, s_hist, s_sel);
    for (uint32_t g = tid; g < total; g += kThreads) {
      const Rec rc = recs[g];
      const uint32_t x = okey(rc.key);
      if (x != 0u && x >= lower) {
        const uint32_t slot = atomicAdd(&s_n, 1u);
        if (slot < (uint32_t)kCapMerge) {
          m_val[slot] = rc.val;
          m_id[slot] = rc.id;
        }
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
#pragma unroll 8
      for (uint32_t j = 0; j < m; ++j) rank += ranks_before(m_val[j], m_id[j], vc0, ic) ? 1u : 0u;
      if (rank < (uint32_t)k) {
        t_val[rank] = vc0;
        t_id[rank] = ic;
      }
    }
    kk = (int)min(m, (uint32_t)k);
  } else {
    flags |= SAS_FLAG_SLOW_SELECT;
    kk = merge_topk_slow(recs, total, lower, k, t_val, t_id, &s_red);
  }
  __syncthreads();

  // ---- 7. sample() tail (tokenizer.js:161-177), double precision -----------
  // exp and division are correctly rounded wherever they run; only the
  // running sums must follow the reference's left-to-right order.
  const double T = p.temperature;
  const bool draw = !greedy && kk > 0;
  if (draw) {
    const double v0 = t_val[0];
    for (int i = tid; i < kk; i += kThreads) t_p[i] = fd_exp((t_val[i] - v0) / T);
  }
  __syncthreads();
  if (draw && tid == 0) {
    double sum = 0.0;
#pragma unroll 8
    for (int i = 0; i < kk; ++i) {
      sum += t_p[i];
      t_pre[i] = sum;
    }
  }
  __syncthreads();
  if (draw) {
    const double sum = t_pre[kk - 1];
    for (int i = tid; i < kk; i += kThreads) t_q[i] = t_p[i] / sum;
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
      double cum = 0.0;
      cut = kk;
      for (int i = 0; i < kk; ++i) {
        cum += t_q[i];
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
    }
    a.out_ids[row] = out_id;
    if (a.out_counts) {
      a.out_counts[2 * row] = greedy ? 0 : kk;
      a.out_counts[2 * row + 1] = greedy ? 0 : cut;
    }
    if (a.out_flags) a.out_flags[row] = flags;
  }
  if (a.out_probs || a.out_cand_ids) {
    const int np = draw ? kk : 0;
    for (int i = tid; i < SAS_MAX_TOP_K; i += kThreads) {
      if (a.out_probs) a.out_probs[(int64_t)row * SAS_MAX_TOP_K + i] = i < np ? t_q[i] : 0.0;
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

int64_t sample_rec_cap(int splits) { return (int64_t)splits * kCapBlock; }

size_t sample_rec_bytes(int rows, int splits) { return (size_t)rows * (size_t)sample_rec_cap(splits) * sizeof(Rec); }

template <int F4>
static hipError_t launch_split(const SampleArgs &a, bool aligned, hipStream_t stream) {
  const dim3 grid((unsigned)(a.rows * a.splits)), block(kThreads);
  if (aligned) hipLaunchKernelGGL((split_kernel<F4, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((split_kernel<F4, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_sample(const SampleArgs &a, int f4, bool aligned, hipStream_t stream) {
  hipError_t e;
  switch (f4) {
    case 8: e = launch_split<8>(a, aligned, stream); break;
    case 4: e = launch_split<4>(a, aligned, stream); break;
    default: e = launch_split<2>(a, aligned, stream); break;
  }
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)a.rows), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sas

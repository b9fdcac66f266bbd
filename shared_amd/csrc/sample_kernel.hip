// sample_kernel.hip - fused logit processing + top-k/top-p sampling for gfx950.
//
// One launch per decode step.  Grid = rows x parts blocks of 256 threads,
// sized so that every block is resident at once (four per CU).  Block
// (row, q) streams a contiguous run of 4096-id chunks of one row:
//
//   1. loads: every chunk's fp32 logits as 16-byte loads (16 values per
//      thread) and its mask words, the next chunk's loads always in flight
//      while the current one is processed.  Every iteration issues the same
//      loads (clamped addresses, a dummy past the part's end) and the hot
//      path touches no other memory, so the compiler never waits for the
//      prefetched chunk early;
//   2. per value: softcap, mask (masked -> NaN, never selected);
//   3. each wave keeps its own candidate list in LDS and a bound (the k-th
//      largest key of its list, shared with the block through an LDS
//      atomic max); values at or above the bound are appended (one ballot
//      prefix per chunk, static slots), the list is re-bounded when it
//      fills.  The first chunk bounds itself by its own k-th largest value;
//   4. history penalties that can only lower a value are applied to the
//      appended values alone (the raw value bounds the penalized one from
//      above); others are applied to every value before the bound test;
//   5. after the last chunk: the part's bound over its four lists (an LDS
//      histogram), its candidates written to its record slots with exact
//      double values, and one arrival atomic on the row's own cache line;
//   6. the row's last part merges: one round of loads brings the counts and
//      a window of every part's records; an LDS histogram bounds the keys to
//      the top k and a few ties, which are ranked by composite 64-bit keys
//      (value, exact-value flag, id);
//   7. the reference's sample() tail in double precision: exp weights and
//      divisions across lanes, each running sum one chain in JS order.
//
// Cross-block data (records, counts, row counters and thresholds) is only
// accessed with agent-scope atomic loads and stores, which are coherent
// across the XCDs' L2 caches without cache maintenance; each block waits
// for its record stores to complete before it counts itself in, so the
// last block, which observes every other block's count, reads complete
// records.  The merging block resets the row's counter and threshold for
// the next launch.
//
// Logits cross HBM once.  Replaces the topk + sampler WGSL pair
// (lib/webgpu-llm/kernels.js:1389-1449, 65-201) and the CPU sample()
// (lib/webgpu-llm/tokenizer.js:151-178).
#include <type_traits>

#include "sas_device.h"
#include "sas_launch.h"

namespace sas {

constexpr int kSpanWordsIds = 65536;             // ids one part may span
constexpr int kF4 = kChunkIds / (4 * kThreads);  // float4 per thread per chunk
constexpr int kE = kF4 * 4;                      // values per thread per chunk
static_assert(kE == 16, "a thread holds 16 values of a chunk");
static_assert(kCtlCnt + kMaxParts <= kCtlStride, "a count per part in the row's control block");
constexpr int kWaveCap = 256;                    // candidates one wave's list holds
constexpr int kHistRegs = 2;                    // history ids per thread loaded with the first chunk
constexpr int kRedoCap = 16;                     // chunk slices a wave may defer (>= chunks per part)
constexpr int kMaxCpp = kSpanWordsIds / kChunkIds;  // chunks per part (the history bitmap's span)
constexpr int kSurvCap = 256;                    // survivors the merge ranks in LDS
constexpr int kMergeSlack = 32;                  // survivors beyond top_k the merge aims for
constexpr int kMergeR = 4;                       // window records per merge thread
constexpr uint32_t kExactFlag = 0x40000000u;     // list entry whose l_val holds the exact value
constexpr uint32_t kIdMask = 0x3FFFFFFFu;
constexpr uint32_t kRecValFlag = 0x80000000u;   // record whose exact value differs from its fp32 key

// LDS used by block-wide reductions.
struct Red {
  int have[kWaves];
  double v[kWaves];
  uint32_t id[kWaves];
};

// The value of the wave's first active lane (wave-uniform values).
__device__ __forceinline__ uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// Agent-scope relaxed accesses: coherent across the XCDs without fences.
__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every vector memory operation this wave issued (stores and
// atomics included) has completed: s_waitcnt vmcnt(0).
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Block-wide search for a bound L on keys (0 = no key): at least `need`
// keys are >= L, and at most `cap` are unless more than that tie at the
// need-th largest key (then L is that key exactly).  Digits of 8 bits run
// from bit `hb` (the highest bit in which the keys may differ; `hprefix`
// holds the bits above it) down to bit 0.  `need` must not exceed the
// number of keys.  for_keys(f) calls f(key) for each of this thread's keys.
// LDS: hist[256], sel[3].
template <typename ForKeys>
__device__ __forceinline__ uint32_t radix_bound(ForKeys for_keys, int hb, uint32_t hprefix, uint32_t need, uint32_t cap,
                                uint32_t *hist, uint32_t *sel) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = hprefix, kr = need, taken = 0u;
  int top = hb + 1;  // bits >= top are fixed by prefix
  for (;;) {
    const int width = top < 8 ? top : 8;
    const int shift = top - width;
    for (int i = tid; i < 256; i += kThreads) hist[i] = 0u;
    __syncthreads();
    for_keys([&](uint32_t x) {
      if (x != 0u && (top == 32 || (x >> top) == prefix)) atomicAdd(&hist[(x >> shift) & ((1u << width) - 1u)], 1u);
    });
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
    prefix = (prefix << width) | bin;
    if (taken + above + cnt <= cap || shift == 0) return prefix << shift;
    top = shift;
    taken += above;
    kr -= above;
  }
}

// radix_bound for one wave alone (the other waves may have left): the
// same bound, with wave barriers.  LDS: hist[256].
template <typename ForKeys>
__device__ __forceinline__ uint32_t wave_radix_bound(ForKeys for_keys, int hb, uint32_t hprefix, uint32_t need, uint32_t cap,
                                     uint32_t *hist) {
  const int lane = threadIdx.x & 63;
  uint32_t prefix = hprefix, kr = need, taken = 0u;
  int top = hb + 1;  // bits >= top are fixed by prefix
  for (;;) {
    const int width = top < 8 ? top : 8;
    const int shift = top - width;
    *reinterpret_cast<uint4 *>(hist + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
    __builtin_amdgcn_wave_barrier();
    for_keys([&](uint32_t x) {
      if (x != 0u && (top == 32 || (x >> top) == prefix)) atomicAdd(&hist[(x >> shift) & ((1u << width) - 1u)], 1u);
    });
    __builtin_amdgcn_wave_barrier();
    // lane l holds bins 255-4l .. 252-4l (largest digits first)
    const uint4 h4 = *reinterpret_cast<const uint4 *>(hist + 252 - 4 * lane);
    const uint32_t c[4] = {h4.w, h4.z, h4.y, h4.x};
    const uint32_t sum = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_incl_scan(sum);
    const uint64_t hit = __ballot(incl >= kr);
    const int first = __ffsll((unsigned long long)hit) - 1;
    uint32_t bin = 0u, above = 0u, cnt = 0u;
    {
      uint32_t acc = incl - sum;
      bool done = false;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (!done && acc + c[j] >= kr) {
          bin = (uint32_t)(255 - 4 * lane - j);
          above = acc;
          cnt = c[j];
          done = true;
        }
        if (!done) acc += c[j];
      }
    }
    bin = (uint32_t)__builtin_amdgcn_readlane((int)bin, first);
    above = (uint32_t)__builtin_amdgcn_readlane((int)above, first);
    cnt = (uint32_t)__builtin_amdgcn_readlane((int)cnt, first);
    __builtin_amdgcn_wave_barrier();  // hist is reused
    prefix = (prefix << width) | bin;
    if (taken + above + cnt <= cap || shift == 0) return prefix << shift;
    top = shift;
    taken += above;
    kr -= above;
  }
}

// Reserves popcount(bits) consecutive LDS list slots for this lane (wave
// prefix of the counts by ballots, one atomic per wave) and returns the
// first.  bits holds at most 32 set bits.
__device__ __forceinline__ uint32_t wave_reserve(uint32_t bits, uint32_t *s_n) {
  const uint32_t cnt = __popc(bits);
  uint32_t pre = 0u, tot = 0u;
#pragma unroll
  for (int b = 0; b < 6; ++b) {
    const uint64_t bb = __ballot((cnt >> b) & 1u);
    pre += lanes_below(bb) << b;
    tot += (uint32_t)__popcll(bb) << b;
  }
  uint32_t base = 0u;
  if (tot && (threadIdx.x & 63) == 0) base = atomicAdd(s_n, tot);
  return __builtin_amdgcn_readlane(base, 0) + pre;
}

// Appends the ids whose predicate holds to an LDS list of `cap` entries,
// one LDS atomic per wave per element slot (the rare paths).
template <int E, int U, typename Pred, typename Key>
__device__ __forceinline__ void emit_each(int lo, Pred pred_of, Key key_of, uint32_t cap, uint32_t *s_n,
                                         uint32_t *s_rec_id, float *s_rec_key) {
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
        if (slot < cap) {
          s_rec_id[slot] = (uint32_t)(lo + 4 * (f * kThreads + tid) + j) | kPenFlag;
          s_rec_key[slot] = key_of(i);
        }
      }
    }
  }
}

// History of one part in LDS: a membership bitmap over the part's ids and
// an open-addressing hash of (id, count).  Ids the full hash could not take
// are counted from the row's history in memory (a slow path).
constexpr int kSpanWords = 2048;   // bitmap words: a part spans at most 65536 ids
constexpr int kHashSlots = 1024;
constexpr uint32_t kEmpty = 0xFFFFFFFFu;

struct PartHist {
  uint32_t bits[kSpanWords];
  uint32_t key[kHashSlots];
  uint32_t cnt[kHashSlots];
  uint32_t over;   // some id did not fit in the hash
};

__device__ __forceinline__ uint32_t hash_slot(uint32_t id) { return (id * 2654435761u) >> 22; }

struct HistView {
  const PartHist *h;      // NULL: no history
  uint32_t plo;           // first id of the part
  const uint32_t *ids;    // the row's history in memory (for the slow path)
  int h0, h1;

  __device__ __forceinline__ bool member(uint32_t id) const {
    const uint32_t off = id - plo;
    return h && ((h->bits[off >> 5] >> (off & 31)) & 1u);
  }
  // Occurrences of a member id.
  __device__ uint32_t count(uint32_t id) const {
    uint32_t s = hash_slot(id);
    for (int probe = 0; probe < kHashSlots; ++probe) {
      const uint32_t k = h->key[s];
      if (k == id) return h->cnt[s];
      if (k == kEmpty) break;
      s = (s + 1u) & (uint32_t)(kHashSlots - 1);
    }
    uint32_t c = 0;
    if (h->over)
      for (int i = h0; i < h1; ++i) c += ids[i] == id ? 1u : 0u;
    return c;
  }
};

// Recomputes one chunk element from global memory and the part's history;
// used by the rare paths so the hot loop keeps only fp32 keys in registers.
// only_wave >= 0 restricts the elements to that wave's slice of the chunk.
struct ElemCtx {
  const float *lrow;
  const uint32_t *mrow;    // the row's mask words, NULL: every id allowed
  HistView hv;
  int lo;
  int vocab;
  const sas_params &p;
  int only_wave;

  __device__ __forceinline__ uint32_t count(uint32_t id) const { return hv.member(id) ? hv.count(id) : 0u; }
  // Element `slot` (0 .. kE-1) of this thread; false if masked, NaN or
  // outside the selected wave.
  __device__ __noinline__ bool value(int slot, double &val, uint32_t &id) const {
    if (only_wave >= 0 && (int)(threadIdx.x >> 6) != only_wave) return false;
    const int f = slot >> 2, j = slot & 3;
    const int q = f * kThreads + (int)threadIdx.x;
    const int e = lo + 4 * q + j;
    if (e >= vocab) return false;
    if (mrow && !((mrow[e >> 5] >> (e & 31)) & 1u)) return false;
    float x = lrow[e];
    if (p.softcap > 0.0f) x = softcap_f32(x, p.softcap);
    if (x != x) return false;
    const uint32_t c = count((uint32_t)e);
    val = c ? penalize((double)x, c, p) : (double)x;
    id = (uint32_t)e;
    return val == val;
  }
};

// Exact value of a candidate whose fp32 logit is read again.
__device__ __forceinline__ double exact_value(const float *lrow, uint32_t id, uint32_t count, const sas_params &p) {
  float x = lrow[id];
  if (p.softcap > 0.0f) x = softcap_f32(x, p.softcap);
  return count ? penalize((double)x, count, p) : (double)x;
}

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

// Exact top-k of one chunk by repeated block argmax, each round taking the
// best element strictly after the previous pick in (value desc, id asc)
// order, among the elements that rank before (fv, fid) if has_floor.  Runs
// only when more candidates than fit tie exactly at the k-th largest key of
// the chunk.  Returns the count.
__device__ __forceinline__ int chunk_topk_slow(const ElemCtx &c, int k, bool has_floor, double fv, uint32_t fid,
                                               uint32_t *s_rec_id, float *s_rec_key, Red *red) {
  double pv = 0.0;
  uint32_t pid = 0;
  int got = 0;
  for (int r = 0; r < k; ++r) {
    bool have = false;
    double bv = 0.0;
    uint32_t bi = 0;
#pragma unroll 1
    for (int s = 0; s < kE; ++s) {
      double val;
      uint32_t id;
      if (!c.value(s, val, id)) continue;
      if (has_floor && !ranks_before(val, id, fv, fid)) continue;
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
      s_rec_id[r] = wi | kPenFlag;
      s_rec_key[r] = rd_f32(wv);
    }
    pv = wv;
    pid = wi;
    ++got;
  }
  __syncthreads();
  return got;
}

// A chunk emitted more values than the list can take (heavy ties or a low
// bound): bound its keys exactly (at least k, at or above `floor_key`, at
// most `cap` unless ties) and emit again; with more than `cap` exact ties,
// fall back to repeated block argmax.  Keys are recomputed from memory.
// Every emitted entry carries kPenFlag (its exact value is recomputed from
// its count).  Returns the count.
__device__ uint32_t overflow_select(const ElemCtx &ec, int k, uint32_t floor_key, uint32_t cap, bool has_floor,
                                    double fv, uint32_t fid, uint32_t *s_rec_id, float *s_rec_key, uint32_t *s_hist,
                                    uint32_t *s_sel, uint32_t *s_on, Red *red) {
  auto key = [&](int i) {
    double val;
    uint32_t id;
    return ec.value(i, val, id) ? okey(rd_f32(val)) : 0u;
  };
  auto for_keys = [&](auto f) {
#pragma unroll 1
    for (int i = 0; i < kE; ++i) f(key(i));
  };
  uint32_t bound = radix_bound(for_keys, 31, 0u, (uint32_t)k, cap, s_hist, s_sel);
  bound = max(bound, floor_key);
  if (threadIdx.x == 0) *s_on = 0u;
  __syncthreads();
  emit_each<kE, 1>(
      ec.lo,
      [&](int i) {
        const uint32_t x = key(i);
        return x != 0u && x >= bound;
      },
      [&](int i) { return fkey(key(i)); }, cap, s_on, s_rec_id, s_rec_key);
  __syncthreads();
  uint32_t n = *s_on;
  if (n > cap) n = (uint32_t)chunk_topk_slow(ec, k, has_floor, fv, fid, s_rec_id, s_rec_key, red);
  return n;
}

// ------------------------------------------------------------------ merge --

// Block-wide max and min; every thread returns them.  LDS: red[2 * kWaves].
__device__ __forceinline__ void block_minmax(uint32_t &mx, uint32_t &mn, uint32_t *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  mx = wave_max_u32(mx);
  mn = wave_min_u32(mn);
  if (lane == 0) {
    red[wave] = mx;
    red[kWaves + wave] = mn;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    mx = max(mx, red[w]);
    mn = min(mn, red[kWaves + w]);
  }
}

// LDS of the merge (overlays the parts' count table and history list).
struct MergeLds {
  uint32_t cnt[kMaxParts];
  uint32_t hist[256];
  uint32_t sel[4];
  uint32_t red32[2 * kWaves];
  double m_val[kSurvCap];       // survivors
  uint32_t m_id[kSurvCap];
  uint32_t m_g[kSurvCap];       // their record slots
  uint32_t m_slot[kSurvCap];    // record slots of the survivors whose exact value is loaded
  uint64_t m_c[kSurvCap];       // survivors' rank keys: (okey, exact-value flag, ~id), larger first
  double t_val[SAS_MAX_TOP_K];  // the ranked top k
  uint32_t t_id[SAS_MAX_TOP_K];
  double t_p[SAS_MAX_TOP_K];    // exp weights (zero past k)
  double t_q[SAS_MAX_TOP_K];    // weights / sum
  double t_pre[SAS_MAX_TOP_K];  // running sums of the weights
  double t_cum[SAS_MAX_TOP_K];  // running sums of weights / sum
  double t_r[SAS_MAX_TOP_K];    // the draw residuals
  uint32_t n, over;
  Red red;
};


__device__ __forceinline__ uint64_t rec_kid(const uint64_t *rrow, int64_t slot) { return ld_agent(rrow + 2 * slot); }
// The fp32 key bits alone (the low word of the record's first half).
__device__ __forceinline__ uint32_t rec_key(const uint64_t *rrow, int64_t slot) {
  return ld_agent(reinterpret_cast<const uint32_t *>(rrow + 2 * slot));
}
__device__ __forceinline__ uint64_t rec_val(const uint64_t *rrow, int64_t slot) {
  return ld_agent(rrow + 2 * slot + 1);
}

// The merge of one row by its last part: bound, rank, sample() tail, outputs.
struct MergeOut {
  uint32_t *ids;
  double *probs;
  uint32_t *cand_ids;
  int32_t *counts;
  uint32_t *flags;
};

// Exact top k over every record of the row by wave 0 alone, k rounds of a
// wave argmax over memory (rare: records beyond the window or ties wider
// than the survivor buffer).  Returns the count.
__device__ int wave_topk_slow(const uint64_t *rrow, const uint32_t *cnt, int S, uint32_t lower, int k,
                              double *t_val, uint32_t *t_id) {
  const int lane = threadIdx.x & 63;
  double pv = 0.0;
  uint32_t pid = 0;
  int got = 0;
  for (int r = 0; r < k; ++r) {
    bool have = false;
    double bv = 0.0;
    uint32_t bi = 0;
    for (int q = 0; q < S; ++q) {
      for (uint32_t j = (uint32_t)lane; j < cnt[q]; j += 64u) {
        const int64_t g = (int64_t)q * kListCap + j;
        const uint64_t kv = rec_kid(rrow, g);
        const uint32_t x = okey(__uint_as_float((uint32_t)kv));
        if (x == 0u || x < lower) continue;
        const double val = __longlong_as_double((long long)rec_val(rrow, g));
        const uint32_t id = (uint32_t)(kv >> 32) & kIdMask;
        if (r > 0 && !ranks_before(pv, pid, val, id)) continue;
        if (!have || ranks_before(val, id, bv, bi)) {
          have = true;
          bv = val;
          bi = id;
        }
      }
    }
    wave_best(have, bv, bi);
    if (!__ballot(have)) break;
    bv = __shfl(bv, 0, 64);
    bi = (uint32_t)__shfl((int)bi, 0, 64);
    if (lane == 0) {
      t_val[r] = bv;
      t_id[r] = bi;
    }
    pv = bv;
    pid = bi;
    ++got;
  }
  __builtin_amdgcn_wave_barrier();
  return got;
}

// The merge of one row by wave 0 of its last part.  One round of loads
// brings the row's bound, the record counts and the first half (key, id) of
// a window of W slots of every part; a wave ballot search bounds the keys
// to the top k and a few ties; only records whose exact value differs from
// their key need a second load.  A bitonic sort ranks the survivors, then
// the sample() tail runs on registers: exp weights and divisions across
// lanes, each running sum in the reference's left-to-right order with its
// operands read lane by lane (no LDS round trips in the chains).
__device__ __forceinline__ void merge_row(const uint64_t *rrow, uint32_t *ctl, int S, int row, double temperature, double top_p,
                          int k, double u_row, MergeOut o, MergeLds &ml) {
  const int lane = threadIdx.x & 63;
  const bool greedy = !(temperature > 0.0);
  constexpr int R = 12;  // window slots per lane
  // window W >= k + 16 slots per part (a part writes k records and its
  // ties), a multiple of 8; slot g of the window is record g % W of part
  // g / W, the division by a multiply (exact for g < 2^12)
  const int W = (k + 16 + 7) & ~7;
  const uint32_t winv = ((1u << 20) + (uint32_t)W - 1u) / (uint32_t)W;
  auto wpart = [&](int g) { return (int)(((uint32_t)g * winv) >> 20); };
  auto wslot = [&](int g) { const int q = wpart(g); return (int64_t)q * kListCap + (g - q * W); };
  const bool windowed = S * W <= R * 64;
  // every load of the round is issued before any result is used
  const uint32_t my_cnt = lane < S ? ld_agent(ctl + kCtlCnt + lane) : 0u;
  uint64_t kid[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = r * 64 + lane;
    kid[r] = windowed && g < S * W ? rec_kid(rrow, wslot(g)) : 0u;
  }
  const uint32_t row_bound_v = ld_agent(ctl + kCtlThr);
  if (lane == 0) {
    // reset for the next launch (after this lane's loads of the same words)
    ctl[0] = 0u;
    ctl[kCtlThr] = 0u;
  }
  if (lane < S) ml.cnt[lane] = my_cnt;
  __builtin_amdgcn_wave_barrier();
  const uint32_t total = wave_sum_u32(my_cnt);
  bool compact = !windowed || __ballot(lane < S && my_cnt > (uint32_t)W) != 0;
  uint32_t flags = 0;
  int kk = 0;
  if (compact && total <= (uint32_t)(R * 64)) {
    // a second round: the records back to back, part by part
    uint32_t pre = lane < S ? my_cnt : 0u;
#pragma unroll
    for (int sh = 1; sh < 64; sh <<= 1) {
      const uint32_t t = (uint32_t)__shfl_up((int)pre, sh, 64);
      if (lane >= sh) pre += t;
    }
    if (lane < S) ml.m_g[lane] = pre - my_cnt;  // first record of part lane
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t j = (uint32_t)(r * 64 + lane);
      kid[r] = 0u;
      if (j < total) {
        int q = 0;
        for (int step = 32; step > 0; step >>= 1)
          if (q + step < S && ml.m_g[q + step] <= j) q += step;
        kid[r] = rec_kid(rrow, (int64_t)q * kListCap + (j - ml.m_g[q]));
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  const uint32_t row_bound = uni(row_bound_v);
  if (compact && total > (uint32_t)(R * 64)) {
    flags |= SAS_FLAG_SLOW_SELECT;
    kk = wave_topk_slow(rrow, ml.cnt, S, row_bound > 0u ? row_bound : 1u, k, ml.t_val, ml.t_id);
  } else {
    // keys (okey images) of the valid slots at or above the row's bound
    uint32_t key[R];
    uint32_t kmax = 0u, kmin = 0xFFFFFFFFu;
    int nv = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = r * 64 + lane;
      const uint32_t x = okey(__uint_as_float((uint32_t)kid[r]));
      const bool valid = compact ? (uint32_t)g < total
                                 : g < S * W && (uint32_t)(g - wpart(g) * W) < ml.cnt[wpart(g)];
      key[r] = valid && x >= row_bound ? x : 0u;
      if (key[r]) {
        kmax = max(kmax, key[r]);
        kmin = min(kmin, key[r]);
      }
      nv += __popcll(__ballot(key[r] != 0u));
    }
    kmax = wave_max_u32(kmax);
    kmin = wave_min_u32(kmin);
    // the largest bound (searched to 12 bits below the highest bit in which
    // the keys differ) that at least k keys reach: a lower bound of the
    // exact k-th key, so the top k all survive
    uint32_t lower = 1u;
    if (nv > k + kMergeSlack && kmax != kmin) {
      const int hb = 31 - __clz(kmax ^ kmin);
      auto for_keys = [&](auto f) {
#pragma unroll
        for (int r = 0; r < R; ++r) f(key[r]);
      };
      lower = max(wave_radix_bound(for_keys, hb, hb == 31 ? 0u : kmax >> (hb + 1), (uint32_t)k,
                                   (uint32_t)(k + kMergeSlack), ml.hist),
                  1u);
    }
    // survivors in LDS: value (the key, or the record's exact value), id
    int m = 0;
    bool need_val = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const bool keep = key[r] != 0u && key[r] >= lower;
      const uint64_t bb = __ballot(keep);
      if (keep) {
        const int d = m + (int)lanes_below(bb);
        if (d < kSurvCap) {
          const uint32_t idf = (uint32_t)(kid[r] >> 32);
          ml.m_id[d] = idf;
          ml.m_val[d] = (double)__uint_as_float((uint32_t)kid[r]);
          // an exact value lies strictly above its round-down key, so it
          // ranks before the plain values of the same key; the ids of the
          // plain ones then decide
          ml.m_c[d] = ((uint64_t)key[r] << 32) | (idf & kRecValFlag) | (0x7FFFFFFFu - (idf & kIdMask));
          if (idf & kRecValFlag) {
            // where the record lies, for the exact value
            const int g = r * 64 + lane;
            int64_t slot;
            if (compact) {
              int q = 0;
              for (int step = 32; step > 0; step >>= 1)
                if (q + step < S && ml.m_g[q + step] <= (uint32_t)g) q += step;
              slot = (int64_t)q * kListCap + ((uint32_t)g - ml.m_g[q]);
            } else {
              slot = wslot(g);
            }
            ml.m_slot[d] = (uint32_t)slot;
            need_val = true;
          }
        }
      }
      m += __popcll(bb);
    }
    __builtin_amdgcn_wave_barrier();
    if (m > kSurvCap) {
      flags |= SAS_FLAG_SLOW_SELECT;
      kk = wave_topk_slow(rrow, ml.cnt, S, lower, k, ml.t_val, ml.t_id);
    } else {
      // exact values of the flagged survivors: loads in flight during the rank
      const bool any_val = __ballot(need_val) != 0;
      double xv[kSurvCap / 64];
      if (any_val) {
#pragma unroll
        for (int t = 0; t < kSurvCap / 64; ++t) {
          const int i = t * 64 + lane;
          xv[t] = 0.0;
          if (i < m && (ml.m_id[i] & kRecValFlag)) xv[t] = __longlong_as_double((long long)rec_val(rrow, ml.m_slot[i]));
        }
      }
      // ---- exact rank ----------------------------------------------------
      // Ranks by the composite keys (one 64-bit compare per pair, LDS
      // broadcast reads): exact, unless two exact values share a key, which
      // takes the double compare.
      kk = min(m, k);
      // keys past m are zero (below every key) up to a multiple of 16
      const int m16 = (m + 15) & ~15;
      for (int i = m + lane; i < m16; i += 64) ml.m_c[i] = 0u;
      __builtin_amdgcn_wave_barrier();
      uint32_t rk[kSurvCap / 64];
      bool clash = false;
#pragma unroll
      for (int t = 0; t < kSurvCap / 64; ++t) {
        const int i = t * 64 + lane;
        rk[t] = 0u;
        if (t * 64 < m) {
          const uint64_t c = i < m ? ml.m_c[i] : ~0ull;
          const bool cf = (c & kRecValFlag) != 0;
          uint32_t rank = 0u;
          for (int j = 0; j < m16; j += 16) {
            uint64_t o[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) o[u] = ml.m_c[j + u];
#pragma unroll
            for (int u = 0; u < 16; ++u) rank += o[u] > c ? 1u : 0u;
          }
          rk[t] = rank;
          if (any_val && cf) {
            // another exact value under the same key
            for (int j = 0; j < m; ++j) {
              const uint64_t o = ml.m_c[j];
              clash |= (o >> 32) == (c >> 32) && (o & kRecValFlag) && o != c;
            }
          }
        }
      }
      if (any_val) {
#pragma unroll
        for (int t = 0; t < kSurvCap / 64; ++t) {
          const int i = t * 64 + lane;
          if (i < m && (ml.m_id[i] & kRecValFlag)) ml.m_val[i] = xv[t];
        }
        __builtin_amdgcn_wave_barrier();
      }
      if (__ballot(clash)) {
        // two exact values under one key: rank by (value, id) in double
#pragma unroll
        for (int t = 0; t < kSurvCap / 64; ++t) {
          const int i = t * 64 + lane;
          if (i < m) {
            const double vc = ml.m_val[i];
            const uint32_t ic = ml.m_id[i] & kIdMask;
            uint32_t rank = 0;
            for (int j = 0; j < m; ++j) rank += ranks_before(ml.m_val[j], ml.m_id[j] & kIdMask, vc, ic) ? 1u : 0u;
            rk[t] = rank;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < kSurvCap / 64; ++t) {
        const int i = t * 64 + lane;
        if (i < m && rk[t] < (uint32_t)k) {
          ml.t_val[rk[t]] = ml.m_val[i];
          ml.t_id[rk[t]] = ml.m_id[i] & kIdMask;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---- sample() tail (tokenizer.js:161-177), double precision, wave 0 ------
  // exp weights and divisions across lanes; each running sum is one chain in
  // the reference's left-to-right order, run by every lane alike on operands
  // read 16 at a time from LDS (a bare add per step), its values stored per
  // batch; the cut, the pick and the edge flags are found from the stored
  // values.
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
    const double p_a = lane < kk ? fd_exp((ml.t_val[lane] - v0) / T) : 0.0;
    const double p_b = lane + 64 < kk ? fd_exp((ml.t_val[lane + 64] - v0) / T) : 0.0;
    ml.t_p[lane] = p_a;
    ml.t_p[lane + 64] = p_b;
    __builtin_amdgcn_wave_barrier();
    const int nb = (kk + 15) >> 4;  // batches of 16 (the weights past kk are zero)
    double run = 0.0;
    for (int b = 0; b < nb; ++b) {
      double x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = ml.t_p[16 * b + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        run += x[u];
        x[u] = run;
      }
      if (lane == 0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) ml.t_pre[16 * b + u] = x[u];
      }
    }
    const double sum = run;
    q_a = p_a / sum;
    q_b = p_b / sum;
    ml.t_q[lane] = q_a;
    ml.t_q[lane + 64] = q_b;
    __builtin_amdgcn_wave_barrier();
    // top-p cut: the first i with p_0/sum + ... + p_i/sum >= top_p
    double cum = 0.0;
    cut = kk;
    for (int b = 0; b < nb; ++b) {
      double x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = ml.t_q[16 * b + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        cum += x[u];
        x[u] = cum;
      }
      if (lane == 0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) ml.t_cum[16 * b + u] = x[u];
      }
      uint32_t hit = 0u;
#pragma unroll
      for (int u = 0; u < 16; ++u) hit |= (x[u] >= top_p ? 1u : 0u) << u;
      hit = uni(hit) & (kk - 16 * b >= 16 ? 0xFFFFu : (1u << (kk - 16 * b)) - 1u);
      if (hit) {
        cut = 16 * b + __builtin_ctz(hit) + 1;
        break;
      }
    }
    __builtin_amdgcn_wave_barrier();
    // r = U * (p_0 + ... + p_{cut-1}), the sum taken left to right; the
    // first i at which r - p_0 - ... - p_i <= 0 is drawn
    const double sub = ml.t_pre[cut - 1];
    double r = u_row * sub;
    int pick = cut - 1;
    const int nc = (cut + 15) >> 4;
    for (int b = 0; b < nc; ++b) {
      double x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = ml.t_p[16 * b + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        r -= x[u];
        x[u] = r;
      }
      if (lane == 0) {
#pragma unroll
        for (int u = 0; u < 16; ++u) ml.t_r[16 * b + u] = x[u];
      }
      uint32_t hit = 0u;
#pragma unroll
      for (int u = 0; u < 16; ++u) hit |= (x[u] <= 0.0 ? 1u : 0u) << u;
      hit = uni(hit) & (cut - 16 * b >= 16 ? 0xFFFFu : (1u << (cut - 16 * b)) - 1u);
      if (hit) {
        pick = 16 * b + __builtin_ctz(hit);
        break;
      }
    }
    __builtin_amdgcn_wave_barrier();
    // edges: a running mass within 1e-6 of top_p up to the cut; a draw
    // residual within 1e-12 of the mass up to the pick
    bool te = false, de = false;
    for (int i = lane; i < kk; i += 64) {
      if (i < cut && fabs(ml.t_cum[i] - top_p) < 1e-6) te = true;
      if (i <= pick && fabs(ml.t_r[i]) <= 1e-12 * sub) de = true;
    }
    if (__ballot(te)) flags |= SAS_FLAG_TOPP_EDGE;
    if (__ballot(de)) flags |= SAS_FLAG_DRAW_EDGE;
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

// ------------------------------------------------------------------ parts --

// Offsets of lane slots in a wave: the prefix of this lane's count and the
// wave's total, by ballots over the count's bits (no LDS).
__device__ __forceinline__ void wave_prefix(uint32_t cnt, uint32_t &pre, uint32_t &tot) {
  pre = 0u;
  tot = 0u;
#pragma unroll
  for (int b = 0; b < 5; ++b) {
    const uint64_t bb = __ballot((cnt >> b) & 1u);
    pre += lanes_below(bb) << b;
    tot += (uint32_t)__popcll(bb) << b;
  }
}


// One wave's candidate list in LDS: fp32 key bits; id with kPenFlag when
// val holds the history count of a penalized value (else the value is the
// key) or kExactFlag when val holds the exact value.
struct WList {
  uint32_t *key;
  uint32_t *id;
  double *val;
};

// Keeps the entries whose key is >= t; returns the new count.  Wave-level:
// every lane reads its entries before any is written (LDS runs a wave's
// instructions in order).
__device__ __forceinline__ uint32_t wave_list_keep(const WList &l, uint32_t n, uint32_t t) {
  const int lane = threadIdx.x & 63;
  uint32_t kb[4], ib[4];
  double vb[4];
  bool keep[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t i = (uint32_t)(j * 64 + lane);
    keep[j] = false;
    kb[j] = 0u;
    ib[j] = 0u;
    vb[j] = 0.0;
    if (i < n) {
      kb[j] = l.key[i];
      ib[j] = l.id[i];
      vb[j] = l.val[i];
      keep[j] = okey(__uint_as_float(kb[j])) >= t;
    }
  }
  uint32_t base = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint64_t bb = __ballot(keep[j]);
    if (keep[j]) {
      const uint32_t d = base + lanes_below(bb);
      l.key[d] = kb[j];
      l.id[d] = ib[j];
      l.val[d] = vb[j];
    }
    base += (uint32_t)__popcll(bb);
  }
  return uni(base);
}

// The redo list: candidates of deferred chunk slices, selected exactly
// after the chunk loop.
struct Redo {
  uint32_t key[kCapBlock];
  uint32_t id[kCapBlock];
  double val[kCapBlock];
  uint32_t slices[kWaves][kRedoCap];
  uint32_t nslices[kWaves];
  uint32_t n;
  double fv;
  uint32_t fid;
  uint32_t has_floor;
};

// Keeps the exact top k of the redo list by (value, id) and records the
// k-th as the floor of later selections.  Block-wide, barriers.
__device__ void redo_topk(Redo &r, int k, const float *lrow, const sas_params &p, const HistView &hv,
                          uint32_t *s_tmp) {
  const int tid = threadIdx.x;
  const uint32_t n = r.n;
  for (uint32_t i = tid; i < n; i += kThreads) {
    const uint32_t idf = r.id[i];
    if (idf & kPenFlag) {
      const uint32_t id = idf & kIdMask;
      r.val[i] = exact_value(lrow, id, hv.member(id) ? hv.count(id) : 0u, p);
      r.id[i] = id | kExactFlag;
    } else if (!(idf & kExactFlag)) {
      r.val[i] = (double)__uint_as_float(r.key[i]);
      r.id[i] = idf | kExactFlag;
    }
  }
  __syncthreads();
  uint32_t keep_bits = 0u;
  constexpr int R = kCapBlock / kThreads;
  uint32_t kb[R], ib[R];
  double vb[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const uint32_t i = (uint32_t)(j * kThreads + tid);
    kb[j] = ib[j] = 0u;
    vb[j] = 0.0;
    if (i < n) {
      kb[j] = r.key[i];
      ib[j] = r.id[i];
      vb[j] = r.val[i];
      uint32_t rank = 0;
      for (uint32_t q = 0; q < n; ++q) rank += ranks_before(r.val[q], r.id[q] & kIdMask, vb[j], ib[j] & kIdMask) ? 1u : 0u;
      if (rank < (uint32_t)k) keep_bits |= 1u << j;
      if (rank == (uint32_t)k - 1u) {
        r.fv = vb[j];
        r.fid = ib[j] & kIdMask;
        r.has_floor = 1u;
      }
    }
  }
  __syncthreads();
  if (tid == 0) *s_tmp = 0u;
  __syncthreads();
  uint32_t slot = wave_reserve(keep_bits, s_tmp);
#pragma unroll
  for (int j = 0; j < R; ++j)
    if ((keep_bits >> j) & 1u) {
      r.key[slot] = kb[j];
      r.id[slot] = ib[j];
      r.val[slot] = vb[j];
      ++slot;
    }
  __syncthreads();
  if (tid == 0) r.n = *s_tmp;
  __syncthreads();
}

// A lower bound, at least `floor`, of the k-th largest of the wave's keys
// (okey images, 0 = none): at least k keys are >= the result unless it is
// floor.  The 16 bits below the highest bit in which floor and the largest
// key differ are searched by ballots; the bits under them stay zero.
template <int N>
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&x)[N], int k, uint32_t floor) {
  uint32_t kmax = 0u;
#pragma unroll
  for (int j = 0; j < N; ++j) kmax = max(kmax, x[j]);
  kmax = wave_max_u32(kmax);
  if (kmax <= floor) return floor;
  const int hb = 31 - __clz(kmax ^ floor);
  uint32_t res = hb == 31 ? 0u : (kmax >> (hb + 1)) << (hb + 1);
  const int lo = hb >= 15 ? hb - 15 : 0;
  for (int b = hb; b >= lo; --b) {
    const uint32_t cand = res | (1u << b);
    int c = 0;
#pragma unroll
    for (int j = 0; j < N; ++j) c += __popcll(__ballot(x[j] >= cand));
    if (c >= k) res = cand;
  }
  return max(res, floor);
}

// Barrier over the block's LDS accesses alone: it waits for this wave's LDS
// operations but not for its global loads, so prefetched chunks stay in
// flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <bool kMask, bool kHist, bool kSoftcap>
__global__ __launch_bounds__(kThreads, 4) void sample_kernel(const SampleArgs a) {
  constexpr size_t kHistBytes = kHist ? sizeof(PartHist) : 16;
  constexpr size_t kRawBytes = kHistBytes > sizeof(MergeLds) ? kHistBytes : sizeof(MergeLds);
  __shared__ __align__(16) unsigned char s_raw[kRawBytes];  // the part's history, then the merge's LDS
  __shared__ uint32_t l_key[kWaves * kWaveCap];
  __shared__ uint32_t l_id[kWaves * kWaveCap];
  __shared__ double l_val[kWaves * kWaveCap];
  __shared__ Redo s_redo;
  __shared__ uint32_t s_bthr;                       // the part's bound (okey image), raised by any wave
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[4];
  __shared__ uint32_t s_on, s_tmp;
  __shared__ int s_last;
  __shared__ Red s_red;
  PartHist &ph = *reinterpret_cast<PartHist *>(s_raw);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows = a.rows, P = a.parts;
  int lb = blockIdx.x;
  // XCD-aware order: consecutive dispatches rotate over the 8 XCDs, so give
  // each XCD a contiguous run of rows; a row's parts then share one L2 for
  // the history, the mask and the records.
  const int nblocks = rows * P;
  if ((nblocks & 7) == 0) lb = (lb & 7) * (nblocks >> 3) + (lb >> 3);
  const int row = lb / P;
  const int part = lb - row * P;
  const int c0 = part * a.cpp;
  const int c1 = min(c0 + a.cpp, a.chunks);
  const int vocab = a.vocab;
  const uint32_t plo = (uint32_t)c0 * kChunkIds;
  const uint32_t pspan = (uint32_t)min(c1 * kChunkIds, vocab) - plo;

  const sas_params p = a.row_params ? a.row_params[row] : a.params;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const double u_row = greedy ? 0.0 : a.uniforms[row];  // read early: the merge needs it last
  const float softcap = kSoftcap ? p.softcap : 0.0f;
  const float *lrow = a.logits + (int64_t)row * a.logits_stride;
  const uint32_t *mrow = kMask ? a.mask + (int64_t)row * a.mask_stride : nullptr;
  const uint32_t *hist_ids = a.hist_ids;
  uint32_t *ctl = a.ctl + (int64_t)row * kCtlStride;

  // ---- chunk loads ---------------------------------------------------------
  // Every lane issues the same loads for every chunk, and nothing reads a
  // loaded value here, so the compiler waits for one chunk's loads while the
  // next chunk's stay in flight.  A float4 is loaded from element
  // max(min(e, vocab - 4), 0): 16 bytes inside the row (rows hold at least 4
  // floats; the loads need 4-byte alignment only).  The float4 that
  // straddles the end of the row is shifted back, and ids past the end are
  // replaced, when the row's last chunk is processed.
  const int last_word = ((vocab + 31) >> 5) - 1;
  auto load_at = [&](int e) { return max(min(e, vocab - 4), 0); };
  auto load_chunk = [&](int c, float4 (&v)[kF4], uint32_t (&mw)[kF4]) __attribute__((always_inline)) {
    const int lo = c * kChunkIds;
#pragma unroll
    for (int f = 0; f < kF4; ++f) {
      const f32x4u t = __builtin_nontemporal_load(reinterpret_cast<const f32x4u *>(lrow + load_at(lo + 4 * (f * kThreads + tid))));
      v[f] = make_float4(t.x, t.y, t.z, t.w);
    }
    if (kMask) {
#pragma unroll
      for (int f = 0; f < kF4; ++f) mw[f] = mrow[max(min((lo >> 5) + f * (kThreads / 8) + (tid >> 3), last_word), 0)];
    }
  };
  // Chunk c, or past the part's end a dummy that reads the row's first
  // cache line: every iteration issues the same loads, so the compiler
  // never has to assume a chunk's loads are the youngest outstanding.
  constexpr int kNoChunk = -(1 << 18);
  auto prefetch = [&](int c, float4 (&v)[kF4], uint32_t (&mw)[kF4]) __attribute__((always_inline)) {
    load_chunk(c < c1 ? c : kNoChunk, v, mw);
  };

  float4 va[kF4], vb[kF4];
  uint32_t ma[kF4], mb[kF4];
  load_chunk(c0, va, ma);

  // ---- the part's history: membership bitmap and (id, count) hash ------------
  // The first ids are loaded with the first chunk, and the barriers wait on
  // LDS alone, so the chunk's loads stay in flight while the tables fill.
  int h0 = 0, h1 = 0;
  if (kHist) {
    h0 = a.hist_offsets[row];
    h1 = a.hist_offsets[row + 1];
  }
  const bool has_hist = kHist && h1 > h0;
  // Penalties that can only lower a value (repetition >= 1, frequency and
  // presence >= 0) are applied to the emitted candidates alone: the raw
  // value bounds the penalized one from above, so no candidate is lost.
  const bool pen_in_loop =
      has_hist && !(p.repetition_penalty >= 1.0 && p.frequency_penalty >= 0.0 && p.presence_penalty >= 0.0);
  uint32_t hreg[kHistRegs];
#pragma unroll
  for (int j = 0; j < kHistRegs; ++j) {
    const int i = h0 + j * kThreads + tid;
    hreg[j] = has_hist && i < h1 ? hist_ids[i] : kEmpty;
  }
  if (tid == 0) s_bthr = 0u;
  if (tid == 0) {
    s_redo.n = 0u;
    s_redo.has_floor = 0u;
  }
  if (tid < kWaves) s_redo.nslices[tid] = 0u;
  if (has_hist) {
    const int words = (int)((pspan + 31u) >> 5);
    for (int w = tid; w < words; w += kThreads) ph.bits[w] = 0u;
    for (int sl = tid; sl < kHashSlots; sl += kThreads) {
      ph.key[sl] = kEmpty;
      ph.cnt[sl] = 0u;
    }
    if (tid == 0) ph.over = 0u;
    lds_barrier();
    auto insert = [&](uint32_t id) {
      const uint32_t off = id - plo;
      if (off >= pspan) return;
      atomicOr(&ph.bits[off >> 5], 1u << (off & 31));
      uint32_t sl = hash_slot(id);
      int probe = 0;
      for (; probe < kHashSlots; ++probe) {
        const uint32_t old = atomicCAS(&ph.key[sl], kEmpty, id);
        if (old == kEmpty || old == id) {
          atomicAdd(&ph.cnt[sl], 1u);
          break;
        }
        sl = (sl + 1u) & (uint32_t)(kHashSlots - 1);
      }
      if (probe == kHashSlots) ph.over = 1u;
    };
#pragma unroll
    for (int j = 0; j < kHistRegs; ++j) insert(hreg[j]);
    for (int i = h0 + kHistRegs * kThreads + tid; i < h1; i += kThreads) insert(hist_ids[i]);
  }
  lds_barrier();
  // The hot path reads the tables straight from LDS (ds_read only, never a
  // generic-pointer load that the compiler would have to wait for together
  // with the prefetched chunks).
  auto hmember = [&](uint32_t id) {
    const uint32_t off = id - plo;
    return (ph.bits[off >> 5] >> (off & 31u)) & 1u;
  };
  auto hcount = [&](uint32_t id) {
    uint32_t sl = hash_slot(id);
    for (int probe = 0; probe < kHashSlots; ++probe) {
      const uint32_t kk = ph.key[sl];
      if (kk == id) return ph.cnt[sl];
      if (kk == kEmpty) break;
      sl = (sl + 1u) & (uint32_t)(kHashSlots - 1);
    }
    uint32_t cnt = 0u;
    if (ph.over)
      for (int i = h0; i < h1; ++i) cnt += hist_ids[i] == id ? 1u : 0u;
    return cnt;
  };

  // ---- this wave's list and bound ------------------------------------------
  const WList wl{l_key + wave * kWaveCap, l_id + wave * kWaveCap, l_val + wave * kWaveCap};
  uint32_t n_w = 0u;    // entries in the wave's list
  uint32_t thr_w = 0u;  // okey bound: at least k values of this wave's slices reach it
  // the list is re-bounded when it reaches this many entries
  const uint32_t n_tight = (uint32_t)(k + max(k, 32));

  // Re-bounds the list by its own k-th largest key (at least the block's
  // bound), drops what falls below, and shares the bound with the block.
  auto tighten = [&]() __attribute__((always_inline)) {
    uint32_t x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = (uint32_t)(j * 64 + lane);
      x[j] = i < n_w ? okey(__uint_as_float(wl.key[i])) : 0u;
    }
    thr_w = wave_kth(x, k, max(thr_w, uni(s_bthr)));
    n_w = wave_list_keep(wl, n_w, thr_w);
    if (lane == 0) atomicMax(&s_bthr, thr_w);
  };

  // ---- one chunk: this wave's slice of 16 values per lane -------------------
  // The first chunk also bounds the slice by its own k-th largest value, so
  // that later chunks emit little.
  auto process = [&](auto first_tag, int c, float4 (&v)[kF4], uint32_t (&mw)[kF4]) {
    constexpr bool kFirst = decltype(first_tag)::value;
    const int lo = c * kChunkIds;
    if (lo + kChunkIds > vocab) {
      // the row's last, partial chunk: the float4 loaded from an earlier
      // element is shifted into place; ids past the vocabulary hold no value
#pragma unroll
      for (int f = 0; f < kF4; ++f) {
        const int e = lo + 4 * (f * kThreads + tid);
        const int sh = e - load_at(e);  // 0 except for the float4 that straddles the end
        if (sh > 0) {
          // sh = 1..3 (the slots past the row's end are replaced below)
          const float ty = v[f].y, tz = v[f].z, tw = v[f].w;
          v[f].x = sh == 1 ? ty : sh == 2 ? tz : tw;
          v[f].y = sh == 1 ? tz : tw;
          v[f].z = tw;
        }
        if (e + 0 >= vocab) v[f].x = qnan();
        if (e + 1 >= vocab) v[f].y = qnan();
        if (e + 2 >= vocab) v[f].z = qnan();
        if (e + 3 >= vocab) v[f].w = qnan();
        if (kMask && (lo >> 5) + f * (kThreads / 8) + (tid >> 3) > last_word) mw[f] = 0u;
      }
    }
#pragma unroll
    for (int f = 0; f < kF4; ++f) {
      if (kSoftcap && softcap > 0.0f) {
        v[f].x = softcap_f32(v[f].x, softcap);
        v[f].y = softcap_f32(v[f].y, softcap);
        v[f].z = softcap_f32(v[f].z, softcap);
        v[f].w = softcap_f32(v[f].w, softcap);
      }
      if (kMask) {
        // bit j of the nibble -> all ones or zero, then one bit-field insert
        // keeps the value or puts a quiet NaN in its place
        const uint32_t sh = 4u * (uint32_t)(tid & 7);
        auto keep = [&](float x, uint32_t bit) {
          const uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)mw[f], sh + bit, 1u);  // 0 or ~0
          return __uint_as_float((m & __float_as_uint(x)) | (~m & 0x7FC00000u));
        };
        v[f].x = keep(v[f].x, 0u);
        v[f].y = keep(v[f].y, 1u);
        v[f].z = keep(v[f].z, 2u);
        v[f].w = keep(v[f].w, 3u);
      }
      if (kHist && pen_in_loop) {
        // penalties that may raise a value: applied before the bound test
        const uint32_t off = (uint32_t)(lo - (int)plo) + 4u * (uint32_t)(f * kThreads + tid);
        const uint32_t hb = (ph.bits[off >> 5] >> (off & 31u)) & 0xFu;
        if (hb) {
          float x[4] = {v[f].x, v[f].y, v[f].z, v[f].w};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (((hb >> j) & 1u) && x[j] == x[j])
              x[j] = rd_f32(penalize((double)x[j], hcount(plo + off + (uint32_t)j), p));
          v[f] = make_float4(x[0], x[1], x[2], x[3]);
        }
      }
    }
    auto elem = [&](int i) -> float {
      const int f = i >> 2, j = i & 3;
      return j == 0 ? v[f].x : j == 1 ? v[f].y : j == 2 ? v[f].z : v[f].w;
    };
    auto elem_id = [&](int i) -> uint32_t { return (uint32_t)(lo + 4 * ((i >> 2) * kThreads + tid) + (i & 3)); };
    float m1 = qnan();
#pragma unroll
    for (int i = 0; i < kE; ++i) m1 = fmaxf(m1, elem(i));

    uint32_t eff = uni(max(thr_w, s_bthr));
    // keys at or below okey(-inf) (0 or truncated) admit every valid value
    auto thr_of = [](uint32_t e) { return e > 0x007FFFFFu ? fkey(e) : -__builtin_inff(); };
    float thr = thr_of(eff);
    if (!__ballot(m1 >= thr)) return;

    auto bits_of = [&](float t) {
      uint32_t b = 0u;
#pragma unroll
      for (int i = 0; i < kE; ++i) b |= (elem(i) >= t ? 1u : 0u) << i;
      return b;
    };
    if (kFirst) {
      uint32_t x[kE];
      // a value that is only an upper bound (penalties not yet applied) is
      // left out of the count: the bound stays a lower bound
#pragma unroll
      for (int i = 0; i < kE; ++i) {
        const bool ub = has_hist && !pen_in_loop && hmember(elem_id(i));
        x[i] = ub ? 0u : okey(elem(i));
      }
      thr_w = wave_kth(x, k, 0u);
      if (lane == 0) atomicMax(&s_bthr, thr_w);
      eff = uni(max(thr_w, s_bthr));
      thr = thr_of(eff);
    }
    uint32_t bits = bits_of(thr);
    uint32_t pre, tot;
    wave_prefix(__popc(bits), pre, tot);
    tot = uni(tot);
    if (n_w + tot > (uint32_t)kWaveCap) {
      // make room: re-bound the list
      if (!kFirst && n_w >= (uint32_t)k) {
        tighten();
        eff = uni(max(thr_w, s_bthr));
        thr = thr_of(eff);
        bits = bits_of(thr);
        wave_prefix(__popc(bits), pre, tot);
        tot = uni(tot);
      }
      if (n_w + tot > (uint32_t)kWaveCap) {
        // more than the list can take (ties, or values rising chunk after
        // chunk): select this slice exactly after the loop
        if (lane == 0) {
          const uint32_t r = s_redo.nslices[wave]++;
          if (r < (uint32_t)kRedoCap) s_redo.slices[wave][r] = (uint32_t)c;
        }
        return;
      }
    }
    uint32_t slot = n_w + pre;
#pragma unroll
    for (int i = 0; i < kE; ++i)
      if ((bits >> i) & 1u) {
        wl.key[slot] = __float_as_uint(elem(i));
        wl.id[slot] = elem_id(i);
        ++slot;
      }
    const uint32_t n0 = n_w;
    n_w += tot;
    if (has_hist) {
      // history members: the exact penalized key and the count
      for (uint32_t i = n0 + (uint32_t)lane; i < n_w; i += 64u) {
        const uint32_t id = wl.id[i];
        if (hmember(id)) {
          const uint32_t cnt = hcount(id);
          if (!pen_in_loop) {
            // the exact value is kept: the records need no second read
            const double ev = penalize((double)__uint_as_float(wl.key[i]), cnt, p);
            wl.key[i] = __float_as_uint(rd_f32(ev));
            wl.id[i] = id | kExactFlag;
            wl.val[i] = ev;
          } else {
            wl.id[i] = id | kPenFlag;
            wl.val[i] = (double)cnt;
          }
        }
      }
    }
    if (n_w >= n_tight) tighten();
  };

  // ---- the chunk loop: the next chunk's loads are in flight during each ----
  using First = std::integral_constant<bool, true>;
  using Next = std::integral_constant<bool, false>;
  prefetch(c0 + 1, vb, mb);
  process(First{}, c0, va, ma);
  for (int c = c0 + 1; c < c1; c += 2) {
    prefetch(c + 1, va, ma);
    process(Next{}, c, vb, mb);
    if (c + 1 >= c1) break;
    prefetch(c + 2, vb, mb);
    process(Next{}, c + 1, va, ma);
  }
  __syncthreads();

  // ---- the part's bound; deferred slices -------------------------------------
  // The rare paths below take the parameters and the history by reference
  // (their addresses escape to out-of-line code): copies of their own keep
  // the chunk loop's values in registers.
  const sas_params p_rare = p;
  const HistView hv{has_hist ? &ph : nullptr, plo, hist_ids, h0, h1};
  // Every list holds all of its wave's values at or above the largest wave
  // bound, so the k-th largest key of their union bounds the part exactly.
  uint32_t pbound = s_bthr;
  n_w = wave_list_keep(wl, n_w, pbound);
  {
    uint32_t key4[4];
    uint32_t kmax = 0u, kmin = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = (uint32_t)(j * 64 + lane);
      key4[j] = i < n_w ? okey(__uint_as_float(wl.key[i])) : 0u;
      if (key4[j]) {
        kmax = max(kmax, key4[j]);
        kmin = min(kmin, key4[j]);
      }
    }
    if (tid == 0) s_tmp = 0u;
    block_minmax(kmax, kmin, s_hist);
    if (lane == 0) atomicAdd(&s_tmp, n_w);
    __syncthreads();
    const uint32_t total = s_tmp;
    __syncthreads();
    if (total > (uint32_t)k && kmax != kmin) {
      const int hb = 31 - __clz(kmax ^ kmin);
      auto for_keys = [&](auto f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) f(key4[j]);
      };
      pbound = max(pbound, radix_bound(for_keys, hb, hb == 31 ? 0u : kmax >> (hb + 1), (uint32_t)k,
                                       (uint32_t)k + 16u, s_hist, s_sel));
    } else if (total > (uint32_t)k) {
      pbound = max(pbound, kmax);
    }
  }
  const uint32_t bound = pbound;
  if (tid == 0) __hip_atomic_fetch_max(ctl + kCtlThr, pbound, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int w = 0; w < kWaves; ++w) {
    const uint32_t ns = min(s_redo.nslices[w], (uint32_t)kRedoCap);
    for (uint32_t r = 0; r < ns; ++r) {
      if (s_redo.n > 0u) redo_topk(s_redo, k, lrow, p_rare, hv, &s_tmp);
      const uint32_t n0 = s_redo.n;
      const ElemCtx ec{lrow, mrow, hv, (int)s_redo.slices[w][r] * kChunkIds, vocab, p_rare, w};
      const uint32_t m = overflow_select(ec, k, bound, (uint32_t)kCapBlock - n0, s_redo.has_floor != 0u, s_redo.fv,
                                         s_redo.fid, s_redo.id + n0, reinterpret_cast<float *>(s_redo.key + n0),
                                         s_hist, s_sel, &s_on, &s_red);
      // every entry of this path carries its history count for the exact value
      for (uint32_t i = tid; i < m; i += kThreads) s_redo.val[n0 + i] = (double)ec.count(s_redo.id[n0 + i] & kIdMask);
      __syncthreads();
      if (tid == 0) s_redo.n = n0 + m;
      __syncthreads();
    }
  }

  // ---- records out ------------------------------------------------------
  if (tid == 0) s_on = 0u;
  __syncthreads();
  uint64_t *rout = a.rec + ((int64_t)row * P + part) * kListCap * 2;
  auto write_entries = [&](const uint32_t *key, const uint32_t *idv, const double *val, uint32_t n, uint32_t i0) {
    for (uint32_t ib = 0; ib < n; ib += 64) {
      const uint32_t i = ib + (uint32_t)lane;
      bool keep = false;
      uint32_t kb = 0u, id = 0u;
      double x = 0.0;
      if (i < n) {
        kb = key[i0 + i];
        keep = okey(__uint_as_float(kb)) >= bound;
        if (keep) {
          const uint32_t idf = idv[i0 + i];
          id = idf & kIdMask;
          x = (idf & kPenFlag)     ? exact_value(lrow, id, (uint32_t)val[i0 + i], p)
              : (idf & kExactFlag) ? val[i0 + i]
                                   : (double)__uint_as_float(kb);
        }
      }
      // one LDS atomic per wave for the slots
      const uint64_t bb = __ballot(keep);
      uint32_t base = 0u;
      if (lane == 0 && bb) base = atomicAdd(&s_on, (uint32_t)__popcll(bb));
      base = __builtin_amdgcn_readlane(base, 0);
      if (keep) {
        const uint32_t slot = base + lanes_below(bb);
        if (slot < (uint32_t)kListCap) {
          if (x != (double)__uint_as_float(kb)) id |= kRecValFlag;
          st_agent(rout + 2 * slot, (uint64_t)kb | ((uint64_t)id << 32));
          st_agent(rout + 2 * slot + 1, (uint64_t)__double_as_longlong(x));
        }
      }
    }
  };
  // each wave writes its own list; wave 0 also the redo list
  write_entries(wl.key, wl.id, wl.val, n_w, 0u);
  if (wave == 0 && s_redo.n) write_entries(s_redo.key, s_redo.id, s_redo.val, s_redo.n, 0u);
  __syncthreads();
  if (tid == 0) st_agent(ctl + kCtlCnt + part, min(s_on, (uint32_t)kListCap));

  // ---- count in; the row's last part merges --------------------------------
  wait_vm();  // this wave's records, count and threshold are complete
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(P - 1);
  __syncthreads();
  // every part of the row has counted in and published its bound
  if (!s_last || wave != 0) return;
  const MergeOut o{a.out_ids, a.out_probs, a.out_cand_ids, a.out_counts, a.out_flags};
  merge_row(a.rec + (int64_t)row * P * kListCap * 2, ctl, P, row, p.temperature, p.top_p, k, u_row, o,
            *reinterpret_cast<MergeLds *>(s_raw));
}

// Parts per row: about `target` blocks in all (every block resident at
// once), at most kMaxParts per row, at least one chunk each.
void choose_parts(int rows, int vocab, int target, int *parts, int *cpp) {
  const int chunks = (vocab + kChunkIds - 1) / kChunkIds;
  const long long want = target > 0 ? target : 1024;
  long long c = rows > 0 ? ((long long)rows * chunks + want - 1) / want : chunks;
  if (c < 1) c = 1;
  if ((chunks + c - 1) / c > kMaxParts) c = (chunks + kMaxParts - 1) / kMaxParts;
  if (c > kMaxCpp) c = kMaxCpp;
  *cpp = (int)c;
  *parts = (int)((chunks + c - 1) / c);
}

static int variant_of(bool mask, bool hist, bool softcap) { return (mask ? 4 : 0) | (hist ? 2 : 0) | (softcap ? 1 : 0); }

template <bool kMask, bool kHist, bool kSoftcap>
static int occupancy_one() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, sample_kernel<kMask, kHist, kSoftcap>, kThreads, 0) !=
      hipSuccess)
    return 0;
  return n;
}

int sample_blocks_per_cu(bool mask, bool hist, bool softcap) {
  switch (variant_of(mask, hist, softcap)) {
    case 0: return occupancy_one<false, false, false>();
    case 1: return occupancy_one<false, false, true>();
    case 2: return occupancy_one<false, true, false>();
    case 3: return occupancy_one<false, true, true>();
    case 4: return occupancy_one<true, false, false>();
    case 5: return occupancy_one<true, false, true>();
    case 6: return occupancy_one<true, true, false>();
    default: return occupancy_one<true, true, true>();
  }
}

size_t sample_rec_bytes(int rows, int parts) { return (size_t)rows * parts * kListCap * 16; }

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
static void launch_one(const SampleArgs &a, hipStream_t stream) {
  hipLaunchKernelGGL((sample_kernel<kMask, kHist, kSoftcap>), dim3((unsigned)(a.rows * a.parts)), dim3(kThreads), 0,
                     stream, a);
}

hipError_t launch_sample(const SampleArgs &a, bool softcap, hipStream_t stream) {
  switch (variant_of(a.mask != nullptr, a.hist_ids != nullptr, softcap)) {
    case 0: launch_one<false, false, false>(a, stream); break;
    case 1: launch_one<false, false, true>(a, stream); break;
    case 2: launch_one<false, true, false>(a, stream); break;
    case 3: launch_one<false, true, true>(a, stream); break;
    case 4: launch_one<true, false, false>(a, stream); break;
    case 5: launch_one<true, false, true>(a, stream); break;
    case 6: launch_one<true, true, false>(a, stream); break;
    default: launch_one<true, true, true>(a, stream); break;
  }
  return hipGetLastError();
}

}  // namespace sas

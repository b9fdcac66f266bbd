// sample_kernel.hip - fused logit processing + top-k/top-p sampling for gfx950.
//
// One launch per decode step.  Grid = rows x splits blocks; block (row, s)
// owns vocabulary chunk [s*CHUNK, (s+1)*CHUNK) of one row:
//
//   1. the chunk's fp32 logits (128-bit loads straight into registers,
//      CHUNK/256 values per thread), its mask words (one 32-bit load per
//      float4; the 8 threads of a word share it), the row's published
//      threshold and its history ids, counted into a packed u16 LDS table;
//   2. per value: softcap, mask (masked -> NaN, never selected), history
//      penalties for the few ids with a count (double precision, kept as a
//      round-down fp32 key; the exact double is recomputed when emitted);
//   3. block threshold: the j-th largest lane max of each wave by a ballot
//      search over order-preserving keys, combined so that >= top_k values
//      are >= it.  It is published to the row (atomic max, not waited on):
//      a chunk of the row that starts later drops everything below the
//      largest threshold published so far, since the row's top_k cannot
//      lie there;
//   4. values >= the threshold (typically a little over top_k of them) are
//      appended to an LDS list (one LDS atomic per wave) and written into
//      the block's own record slots with their count;
//   5. the block counts itself in on the row (one atomic on a counter with
//      a cache line to itself); the row's last block merges:
//   6. a radix search over the row's record keys (8-bit digits starting at
//      the highest bit in which they differ) finds a bound keeping at least
//      top_k and at most top_k + kMergeSlack records; the survivors are
//      ranked exactly by (value desc, id asc) in double;
//   7. the reference's sample() tail in double precision: exp weights and
//      divisions across lanes, the running sums sequentially in JS order.
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
#include "sas_device.h"
#include "sas_launch.h"

namespace sas {

template <int F4>
struct SplitLds {
  static constexpr int kChunk = F4 * 1024;
  static constexpr int kCountWords = kChunk / 2;  // two u16 counts per word
};

constexpr int kHistRegs = 4;     // history ids per thread held in registers
constexpr int kSurvCap = 256;    // survivors the merge ranks in LDS
constexpr int kMergeSlack = 32;  // survivors beyond top_k the merge aims for
constexpr int kMergeRegs = 32;   // blocks per row whose record keys the merge holds in registers

// LDS used by block-wide reductions.
struct Red {
  int have[kWaves];
  double v[kWaves];
  uint32_t id[kWaves];
};

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
__device__ uint32_t radix_bound(ForKeys for_keys, int hb, uint32_t hprefix, uint32_t need, uint32_t cap,
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

// Appends the ids whose predicate holds to the LDS candidate list with one
// LDS atomic per wave per element slot (the rare paths).
template <int E, int U, typename Pred, typename Key>
__device__ __forceinline__ void emit_each(int lo, uint32_t penbits, Pred pred_of, Key key_of, uint32_t *s_n,
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
        if (slot < (uint32_t)kCapBlock) {
          const uint32_t id = (uint32_t)(lo + 4 * (f * kThreads + tid) + j);
          s_rec_id[slot] = id | (((penbits >> i) & 1u) ? kPenFlag : 0u);
          s_rec_key[slot] = key_of(i);
        }
      }
    }
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

// More than kCapBlock values passed the wave thresholds (few valid lanes or
// heavy ties): bound the block's keys exactly (at least k, at or above
// `floor_key`) and emit again; with more than kCapBlock exact ties, fall
// back to repeated block argmax.  The keys are recomputed from memory, so
// nothing of the hot path's registers is live here.  Returns the count.
template <int E>
__device__ uint32_t overflow_select(const ElemCtx &ec, int k, uint32_t floor_key, uint32_t *s_rec_id,
                                                 float *s_rec_key, uint32_t *s_hist, uint32_t *s_sel,
                                                 uint32_t *s_n, Red *red) {
  auto key = [&](int i) {
    double val;
    uint32_t id;
    return ec.value(i, val, id) ? okey(rd_f32(val)) : 0u;
  };
  auto for_keys = [&](auto f) {
#pragma unroll 4
    for (int i = 0; i < E; ++i) f(key(i));
  };
  uint32_t bound = radix_bound(for_keys, 31, 0u, (uint32_t)k, (uint32_t)kCapBlock, s_hist, s_sel);
  bound = max(bound, floor_key);
  if (threadIdx.x == 0) *s_n = 0u;
  __syncthreads();
  // every record of this path recomputes its exact value when written
  emit_each<E, 4>(
      ec.lo, ~0u,
      [&](int i) {
        const uint32_t x = key(i);
        return x != 0u && x >= bound;
      },
      [&](int i) { return fkey(key(i)); }, s_n, s_rec_id, s_rec_key);
  __syncthreads();
  uint32_t n = *s_n;
  if (n > (uint32_t)kCapBlock) n = (uint32_t)block_topk_slow(ec, E, k, s_rec_id, s_rec_key, red);
  return n;
}

// ------------------------------------------------------------------ merge --

// Block-wide max and min; every thread returns them.  LDS: red[2 * kWaves].
__device__ __forceinline__ void block_minmax(uint32_t &mx, uint32_t &mn, uint32_t *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    mx = max(mx, (uint32_t)__shfl_xor((int)mx, s, 64));
    mn = min(mn, (uint32_t)__shfl_xor((int)mn, s, 64));
  }
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

// A row's candidate records: block b's j-th at slot b*kCapBlock + j, read
// with agent-scope loads.
struct RowRecs {
  const uint32_t *key;  // fp32 bits
  const uint32_t *id;
  const uint64_t *val;  // fp64 bits
  __device__ uint32_t okey_at(int64_t g) const { return okey(__uint_as_float(ld_agent(key + g))); }
  __device__ double val_at(int64_t g) const { return __longlong_as_double((long long)ld_agent(val + g)); }
  __device__ uint32_t id_at(int64_t g) const { return ld_agent(id + g); }
};

// LDS of the merge; overlays the split phase's count table.
struct MergeLds {
  uint32_t cntb[kMaxSplits];
  uint32_t pre[kMaxSplits + 1];
  uint32_t hist[256];
  uint32_t sel[4];
  uint32_t red32[2 * kWaves];
  uint32_t m_slot[kSurvCap];     // survivors' record slots
  double m_val[kSurvCap];
  uint32_t m_id[kSurvCap];
  double t_val[SAS_MAX_TOP_K];   // ranked top-k values
  uint32_t t_id[SAS_MAX_TOP_K];
  double t_p[SAS_MAX_TOP_K];     // exp weights
  double t_pre[SAS_MAX_TOP_K];   // their running sums
  double t_q[SAS_MAX_TOP_K];     // weights / sum
  uint32_t n, lower;
  Red red;
};

// Exact top-k over the records whose key maps to >= lower when more than
// kSurvCap of them survive (degenerate ties); repeated block argmax.
__device__ __forceinline__ int merge_topk_slow(const RowRecs &rr, const uint32_t *cnt, int S, uint32_t lower,
                                               int k, double *t_val, uint32_t *t_id, Red *red) {
  double pv = 0.0;
  uint32_t pid = 0;
  int got = 0;
  for (int r = 0; r < k; ++r) {
    bool have = false;
    double bv = 0.0;
    uint32_t bi = 0;
    for (int b = 0; b < S; ++b) {
      for (uint32_t j = threadIdx.x; j < cnt[b]; j += kThreads) {
        const int64_t g = (int64_t)b * kCapBlock + j;
        const uint32_t x = rr.okey_at(g);
        if (x == 0u || x < lower) continue;
        const double val = rr.val_at(g);
        const uint32_t id = rr.id_at(g);
        if (r > 0 && !ranks_before(pv, pid, val, id)) continue;
        if (!have || ranks_before(val, id, bv, bi)) {
          have = true;
          bv = val;
          bi = id;
        }
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

// The merge of one row by its last block: bound, rank, sample() tail, outputs.
__device__ void merge_row(const SampleArgs &a, int row, const sas_params &p, MergeLds &ml) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int S = a.splits;
  const int64_t r0 = (int64_t)row * S * kCapBlock;
  const RowRecs rr{reinterpret_cast<const uint32_t *>(a.rkey) + r0, a.rid + r0,
                   reinterpret_cast<const uint64_t *>(a.rval) + r0};
  const bool in_regs = S <= kMergeRegs;
  const bool greedy = !(p.temperature > 0.0);
  const double u_row = greedy ? 0.0 : a.uniforms[row];

  // Thread t holds slot t of every block in registers: the loads are
  // in-bounds whatever the counts, all in flight at once (issued before the
  // counts are known), and a slot at or beyond its block's count is dropped.
  uint32_t key[kMergeRegs];
  if (in_regs) {
#pragma unroll
    for (int b = 0; b < kMergeRegs; ++b) key[b] = b < S ? ld_agent(rr.key + (int64_t)b * kCapBlock + tid) : 0u;
  }

  // ---- counts per block, offsets -----------------------------------------
  for (int b = tid; b < S; b += kThreads) ml.cntb[b] = ld_agent(a.counts + (int64_t)row * S + b);
  if (tid == 0) ml.n = 0u;
  __syncthreads();
  if (wave == 0) {
    uint32_t carry = 0;
    for (int b0 = 0; b0 < S; b0 += 64) {
      const int b = b0 + lane;
      const uint32_t nb = b < S ? ml.cntb[b] : 0u;
      const uint32_t inc = wave_incl_scan(nb);
      if (b < S) ml.pre[b] = carry + inc - nb;
      carry += __shfl(inc, 63, 64);
    }
    if (lane == 0) ml.pre[S] = carry;
  }
  __syncthreads();
  const uint32_t total = ml.pre[S];
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const uint32_t need = min((uint32_t)k, total);
  const uint32_t cap = min((uint32_t)kSurvCap, (uint32_t)k + (uint32_t)kMergeSlack);

  // ---- 6. bound, survivors -----------------------------------------------
  if (in_regs) {
    uint32_t valid = 0u;
#pragma unroll
    for (int b = 0; b < kMergeRegs; ++b)
      if (b < S && (uint32_t)tid < ml.cntb[b]) valid |= 1u << b;
    uint32_t kmax = 0u, kmin = 0xFFFFFFFFu;
#pragma unroll
    for (int b = 0; b < kMergeRegs; ++b) {
      key[b] = ((valid >> b) & 1u) ? okey(__uint_as_float(key[b])) : 0u;
      if (key[b]) {
        kmax = max(kmax, key[b]);
        kmin = min(kmin, key[b]);
      }
    }
    block_minmax(kmax, kmin, ml.red32);
    uint32_t lower = 1u;
    if (total > cap && kmax != kmin) {
      const int hb = 31 - __clz(kmax ^ kmin);
      auto for_keys = [&](auto f) {
#pragma unroll
        for (int b = 0; b < kMergeRegs; ++b) f(key[b]);
      };
      lower = radix_bound(for_keys, hb, hb == 31 ? 0u : kmax >> (hb + 1), need, cap, ml.hist, ml.sel);
    } else if (total > cap) {
      lower = kmax;  // every key is equal
    }
    uint32_t bits = 0u;
#pragma unroll
    for (int b = 0; b < kMergeRegs; ++b) bits |= (key[b] != 0u && key[b] >= lower ? 1u : 0u) << b;
    uint32_t slot = wave_reserve(bits, &ml.n);
#pragma unroll
    for (int b = 0; b < kMergeRegs; ++b)
      if ((bits >> b) & 1u) {
        if (slot < (uint32_t)kSurvCap) ml.m_slot[slot] = (uint32_t)b * kCapBlock + tid;
        ++slot;
      }
    ml.lower = lower;
  } else {
    // many blocks: the keys are read from memory on every pass
    uint32_t kmax = 0u, kmin = 0xFFFFFFFFu;
    for (int b = 0; b < S; ++b)
      if ((uint32_t)tid < ml.cntb[b]) {
        const uint32_t ok = rr.okey_at((int64_t)b * kCapBlock + tid);
        kmax = max(kmax, ok);
        kmin = min(kmin, ok);
      }
    block_minmax(kmax, kmin, ml.red32);
    uint32_t lower = 1u;
    if (total > cap && kmax != kmin) {
      const int hb = 31 - __clz(kmax ^ kmin);
      auto for_keys = [&](auto f) {
        for (int b = 0; b < S; ++b)
          if ((uint32_t)tid < ml.cntb[b]) f(rr.okey_at((int64_t)b * kCapBlock + tid));
      };
      lower = radix_bound(for_keys, hb, hb == 31 ? 0u : kmax >> (hb + 1), need, cap, ml.hist, ml.sel);
    } else if (total > cap) {
      lower = kmax;
    }
    for (int b = 0; b < S; ++b)
      if ((uint32_t)tid < ml.cntb[b]) {
        const uint32_t g = (uint32_t)b * kCapBlock + tid;
        const uint32_t x = rr.okey_at(g);
        if (x != 0u && x >= lower) {
          const uint32_t slot = atomicAdd(&ml.n, 1u);
          if (slot < (uint32_t)kSurvCap) ml.m_slot[slot] = g;
        }
      }
    ml.lower = lower;
  }
  __syncthreads();
  const uint32_t m = ml.n;
  const uint32_t lower = ml.lower;
  // the survivors' values and ids, one round of loads
  if ((uint32_t)tid < min(m, (uint32_t)kSurvCap)) {
    const uint32_t g = ml.m_slot[tid];
    ml.m_val[tid] = rr.val_at(g);
    ml.m_id[tid] = rr.id_at(g);
  }

  // ---- exact rank --------------------------------------------------------
  int kk = 0;  // candidates ranked into t_val/t_id
  uint32_t flags = 0;
  if (m <= (uint32_t)kSurvCap) {
    // pad to a multiple of 4 with entries that never rank before another
    const uint32_t mp = (m + 3u) & ~3u;
    if ((uint32_t)tid >= m && (uint32_t)tid < mp) {
      ml.m_val[tid] = -__builtin_inf();
      ml.m_id[tid] = 0xFFFFFFFFu;
    }
    __syncthreads();
    if ((uint32_t)tid < m) {
      const double vc = ml.m_val[tid];
      const uint32_t ic = ml.m_id[tid];
      uint32_t rank = 0;
      for (uint32_t j = 0; j < mp; j += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const double vj = ml.m_val[j + u];
          const uint32_t ij = ml.m_id[j + u];
          rank += (uint32_t)((vj > vc) | ((vj == vc) & (ij < ic)));
        }
      }
      if (rank < (uint32_t)k) {
        ml.t_val[rank] = vc;
        ml.t_id[rank] = ic;
      }
    }
    kk = (int)min(m, (uint32_t)k);
  } else {
    flags |= SAS_FLAG_SLOW_SELECT;
    kk = merge_topk_slow(rr, ml.cntb, S, lower, k, ml.t_val, ml.t_id, &ml.red);
  }
  __syncthreads();
  if (wave != 0) return;

  // ---- 7. sample() tail (tokenizer.js:161-177), double precision -----------
  // exp and division are correctly rounded in any lane, so the weights and
  // their normalised values are computed across lanes; the running sums
  // follow the reference's left-to-right order in lane 0, which reads its
  // operands from LDS eight at a time.
  const bool draw = !greedy && kk > 0;
  uint32_t out_id = SAS_NO_TOKEN;
  int cut = 0;
  if (kk == 0) {
    flags |= SAS_FLAG_EMPTY_ROW;
  } else if (greedy) {
    out_id = ml.t_id[0];
  } else {
    const double T = p.temperature;
    const double v0 = ml.t_val[0];
    for (int i = lane; i < kk; i += 64) ml.t_p[i] = fd_exp((ml.t_val[i] - v0) / T);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
      double run = 0.0;
      for (int i = 0; i < kk; i += 8) {
        double x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = ml.t_p[min(i + u, kk - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i + u < kk) {
            run += x[u];
            ml.t_pre[i + u] = run;
          }
      }
    }
    __builtin_amdgcn_wave_barrier();
    const double sum = ml.t_pre[kk - 1];
    for (int i = lane; i < kk; i += 64) ml.t_q[i] = ml.t_p[i] / sum;
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
      // top-p cut: the first i with p_0/sum + ... + p_i/sum >= top_p
      double cum = 0.0;
      cut = kk;
      for (int i = 0; i < kk && cut == kk; i += 8) {
        double x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = ml.t_q[min(i + u, kk - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i + u < kk && cut == kk) {
            cum += x[u];
            if (fabs(cum - p.top_p) < 1e-6) flags |= SAS_FLAG_TOPP_EDGE;
            if (cum >= p.top_p) cut = i + u + 1;
          }
      }
      // r = U * (p_0 + ... + p_{cut-1}), the sum taken left to right; the
      // first i at which r - p_0 - ... - p_i <= 0 is drawn
      const double sub = ml.t_pre[cut - 1];
      double r = u_row * sub;
      int pick = cut - 1;
      bool found = false;
      for (int i = 0; i < cut && !found; i += 8) {
        double x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = ml.t_p[min(i + u, cut - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i + u < cut && !found) {
            r -= x[u];
            if (fabs(r) <= 1e-12 * sub) flags |= SAS_FLAG_DRAW_EDGE;
            if (r <= 0.0) {
              pick = i + u;
              found = true;
            }
          }
      }
      out_id = ml.t_id[pick];
    }
  }
  if (lane == 0) {
    a.out_ids[row] = out_id;
    if (a.out_counts) {
      a.out_counts[2 * row] = draw ? kk : 0;
      a.out_counts[2 * row + 1] = draw ? cut : 0;
    }
    if (a.out_flags) a.out_flags[row] = flags;
  }
  const int np = draw ? kk : 0;
  if (a.out_probs) {
    double *op = a.out_probs + (int64_t)row * SAS_MAX_TOP_K;
    for (int i = lane; i < SAS_MAX_TOP_K; i += 64) op[i] = i < np ? ml.t_q[i] : 0.0;
  }
  if (a.out_cand_ids) {
    uint32_t *oc = a.out_cand_ids + (int64_t)row * SAS_MAX_TOP_K;
    for (int i = lane; i < SAS_MAX_TOP_K; i += 64) oc[i] = i < np ? ml.t_id[i] : SAS_NO_TOKEN;
  }
}

template <int F4, bool kMask, bool kHist, bool kSoftcap>
__global__ __launch_bounds__(kThreads) void sample_kernel(const SampleArgs a) {
  using L = SplitLds<F4>;
  constexpr int kChunk = L::kChunk;
  constexpr int E = F4 * 4;
  static_assert(E <= 32, "candidate bit masks are 32-bit");

  constexpr size_t kCntBytes = kHist ? L::kCountWords * 4 : 16;
  constexpr size_t kRawBytes = kCntBytes > sizeof(MergeLds) ? kCntBytes : sizeof(MergeLds);
  __shared__ __align__(16) unsigned char s_raw[kRawBytes];  // count table, then the merge's LDS
  uint32_t *s_cnt = reinterpret_cast<uint32_t *>(s_raw);
  __shared__ uint32_t s_rec_id[kCapBlock];
  __shared__ float s_rec_key[kCapBlock];
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[3];
  __shared__ uint32_t s_wkey[2 * kWaves];
  __shared__ uint32_t s_n;
  __shared__ int s_last;
  __shared__ Red s_red;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows = a.rows, S = a.splits;
  int lb = blockIdx.x;
  // XCD-aware order: consecutive dispatches rotate over the 8 XCDs, so give
  // each XCD a contiguous run of rows; a row's splits then share one L2 for
  // the history and mask reads.
  const int nblocks = rows * S;
  if ((nblocks & 7) == 0) lb = (lb & 7) * (nblocks >> 3) + (lb >> 3);
  const int row = lb / S;
  const int split = lb - row * S;
  const int lo = split * kChunk;
  const int vocab = a.vocab;

  const sas_params p = a.row_params ? a.row_params[row] : a.params;
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  const float *lrow = a.logits + (int64_t)row * a.logits_stride;
  const uint32_t *mrow = kMask ? a.mask + (int64_t)row * a.mask_stride : nullptr;

  uint32_t *ctl = a.ctl + (int64_t)row * kCtlStride;  // [0] arrivals, [kCtlThr] threshold key

  // ---- 1. loads --------------------------------------------------------
  // the row's threshold as published by the chunks that finished earlier
  const uint32_t row_key0 = ld_agent(ctl + kCtlThr);
  float4 v[F4];
  if (a.aligned && lo + kChunk <= vocab) {
    const f32x4 *src = reinterpret_cast<const f32x4 *>(lrow + lo) + tid;
#pragma unroll
    for (int f = 0; f < F4; ++f) {
      const f32x4 t = __builtin_nontemporal_load(src + f * kThreads);
      v[f] = make_float4(t.x, t.y, t.z, t.w);
    }
  } else {
    // a partial chunk or an unaligned row
#pragma unroll
    for (int f = 0; f < F4; ++f) {
      const int e = lo + 4 * (f * kThreads + tid);
      v[f].x = e + 0 < vocab ? lrow[e + 0] : qnan();
      v[f].y = e + 1 < vocab ? lrow[e + 1] : qnan();
      v[f].z = e + 2 < vocab ? lrow[e + 2] : qnan();
      v[f].w = e + 3 < vocab ? lrow[e + 3] : qnan();
    }
  }
  // mask word of float4 f: word (lo + 4q) / 32 with q = f*256 + tid
  uint32_t mw[kMask ? F4 : 1];
  if (kMask) {
    const int nw = (vocab + 31) >> 5;
#pragma unroll
    for (int f = 0; f < F4; ++f) {
      const int w = (lo >> 5) + f * (kThreads / 8) + (tid >> 3);
      mw[f] = w < nw ? mrow[w] : 0u;
    }
  }
  int h0 = 0, h1 = 0;
  if (kHist) {
    h0 = a.hist_offsets[row];
    h1 = a.hist_offsets[row + 1];
  }
  const bool has_hist = kHist && h1 > h0;
  if (has_hist) {
    uint32_t hreg[kHistRegs];
#pragma unroll
    for (int j = 0; j < kHistRegs; ++j) {
      const int i = h0 + j * kThreads + tid;
      hreg[j] = i < h1 ? a.hist_ids[i] : 0xFFFFFFFFu;
    }
    uint4 *c4 = reinterpret_cast<uint4 *>(s_cnt);
    for (int w = tid; w < L::kCountWords / 4; w += kThreads) c4[w] = make_uint4(0u, 0u, 0u, 0u);
    if (tid == 0) s_n = 0u;
    __syncthreads();
    auto count = [&](uint32_t id) {
      const uint32_t off = id - (uint32_t)lo;
      if (off < (uint32_t)kChunk && id < (uint32_t)vocab) atomicAdd(&s_cnt[off >> 1], 1u << ((off & 1u) * 16u));
    };
#pragma unroll
    for (int j = 0; j < kHistRegs; ++j) count(hreg[j]);
    for (int i = h0 + kHistRegs * kThreads + tid; i < h1; i += kThreads) count(a.hist_ids[i]);
    __syncthreads();
  } else if (tid == 0) {
    s_n = 0u;  // published by the threshold barrier below
  }
  const ElemCtx ec{lrow, mrow, has_hist ? s_cnt : nullptr, lo, vocab, p};

  // ---- 2. values (in place in v) -----------------------------------------
  uint32_t penbits = 0;
  float tmax = qnan();  // stays NaN in a lane without a valid value
#pragma unroll
  for (int f = 0; f < F4; ++f) {
    if (kSoftcap && p.softcap > 0.0f) {
      v[f].x = softcap_f32(v[f].x, p.softcap);
      v[f].y = softcap_f32(v[f].y, p.softcap);
      v[f].z = softcap_f32(v[f].z, p.softcap);
      v[f].w = softcap_f32(v[f].w, p.softcap);
    }
    if (kMask) {
      const uint32_t nib = mw[f] >> (4 * (tid & 7));
      v[f].x = (nib & 1u) ? v[f].x : qnan();
      v[f].y = (nib & 2u) ? v[f].y : qnan();
      v[f].z = (nib & 4u) ? v[f].z : qnan();
      v[f].w = (nib & 8u) ? v[f].w : qnan();
    }
    if (has_hist) {
      const int q = f * kThreads + tid;
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
  // neither, every valid value passes.  Keys are searched to 16 bits: the
  // bound only gets lower, the guarantee holds.
  const int jth = (k + kWaves - 1) / kWaves;
  const int mth = (k + jth - 1) / jth;
  const uint32_t lkey = okey(tmax);
  const uint32_t tw = wave_jth_largest_key16(lkey, jth);
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
    const uint32_t tk = wave_jth_largest_key16(lkey, k);
    if (lane == 0) s_wkey[kWaves + wave] = tk;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tkey = max(tkey, s_wkey[kWaves + w]);
  }
  // publish; nothing waits for the result
  if (tid == 0 && tkey > row_key0)
    __hip_atomic_fetch_max(ctl + kCtlThr, tkey, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // keys below okey(-inf) + 1 (0 or truncated) admit every valid value
  const uint32_t ekey = max(tkey, row_key0);
  const float thr = ekey > 0x007FFFFFu ? fkey(ekey) : -__builtin_inff();

  // ---- 4. emission -----------------------------------------------------
  // per-lane bit mask of passing slots, wave prefix of the counts by
  // ballots, one LDS atomic per wave
  uint32_t bits = 0u;
#pragma unroll
  for (int i = 0; i < E; ++i) bits |= (elem(i) >= thr ? 1u : 0u) << i;
  if (__ballot(bits != 0u)) {
    uint32_t slot = wave_reserve(bits, &s_n);
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((bits >> i) & 1u) {
        if (slot < (uint32_t)kCapBlock) {
          const int f = i >> 2, j = i & 3;
          s_rec_id[slot] = (uint32_t)(lo + 4 * (f * kThreads + tid) + j) | (((penbits >> i) & 1u) ? kPenFlag : 0u);
          s_rec_key[slot] = elem(i);
        }
        ++slot;
      }
    }
  }
  __syncthreads();
  uint32_t n = s_n;
  if (n > (uint32_t)kCapBlock) n = overflow_select<E>(ec, k, ekey, s_rec_id, s_rec_key, s_hist, s_sel, &s_n, &s_red);

  // ---- records out: the block's own slots ---------------------------------
  const int64_t slot0 = (int64_t)row * S + split;
  const int64_t r0 = slot0 * kCapBlock;
  for (int i = tid; i < (int)n; i += kThreads) {
    const uint32_t idf = s_rec_id[i];
    const float kk = s_rec_key[i];
    st_agent(reinterpret_cast<uint32_t *>(a.rkey) + r0 + i, __float_as_uint(kk));
    st_agent(a.rid + r0 + i, idf & ~kPenFlag);
    st_agent(reinterpret_cast<uint64_t *>(a.rval) + r0 + i, (uint64_t)__double_as_longlong(ec.exact(idf, kk)));
  }
  if (tid == 0) st_agent(a.counts + slot0, n);

  // ---- 5. count in; the row's last block merges ----------------------------
  wait_vm();  // this wave's records, count and threshold are complete
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(ctl, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(S - 1);
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) {
    // every block of the row has counted in and published: reset for the next launch
    ctl[0] = 0u;
    ctl[kCtlThr] = 0u;
  }
  merge_row(a, row, p, *reinterpret_cast<MergeLds *>(s_raw));
}

// Chunk size (float4 loads per thread): the largest that still gives every
// CU several blocks; then grown while a row would have more splits than the
// merge holds in registers.
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
  while (pick < 8 && (vocab + pick * 1024 - 1) / (pick * 1024) > kMergeRegs) pick *= 2;
  return pick;
}

size_t sample_rec_bytes(int rows, int splits) {
  return (size_t)rows * splits * kCapBlock * (sizeof(float) + sizeof(uint32_t) + sizeof(double));
}
size_t sample_count_bytes(int rows, int splits) { return (size_t)rows * splits * sizeof(uint32_t); }

template <int F4, bool kMask, bool kHist, bool kSoftcap>
static void launch_one(const SampleArgs &a, hipStream_t stream) {
  hipLaunchKernelGGL((sample_kernel<F4, kMask, kHist, kSoftcap>), dim3((unsigned)(a.rows * a.splits)),
                     dim3(kThreads), 0, stream, a);
}

template <int F4>
static void launch_f4(const SampleArgs &a, bool softcap, hipStream_t stream) {
  const int v = (a.mask ? 4 : 0) | (a.hist_ids ? 2 : 0) | (softcap ? 1 : 0);
  switch (v) {
    case 0: launch_one<F4, false, false, false>(a, stream); break;
    case 1: launch_one<F4, false, false, true>(a, stream); break;
    case 2: launch_one<F4, false, true, false>(a, stream); break;
    case 3: launch_one<F4, false, true, true>(a, stream); break;
    case 4: launch_one<F4, true, false, false>(a, stream); break;
    case 5: launch_one<F4, true, false, true>(a, stream); break;
    case 6: launch_one<F4, true, true, false>(a, stream); break;
    default: launch_one<F4, true, true, true>(a, stream); break;
  }
}

hipError_t launch_sample(const SampleArgs &a, int f4, bool softcap, hipStream_t stream) {
  switch (f4) {
    case 8: launch_f4<8>(a, softcap, stream); break;
    case 4: launch_f4<4>(a, softcap, stream); break;
    default: launch_f4<2>(a, softcap, stream); break;
  }
  return hipGetLastError();
}

}  // namespace sas

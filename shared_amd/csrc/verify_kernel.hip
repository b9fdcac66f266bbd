// verify_kernel.hip - speculative verification by rejection sampling
// (Leviathan et al. 2023, "Fast Inference from Transformers via Speculative
// Decoding"; Chen et al. 2023, "Accelerating Large Language Model Decoding
// with Speculative Sampling").
//
// The reference verifies drafts by an exact-match cascade
// (lib/webgpu-llm/kernels.js:328-339, acceptSpec); this path implements the
// distribution-preserving rule the sampling API needs at temperature > 0:
//
//   p_j = softmax(target row j / T), q_j = softmax(draft row j / T), both over
//   allowed, non-NaN ids.  Position j accepts draft d_j iff
//   d_j < vocab and p_j(d_j) > 0 and U1 * q_j(d_j) <= p_j(d_j).  The first
//   rejected position a draws from max(0, p_a - q_a) (from p_a when that is
//   all zero) with U2; when every draft is accepted the bonus position L
//   draws from p_L with its U2.  A draw returns the smallest id whose
//   running weight (ascending ids) exceeds U2 * total.
//
// Three launches, each reading what the previous one wrote:
//   1. verify_stats_kernel, one block per (position, 4096-id chunk): reads
//      the target chunk, the draft chunk and the mask words once, and writes
//      the chunk's max and sum of exp((x - max) / T) for both rows.  This is
//      the pass that streams the whole input.
//   2. verify_decide_kernel, one block per (sequence, chunk): combines the
//      chunk statistics of the sequence's positions (every block the same
//      way, in the same order, so they agree bit for bit), decides the
//      accepted prefix, and for the one position that draws, writes its
//      chunk's residual mass and target mass.  Only that position's rows are
//      read again.
//   3. verify_draw_kernel, one block per sequence: finds the chunk in which
//      U2 * total falls, scans that chunk's ids in ascending order, and
//      writes the tokens.
//
// The weights that are summed (softmax normalizers, residual and target
// masses, the draw's running sums) are exp_sum of (x - max) * (1 / T) and
// products with reciprocals of the normalizers: within a few ulp of the
// host oracle's fdlibm exp and divisions, a difference of the same order as
// that of the summation order, which differs from a sequential loop anyway.
// The acceptance test p(d) >= U1 q(d) uses fdlibm exp and divisions.
#include <hip/hip_runtime.h>

#include <cmath>

#include "sas_device.h"
#include "sas_launch.h"
#include "shared_amd_sampler.h"

namespace sas {
namespace {

constexpr int kPerThread = kVChunk / kThreads;  // 16 ids per thread
typedef double f64x2 __attribute__((ext_vector_type(2)));
static_assert(kPerThread == 16, "a thread owns four float4 of a chunk");

__device__ __forceinline__ double dneg_inf() { return -__longlong_as_double(0x7ff0000000000000ll); }

__device__ __forceinline__ double wave_max_d(double x) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) x = fmax(x, __shfl_xor(x, s, 64));
  return x;
}

// Butterfly sum: lane i adds x_i + x_(i^s) and lane i^s adds the same two
// numbers, so every lane ends with the identical sum.
__device__ __forceinline__ double wave_sum_d(double x) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) x += __shfl_xor(x, s, 64);
  return x;
}

__device__ __forceinline__ double wave_incl_scan_d(double x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    double y = __shfl_up(x, s, 64);
    if (lane >= s) x += y;
  }
  return x;
}

// Strided chunk layout (passes 1 and 2): thread t owns ids
// base + (f * 256 + t) * 4 + k, f, k in 0..3, loaded as four coalesced float4.
__device__ __forceinline__ void load_strided(const float *row, int64_t base, int vocab, bool aligned,
                                             float x[kPerThread]) {
  const int tid = threadIdx.x;
  if (aligned && base + kVChunk <= vocab) {
    const f32x4 *p = reinterpret_cast<const f32x4 *>(row + base);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      f32x4 v = __builtin_nontemporal_load(p + f * kThreads + tid);
      x[f * 4 + 0] = v.x;
      x[f * 4 + 1] = v.y;
      x[f * 4 + 2] = v.z;
      x[f * 4 + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // clamped into the row: every load issued, none behind a branch
        const int64_t id = base + (f * kThreads + tid) * 4 + k;
        const float t = row[min(id, (int64_t)vocab - 1)];
        x[f * 4 + k] = id < vocab ? t : 0.0f;
      }
  }
}

// Bit f*4+k set: id base + (f*256+t)*4 + k is below vocab and its mask bit
// is set.  The four mask words are loaded unconditionally (clamped into the
// row), so that they are in flight together.
template <bool kMask>
__device__ __forceinline__ uint32_t allow_strided(const uint32_t *mrow, int64_t base, int vocab) {
  const int tid = threadIdx.x;
  const int64_t last_word = ((int64_t)vocab + 31) / 32 - 1;
  uint32_t mw[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int64_t id0 = base + (f * kThreads + tid) * 4;
    mw[f] = kMask ? mrow[min(id0 >> 5, last_word)] : ~0u;
  }
  uint32_t bits = 0;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int64_t id0 = base + (f * kThreads + tid) * 4;
    // ids of the four below vocab: 0 .. 4 (no branch, so the loads stay
    // ahead of every use)
    const int left = (int)min(max((int64_t)vocab - id0, (int64_t)0), (int64_t)4);
    bits |= ((mw[f] >> (uint32_t)(id0 & 31)) & ((1u << left) - 1u)) << (f * 4);
  }
  return bits;
}

// Places n items per lane in one list for the wave: `pre` the lane's first
// slot (the items of the lanes below it), `tot` the wave's total.  n < 32.
__device__ __forceinline__ void wave_place(uint32_t n, uint32_t &pre, uint32_t &tot) {
  pre = 0u;
  tot = 0u;
#pragma unroll
  for (int bit = 0; bit < 5; ++bit) {
    const uint64_t bb = __ballot((n >> bit) & 1u);
    pre += lanes_below(bb) << bit;
    tot += (uint32_t)__popcll(bb) << bit;
  }
}

// A wave's allowed values of one side, packed, when they are few.
constexpr int kCompact = 256;
// pk_n words: the wave's allowed ids' values were packed for both rows
// (a draft value may be NaN), or for the target row only (a position
// without a draft); the count in the low bits.  0: not packed (more than
// kCompact allowed, or a target value among them is NaN).
constexpr uint32_t kPkJoint = 1u << 30;
constexpr uint32_t kPkTarget = 1u << 29;
constexpr uint32_t kPkCount = 0xFFFFu;

struct StatsLds {
  float m[kWaves][2];
  double z[kWaves][2];
  float cv[kWaves][2][kCompact];
};

__device__ __forceinline__ uint32_t nan_free(const float x[kPerThread], uint32_t ok) {
#pragma unroll
  for (int i = 0; i < kPerThread; ++i)
    if (x[i] != x[i]) ok &= ~(1u << i);
  return ok;
}

// Sum over the wave of exp((x - M) / T) for the allowed values of one side:
// packed into the wave's LDS slots first when at most kCompact of the
// wave's 1,024 are allowed (a sparse mask), so that only those are
// exponentiated; every lane's result is the wave's.
__device__ __forceinline__ double side_sum(const float x[kPerThread], uint32_t ok, double M, double inv_t,
                                           float *cv) {
  const int lane = threadIdx.x & 63;
  uint32_t pre, tot;
  wave_place((uint32_t)__popc(ok), pre, tot);
  double z = 0.0;
  if (tot <= (uint32_t)kCompact) {
    uint32_t j = pre;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      if ((ok >> i) & 1u) cv[j++] = x[i];
    wave_lds_sync();
    for (uint32_t e = (uint32_t)lane; e < tot; e += 64u) z += exp_sum(((double)cv[e] - M) * inv_t);
  } else {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const double w = exp_sum(((double)x[i] - M) * inv_t);
      z += ((ok >> i) & 1u) ? w : 0.0;
    }
  }
  return wave_sum_d(z);
}

// Seven waves per SIMD (72 VGPRs): the kernel hides its loads behind the
// other waves.
template <bool kMask>
__global__ __launch_bounds__(kThreads, 7) void verify_stats_kernel(VerifyArgs a) {
  __shared__ StatsLds l;
  const int c = blockIdx.x, pos = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int P1 = a.L + 1;
  const int s = pos / P1, j = pos - s * P1;
  const int64_t base = (int64_t)c * kVChunk;
  const bool has_draft = j < a.L;
  float xt[kPerThread], xq[kPerThread];
  load_strided(a.target + (int64_t)pos * a.stride, base, a.vocab, a.aligned, xt);
  if (has_draft) load_strided(a.draft + ((int64_t)s * a.L + j) * a.stride, base, a.vocab, a.aligned, xq);
  const uint32_t ok = allow_strided<kMask>(kMask ? a.mask + (int64_t)pos * a.mask_stride : nullptr, base, a.vocab);
  if (has_draft && tid == 0) {
    // the block whose chunk holds the position's draft token records the
    // token's two logits for the acceptance test (NaN when masked)
    const uint32_t d = a.draft_ids[(int64_t)s * a.L + j];
    if (d < (uint32_t)a.vocab && (int64_t)(d / kVChunk) == (int64_t)c) {
      const bool allowed = !kMask || ((a.mask[(int64_t)pos * a.mask_stride + (d >> 5)] >> (d & 31)) & 1u);
      a.dtok[2 * pos] = allowed ? a.target[(int64_t)pos * a.stride + d] : __builtin_nanf("");
      a.dtok[2 * pos + 1] = allowed ? a.draft[((int64_t)s * a.L + j) * a.stride + d] : __builtin_nanf("");
    }
  }
  // The wave's allowed ids, when at most kCompact of its 1,024 (a sparse
  // mask): both rows' values packed into the wave's LDS slots in id order,
  // NaNs included, so that the NaN tests, the maxima and the exponentials
  // run over those values only.  Otherwise every value is tested in the
  // registers.
  uint32_t pre, tot;
  wave_place((uint32_t)__popc(ok), pre, tot);
  const bool packed = tot <= (uint32_t)kCompact;  // uniform over the wave
  float *cvt = l.cv[wave][0], *cvq = l.cv[wave][1];
  float mt = -__builtin_inff(), mq = -__builtin_inff();
  uint32_t okt = 0u, okq = 0u;
  bool tnan = false;  // a packed target value is NaN
  if (packed) {
    uint32_t jj = pre;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      if ((ok >> i) & 1u) {
        cvt[jj] = xt[i];
        if (has_draft) cvq[jj] = xq[i];
        ++jj;
      }
    wave_lds_sync();
    // a NaN compares false: it never becomes a maximum
    for (uint32_t e = (uint32_t)lane; e < tot; e += 64u) {
      const float t = cvt[e];
      tnan |= t != t;
      mt = t > mt ? t : mt;
      if (has_draft) {
        const float q = cvq[e];
        mq = q > mq ? q : mq;
      }
    }
  } else {
    okt = nan_free(xt, ok);
    okq = has_draft ? nan_free(xq, ok) : 0u;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      if ((okt >> i) & 1u) mt = fmaxf(mt, xt[i]);
      if ((okq >> i) & 1u) mq = fmaxf(mq, xq[i]);
    }
    // opaque copies: the bit tests below are made again from the words, not
    // kept from the loop above (32 lane masks would not fit the SGPRs)
    asm volatile("" : "+v"(okt), "+v"(okq));
  }
  // the chunk's maxima of both rows (allowed, not NaN)
  mt = wave_max(mt);
  mq = wave_max(mq);
  if (lane == 0) {
    l.m[wave][0] = mt;
    l.m[wave][1] = mq;
  }
  __syncthreads();
  float bt = l.m[0][0], bq = l.m[0][1];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    bt = fmaxf(bt, l.m[w][0]);
    bq = fmaxf(bq, l.m[w][1]);
  }
  // sums of exp((x - max) / T)
  const double Mt = (double)bt, Mq = (double)bq;
  double zt, zq;
  uint32_t pk = 0u;  // how the wave's values were packed for the decide pass
  if (packed) {
    double st = 0.0, sq = 0.0;
    for (uint32_t e = (uint32_t)lane; e < tot; e += 64u) {
      const float t = cvt[e];
      if (t == t) st += exp_sum(((double)t - Mt) * a.inv_t);
      if (has_draft) {
        const float q = cvq[e];
        if (q == q) sq += exp_sum(((double)q - Mq) * a.inv_t);
      }
    }
    zt = wave_sum_d(st);
    zq = has_draft ? wave_sum_d(sq) : 0.0;
    // the decide pass takes packed target values that are not NaN (a NaN
    // draft value it tests itself)
    if (__ballot(tnan) == 0ull) pk = (has_draft ? kPkJoint : kPkTarget) | tot;
  } else {
    zt = side_sum(xt, okt, Mt, a.inv_t, cvt);
    zq = has_draft ? side_sum(xq, okq, Mq, a.inv_t, cvq) : 0.0;
  }
  if (lane == 0) {
    l.z[wave][0] = zt;
    l.z[wave][1] = zq;
  }
  // the wave's packed values (in the order the decide pass packs them from
  // the rows, so that its sums are the same) and how they were packed
  {
    const int64_t w = ((int64_t)pos * a.chunks + c) * kWaves + wave;
    float *pv = a.pk_v + w * (2 * kCompact);
    for (uint32_t e = (uint32_t)lane; pk && e < tot; e += 64u) {
      pv[e] = cvt[e];
      if (pk & kPkJoint) pv[kCompact + e] = cvq[e];
    }
    if (lane == 0) a.pk_n[w] = pk;
  }
  __syncthreads();
  if (tid == 0) {
    double t = l.z[0][0], q = l.z[0][1];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      t += l.z[w][0];
      q += l.z[w][1];
    }
    double *o = a.stats + ((int64_t)pos * a.chunks + c) * 4;
    o[0] = Mt;
    o[1] = t;
    o[2] = has_draft ? Mq : dneg_inf();
    o[3] = q;
  }
}

struct Decided {
  int a;         // accepted drafts; the position that draws
  double mt, zt, mq, zq;
};

struct DecideLds {
  double m[SAS_MAX_DRAFT + 1][2];
  double z[SAS_MAX_DRAFT + 1][2];
  int acc[SAS_MAX_DRAFT];
  double red[kWaves][2];
  float ct[kWaves][kCompact];  // a wave's allowed target values, packed
  float cq[kWaves][kCompact];  // and the draft values of the same ids
};

// Softmax statistics of every position of sequence s from the chunk
// statistics, then the accepted prefix.  Identical in every block.
__device__ Decided decide(const VerifyArgs &a, int s, DecideLds &l) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = a.L, P1 = L + 1;
  const double T = a.temperature;
  // the acceptance inputs (loaded with the statistics: nothing depends on them)
  uint32_t d = 0u;
  float dxt = 0.0f, dxq = 0.0f;
  double u1 = 0.0;
  if (tid < L) {
    const int pos = s * P1 + tid;
    d = a.draft_ids[(int64_t)s * L + tid];
    dxt = a.dtok[2 * pos];
    dxq = a.dtok[2 * pos + 1];
    u1 = a.uniforms[(int64_t)pos * 2];
  }
  if (a.chunks <= 64 && P1 <= 2 * kWaves) {
    // at most two positions per wave and one chunk per lane: both
    // positions' statistics are loaded at once (clamped into the existing
    // ones), then combined as below
    const bool cok = lane < a.chunks;
    const int c = min(lane, a.chunks - 1);
    f64x2 st[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = min(wave + kWaves * i, P1 - 1);
      const f64x2 *p = reinterpret_cast<const f64x2 *>(a.stats + ((int64_t)(s * P1 + j) * a.chunks + c) * 4);
      st[i][0] = p[0];  // (max, sum) of the target row
      st[i][1] = p[1];  // and of the draft row
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = wave + kWaves * i;
      if (j < P1) {
        for (int side = 0; side < (j < L ? 2 : 1); ++side) {
          const double mc = st[i][side].x, zc = cok ? st[i][side].y : 0.0;
          const double m = wave_max_d(fmax(dneg_inf(), cok ? mc : dneg_inf()));
          double z = 0.0;
          if (zc > 0.0) z += zc * exp_sum((mc - m) * a.inv_t);
          z = wave_sum_d(z);
          if (lane == 0) {
            l.m[j][side] = m;
            l.z[j][side] = z;
          }
        }
      }
    }
  } else {
    for (int j = wave; j < P1; j += kWaves) {
      const double *st = a.stats + (int64_t)(s * P1 + j) * a.chunks * 4;
      for (int side = 0; side < (j < L ? 2 : 1); ++side) {
        double m = dneg_inf();
        for (int c = lane; c < a.chunks; c += 64) m = fmax(m, st[c * 4 + side * 2]);
        m = wave_max_d(m);
        double z = 0.0;
        for (int c = lane; c < a.chunks; c += 64) {
          const double zc = st[c * 4 + side * 2 + 1];
          if (zc > 0.0) z += zc * exp_sum((st[c * 4 + side * 2] - m) * a.inv_t);
        }
        z = wave_sum_d(z);
        if (lane == 0) {
          l.m[j][side] = m;
          l.z[j][side] = z;
        }
      }
    }
  }
  __syncthreads();
  if (tid < L) {
    const int j = tid;
    double pd = 0.0, qd = 0.0;
    const bool in_vocab = d < (uint32_t)a.vocab;
    if (in_vocab) {
      // dtok: written by the statistics pass for every in-vocabulary draft
      // token (NaN when masked)
      const double wt = dxt == dxt ? fd_exp(((double)dxt - l.m[j][0]) / T) : 0.0;
      const double wq = dxq == dxq ? fd_exp(((double)dxq - l.m[j][1]) / T) : 0.0;
      pd = wt / l.z[j][0];
      qd = wq / l.z[j][1];
    }
    l.acc[j] = in_vocab && pd > 0.0 && u1 * qd <= pd;
  }
  __syncthreads();
  Decided r;
  r.a = L;
  for (int j = 0; j < L; ++j)
    if (!l.acc[j]) {
      r.a = j;
      break;
    }
  r.mt = l.m[r.a][0];
  r.zt = l.z[r.a][0];
  r.mq = r.a < L ? l.m[r.a][1] : 0.0;
  r.zq = r.a < L ? l.z[r.a][1] : 0.0;
  return r;
}

// Residual weight max(0, p - q) and target weight exp((x - M) / T) of one
// id whose target value is allowed and not NaN.  izt, izq: 1 / zt, 1 / zq.
struct Weights {
  double mt, izt, mq, izq, inv_t;
  bool resid;
  __device__ __forceinline__ void at(float xt, float xq, bool q_ok, double &wt, double &r) const {
    wt = exp_sum(((double)xt - mt) * inv_t);
    r = 0.0;
    if (resid) {
      const double wq = q_ok ? exp_sum(((double)xq - mq) * inv_t) : 0.0;
      const double d = wt * izt - wq * izq;
      r = d > 0.0 ? d : 0.0;
    }
  }
};

template <bool kMask>
__global__ __launch_bounds__(kThreads) void verify_decide_kernel(VerifyArgs a) {
  __shared__ DecideLds l;
  const int c = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const Decided d = decide(a, s, l);
  const int P1 = a.L + 1;
  const int pos = s * P1 + d.a;
  const bool resid = d.a < a.L;
  const int64_t base = (int64_t)c * kVChunk;
  const Weights w{d.mt, 1.0 / d.zt, d.mq, resid ? 1.0 / d.zq : 0.0, a.inv_t, resid};
  double pm = 0.0, rs = 0.0;
  // the wave's allowed ids as the statistics pass packed them (both rows,
  // or the target row where no residual is drawn); else the rows again
  const int64_t wpk = ((int64_t)pos * a.chunks + c) * kWaves + wave;
  const uint32_t pk = a.pk_n[wpk];
  if (resid ? (pk & kPkJoint) != 0u : (pk & (kPkJoint | kPkTarget)) != 0u) {
    const float *pv = a.pk_v + wpk * (2 * kCompact);
    const uint32_t tot = pk & kPkCount;
    for (uint32_t e = (uint32_t)lane; e < tot; e += 64u) {
      const float vq = resid ? pv[kCompact + e] : 0.0f;
      double wt, r;
      w.at(pv[e], vq, resid && vq == vq, wt, r);
      pm += wt;
      rs += r;
    }
  } else {
    float xt[kPerThread], xq[kPerThread];
    load_strided(a.target + (int64_t)pos * a.stride, base, a.vocab, a.aligned, xt);
    if (resid) load_strided(a.draft + ((int64_t)s * a.L + d.a) * a.stride, base, a.vocab, a.aligned, xq);
    const uint32_t ok = nan_free(xt, allow_strided<kMask>(kMask ? a.mask + (int64_t)pos * a.mask_stride : nullptr,
                                                           base, a.vocab));
    // the allowed ids' values, packed per wave when few (a sparse mask)
    uint32_t pre, tot;
    wave_place((uint32_t)__popc(ok), pre, tot);
    if (tot <= (uint32_t)kCompact) {
      uint32_t jj = pre;
#pragma unroll
      for (int i = 0; i < kPerThread; ++i)
        if ((ok >> i) & 1u) {
          l.ct[wave][jj] = xt[i];
          l.cq[wave][jj] = resid ? xq[i] : 0.0f;
          ++jj;
        }
      wave_lds_sync();
      for (uint32_t e = (uint32_t)lane; e < tot; e += 64u) {
        const float vq = l.cq[wave][e];
        double wt, r;
        w.at(l.ct[wave][e], vq, resid && vq == vq, wt, r);
        pm += wt;
        rs += r;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kPerThread; ++i)
        if ((ok >> i) & 1u) {
          double wt, r;
          w.at(xt[i], resid ? xq[i] : 0.0f, resid && xq[i] == xq[i], wt, r);
          pm += wt;
          rs += r;
        }
    }
  }
  pm = wave_sum_d(pm);
  rs = wave_sum_d(rs);
  if (lane == 0) {
    l.red[wave][0] = rs;
    l.red[wave][1] = pm;
  }
  __syncthreads();
  if (tid == 0) {
    double r = l.red[0][0], p = l.red[0][1];
#pragma unroll
    for (int v = 1; v < kWaves; ++v) {
      r += l.red[v][0];
      p += l.red[v][1];
    }
    double *o = a.part + ((int64_t)s * a.chunks + c) * 2;
    o[0] = r;
    o[1] = p;
    if (c == 0) {
      double *q = a.seqrec + (int64_t)s * 8;
      q[0] = (double)d.a;
      q[1] = d.mt;
      q[2] = d.zt;
      q[3] = d.mq;
      q[4] = d.zq;
    }
  }
}

struct DrawLds {
  double wsum[kWaves];
  int chunk;
  int resid;
  int last_mode;
  double before;
  double target;
  uint32_t found;
  uint32_t last;
  uint32_t wcnt[kWaves];
  float pt[kVChunk];     // the drawing chunk's allowed ids, ascending: target value,
  float pq[kVChunk];     // draft value,
  uint16_t pid[kVChunk]; // offset in the chunk,
  double pw[kVChunk];    // and weight
};

template <bool kMask>
__global__ __launch_bounds__(kThreads) void verify_draw_kernel(VerifyArgs a) {
  __shared__ DrawLds l;
  const int s = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = a.L, P1 = L + 1;
  const int C = a.chunks;
  const double *part = a.part + (int64_t)s * C * 2;
  // Loads that do not wait for the accepted count come first: wave 0's
  // chunk masses (one chunk per lane when there are at most 64) and the
  // second uniform of every position of the sequence (P1 <= 64).
  f64x2 pc = {0.0, 0.0};
  if (wave == 0 && C <= 64) pc = *reinterpret_cast<const f64x2 *>(part + 2 * min(lane, C - 1));
  const double u2c = a.uniforms[((int64_t)s * P1 + min(lane, P1 - 1)) * 2 + 1];
  const double *q = a.seqrec + (int64_t)s * 8;
  const int acc = (int)q[0];
  const int pos = s * P1 + acc;
  const double u2 = __shfl(u2c, acc, 64);
  if (tid == 0) {
    l.found = SAS_NO_TOKEN;
    l.last = 0;
    l.chunk = -1;
    l.last_mode = 1;
  }
  if (tid <= L && tid != acc)
    a.out_tokens[(int64_t)s * P1 + tid] = tid < acc ? a.draft_ids[(int64_t)s * L + tid] : SAS_NO_TOKEN;
  if (tid == 0) a.out_accepted[s] = acc;

  // Which weights draw: the residual unless it is all zero, else the target.
  if (wave == 0) {
    const int R = (C + 63) / 64;
    const int c0 = lane * R, c1 = min(C, c0 + R);
    // chunk c's residual (col 0) or target (col 1) mass; with one chunk
    // per lane (c == lane) from the registers
    auto wpart = [&](int c, int col) __attribute__((always_inline)) -> double {
      if (C <= 64) return col ? pc.y : pc.x;
      return part[c * 2 + col];
    };
    bool resid = acc < L;
    if (resid) {
      double v = 0.0;
      for (int c = c0; c < c1; ++c) v += wpart(c, 0);
      v = wave_incl_scan_d(v);
      resid = __shfl(v, 63, 64) > 0.0;
    }
    const int col = resid ? 0 : 1;
    double v = 0.0;
    for (int c = c0; c < c1; ++c) v += wpart(c, col);
    const double incl = wave_incl_scan_d(v);
    double excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = 0.0;
    const double tot = __shfl(incl, 63, 64);
    const double target = u2 * tot;
    // first chunk whose running total passes the target
    int hit = -1;
    double cum = excl, hit_before = 0.0;
    int lastc = -1;
    double last_before = 0.0;
    for (int c = c0; c < c1; ++c) {
      const double wc = wpart(c, col);
      if (!(wc > 0.0)) continue;
      lastc = c;
      last_before = cum;
      const double nxt = cum + wc;
      if (hit < 0 && nxt > target) {
        hit = c;
        hit_before = cum;
      }
      cum = nxt;
    }
    const uint64_t hits = __ballot(hit >= 0);
    const uint64_t lasts = __ballot(lastc >= 0);
    if (tot > 0.0) {
      if (hits) {
        const int src = __ffsll((long long)hits) - 1;
        const int hc = __shfl(hit, src, 64);
        const double hb = __shfl(hit_before, src, 64);
        if (lane == 0) {
          l.chunk = hc;
          l.before = hb;
          l.last_mode = 0;
        }
      } else if (lasts) {
        const int src = 63 - __clzll((long long)lasts);
        const int lc = __shfl(lastc, src, 64);
        const double lb = __shfl(last_before, src, 64);
        if (lane == 0) {
          l.chunk = lc;
          l.before = lb;
          l.last_mode = 1;
        }
      }
    }
    if (lane == 0) {
      l.target = target;
      l.resid = resid;
    }
  }
  __syncthreads();
  const int chunk = l.chunk;
  if (chunk < 0) {
    if (tid == 0) a.out_tokens[(int64_t)s * P1 + acc] = SAS_NO_TOKEN;
    return;
  }
  const bool resid = l.resid != 0;
  const double target = l.target, before = l.before;
  const bool last_mode = l.last_mode != 0;

  // The chunk's allowed ids in ascending order, packed: thread t reads ids
  // chunk*4096 + 16t .. +15, and entry e of the packed list goes to thread
  // e / per (per = ceil(entries / 256)), so every thread holds a run of
  // consecutive ids.
  const int64_t id0 = (int64_t)chunk * kVChunk + (int64_t)tid * kPerThread;
  const float *trow = a.target + (int64_t)pos * a.stride;
  const float *drow = resid ? a.draft + ((int64_t)s * L + acc) * a.stride : nullptr;
  uint32_t bits = 0;
  if (id0 < a.vocab) {
    bits = a.mask ? (a.mask[(int64_t)pos * a.mask_stride + (id0 >> 5)] >> (id0 & 31)) & 0xFFFFu : 0xFFFFu;
    const int64_t left = a.vocab - id0;
    if (left < kPerThread) bits &= (1u << left) - 1u;
  }
  float vt[kPerThread], vq[kPerThread];
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    vt[i] = (bits >> i) & 1u ? trow[id0 + i] : 0.0f;
    vq[i] = resid && ((bits >> i) & 1u) ? drow[id0 + i] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kPerThread; ++i)
    if (vt[i] != vt[i]) bits &= ~(1u << i);
  // block-wide exclusive prefix of the per-thread counts (thread order)
  const uint32_t n = (uint32_t)__popc(bits);
  uint32_t pre = 0u, tot = 0u;
#pragma unroll
  for (int bit = 0; bit < 5; ++bit) {
    const uint64_t bb = __ballot((n >> bit) & 1u);
    pre += lanes_below(bb) << bit;
    tot += (uint32_t)__popcll(bb) << bit;
  }
  if (lane == 0) l.wcnt[wave] = tot;
  __syncthreads();
  uint32_t start_e = pre, total_e = 0u;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    start_e += v < wave ? l.wcnt[v] : 0u;
    total_e += l.wcnt[v];
  }
  {
    uint32_t e = start_e;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      if ((bits >> i) & 1u) {
        l.pt[e] = vt[i];
        l.pq[e] = vq[i];
        l.pid[e] = (uint16_t)(tid * kPerThread + i);
        ++e;
      }
  }
  __syncthreads();
  const Weights w{q[1], 1.0 / q[2], q[3], resid ? 1.0 / q[4] : 0.0, a.inv_t, resid};
  const uint32_t per = (total_e + kThreads - 1) / kThreads;
  const uint32_t e0 = min((uint32_t)tid * per, total_e), e1 = min(e0 + per, total_e);
  double mine = 0.0;
  for (uint32_t e = e0; e < e1; ++e) {
    const float xq = l.pq[e];
    double wt, r;
    w.at(l.pt[e], xq, resid && xq == xq, wt, r);
    const double wv = resid ? r : wt;
    l.pw[e] = wv;
    mine += wv;
  }
  // exclusive prefix of the per-thread sums in thread order
  const double incl = wave_incl_scan_d(mine);
  if (lane == 63) l.wsum[wave] = incl;
  __syncthreads();
  double start = before;
  for (int v = 0; v < wave; ++v) start += l.wsum[v];
  double ex = __shfl_up(incl, 1, 64);
  if (lane == 0) ex = 0.0;
  start += ex;
  uint32_t found = SAS_NO_TOKEN, last = 0;
  bool any = false;
  double cum = start;
  for (uint32_t e = e0; e < e1; ++e) {
    const double wv = l.pw[e];
    if (wv > 0.0) {
      const uint32_t id = (uint32_t)((int64_t)chunk * kVChunk + l.pid[e]);
      any = true;
      last = id;
      cum += wv;
      if (found == SAS_NO_TOKEN && cum > target) found = id;
    }
  }
  if (!last_mode && found != SAS_NO_TOKEN) atomicMin(&l.found, found);
  if (any) atomicMax(&l.last, last + 1u);
  __syncthreads();
  if (tid == 0) {
    uint32_t tok = l.found;
    if (last_mode || tok == SAS_NO_TOKEN) tok = l.last ? l.last - 1u : SAS_NO_TOKEN;
    a.out_tokens[(int64_t)s * P1 + acc] = tok;
  }
}

}  // namespace

size_t verify_scratch_bytes(int seqs, int L, int vocab) {
  const size_t chunks = ((size_t)vocab + kVChunk - 1) / kVChunk;
  const size_t positions = (size_t)seqs * (L + 1);
  return (positions * chunks * 4 + (size_t)seqs * chunks * 2 + (size_t)seqs * 8) * sizeof(double) +
         positions * 2 * sizeof(float) + positions * chunks * kWaves * sizeof(uint32_t) +
         positions * chunks * kWaves * 2 * kCompact * sizeof(float);
}

hipError_t launch_verify(const VerifyArgs &a, hipStream_t stream) {
  const dim3 block(kThreads);
  const dim3 g1(a.chunks, a.seqs * (a.L + 1)), g2(a.chunks, a.seqs), g3(a.seqs);
  if (a.mask) {
    hipLaunchKernelGGL(verify_stats_kernel<true>, g1, block, 0, stream, a);
    hipLaunchKernelGGL(verify_decide_kernel<true>, g2, block, 0, stream, a);
    hipLaunchKernelGGL(verify_draw_kernel<true>, g3, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL(verify_stats_kernel<false>, g1, block, 0, stream, a);
    hipLaunchKernelGGL(verify_decide_kernel<false>, g2, block, 0, stream, a);
    hipLaunchKernelGGL(verify_draw_kernel<false>, g3, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace sas

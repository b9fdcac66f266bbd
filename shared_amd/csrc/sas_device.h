// sas_device.h - device-side helpers shared by the sampling kernels (gfx950).
//
// Every translation unit that includes this is compiled with
// -ffp-contract=off: the double-precision tail must round each operation
// separately, exactly as a JS engine does in sample()
// (lib/webgpu-llm/tokenizer.js:163-177).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared_amd_sampler.h"

namespace sas {

constexpr int kThreads = 256;           // 4 wave64s per block
constexpr int kWaves = kThreads / 64;
constexpr int kCapBlock = 256;          // candidates one exact chunk selection may emit
constexpr uint32_t kPenFlag = 0x80000000u;

// The waves that bound a part, and the rank each takes: lane l of wave w
// holds the part's ids from per * (64 w + l) on, `nids` ids in all.  Each
// of the first nw waves has j lane maxima at or above its j-th largest, so
// nw j >= k values of the part reach the smallest of those results.  A wave
// with fewer than j lanes that hold an id cannot bound (its result would be
// "no value"), so nw is the most waves whose last one has j = ceil(k / nw)
// such lanes; the other waves take no part.
struct BoundRank {
  int nw, j;
};
__device__ __forceinline__ BoundRank bound_rank(int nids, int per, int k) {
  // unrolled: every divisor a constant (no integer division instruction)
#pragma unroll
  for (int nw = kWaves; nw > 1; --nw) {
    const int j = (k + nw - 1) / nw;
    if ((nids - per * 64 * (nw - 1) + per - 1) / per >= j) return {nw, j};
  }
  return {1, k};
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
// A float4 that needs 4-byte alignment only (global loads take it as one 16-byte access).
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ float qnan() { return __builtin_nanf(""); }

// fp64 -> fp32 rounding toward -inf.  Monotone, and val >= t implies
// rd(val) >= t for every fp32 t, so fp32 keys can filter double values.
__device__ __forceinline__ float rd_f32(double d) {
  float f = (float)d;
  if ((double)f > d) {
    uint32_t b = __float_as_uint(f);
    if (f > 0.0f) b -= 1u;
    else if (f == 0.0f) b = 0x80000001u;
    else b += 1u;
    f = __uint_as_float(b);
  }
  return f;
}

// History penalty of a token seen `count` > 0 times: CTRL repetition
// (sign-wise), then OpenAI frequency and presence.  Presence alone is the
// reference's rule (tokenizer.js:157).
__device__ __forceinline__ double penalize(double v, uint32_t count, const sas_params &p) {
  double r = p.repetition_penalty;
  v = v > 0.0 ? v / r : v * r;
  v = v - p.frequency_penalty * (double)count;
  v = v - p.presence_penalty;
  return v;
}

// exp(x) by fdlibm's e_exp.c algorithm (Sun Microsystems, 1993): reduce
// x = k*ln2 + r with ln2 split in a 32-bit-exact high part and a low part,
// approximate exp(r) with the degree-5 Remez rational form, scale by 2^k.
// V8's Math.exp is this algorithm, so probabilities come out bit-identical
// to the reference's JS sample().
//
// Written without branches (lanes of a wave take different paths): every
// path is computed and the result selected.  The paths fdlibm keeps apart
// are one formula here, bit for bit:
//   - |x| in (ln2/2, 1.5 ln2) uses k = +-1, hi = x -+ ln2_hi, lo = +-ln2_lo,
//     which is k*ln2_hi and k*ln2_lo for k = +-1 (exact products);
//   - |x| <= ln2/2 uses k = 0 and no reduction: with k = 0, hi = x - 0 = x,
//     lo = 0, and 1 - ((0 + q) - x) is fdlibm's 1 - (q - x);
//   - fdlibm's (x*c)/(c-2) and (x*c)/(2-c) are one quotient and its exact
//     negation (IEEE subtraction and division are sign-symmetric), so
//     lo - (x*c)/(2-c) is lo + q to the bit.
// Specials (NaN, infinities, overflow, underflow, |x| < 2^-28, x == 1)
// are selected last, as fdlibm returns them before the reduction.
__device__ __forceinline__ double fd_exp(double x) {
  const double inv_ln2 = 1.44269504088896338700e+00;
  const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
  const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03,
               P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06,
               P5 = 4.13813679705723846039e-08;
  const double over = 7.09782712893383973096e+02, under = -7.45133219101941108420e+02;
  const double two_m1000 = 9.33263618503218878990e-302;
  const uint64_t bits = (uint64_t)__double_as_longlong(x);
  const uint32_t hx = (uint32_t)(bits >> 32) & 0x7fffffffu;
  const bool neg = (bits >> 63) != 0u;
  const bool reduce = hx > 0x3fd62e42u;   // |x| > ln2 / 2
  const bool one = hx < 0x3FF0A2B2u;      // |x| < 1.5 ln2
  // clamped so the conversion is defined for every x; |x| <= 745 is unchanged
  const double xc = fmin(fmax(x, -1100.0), 1100.0);
  const int kg = (int)(inv_ln2 * xc + (neg ? -0.5 : 0.5));
  const int k = reduce ? (one ? (neg ? -1 : 1) : kg) : 0;
  const double t = (double)k;
  const double hi = x - t * ln2_hi;
  const double lo = t * ln2_lo;
  const double r = hi - lo;
  const double rr = r * r;
  const double c = r - rr * (P1 + rr * (P2 + rr * (P3 + rr * (P4 + rr * P5))));
  const double q = (r * c) / (c - 2.0);
  const double y = 1.0 - ((lo + q) - hi);
  const int ke = k >= -1021 ? k : k + 1000;
  const double scale = __longlong_as_double((long long)((uint64_t)((0x3ffu + (uint32_t)ke) & 0x7ffu) << 52));
  double res = k >= -1021 ? y * scale : y * scale * two_m1000;
  if (k == 1024) res = y * 2.0 * 8.988465674311579539e307;
  if (reduce && one && x == 1.0) res = 2.718281828459045;
  if (hx < 0x3e300000u) res = 1.0 + x;    // |x| < 2^-28
  if (x < under) res = 0.0;
  if (x > over) res = __longlong_as_double(0x7ff0000000000000ll);
  if (hx >= 0x7ff00000u) res = (((hx & 0xfffffu) | (uint32_t)bits) != 0u) ? x + x : (neg ? 0.0 : x);
  return res;
}

// e^x for sums of many weights, where the order of the additions already
// differs from a sequential loop: within 2 ulp of the exact value, with no
// division.  x = k ln2 + r (|r| <= ln2 / 2, ln2 split in two parts), e^r by
// its Taylor series to degree 13 (truncation below 2^-60 relative), scaled
// by 2^k with ldexp (subnormal results included).  x = -inf gives 0; x past
// 709.78 overflows to +inf; NaN stays NaN.
__device__ __forceinline__ double exp_sum(double x) {
  const double inv_ln2 = 1.44269504088896338700e+00;
  const double ln2_hi = 6.93147180369123816490e-01, ln2_lo = 1.90821492927058770002e-10;
  const double xc = fmin(fmax(x, -1100.0), 1100.0);
  const double k = rint(xc * inv_ln2);
  const double r = fma(-k, ln2_lo, fma(-k, ln2_hi, xc));
  double p = 1.0 / 6227020800.0;  // 1/13!
  p = fma(p, r, 1.0 / 479001600.0);
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  const double res = __builtin_amdgcn_ldexp(p, (int)k);
  return x == x ? res : x;
}

// tanh of an fp32 value, rounded once to fp32 from a double-precision
// evaluation: an odd Taylor polynomial below 2^-9, (e^2x - 1)/(e^2x + 1)
// with the fdlibm exp above, 1 from 9.5 on.  Only correctly rounded double
// operations and fd_exp are used, so the host oracle computes the same bits.
__device__ __forceinline__ float tanh_f32(float x) {
  const double ax = fabs((double)x);
  double r;
  if (!(ax == ax)) return x;
  if (ax >= 9.5) {
    r = 1.0;
  } else if (ax < 0.001953125) {
    const double x2 = ax * ax;
    r = ax * (1.0 - x2 * (1.0 / 3.0 - x2 * (2.0 / 15.0 - x2 * (17.0 / 315.0))));
  } else {
    const double t = fd_exp(2.0 * ax);
    r = (t - 1.0) / (t + 1.0);
  }
  return copysignf((float)r, x);
}

// Gemma's final-logit softcap cap*tanh(x/cap) in fp32 (kernels.js:1393-1395;
// cap 30, gemma-config.js:47).
__device__ __forceinline__ float softcap_f32(float x, float cap) {
  const float q = x / cap;
  return cap * tanh_f32(q);
}

// (v desc, id asc): the order of the reference's stable descending sort
// over an id-ascending candidate list (tokenizer.js:160).
__device__ __forceinline__ bool ranks_before(double va, uint32_t ia, double vb, uint32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// LDS writes of a wave visible to the wave's other lanes.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Order-preserving map of an fp32 key to uint32 (larger float, larger
// uint); NaN maps to 0, which marks "no key".
__device__ __forceinline__ uint32_t okey(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return 0u;
  if (u == 0x80000000u) u = 0u;  // -0 and +0 are one value: one key
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inverse of okey for nonzero images.
__device__ __forceinline__ float fkey(uint32_t x) {
  return __uint_as_float((x & 0x80000000u) ? (x & 0x7FFFFFFFu) : ~x);
}

// j-th largest (1-based) of the 64 lane keys of a wave (okey images, 0 =
// none); 0 when fewer than j lanes hold a key.  Bit-by-bit search from the
// top: each step is one compare and a ballot count, no cross-lane moves.
__device__ __forceinline__ uint32_t wave_jth_largest_key(uint32_t u, int j) {
  uint32_t res = 0u;
#pragma unroll
  for (int b = 31; b >= 0; --b) {
    const uint32_t cand = res | (1u << b);
    if (__popcll(__ballot(u >= cand)) >= j) res = cand;
  }
  return res;
}

// As wave_jth_largest_key searched to the top 16 bits only: the largest
// key with zero low half that at least j lane keys reach.  A lower bound of
// the exact j-th largest, at half the steps.
__device__ __forceinline__ uint32_t wave_jth_largest_key16(uint32_t u, int j) {
  uint32_t res = 0u;
#pragma unroll
  for (int b = 31; b >= 16; --b) {
    const uint32_t cand = res | (1u << b);
    if (__popcll(__ballot(u >= cand)) >= j) res = cand;
  }
  return res;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) x = fmaxf(x, __shfl_xor(x, s, 64));
  return x;
}

// Best (value, id) over the wave under ranks_before; lanes without a
// candidate pass have = false.
__device__ __forceinline__ void wave_best(bool &have, double &v, uint32_t &id) {
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    int oh = __shfl_xor((int)have, s, 64);
    double ov = __shfl_xor(v, s, 64);
    uint32_t oi = (uint32_t)__shfl_xor((int)id, s, 64);
    if (oh && (!have || ranks_before(ov, oi & ~kPenFlag, v, id & ~kPenFlag))) {
      have = true;
      v = ov;
      id = oi;
    }
  }
}

// DPP lane moves (GFX9 encodings).  dpp0: lanes whose source lies outside
// their row (or in a row that row_mask leaves out) read 0; dppx: every
// source lies inside the row.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ uint32_t dpp0(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kCtrl, kRowMask, 0xF, true);
}
template <int kCtrl>
__device__ __forceinline__ uint32_t dppx(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, kCtrl, 0xF, 0xF, false);
}
constexpr int kDppQuad1032 = 0xB1, kDppQuad2301 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// Inclusive prefix sum over the wave: Hillis-Steele within each row of 16
// lanes, then the rows' totals broadcast forward.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dpp0<kDppRowShr1>(x);
  x += dpp0<kDppRowShr2>(x);
  x += dpp0<kDppRowShr4>(x);
  x += dpp0<kDppRowShr8>(x);
  x += dpp0<kDppRowBcast15, 0xA>(x);
  x += dpp0<kDppRowBcast31, 0xC>(x);
  return x;
}

// Wave-wide reductions: pairs, quads, eights and rows of 16 by DPP, then the
// four rows' results (wave-uniform).
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t x, Op op) {
  x = op(x, dppx<kDppQuad1032>(x));
  x = op(x, dppx<kDppQuad2301>(x));
  x = op(x, dppx<kDppRowHalfMirror>(x));
  x = op(x, dppx<kDppRowMirror>(x));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 16),
                 r2 = (uint32_t)__builtin_amdgcn_readlane((int)x, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
  return op(op(r0, r1), op(r2, r3));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  return wave_reduce(x, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
// A wave's bound at rank j: a key that at least j lane keys reach.  Rank 1
// (greedy rows) takes the wave's largest key exactly; other ranks the 16-bit
// lower bound of wave_jth_largest_key16, at half the ballot steps of the
// exact search.
__device__ __forceinline__ uint32_t wave_rank_key(uint32_t u, int j) {
  return j == 1 ? wave_max_u32(u) : wave_jth_largest_key16(u, j);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  return wave_reduce(x, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t x) {
  return wave_reduce(x, [](uint32_t a, uint32_t b) { return a + b; });
}

// The value of the wave's first active lane (wave-uniform values).
__device__ __forceinline__ uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

// Barrier over the block's LDS accesses alone: it waits for this wave's LDS
// operations but not for its global loads, so loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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

}  // namespace sas

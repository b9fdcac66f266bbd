// lmhead_kernel.hip - the LM head with the sampling step's parts pass fused
// into its epilogue (gfx950).
//
// The decode head of the reference is a projection of the final-normed
// hidden state onto every vocabulary row, then a topk pass that reads the
// logits back (lib/webgpu-llm/model.js:466-471, gemma-model.js:786-799).
// Here the logits never leave the chip: the block that computes a part's
// logits also masks, penalizes and bounds them and writes only the part's
// candidate records, in the records format of the sampling kernels.
//
// lmh_parts_kernel: grid = parts (kLmhSpan ids each), 256 threads, every
// row of the call (<= SAS_LMH_MAX_ROWS).  The rows' hidden states are staged
// once in LDS.  Eight lanes share one id: lane g of the group sums the
// hidden indices 64 c + 8 g .. + 7 (c ascending) as one f32 fused
// multiply-add chain, so each load of the group is a whole 128-byte line of
// the weight row; the eight partial sums then add in one fixed tree.  That
// order is the one the host oracle follows.  The bf16 weight widens exactly
// to f32 (bits << 16, ggml/kernels.js:31-33), so each product is the
// reference's f32 product.
// The epilogue, per row: softcap, mask, history membership, the part's
// bound (every wave's j-th largest lane maximum, the smallest of the four:
// 4 j >= k values reach it), the values at or above it as records, the
// members' penalized doubles as member records, the part's info word.
//
// lmh_group_kernel: one block per (row, kLmhGroup consecutive parts) keeps
// the records at or above the group's k-th largest key (at or above the
// largest of the parts' bounds: that part alone holds k values above it)
// and writes them as one part of the merge kernel, which then draws as for
// sas_sample.
#include "sas_device.h"
#include "sas_launch.h"

namespace sas {

constexpr int kLmhIds = kLmhSpan / kThreads;  // ids per lane
static_assert(kLmhIds == 2, "a lane owns two ids of its part");
constexpr int kLmhStep = 64;                   // hidden values per load step: 128 bytes of a weight row
constexpr int kLmhHash = 512;                  // (id, count) hash slots of a part's history members
constexpr uint32_t kLmhEmpty = 0xFFFFFFFFu;

// The epilogue's tables, one set per row of the call: the rows are
// selected together, so each barrier serves all of them.
template <int R>
struct LmhLds {
  uint32_t hkey[R][kLmhHash];
  uint32_t hcnt[R][kLmhHash];
  uint32_t hbits[R][kLmhSpan / 32];  // history membership of the part's ids
  uint32_t thr[R][kWaves];           // each wave's bound key
  uint32_t nw[R][kWaves];            // each wave's plain records
  uint32_t nmem[R];                  // members kept at or above the bound
  uint32_t nmw[R];                   // member records written
  uint32_t hover[R];                 // some history id did not fit in the hash
  uint32_t nx, slow;                 // an exact selection's plain records, and whether one ran
  uint32_t hist[256];                // block_select96
  uint32_t sel[4];
};

__device__ __forceinline__ uint32_t lmh_slot(uint32_t id) { return (id * 2654435761u) >> 23; }
static_assert(kLmhHash == 512, "lmh_slot yields 9 bits");

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// What the epilogue of one row reads from memory, loaded when the block
// starts so that no round trip waits after the dot products: the row's
// history range, its first 2 x 256 history ids, the mask word of this
// lane's two ids.
struct LmhPre {
  int h0, h1;
  const uint32_t *ids;  // the history: hist_ids, or the row's ring slots
  uint32_t hid[2];
  uint32_t mword;
};

// The history range and the mask word (no load depends on another)...
__device__ __forceinline__ void lmh_prefetch_range(const SampleArgs &a, int row, int id0, LmhPre &q) {
  q.h0 = 0;
  q.h1 = 0;
  q.ids = a.hist_ids;
  if (a.ring) {
    // a decode step's penalty ring: its first min(count, ring_len) slots
    const uint32_t *rg = a.ring + (int64_t)row * (a.ring_len + 1);
    q.ids = rg + 1;
    q.h1 = (int)min(rg[0], (uint32_t)a.ring_len);
  } else if (a.hist_ids) {
    const int64_t o0 = min(max((int64_t)a.hist_offsets[row], (int64_t)0), a.hist_count);
    const int64_t o1 = min(max((int64_t)a.hist_offsets[row + 1], o0), min(a.hist_count, o0 + SAS_MAX_HISTORY));
    q.h0 = (int)o0;
    q.h1 = (int)o1;
  }
  // id0 is even: both ids share one mask word
  q.mword = a.mask && id0 < a.vocab ? a.mask[(int64_t)row * a.mask_stride + (id0 >> 5)] : ~0u;
}

// ... then the first history ids, once the range is known.
__device__ __forceinline__ void lmh_prefetch_ids(LmhPre &q) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = q.h0 + j * kThreads + (int)threadIdx.x;
    q.hid[j] = i < q.h1 ? q.ids[i] : kLmhEmpty;
  }
}

// The part's selection for every row of the call: values v[r][0..1] of ids
// id0, id0 + 1 (raw logits), each row's parameters and history; writes each
// row's records and info word.  A member is penalized by the lane that holds
// it (its count from the row's hash) and kept when it reaches the bound,
// which comes from the plain values only.
template <int R>
__device__ __forceinline__ void lmh_select_rows(const LmhArgs &L, LmhLds<R> &S, int part, const float (&v_in)[R][2],
                                                int id0, const LmhPre (&pf)[R]) {
  const SampleArgs &a = L.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int vocab = a.vocab;
  const int base = part * kLmhSpan;
  const int nids = min(kLmhSpan, vocab - base);
  // ---- history: each row's ids inside the part, in a bitmap and a hash ----
#pragma unroll
  for (int r = 0; r < R; ++r) {
    for (int s2 = tid; s2 < kLmhHash; s2 += kThreads) {
      S.hkey[r][s2] = kLmhEmpty;
      S.hcnt[r][s2] = 0u;
    }
    if (tid < kLmhSpan / 32) S.hbits[r][tid] = 0u;
    if (tid == 0) {
      S.nmem[r] = 0u;
      S.nmw[r] = 0u;
      S.hover[r] = 0u;
    }
  }
  __syncthreads();
  auto insert = [&](int r, uint32_t id) __attribute__((always_inline)) {
    const uint32_t off = id - (uint32_t)base;
    if (off >= (uint32_t)nids) return;
    atomicOr(&S.hbits[r][off >> 5], 1u << (off & 31u));
    uint32_t sl = lmh_slot(id);
    int probe = 0;
    for (; probe < kLmhHash; ++probe) {
      const uint32_t old = atomicCAS(&S.hkey[r][sl], kLmhEmpty, id);
      if (old == kLmhEmpty || old == id) {
        atomicAdd(&S.hcnt[r][sl], 1u);
        break;
      }
      sl = (sl + 1u) & (uint32_t)(kLmhHash - 1);
    }
    if (probe == kLmhHash) S.hover[r] = 1u;
  };
#pragma unroll
  for (int r = 0; r < R; ++r) {
    // the first 2 x 256 ids came with the block's first loads (kLmhEmpty past
    // the range: never inside the part)
    insert(r, pf[r].hid[0]);
    insert(r, pf[r].hid[1]);
    for (int i = pf[r].h0 + 2 * kThreads + tid; i < pf[r].h1; i += kThreads) insert(r, pf[r].ids[i]);
  }
  __syncthreads();
  auto hcount = [&](int r, uint32_t id) -> uint32_t {
    uint32_t sl = lmh_slot(id);
    for (int probe = 0; probe < kLmhHash; ++probe) {
      const uint32_t kk = S.hkey[r][sl];
      if (kk == id) return S.hcnt[r][sl];
      if (kk == kLmhEmpty) break;
      sl = (sl + 1u) & (uint32_t)(kLmhHash - 1);
    }
    uint32_t c = 0u;
    if (S.hover[r])
      for (int i = pf[r].h0; i < pf[r].h1; ++i) c += pf[r].ids[i] == id ? 1u : 0u;
    return c;
  };
  // ---- values: softcap, mask, membership; members penalized here; the bound ----
  sas_params p[R];
  int kr[R];
  float pv[R][2];   // plain candidates (NaN: none)
  bool mem[R][2];   // allowed history members
  double mv[R][2];  // their penalized values
#pragma unroll
  for (int r = 0; r < R; ++r) {
    p[r] = a.params;
    if (a.row_params) p[r] = load_row_params(a.row_params + r);
    kr[r] = !(p[r].temperature > 0.0) ? 1 : min(max(p[r].top_k, 1), SAS_MAX_TOP_K);
    const uint32_t *mrow = a.mask ? a.mask + (int64_t)r * a.mask_stride : nullptr;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int id = id0 + j;
      float x = v_in[r][j];
      if (p[r].softcap > 0.0f) x = softcap_f32(x, p[r].softcap);
      bool ok = id < vocab && x == x;
      if (ok && mrow) ok = ((pf[r].mword >> (id & 31)) & 1u) != 0u;
      const uint32_t off = (uint32_t)(id - base);
      const bool hm = ok && off < (uint32_t)nids && ((S.hbits[r][off >> 5] >> (off & 31u)) & 1u) != 0u;
      mem[r][j] = hm;
      pv[r][j] = ok && !hm ? x : qnan();
      mv[r][j] = hm ? penalize((double)x, hcount(r, (uint32_t)id), p[r]) : 0.0;
    }
    const float m = fmaxf(pv[r][0], pv[r][1]);
    const uint32_t tw = wave_jth_largest_key16(okey(m), (kr[r] + kWaves - 1) / kWaves);
    if (lane == 0) S.thr[r][wave] = tw;
  }
  __syncthreads();
  // ---- plain records: each wave's after the waves before it; members kept ----
  uint32_t tkey[R], pre[R];
  float tf[R];
  bool k0[R], k1[R], m0[R], m1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    tkey[r] = min(min(S.thr[r][0], S.thr[r][1]), min(S.thr[r][2], S.thr[r][3]));
    tf[r] = tkey[r] > 0x007FFFFFu ? fkey(tkey[r]) : -__builtin_inff();
    k0[r] = pv[r][0] >= tf[r];  // NaN never passes
    k1[r] = pv[r][1] >= tf[r];
    const uint32_t c = (k0[r] ? 1u : 0u) + (k1[r] ? 1u : 0u);
    const uint64_t b0 = __ballot(c & 1u), b1 = __ballot((c >> 1) & 1u);
    pre[r] = lanes_below(b0) + 2u * lanes_below(b1);
    if (lane == 0) S.nw[r][wave] = (uint32_t)__popcll(b0) + 2u * (uint32_t)__popcll(b1);
    m0[r] = mem[r][0] && mv[r][0] >= (double)tf[r];  // NaN never passes
    m1[r] = mem[r][1] && mv[r][1] >= (double)tf[r];
    const uint32_t nm = (m0[r] ? 1u : 0u) + (m1[r] ? 1u : 0u);
    if (nm) atomicAdd(&S.nmem[r], nm);
  }
  __syncthreads();
  // ---- records, row by row (a row past its member slots selects exactly) ----
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint32_t off = 0u;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) off += w < wave ? S.nw[r][w] : 0u;
    const uint32_t nplain = S.nw[r][0] + S.nw[r][1] + S.nw[r][2] + S.nw[r][3];
    const uint32_t nmem = S.nmem[r];
    const int64_t pq = (int64_t)r * a.parts + part;
    uint64_t *rrow = a.rec + pq * kListCap;
    uint4 *mrow4 = a.mrec + pq * kMemSlots;
    uint32_t np_out = nplain, nm_out = nmem, slow = 0u;
    auto put_member = [&](uint32_t d, double val, uint32_t id) __attribute__((always_inline)) {
      uint64_t *w = reinterpret_cast<uint64_t *>(mrow4 + d);
      w[0] = (uint64_t)__float_as_uint(rd_f32(val)) | ((uint64_t)id << 32);
      w[1] = (uint64_t)__double_as_longlong(val);
    };
    if (nmem <= (uint32_t)kMemSlots) {
      uint32_t j = off + pre[r];
      if (k0[r]) rrow[j++] = (uint64_t)__float_as_uint(pv[r][0]) | ((uint64_t)(uint32_t)id0 << 32);
      if (k1[r]) rrow[j] = (uint64_t)__float_as_uint(pv[r][1]) | ((uint64_t)(uint32_t)(id0 + 1) << 32);
      if (m0[r]) put_member(atomicAdd(&S.nmw[r], 1u), mv[r][0], (uint32_t)id0);
      if (m1[r]) put_member(atomicAdd(&S.nmw[r], 1u), mv[r][1], (uint32_t)(id0 + 1));
    } else {
      // more members above the bound than a part's member slots hold: the
      // part's exact top k over (value, id), every value computed again
      const uint32_t *mrow = a.mask ? a.mask + (int64_t)r * a.mask_stride : nullptr;
      auto for_elems = [&](auto f) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int id = id0 + j;
          float x = v_in[r][j];
          if (p[r].softcap > 0.0f) x = softcap_f32(x, p[r].softcap);
          bool ok = id < vocab && x == x;
          if (ok && mrow) ok = ((mrow[id >> 5] >> (id & 31)) & 1u) != 0u;
          double val = (double)x;
          if (ok && mem[r][j]) val = mv[r][j];
          ok = ok && val == val;
          f(key96(val, (uint32_t)id), ok, val, (uint32_t)id, mem[r][j]);
        }
      };
      uint32_t nval = 0u;
      for_elems([&](const Key96 &, bool ok, double, uint32_t, bool) { nval += ok ? 1u : 0u; });
      if (tid == 0) S.sel[3] = 0u;
      __syncthreads();
      atomicAdd(&S.sel[3], nval);
      __syncthreads();
      const uint32_t need = min(S.sel[3], (uint32_t)kr[r]);
      __syncthreads();
      if (tid == 0) {
        S.nx = 0u;
        S.nmw[r] = 0u;
      }
      __syncthreads();
      if (need > 0u) {
        const Key96 kth = block_select96(
            [&](auto f) { for_elems([&](const Key96 &kx, bool ok, double, uint32_t, bool) { f(kx, ok); }); }, need,
            S.hist, S.sel);
        for_elems([&](const Key96 &kx, bool ok, double val, uint32_t id, bool member) {
          if (ok && key_ge(kx, kth)) {
            if (member) put_member(atomicAdd(&S.nmw[r], 1u), val, id);
            else rrow[atomicAdd(&S.nx, 1u)] = (uint64_t)__float_as_uint((float)val) | ((uint64_t)id << 32);
          }
        });
      }
      __syncthreads();
      np_out = S.nx;
      nm_out = S.nmw[r];
      slow = 1u;
      __syncthreads();  // S.nx and S.sel are reused by the next row
    }
    if (tid == 0)
      a.pinfo[(int64_t)r * pinfo_stride(a.parts) + part] =
          (uint64_t)(np_out | (nm_out << 16) | (slow ? kPinfoSlow : 0u)) | ((uint64_t)tkey[r] << 32);
  }
}

// ---- GGUF heads: the Q8_1 operand on chip, exact integer block dots ----

// GGUF rows are staged through LDS: 8 items of a row at a time (a stage:
// 8 blocks of Q8_0 / Q4_0, 8 units = 2 super-blocks of Q6_K), loaded as the
// 16-byte aligned chunks that cover them, so the 8 lanes of a row read 128
// contiguous bytes per load and every load is a whole aligned chunk.  A
// chunk that holds one byte of the head lies in the head's pages, so the
// few bytes it holds past either end of the stage are safe to read.
template <int kFmt>
struct QStage {
  static constexpr int bytes = kFmt == SAS_HEAD_Q6_K ? 420 : kFmt == SAS_HEAD_Q8_0 ? 272 : 144;
  static constexpr int chunks = (bytes + 14 + 15) / 16;  // the stage starts 0 .. 14 bytes into its first chunk
  static constexpr int loads = (chunks + 7) / 8;         // per lane
  static constexpr int pitch = 4 * (chunks + 1);         // LDS dwords per row (one chunk of bank skew)
  static constexpr int depth = 4;                        // stages in flight per wave
};

__device__ __forceinline__ float f16_value(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// N words that start `sh` bytes (0 or 2) into u[0]: the N + 1 dwords
// read from LDS, shifted.
template <int N>
__device__ __forceinline__ void words_of(const uint32_t (&u)[N + 1], uint32_t sh, uint32_t (&out)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(u[i + 1], u[i], sh);
}
template <int N>
__device__ __forceinline__ void lds_dwords(const uint32_t *p, uint32_t (&u)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) u[i] = p[i];
}

// The Q8_1 operand of R hidden rows, in LDS, packed per item so that a
// lane reads its item's operand from one base address in whole 16-byte
// loads: kQOpWords dwords per item, rows one after another.
//   Q8_0 / Q4_0, per 32-value block: q (8 words, four int8 each), d8, s8
//     (the f16 d and d * sum(q), as f32), 2 words of padding;
//   Q6_K, per 64-value unit u (super-block u / 4, half h = (u / 2) % 2,
//     16-value half lh = u % 2): for its quarters qt = 0 .. 3 (the Q8_1
//     block 8 (u / 4) + 4 h + qt, its half lh): the 16 q (4 words each,
//     quarter after quarter), then -32 x each quarter's sum of q, then each
//     quarter's d8.
// One 32-value block per thread per round (q8.js:27-42): amax,
// d = amax / 127, q = round-half-even(x * (1 / d)), the f16 d and d * sum(q).
template <int kFmt>
constexpr int kQOpWords = kFmt == SAS_HEAD_Q6_K ? 24 : 12;
template <int kFmt>
__host__ __device__ constexpr int q_items(int dim) {
  return kFmt == SAS_HEAD_Q6_K ? dim / 64 : dim / 32;
}

template <int R, int kFmt>
__device__ __forceinline__ void q81_stage(const LmhArgs &L, uint32_t *U) {
  const int dim = L.dim, nq = dim / 32, rw = q_items<kFmt>(dim) * kQOpWords<kFmt>;
  for (int t = threadIdx.x; t < R * nq; t += kThreads) {
    const int r = t / nq, b = t - r * nq;
    const float *h = L.hidden + (int64_t)r * L.hidden_stride + 32 * b;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = h[i];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    const float d = amax / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t w[8];
    int sum = 0, half = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t x = 0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float xs = v[4 * j + i] * inv;
        const float rq = xs != xs ? 0.0f : fminf(fmaxf(rintf(xs), -128.0f), 127.0f);
        const int qi = (int)rq;
        sum += qi;
        x |= ((uint32_t)qi & 0xFFu) << (8 * i);
      }
      w[j] = x;
      if (j == 3) half = sum;
    }
    const float d16 = (float)(_Float16)d;
    uint32_t *ur = U + r * rw;
    if constexpr (kFmt == SAS_HEAD_Q6_K) {
      const int sb = b >> 3, hh = (b >> 2) & 1, qt = b & 3;
#pragma unroll
      for (int lh = 0; lh < 2; ++lh) {
        uint32_t *o = ur + (sb * 4 + hh * 2 + lh) * 24;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[4 * qt + j] = w[4 * lh + j];
        o[16 + qt] = (uint32_t)(-32 * (lh ? sum - half : half));
        o[20 + qt] = __float_as_uint(d16);
      }
    } else {
      uint32_t *o = ur + b * 12;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = w[j];
      o[8] = __float_as_uint(d16);
      o[9] = __float_as_uint((float)(_Float16)(d * (float)sum));
    }
  }
}

// Where a lane's item lies in its row's staged copy: `c0` its byte offset
// from the stage's first byte, and the LDS dword index of each field for a
// stage that starts at dword 0 (the stage adds its own base).
template <int kFmt>
struct QLane {
  uint32_t c0, row;  // Q8_0 / Q4_0: the block (its f16 d, then its values)
};
template <>
struct QLane<SAS_HEAD_Q6_K> {
  uint32_t c0, la, lb, qh, sc, d;  // Q6_K: the unit's ql spans, qh span, scales, the super-block's d
  uint32_t lh8;                    // 8 lh: the bit offset of the unit's scales in a scale word
};

// Item g of a stage of the lane's row, whose copy starts at LDS dword `row`.
template <int kFmt>
__device__ __forceinline__ QLane<kFmt> q_lane(int g, uint32_t row) {
  QLane<kFmt> ln;
  if constexpr (kFmt == SAS_HEAD_Q6_K) {
    // unit g % 4 (half h, quarter pair lh) of the stage's super-block g / 4
    const uint32_t h = (uint32_t)(g & 3) >> 1, lh = (uint32_t)g & 1u;
    ln.c0 = 210u * (uint32_t)(g >> 2);
    ln.la = row + h * 16u + lh * 4u;        // byte h*64 + lh*16
    ln.lb = ln.la + 8u;                     // byte h*64 + 32 + lh*16
    ln.qh = row + 32u + h * 8u + lh * 4u;   // byte 128 + h*32 + lh*16
    ln.sc = row + 48u + h * 2u;             // byte 192 + h*8: scales h*8 .. h*8 + 7
    ln.d = row + 52u;                       // byte 208
    ln.lh8 = 8u * lh;
  } else {
    ln.c0 = (uint32_t)((kFmt == SAS_HEAD_Q8_0 ? 34 : 18) * g);
    ln.row = row;
  }
  return ln;
}

// A lane's Q8_1 operand for its item, read from LDS where it is used: `u`
// the item's words for row 0, `rw` words between rows.
struct QOp {
  const uint32_t *u;
  int rw;
  // Q8_0 / Q4_0: the block's 32 values, d and the f16 of d * sum
  __device__ __forceinline__ void block(int r, int32_t (&q)[8], float &d, float &sd) const {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *p = reinterpret_cast<const u32x4 *>(u + r * rw);
    const u32x4 a0 = p[0], a1 = p[1], a2 = p[2];
    q[0] = (int32_t)a0.x;
    q[1] = (int32_t)a0.y;
    q[2] = (int32_t)a0.z;
    q[3] = (int32_t)a0.w;
    q[4] = (int32_t)a1.x;
    q[5] = (int32_t)a1.y;
    q[6] = (int32_t)a1.z;
    q[7] = (int32_t)a1.w;
    d = __uint_as_float(a2.x);
    sd = __uint_as_float(a2.y);
  }
  // Q6_K: quarter qt of the unit, -32 x its sum, its Q8_1 block's d
  __device__ __forceinline__ void quarter(int r, int qt, int32_t (&q4)[4], int32_t &zq, float &dq) const {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const uint32_t *b = u + r * rw;
    const u32x4 a = reinterpret_cast<const u32x4 *>(b)[qt];
    q4[0] = (int32_t)a.x;
    q4[1] = (int32_t)a.y;
    q4[2] = (int32_t)a.z;
    q4[3] = (int32_t)a.w;
    zq = (int32_t)b[16 + qt];
    dq = __uint_as_float(b[20 + qt]);
  }
};

// The dwords of a lane's item of a stage, read from its row's copy in LDS
// one stage ahead of their use (so that the LDS round trip overlaps the
// previous stage's arithmetic).
template <int kFmt>
struct QRaw {
  uint32_t w[kFmt == SAS_HEAD_Q8_0 ? 9 : 5];  // Q8_0 / Q4_0: the values' dwords
  uint32_t d;                                // the dword of the f16 d
  uint32_t x0;                               // the item's first byte in the copy
};
template <>
struct QRaw<SAS_HEAD_Q6_K> {
  uint32_t la[5], lb[5], qh[5], sc[3], d;
  uint32_t x0;
};

template <int kFmt>
__device__ __forceinline__ void q_fetch(const uint32_t *stg, const QLane<kFmt> &ln, uint32_t off, QRaw<kFmt> &x) {
  const uint32_t x0 = off + ln.c0;  // the item's first byte (even)
  x.x0 = x0;
  if constexpr (kFmt == SAS_HEAD_Q8_0 || kFmt == SAS_HEAD_Q4_0) {
    lds_dwords(stg + ln.row + ((x0 + 2u) >> 2), x.w);
    x.d = stg[ln.row + (x0 >> 2)];
  } else {
    // every field of the unit starts a multiple of 4 bytes after x0: one
    // dword base and one shift for all
    const uint32_t bdw = x0 >> 2;
    lds_dwords(stg + ln.la + bdw, x.la);
    lds_dwords(stg + ln.lb + bdw, x.lb);
    lds_dwords(stg + ln.qh + bdw, x.qh);
    lds_dwords(stg + ln.sc + bdw, x.sc);
    x.d = stg[ln.d + bdw];
  }
}

// Adds the lane's item (fetched by q_fetch) to acc[r] for every row, in the
// order of the header.
template <int R, int kFmt>
__device__ __forceinline__ void q_terms(const QRaw<kFmt> &x, const QLane<kFmt> &ln, const QOp &op, float (&acc)[R]) {
  if constexpr (kFmt == SAS_HEAD_Q8_0 || kFmt == SAS_HEAD_Q4_0) {
    constexpr int NW = kFmt == SAS_HEAD_Q8_0 ? 8 : 4;
    uint32_t wv[NW];
    words_of<NW>(x.w, (x.x0 + 2u) & 3u, wv);
    const float dw = f16_value(x.d >> (8u * (x.x0 & 2u)));
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int32_t q[8];
      float d8b, s8b;
      op.block(r, q, d8b, s8b);
      int dot = 0;
      if constexpr (kFmt == SAS_HEAD_Q8_0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) dot = __builtin_amdgcn_sdot4((int)wv[j], q[j], dot, false);
        acc[r] = acc[r] + ((float)dot * dw) * d8b;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dot = __builtin_amdgcn_sdot4((int)(wv[j] & 0x0F0F0F0Fu), q[j], dot, false);
          dot = __builtin_amdgcn_sdot4((int)((wv[j] >> 4) & 0x0F0F0F0Fu), q[4 + j], dot, false);
        }
        acc[r] = acc[r] + (((float)dot * dw) * d8b - (8.0f * dw) * s8b);
      }
    }
  } else {
    const uint32_t sh = x.x0 & 3u;
    uint32_t la[4], lb[4], qh[4], sc[2];
    words_of<4>(x.la, sh, la);
    words_of<4>(x.lb, sh, lb);
    words_of<4>(x.qh, sh, qh);
    words_of<2>(x.sc, sh, sc);  // scales h*8 .. h*8 + 7
    const float dq = f16_value(x.d >> (8u * sh));
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      // the 16 six-bit values q of quarter qt, one per byte (0 .. 63): the
      // low or high nibbles of its ql span, bits 2 qt, 2 qt + 1 of qh moved
      // to bits 4, 5.  sum (q - 32) q8 = sum q q8 - 32 sum q8, exactly.
      const uint32_t *src = (qt & 1) ? lb : la;
      uint32_t raw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t nib = qt >= 2 ? src[j] >> 4 : src[j];
        const uint32_t hi = qt == 3 ? qh[j] >> 2 : qh[j] << (4 - 2 * qt);
        raw[j] = (nib & 0x0F0F0F0Fu) | (hi & 0x30303030u);
      }
      // scale byte h*8 + lh + 2 qt: word qt >> 1, byte lh + 2 (qt & 1)
      const uint32_t sw = sc[qt >> 1];
      const float scv = (float)(int)(int8_t)(uint8_t)(sw >> (ln.lh8 + 16u * (uint32_t)(qt & 1)));
      const float ds = dq * scv;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        int32_t q4[4], zq;
        float d8q;
        op.quarter(r, qt, q4, zq, d8q);
        int dot = __builtin_amdgcn_sdot4((int)raw[0], q4[0], zq, false);
        dot = __builtin_amdgcn_sdot4((int)raw[1], q4[1], dot, false);
        dot = __builtin_amdgcn_sdot4((int)raw[2], q4[2], dot, false);
        dot = __builtin_amdgcn_sdot4((int)raw[3], q4[3], dot, false);
        acc[r] = acc[r] + (ds * d8q) * (float)dot;
      }
    }
  }
}

template <int R, int kFmt>
__global__ __launch_bounds__(kThreads, 2) void lmh_parts_kernel(const LmhArgs L) {
  // bf16: [R][dim] hidden states; GGUF: their Q8_1 operand
  extern __shared__ __attribute__((aligned(16))) float xs[];
  __shared__ LmhLds<R> S;
  __shared__ float s_logit[R][kLmhSpan];  // the part's logits, row by row
  // GGUF: each wave's staged rows (8 rows of one stage)
  __shared__ __attribute__((aligned(16))) uint32_t stg[kFmt == SAS_HEAD_BF16 ? 4 : kWaves * 8 * QStage<kFmt>::pitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int part = blockIdx.x;
  const int base = part * kLmhSpan;
  const int dim = L.dim;
  const int vocab = L.s.vocab;
  // ---- the dot products.  Lanes work in groups of 8 on one id: lane g of
  // the group takes hidden indices 64 c + 8 g .. + 7 (c = 0, 1, ...), so a
  // group reads whole 128-byte lines of the weight row and a wave eight of
  // them per load.  Group grp (32 per block) takes ids base + grp + 32 m,
  // m = 0 .. 15: at each m the block reads 32 consecutive rows.  (GGUF
  // heads: lane g takes blocks or units g, g + 8, ... of the row.) ----
  const int g = lane & 7;
  const int grp = (wave << 3) | (lane >> 3);
  LmhPre pre[R];
  if constexpr (kFmt == SAS_HEAD_BF16) {
    const int C = dim / kLmhStep;              // 128-byte steps per weight row
    constexpr int kQ = 4;                       // steps per batch of loads
    const int nb = C / kQ;                      // batches per id (dim is a multiple of 256)
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const uint16_t *W = static_cast<const uint16_t *>(L.weight);
    auto wrow = [&](int m) __attribute__((always_inline)) {
      const int id = min(base + grp + 32 * m, vocab - 1);  // loads stay inside the head
      return W + (int64_t)id * L.weight_stride + 8 * g;
    };
    u32x4 nxt[kQ], nx2[kQ];
    auto load_into = [&](u32x4 (&dst)[kQ], int m, int cb) __attribute__((always_inline)) {
      const uint16_t *w = wrow(m) + (int64_t)cb * kQ * kLmhStep;
#pragma unroll
      for (int q = 0; q < kQ; ++q) dst[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + q * kLmhStep));
    };
    // batches in the flattened order (m, cb): two in flight ahead of the one computed
    const int total = (kLmhSpan / 32) * nb;
    load_into(nxt, 0, 0);
    if (total > 1) load_into(nx2, nb > 1 ? 0 : 1, nb > 1 ? 1 : 0);
    // while the first batches are in flight: the epilogue's inputs (read at
    // the end, loaded now so that no round trip waits after the dot
    // products) and the rows' hidden states into LDS
#pragma unroll
    for (int r = 0; r < R; ++r) lmh_prefetch_range(L.s, r, base + kLmhIds * tid, pre[r]);
    for (int r = 0; r < R; ++r) {
      const float *h = L.hidden + (int64_t)r * L.hidden_stride;
      for (int i = tid; i < dim; i += kThreads) xs[r * dim + i] = h[i];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) lmh_prefetch_ids(pre[r]);
    __syncthreads();  // the hidden states are in LDS
    for (int m = 0; m < kLmhSpan / 32; ++m) {
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.0f;
      for (int cb = 0; cb < nb; ++cb) {
        u32x4 cur[kQ];
#pragma unroll
        for (int q = 0; q < kQ; ++q) {
          cur[q] = nxt[q];
          nxt[q] = nx2[q];
        }
        // the batch two ahead in flight
        const int t2 = m * nb + cb + 2;
        if (t2 < total) load_into(nx2, t2 / nb, t2 - (t2 / nb) * nb);
#pragma unroll
        for (int q = 0; q < kQ; ++q) {
          const int k = (cb * kQ + q) * kLmhStep + 8 * g;  // hidden indices k .. k + 7
          const uint32_t w4[4] = {cur[q].x, cur[q].y, cur[q].z, cur[q].w};
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const float4 *xp = reinterpret_cast<const float4 *>(xs + r * dim + k);
            const float4 x0 = xp[0], x1 = xp[1];
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
              acc[r] = __builtin_fmaf(bf16_lo(w4[h]), xv[2 * h], acc[r]);
              acc[r] = __builtin_fmaf(bf16_hi(w4[h]), xv[2 * h + 1], acc[r]);
            }
          }
        }
      }
      // the group's eight partial sums, in one fixed tree: lane 0 of the
      // group holds ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7))
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v = acc[r];
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 4, 64);
        if (g == 0) s_logit[r][grp + 32 * m] = v;
      }
    }
  } else {
    using St = QStage<kFmt>;
    constexpr int J = St::loads, D = St::depth, NM = kLmhSpan / 32;
    static_assert(NM % D == 0, "the ring divides a pass over the wave's batches");
    const uint8_t *W = static_cast<const uint8_t *>(L.weight);
    // items per id: blocks (Q8_0, Q4_0) or 64-value units (Q6_K); lane g
    // takes g, g + 8, ...: item g of each stage of its row
    const int items = kFmt == SAS_HEAD_Q6_K ? dim / 64 : dim / 32;
    const int rowbytes = kFmt == SAS_HEAD_Q6_K ? 210 * (dim / 256) : (kFmt == SAS_HEAD_Q8_0 ? 34 : 18) * (dim / 32);
    const int per = (items + 7) / 8;  // stages per id
    // Stage (m, c) of the wave: items 8 c .. 8 c + 7 of ids base + 8 wave +
    // 32 m + 0 .. 7 (this lane: its group's id), m outer, c inner: a row's
    // stages follow one another, so the line two stages share comes from
    // L2 the second time.  The loads are plain (cached) loads for that.
    const uint32_t rbi = (uint32_t)((wave * 8 + (lane >> 3)) * St::pitch);  // the lane's row copy in stg
    const QLane<kFmt> ln = q_lane<kFmt>(g, rbi);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    struct Ring {
      u32x4 v[J];
      uint32_t off;  // the stage's first byte in its first chunk; chunks in use << 8
    };
    Ring ring[D];
    // byte offsets into the head are 32-bit (the host checks that it spans
    // less than 4 GiB); the head is 16-byte aligned
    const uint32_t wstride = (uint32_t)L.weight_stride;
    auto stage_load = [&](int c2, int m2, Ring &s) __attribute__((always_inline)) {
      const uint32_t id = (uint32_t)min(base + grp + 32 * m2, vocab - 1);  // loads stay inside the head
      const uint32_t o = id * wstride + (uint32_t)(St::bytes * c2);        // the stage's first byte
      const uint32_t off = o & 15u;
      const uint32_t nch = (off + (uint32_t)min(St::bytes, rowbytes - St::bytes * c2) + 15u) >> 4;
      const uint32_t o16 = o - off;
      // chunks g, g + 8, ... (past the last: the last again, so that every
      // lane loads and no branch splits the loads in flight)
#pragma unroll
      for (int j = 0; j < J; ++j)
        s.v[j] = *reinterpret_cast<const u32x4 *>(W + (o16 + 16u * min((uint32_t)(g + 8 * j), nch - 1u)));
      s.off = off | (nch << 8);
    };
    int cl = 0, ml = 0;  // the next stage to load
    auto advance = [&]() __attribute__((always_inline)) {
      if (++cl == per) {
        cl = 0;
        ++ml;
      }
    };
    // the chunks of the stage in slot rs into the row's copy (the wave's LDS
    // operations run in order, so the reads that follow see them and the
    // previous stage's reads came first), then the slot loads the stage D
    // ahead (past the last stage: the last stage again); returns the
    // stage's offset
    auto stage_take = [&](Ring &rs) __attribute__((always_inline)) {
      const uint32_t off = rs.off & 0xFFu, nch = rs.off >> 8;
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < J; ++j)
        *reinterpret_cast<u32x4 *>(stg + rbi + 4u * min((uint32_t)(g + 8 * j), nch - 1u)) = rs.v[j];
      __asm__ volatile("" ::: "memory");
      const bool more = ml < NM;
      stage_load(more ? cl : per - 1, more ? ml : NM - 1, rs);
      advance();
      return off;
    };
#pragma unroll
    for (int d = 0; d < D; ++d) {
      stage_load(cl, ml, ring[d]);  // D <= NM stages: all exist
      advance();
    }
#pragma unroll
    for (int r = 0; r < R; ++r) lmh_prefetch_range(L.s, r, base + kLmhIds * tid, pre[r]);
    uint32_t *U = reinterpret_cast<uint32_t *>(xs);
    const int rw = items * kQOpWords<kFmt>;
    q81_stage<R, kFmt>(L, U);
#pragma unroll
    for (int r = 0; r < R; ++r) lmh_prefetch_ids(pre[r]);
    __syncthreads();  // the Q8_1 operand is in LDS
    // an id's eight partial sums, in one fixed tree: lane 0 of the group
    // holds ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7))
    auto id_done = [&](float (&a)[R], int m2) __attribute__((always_inline)) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float v = a[r];
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 4, 64);
        if (g == 0) s_logit[r][grp + 32 * m2] = v;
      }
    };
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    int m = 0, c = 0;  // the stage computed
    // the fields of stage t + 1 are read while stage t is computed (after
    // the last stage: the last stage's copy again, unused)
    QRaw<kFmt> cur;
    q_fetch<kFmt>(stg, ln, stage_take(ring[0]), cur);
    for (int t0 = 0; t0 < NM * per; t0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        QRaw<kFmt> nxt;
        q_fetch<kFmt>(stg, ln, stage_take(ring[(d + 1) % D]), nxt);
        const int it = 8 * c + g;
        if (it < items) q_terms<R, kFmt>(cur, ln, QOp{U + it * kQOpWords<kFmt>, rw}, acc);
        cur = nxt;
        if (c == per - 1) {
          id_done(acc, m);
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r] = 0.0f;
          c = 0;
          ++m;
        } else {
          ++c;
        }
      }
    }
  }
  __syncthreads();
  // ---- the epilogue, all rows together: lane t takes ids base + 2 t, + 1 ----
  const int id0 = base + kLmhIds * tid;
  float v[R][2];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    v[r][0] = s_logit[r][kLmhIds * tid];
    v[r][1] = s_logit[r][kLmhIds * tid + 1];
    if (L.out_logits) {
      float *o = L.out_logits + (int64_t)r * vocab;
      if (id0 < vocab) o[id0] = v[r][0];
      if (id0 + 1 < vocab) o[id0 + 1] = v[r][1];
    }
  }
  lmh_select_rows<R>(L, S, part, v, id0, pre);
}

// One block per (row, group of kLmhGroup parts).  The records kept are
// those at or above the group's k-th largest key (round-down keys for the
// members: a member whose value reaches a key's value has a key that
// reaches it), so a merge part holds about k records whatever the spread
// of the parts' bounds.
__global__ __launch_bounds__(kThreads) void lmh_group_kernel(const LmhArgs L) {
  __shared__ uint32_t s_np[kLmhGroup], s_nm[kLmhGroup], s_nw[kWaves], s_nmw, s_slow, s_over, s_n;
  __shared__ uint32_t s_hist[256], s_sel[4];
  const SampleArgs &a = L.s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.x / L.gparts, g = blockIdx.x - row * L.gparts;
  const int q0 = g * kLmhGroup;
  const int nq = min(kLmhGroup, a.parts - q0);
  sas_params p = a.params;
  if (a.row_params) p = load_row_params(a.row_params + row);
  const bool greedy = !(p.temperature > 0.0);
  const int k = greedy ? 1 : min(max(p.top_k, 1), SAS_MAX_TOP_K);
  // ---- every plain and member slot of the group's parts, loaded before
  // the counts are known (all slots lie inside the parts' records) ----
  const int q = tid >> 5, s0 = tid & 31;
  const uint64_t *src = a.rec + ((int64_t)row * a.parts + q0 + min(q, nq - 1)) * kListCap;
  const uint4 *msrc = a.mrec + ((int64_t)row * a.parts + q0 + min(q, nq - 1)) * kMemSlots;
  constexpr int kPer = kLmhSpan / 32;                // plain slots per thread
  constexpr int kMPer = (kMemSlots + 31) / 32;       // member slots per thread
  static_assert(kPer * 32 <= kListCap, "plain slots inside a part's records");
  uint64_t rc[kPer];
  uint4 mr[kMPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) rc[i] = src[s0 + 32 * i];
#pragma unroll
  for (int i = 0; i < kMPer; ++i) {
    const int j = s0 + 32 * i;
    mr[i] = j < kMemSlots ? msrc[j] : make_uint4(0u, 0u, 0u, 0u);
  }
  // ---- the parts' info words: counts, bounds, slow flags ----
  uint32_t bound = 0u, slow = 0u;
#pragma unroll
  for (int q = 0; q < kLmhGroup; ++q) {
    if (q < nq) {
      const uint64_t info = a.pinfo[(int64_t)row * pinfo_stride(a.parts) + q0 + q];
      bound = max(bound, (uint32_t)(info >> 32));
      slow |= (uint32_t)info & kPinfoSlow;
      if (tid == 0) {
        // within the part's slots whatever the word holds
        s_np[q] = min((uint32_t)info & 0x7FFFu, (uint32_t)kLmhSpan);
        s_nm[q] = min(((uint32_t)info >> 16) & 0x7FFFu, (uint32_t)kMemSlots);
      }
    }
  }
  if (tid == 0) {
    s_nmw = 0u;
    s_over = 0u;
    s_n = 0u;
    s_slow = slow ? 1u : 0u;
  }
  __syncthreads();
  // the largest part bound: that part alone holds k values above it, and
  // every part recorded every value at or above its own (smaller) bound
  const uint32_t bkey = bound > 0x007FFFFFu ? bound : 0u;
  const int64_t gq = (int64_t)row * L.gparts + g;
  uint64_t *grec = L.g_rec + gq * kListCap;
  uint4 *gmem = L.g_mrec + gq * kMemSlots;
  // ---- the candidates: slots below the parts' counts, at or above bkey ----
  const uint32_t npq = q < nq ? s_np[q] : 0u;
  const uint32_t nmq = q < nq ? s_nm[q] : 0u;
  uint32_t rk[kPer];  // keys (0: not a candidate)
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t j = (uint32_t)(s0 + 32 * i);
    const uint32_t kk = j < npq ? okey(__uint_as_float((uint32_t)rc[i])) : 0u;
    rk[i] = kk >= bkey ? kk : 0u;
  }
  uint32_t mk[kMPer];
#pragma unroll
  for (int i = 0; i < kMPer; ++i) {
    const uint32_t j = (uint32_t)(s0 + 32 * i);
    const uint32_t kk = j < nmq ? okey(__uint_as_float(mr[i].x)) : 0u;
    mk[i] = kk >= bkey ? kk : 0u;
  }
  // ---- the group's k-th largest key: a radix select, 8 bits a pass from
  // the top, each pass an LDS histogram of the keys that match the bits
  // found so far ----
  {
    uint32_t n = 0u;
#pragma unroll
    for (int i = 0; i < kPer; ++i) n += rk[i] != 0u ? 1u : 0u;
#pragma unroll
    for (int i = 0; i < kMPer; ++i) n += mk[i] != 0u ? 1u : 0u;
    n = wave_sum_u32(n);
    if (lane == 0) atomicAdd(&s_n, n);
  }
  __syncthreads();
  uint32_t t = bkey;
  if (s_n > (uint32_t)k) {
    uint32_t res = 0u, need = (uint32_t)k;
    for (int pass = 0; pass < 4; ++pass) {
      const int sh = 24 - 8 * pass;
      const uint32_t hm = sh == 24 ? 0u : ~0u << (sh + 8);  // the bits found so far
      s_hist[tid] = 0u;
      __syncthreads();
      auto add = [&](uint32_t kk) __attribute__((always_inline)) {
        if (kk != 0u && (kk & hm) == (res & hm)) atomicAdd(&s_hist[(kk >> sh) & 0xFFu], 1u);
      };
#pragma unroll
      for (int i = 0; i < kPer; ++i) add(rk[i]);
#pragma unroll
      for (int i = 0; i < kMPer; ++i) add(mk[i]);
      __syncthreads();
      if (wave == 0) {
        // bins 4 lane .. 4 lane + 3; suf = keys in the bins of this lane and above
        const uint32_t c0 = s_hist[4 * lane], c1 = s_hist[4 * lane + 1], c2 = s_hist[4 * lane + 2],
                       c3 = s_hist[4 * lane + 3];
        const uint32_t s4 = c0 + c1 + c2 + c3;
        uint32_t suf = s4;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const uint32_t y = (uint32_t)__shfl_down((int)suf, d, 64);
          if (lane + d < 64) suf += y;
        }
        const uint32_t above = suf - s4;
        if (above < need && need <= suf) {
          uint32_t acc = above, d;
          if (acc + c3 >= need) {
            d = 3;
          } else if ((acc += c3) + c2 >= need) {
            d = 2;
          } else if ((acc += c2) + c1 >= need) {
            d = 1;
          } else {
            acc += c1;
            d = 0;
          }
          s_sel[0] = 4u * (uint32_t)lane + d;
          s_sel[1] = need - acc;
        }
      }
      __syncthreads();
      res |= s_sel[0] << sh;
      need = s_sel[1];
    }
    t = res;
  }
  // ---- the records at or above t ----
  uint32_t keep = 0u;
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (rk[i] != 0u && rk[i] >= t) keep |= 1u << i;
  const uint32_t mine = (uint32_t)__popc(keep);
  uint32_t pre = 0u, tot = 0u;
#pragma unroll
  for (int bit = 0; bit < 5; ++bit) {
    const uint64_t bb = __ballot((mine >> bit) & 1u);
    pre += lanes_below(bb) << bit;
    tot += (uint32_t)__popcll(bb) << bit;
  }
  if (lane == 0) s_nw[wave] = tot;
  __syncthreads();
  uint32_t off = 0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) off += w < wave ? s_nw[w] : 0u;
  const uint32_t nplain = s_nw[0] + s_nw[1] + s_nw[2] + s_nw[3];
  if (nplain > (uint32_t)kListCap) {
    if (tid == 0) s_over = 1u;
  } else {
    uint32_t j = off + pre;
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if ((keep >> i) & 1u) grec[j++] = rc[i];
  }
#pragma unroll
  for (int i = 0; i < kMPer; ++i) {
    if (mk[i] != 0u && mk[i] >= t) {
      const uint32_t d = atomicAdd(&s_nmw, 1u);
      if (d < (uint32_t)kMemSlots) gmem[d] = mr[i];
      else s_over = 1u;
    }
  }
  __syncthreads();
  uint32_t np_out = nplain, nm_out = s_nmw;
  if (s_over) {
    // more records at the key than a merge part holds (ties): the group's
    // exact top k over (value, id) from the parts' records
    auto for_recs = [&](auto f) {
      for (int i = 0; i < kPer; ++i) {
        const uint32_t j = (uint32_t)(s0 + 32 * i);
        const bool ok = j < npq;
        double v = 0.0;
        uint32_t id = 0u;
        if (ok) {
          const uint64_t r = src[j];
          v = (double)__uint_as_float((uint32_t)r);
          id = (uint32_t)(r >> 32);
        }
        f(key96(v, id), ok, v, id, false, 0u);
      }
      for (int i = 0; i < kMPer; ++i) {
        const uint32_t j = (uint32_t)(s0 + 32 * i);
        const bool ok = j < nmq;
        double v = 0.0;
        uint32_t id = 0u, kb = 0u;
        if (ok) {
          const uint4 m = msrc[j];
          v = __longlong_as_double((long long)(((uint64_t)m.w << 32) | m.z));
          id = m.y;
          kb = m.x;
        }
        f(key96(v, id), ok, v, id, true, kb);
      }
    };
    uint32_t nval = 0u;
    for_recs([&](const Key96 &, bool ok, double, uint32_t, bool, uint32_t) { nval += ok ? 1u : 0u; });
    if (tid == 0) s_sel[3] = 0u;
    __syncthreads();
    atomicAdd(&s_sel[3], nval);
    __syncthreads();
    const uint32_t need = min(s_sel[3], (uint32_t)k);
    __syncthreads();
    if (tid == 0) {
      s_nw[0] = 0u;
      s_nmw = 0u;
      s_slow = 1u;
    }
    __syncthreads();
    if (need > 0u) {
      const Key96 kth = block_select96(
          [&](auto f) {
            for_recs([&](const Key96 &kx, bool ok, double, uint32_t, bool, uint32_t) { f(kx, ok); });
          },
          need, s_hist, s_sel);
      for_recs([&](const Key96 &kx, bool ok, double v, uint32_t id, bool member, uint32_t kb) {
        if (ok && key_ge(kx, kth)) {
          if (member) {
            const uint64_t db = (uint64_t)__double_as_longlong(v);
            gmem[atomicAdd(&s_nmw, 1u)] = make_uint4(kb, id, (uint32_t)db, (uint32_t)(db >> 32));
          } else {
            grec[atomicAdd(&s_nw[0], 1u)] = (uint64_t)__float_as_uint((float)v) | ((uint64_t)id << 32);
          }
        }
      });
    }
    __syncthreads();
    np_out = s_nw[0];
    nm_out = s_nmw;
  }
  if (tid == 0)
    L.g_pinfo[(int64_t)row * pinfo_stride(L.gparts) + g] =
        (uint64_t)(np_out | (nm_out << 16) | (s_slow ? kPinfoSlow : 0u)) | ((uint64_t)max(t, bound) << 32);
}

size_t lmh_scratch_bytes(int rows, int vocab) {
  const int parts = (vocab + kLmhSpan - 1) / kLmhSpan;
  const int gparts = (parts + kLmhGroup - 1) / kLmhGroup;
  return sample_rec_bytes(rows, parts) + sample_rec_bytes(rows, gparts) + 256;
}

void lmh_layout(LmhArgs *a, void *scratch) {
  const int rows = a->s.rows;
  const int parts = (a->s.vocab + kLmhSpan - 1) / kLmhSpan;
  const int gparts = (parts + kLmhGroup - 1) / kLmhGroup;
  uint64_t *p = reinterpret_cast<uint64_t *>(scratch);
  a->s.parts = parts;
  a->s.span = kLmhSpan;
  a->s.rec = p;
  a->s.mrec = reinterpret_cast<uint4 *>(p + (size_t)rows * parts * kListCap);
  a->s.pinfo = reinterpret_cast<uint64_t *>(a->s.mrec + (size_t)rows * parts * kMemSlots);
  uint64_t *g = a->s.pinfo + (size_t)rows * pinfo_stride(parts);
  g = reinterpret_cast<uint64_t *>((reinterpret_cast<uintptr_t>(g) + 255) & ~uintptr_t(255));
  a->gparts = gparts;
  a->g_rec = g;
  a->g_mrec = reinterpret_cast<uint4 *>(g + (size_t)rows * gparts * kListCap);
  a->g_pinfo = reinterpret_cast<uint64_t *>(a->g_mrec + (size_t)rows * gparts * kMemSlots);
}

template <int R, int kFmt>
static hipError_t launch_parts(const LmhArgs &a, hipStream_t stream) {
  // bf16: the f32 hidden rows; GGUF: the packed Q8_1 operand of every row
  const size_t lds = kFmt == SAS_HEAD_BF16 ? (size_t)R * a.dim * sizeof(float)
                                           : (size_t)R * q_items<kFmt>(a.dim) * kQOpWords<kFmt> * sizeof(uint32_t);
  hipLaunchKernelGGL((lmh_parts_kernel<R, kFmt>), dim3((unsigned)a.s.parts), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

template <int kFmt>
static hipError_t launch_parts_rows(const LmhArgs &a, hipStream_t stream) {
  switch (a.s.rows) {
    case 1: return launch_parts<1, kFmt>(a, stream);
    case 2: return launch_parts<2, kFmt>(a, stream);
    case 3: return launch_parts<3, kFmt>(a, stream);
    default: return launch_parts<4, kFmt>(a, stream);
  }
}

hipError_t launch_lm_head_sample(const LmhArgs &a, bool softcap, hipStream_t stream) {
  (void)softcap;  // the epilogue reads each row's softcap itself
  hipError_t e;
  switch (a.format) {
    case SAS_HEAD_Q8_0: e = launch_parts_rows<SAS_HEAD_Q8_0>(a, stream); break;
    case SAS_HEAD_Q4_0: e = launch_parts_rows<SAS_HEAD_Q4_0>(a, stream); break;
    case SAS_HEAD_Q6_K: e = launch_parts_rows<SAS_HEAD_Q6_K>(a, stream); break;
    default: e = launch_parts_rows<SAS_HEAD_BF16>(a, stream); break;
  }
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lmh_group_kernel, dim3((unsigned)(a.s.rows * a.gparts)), dim3(kThreads), 0, stream, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  SampleArgs m = a.s;
  m.rec = a.g_rec;
  m.mrec = a.g_mrec;
  m.pinfo = a.g_pinfo;
  m.parts = a.gparts;
  m.span = kLmhSpan * kLmhGroup;
  return launch_merge(m, stream);
}

}  // namespace sas

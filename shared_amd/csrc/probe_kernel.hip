// probe_kernel.hip - measurement probes (libsas_probe.so), never loaded by
// the sampling library.  They time the HBM stream the sampling kernels
// read: the plain read, and reads that skip the logits a grammar mask
// disallows at 16-, 32-, 64- and 128-byte granularity.  One more checks a
// property of the HIP runtime that a kernel design relied on: whether
// hipMemset (the null stream) is ordered before work on a non-blocking
// stream.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <chrono>

#include "sas_probe.h"

namespace {

constexpr int kThreads = 256;
constexpr int kSpan = 8192;  // ids per block of the masked probe
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));

// A block reads its contiguous share of n4 float4s, eight 16-byte loads
// per thread in flight per round, and folds them into one value that is
// stored only if it equals an impossible bit pattern.
__global__ __launch_bounds__(kThreads) void read_kernel(const float4 *src, int64_t n4, float *sink) {
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(b0 + per, n4);
  float m = 0.0f;
  for (int64_t r = b0 + threadIdx.x; r < b1; r += 8 * kThreads) {
    f32x4u v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = r + (int64_t)u * kThreads;
      v[u] = i < b1 ? __builtin_nontemporal_load(reinterpret_cast<const f32x4u *>(src + i)) : f32x4u{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) m = fmaxf(m, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
  }
  if (__float_as_uint(m) == 0x7FBADBADu) sink[blockIdx.x & 255] = m;
}

// Block b: row b / (vocab / kSpan), ids [q * kSpan, (q + 1) * kSpan).
// Thread t's float4 f covers ids 1024 f + 4 t .. + 3, whose mask word is
// 32 f + t / 8 (nibble t % 8).
template <int kMode>
__global__ __launch_bounds__(kThreads) void masked_kernel(const float *logits, const uint32_t *mask, int vocab,
                                                          float *sink) {
  const int per_row = vocab / kSpan;
  const int row = blockIdx.x / per_row, q = blockIdx.x - row * per_row, t = threadIdx.x;
  const float *lr = logits + (int64_t)row * vocab + (int64_t)q * kSpan;
  const uint32_t *mr = mask + (int64_t)row * (vocab / 32) + q * (kSpan / 32);
  uint32_t w[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) w[f] = mr[32 * f + (t >> 3)];
  f32x4u v[8];
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    bool ld = true;
    if (kMode == 1) ld = ((w[f] >> (4 * (t & 7))) & 0xFu) != 0u;
    if (kMode == 4) ld = ((w[f] >> (8 * ((t & 7) >> 1))) & 0xFFu) != 0u;
    if (kMode == 3) ld = ((w[f] >> (16 * ((t & 7) >> 2))) & 0xFFFFu) != 0u;
    if (kMode == 2) ld = w[f] != 0u;
    if (kMode == 5) ld = w[f] != 0x9E3779B9u || t >= 0;  // waits for the word; always true
    v[f] = ld ? __builtin_nontemporal_load(reinterpret_cast<const f32x4u *>(lr + 1024 * f + 4 * t))
              : f32x4u{0, 0, 0, 0};
  }
  float m = -3.0e38f;
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    const uint32_t nib = (w[f] >> (4 * (t & 7))) & 0xFu;
    if (nib & 1u) m = fmaxf(m, v[f].x);
    if (nib & 2u) m = fmaxf(m, v[f].y);
    if (nib & 4u) m = fmaxf(m, v[f].z);
    if (nib & 8u) m = fmaxf(m, v[f].w);
  }
  if (__float_as_uint(m) == 0x7FBADBADu) sink[blockIdx.x & 255] = m;
}

// Reads 128 words of b (n words): the last 64 and 64 spread over it.
__global__ void peek_kernel(const uint32_t *b, size_t n, uint32_t *out) {
  const int t = threadIdx.x;
  if (t < 64) out[t] = b[n - 1 - t];
  else if (t < 128) out[t] = b[(size_t)(t - 64) * (n / 64)];
}

template <int kMode>
void launch_masked(const float *logits, const uint32_t *mask, int rows, int vocab, float *sink, hipStream_t st) {
  hipLaunchKernelGGL(masked_kernel<kMode>, dim3((unsigned)(rows * (vocab / kSpan))), dim3(kThreads), 0, st, logits,
                     mask, vocab, sink);
}

}  // namespace

extern "C" {

int sasp_read(const void *src, size_t bytes, int32_t blocks, float *sink, void *stream) {
  if (!src || !sink || bytes == 0 || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 || blocks < 1) return -1;
  hipLaunchKernelGGL(read_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const float4 *>(src), (int64_t)(bytes / 16), sink);
  return (int)hipGetLastError();
}

int sasp_masked_read(const float *logits, const uint32_t *mask, int32_t rows, int32_t vocab, int32_t mode,
                     float *sink, void *stream) {
  if (!logits || !mask || !sink || rows < 1 || vocab < kSpan || vocab % kSpan ||
      (int64_t)rows * (vocab / kSpan) > INT32_MAX || reinterpret_cast<uintptr_t>(logits) % 4)
    return -1;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (mode) {
    case 0: launch_masked<0>(logits, mask, rows, vocab, sink, st); break;
    case 1: launch_masked<1>(logits, mask, rows, vocab, sink, st); break;
    case 2: launch_masked<2>(logits, mask, rows, vocab, sink, st); break;
    case 3: launch_masked<3>(logits, mask, rows, vocab, sink, st); break;
    case 4: launch_masked<4>(logits, mask, rows, vocab, sink, st); break;
    case 5: launch_masked<5>(logits, mask, rows, vocab, sink, st); break;
    default: return -1;
  }
  return (int)hipGetLastError();
}

int sasp_memset_order(size_t bytes, int32_t reps, sasp_memset_result *out) {
  if (!out || reps < 1 || bytes < 4096 || bytes % 4) return -1;
  const size_t n = bytes / 4;
  uint32_t *b = nullptr, *peek = nullptr;
  hipStream_t s = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = hipMalloc(&b, bytes);
  if (e == hipSuccess) e = hipMalloc(&peek, 128 * sizeof(uint32_t));
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  out->reps = reps;
  out->stale_runs = 0;
  out->host_us = 0.0;
  // the first hipMemset of a process also initializes the runtime's fill
  // path: one untimed call first
  if (e == hipSuccess) e = hipMemset(b, 0, bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  for (int r = 0; e == hipSuccess && r < reps; ++r) {
    // every word 0xFFFFFFFF, finished; then hipMemset to 0 and, at once, a
    // kernel on the non-blocking stream that reads 128 of the words
    e = hipMemsetAsync(b, 0xFF, bytes, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) break;
    const auto t0 = std::chrono::steady_clock::now();
    e = hipMemset(b, 0, bytes);
    const auto t1 = std::chrono::steady_clock::now();
    if (e != hipSuccess) break;
    hipLaunchKernelGGL(peek_kernel, dim3(1), dim3(128), 0, s, b, n, peek);
    if ((e = hipGetLastError()) != hipSuccess) break;
    if ((e = hipDeviceSynchronize()) != hipSuccess) break;
    uint32_t h[128];
    if ((e = hipMemcpy(h, peek, sizeof h, hipMemcpyDeviceToHost)) != hipSuccess) break;
    int stale = 0;
    for (int i = 0; i < 128; ++i) stale += h[i] != 0u;
    out->stale_runs += stale > 0;
    out->host_us += std::chrono::duration<double, std::micro>(t1 - t0).count() / reps;
  }
  // the same fill timed on a stream
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventRecord(e0, s);
  if (e == hipSuccess) e = hipMemsetAsync(b, 0, bytes, s);
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  out->fill_us = 1000.0 * ms;
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (s) (void)hipStreamDestroy(s);
  if (peek) (void)hipFree(peek);
  if (b) (void)hipFree(b);
  return (int)e;
}

}  // extern "C"

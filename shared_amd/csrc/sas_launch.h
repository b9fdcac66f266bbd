// sas_launch.h - host <-> kernel contract of the sampling kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared_amd_sampler.h"

namespace sas {

// Kernel arguments of the split and merge kernels (validated by sas_sample).
constexpr int kCtlStride = 64;  // words per row: 256 bytes
constexpr int kCtlThr = 32;     // second 128-byte line

struct SampleArgs {
  const float *logits;
  int64_t logits_stride;
  const uint32_t *mask;
  int64_t mask_stride;
  const uint32_t *hist_ids;
  const int32_t *hist_offsets;
  const double *uniforms;
  const sas_params *row_params;
  sas_params params;
  uint32_t *out_ids;
  double *out_probs;
  uint32_t *out_cand_ids;
  int32_t *out_counts;
  uint32_t *out_flags;
  // Candidate records: block (row, split) writes up to kCapBlock records at
  // recs[(row * splits + split) * kCapBlock] and their number at
  // counts[row * splits + split]; the merge kernel, next in stream order,
  // reads them.
  float *rkey;        // [rows][splits][kCapBlock] fp32 key (round-down of the value)
  uint32_t *rid;      // [rows][splits][kCapBlock] token id
  double *rval;       // [rows][splits][kCapBlock] exact value
  uint32_t *counts;   // [rows][splits]
  // Per row kCtlStride words, zero between launches: [0] blocks counted in,
  // [kCtlThr] the largest published threshold key; each on a cache line of
  // its own so that atomics of different rows never queue on one line.
  uint32_t *ctl;      // [rows][kCtlStride]
  int32_t vocab;
  int32_t rows;
  int32_t splits;
  bool aligned;       // logits rows start 16-byte aligned
};

// float4 loads per thread (chunk = f4 * 1024 ids) for a batch shape.
int choose_f4(int rows, int vocab);
// Launches the sampling kernel on `stream`.  softcap:
// some row may have a softcap (row_params, or params.softcap > 0).
hipError_t launch_sample(const SampleArgs &a, int f4, bool softcap, hipStream_t stream);

// Scratch bytes of the record slots and their counts for a batch shape.
size_t sample_rec_bytes(int rows, int splits);
size_t sample_count_bytes(int rows, int splits);

}  // namespace sas

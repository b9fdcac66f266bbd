// sas_launch.h - host <-> kernel contract of the sampling kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared_amd_sampler.h"

namespace sas {

struct Rec;

// Kernel arguments of the split and merge kernels (validated by sas_sample).
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
  // Candidate records, rec_cap slots per row.  Split blocks append at
  // counters[row] (relaxed atomic reservation); the merge kernel, next in
  // stream order, reads them and resets the counter to zero.
  Rec *recs;          // [rows][rec_cap]
  uint32_t *counters; // [rows], zero between launches
  int64_t rec_cap;
  int32_t vocab;
  int32_t rows;
  int32_t splits;
};

// float4 loads per thread (chunk = f4 * 1024 ids) for a batch shape.
int choose_f4(int rows, int vocab);
// Launches the split kernel then the merge kernel on `stream`.
hipError_t launch_sample(const SampleArgs &a, int f4, bool aligned, hipStream_t stream);

// Record slots per row for a split count.
int64_t sample_rec_cap(int splits);
// Scratch bytes of the record arrays for `rows` rows.
size_t sample_rec_bytes(int rows, int splits);

}  // namespace sas

// sas_launch.h - host <-> kernel contract of the sampling kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared_amd_sampler.h"

namespace sas {

struct Rec;
struct BlockHdr;

// Kernel arguments of sample_rows_kernel (validated by sas_sample).
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
  Rec *recs;          // [rows][splits][kCapBlock]
  BlockHdr *hdrs;     // [rows][splits]
  uint32_t *counters; // [rows], zero between launches
  int32_t vocab;
  int32_t rows;
  int32_t splits;
};

// float4 loads per thread (chunk = f4 * 1024 ids) for a batch shape.
int choose_f4(int rows, int vocab);
hipError_t launch_sample(const SampleArgs &a, int f4, bool aligned, hipStream_t stream);

// Scratch bytes sas_sample needs for a shape.
size_t sample_rec_bytes(int rows, int splits);
size_t sample_hdr_bytes(int rows, int splits);

}  // namespace sas

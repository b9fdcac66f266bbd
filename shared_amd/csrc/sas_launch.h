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

// ---------------------------------------------------------------- verify --
// Positions are the rows of target_logits: position p = seq * (L + 1) + j,
// j = 0..L; draft row seq * L + j pairs with target row p for j < L.  The
// vocabulary is cut into chunks of kVChunk ids.
constexpr int kVChunk = 4096;

struct VerifyArgs {
  const float *target;
  const float *draft;
  int64_t stride;
  const uint32_t *mask;      // [positions][mask_stride] or null
  int64_t mask_stride;
  const uint32_t *draft_ids; // [seqs][L]
  const double *uniforms;    // [seqs][L + 1][2]
  double temperature;
  uint32_t *out_tokens;      // [seqs][L + 1]
  int32_t *out_accepted;     // [seqs]
  // Scratch, each written before it is read within one call:
  double *stats;   // [positions][chunks][4]: target max, target sum, draft max, draft sum
  double *part;    // [seqs][chunks][2]: residual mass, target mass of the decided position
  double *seqrec;  // [seqs][8]: decided position, its target max / sum, draft max / sum
  int32_t vocab;
  int32_t seqs;
  int32_t L;
  int32_t chunks;
  bool aligned;    // both logits arrays start 16-byte aligned and stride % 4 == 0
};

size_t verify_scratch_bytes(int seqs, int L, int vocab);
// The three verify launches, in stream order on `stream`.
hipError_t launch_verify(const VerifyArgs &a, hipStream_t stream);

}  // namespace sas

// sas_launch.h - host <-> kernel contract of the sampling kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared_amd_sampler.h"

namespace sas {

// Kernel arguments of the sampling kernel (validated by sas_sample).
//
// A row's vocabulary is cut into chunks of kChunkIds ids; block (row, part)
// streams chunks [part * cpp, (part + 1) * cpp) of the row.
constexpr int kChunkIds = 4096;
constexpr int kMaxParts = 64;   // blocks per row; the merge holds one count per part
constexpr int kListCap = 2048;  // record slots of one part in HBM
constexpr int kCtlStride = 128; // words per row of the control block: 512 bytes
constexpr int kCtlThr = 32;     // second 128-byte line: the largest published threshold key
constexpr int kCtlCnt = 64;     // third and fourth lines: records written by each part (<= kMaxParts)

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
  // Candidate records: part (row, q) writes its records at
  // rec[((row * parts + q) * kListCap + j) * 2 + {0, 1}] = {fp32 key bits |
  // id << 32, exact value bits} and their number at ctl[row][kCtlCnt + q];
  // the row's last part reads them.
  uint64_t *rec;
  // Per row kCtlStride words, [0] and [kCtlThr] zero between launches:
  // [0] parts counted in, [kCtlThr] the largest published threshold key,
  // [kCtlCnt + q] records of part q.  Each row has 512 bytes of its own so
  // that atomics of different rows never queue on one cache line.
  uint32_t *ctl;
  int32_t vocab;
  int32_t rows;
  int32_t parts;   // blocks per row
  int32_t cpp;     // chunks per part
  int32_t chunks;  // chunks per row
};

// Blocks per row and chunks per part for a batch shape, aiming at `target`
// blocks in all.
void choose_parts(int rows, int vocab, int target, int *parts, int *cpp);
// Blocks of the sampling kernel variant that fit on one CU at once.
int sample_blocks_per_cu(bool mask, bool hist, bool softcap);
// Launches the sampling kernel on `stream`.  softcap: some row may have a
// softcap (row_params, or params.softcap > 0).
hipError_t launch_sample(const SampleArgs &a, bool softcap, hipStream_t stream);

// Scratch bytes of the record slots for a batch shape.
size_t sample_rec_bytes(int rows, int parts);
// Copies rows of vocab < 4 logits into dst[rows][4], NaN past vocab.
hipError_t launch_pad_rows(const float *src, int64_t stride, int vocab, int rows, float *dst, hipStream_t stream);

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

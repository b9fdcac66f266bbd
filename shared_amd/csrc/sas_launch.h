// sas_launch.h - host <-> kernel contract of the sampling kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared_amd_sampler.h"

namespace sas {

// Kernel arguments of the sampling kernel (validated by sas_sample).
//
// A row's vocabulary is cut into parts of `span` ids.  Block (row, part)
// runs over ids [part * span, (part + 1) * span) in passes of kSpanPass ids
// (8 float4 per thread) and writes the part's candidates (every allowed
// value at or above the part's bound) as records; the block that finishes
// its row last selects the row's top k from every part's records and draws.
constexpr int kSpanPass = 8192;   // ids of one pass of a block
constexpr int kMaxSpan = 65536;   // ids one part may span (a multiple of kSpanPass above it)
constexpr int kMaxParts = 64;     // blocks per row
constexpr int kListCap = 640;     // records one part may write
constexpr int kMemSlots = kListCap / 2;       // member records (16 bytes) of a part
constexpr uint32_t kPinfoSlow = 0x80000000u;  // pinfo bit: the part took the exact slow selection

// Part counts of a row (pinfo) per 128-byte line: rows never share a line.
__host__ __device__ constexpr int pinfo_stride(int parts) { return (parts + 15) & ~15; }

struct SampleArgs {
  const float *logits;
  int64_t logits_stride;
  const uint32_t *mask;
  int64_t mask_stride;
  const uint32_t *hist_ids;
  const int32_t *hist_offsets;
  int64_t hist_count;   // ids in hist_ids: every row's range is clamped into [0, hist_count]
  const double *uniforms;
  const sas_params *row_params;
  sas_params params;
  uint32_t *out_ids;
  double *out_probs;
  uint32_t *out_cand_ids;
  int32_t *out_counts;
  uint32_t *out_flags;
  // Records: part (row, q) writes its candidates, unordered, to its own
  // slots: plain values rec[(row * parts + q) * kListCap + j] = {fp32 value
  // bits, id} (the value after the mask and softcap), and history members
  // mrec[(row * parts + q) * (kListCap / 2) + j] = {fp32 bits of the
  // penalized value rounded toward -inf, id, the penalized double}; pinfo[row * pinfo_stride(parts) + q] =
  // {plain count | member count << 16, bound key << 32}.
  uint64_t *rec;
  uint4 *mrec;
  uint64_t *pinfo;
  // In-graph feedback (sas_sample_step), all null for sas_sample: per-row
  // {stopped, iteration}, the sampled matrix, the next input tokens, the
  // penalty ring {count, ids[ring_len]} (the history when set), stop ids
  // [rows][4] and PCG seeds.
  uint32_t *st_state;
  uint32_t *st_sampled;
  uint32_t *st_next;
  uint32_t *ring;
  const uint32_t *stop_ids;
  const uint32_t *seeds;
  int32_t st_max_steps;
  int32_t ring_len;
  // Exact-match speculative rounds (sas_spec_exact): `group` consecutive
  // rows (a sequence's verify rows) share one history range, one row of
  // row_params and one seed; row j of a group draws with
  // pcg(spec_seeds[seq] ^ spec_round * 0x9E3779B9 ^ j * 0x85EBCA6B).
  // group 0 or 1: every row is its own.
  const uint32_t *spec_seeds;
  uint32_t spec_round;
  int32_t group;
  // Chained rounds (sas_spec_step): per sequence {frozen, round, pos,
  // accepted}.  A frozen sequence's rows read nothing; the others draw with
  // their own round; the ring above is then indexed by sequence.
  const uint32_t *sp_state;
  // Long histories bucketed by part before the parts kernel: the ids of
  // history row h (a row, or a group's sequence) that fall in part q are
  // hb_ids[hb_offs[h * (parts + 1) + q] .. hb_offs[h * (parts + 1) + q + 1]).
  // Null: every part scans its row's whole history.
  uint32_t *hb_ids;
  int32_t *hb_offs;
  int32_t vocab;
  int32_t rows;
  int32_t parts;   // blocks per row
  int32_t span;    // ids per part: a multiple of 1024, and of kSpanPass above it
};

// Parts per row and ids per part for a batch shape: spans of one pass
// (fewer, larger parts) unless the grid would hold fewer than
// `min_blocks` blocks; at most kMaxParts parts per row.
void choose_parts(int rows, int vocab, int min_blocks, int *parts, int *span);
// The merge launch alone (one block per row) over `a`'s records.
hipError_t launch_merge(const SampleArgs &a, hipStream_t stream);
// Launches the sampling kernel on `stream`.  softcap: some row may have a
// softcap (row_params, or params.softcap > 0).
hipError_t launch_sample(const SampleArgs &a, bool softcap, hipStream_t stream);

// The commit of a chained round (sas_spec_step), all null for
// sas_spec_exact: per sequence {frozen, round, pos, accepted}, the ring,
// the round log [seqs][max_rounds][2 + L] and the next input tokens.
struct SpecCommit {
  uint32_t *state;
  uint32_t *ring;
  int32_t ring_len;
  uint32_t *log;
  int32_t max_rounds;
  uint32_t *next_tokens;
};

// The exact-match cascade of sas_spec_exact, one thread per sequence:
// picks [seqs][L + 1], drafts [seqs][L], stop ids [seqs][4] or null; with
// c.state, the round's commit too.
hipError_t launch_spec_cascade(const uint32_t *picks, const uint32_t *drafts, const uint32_t *stop_ids, int seqs,
                               int L, int32_t *accepted, uint32_t *next, const SpecCommit &c, hipStream_t stream);

// Histories of at least this many ids per row on average are bucketed by
// part first (one more launch): each part then reads its own ids only.
constexpr int64_t kBucketMinIds = 1024;


// Scratch bytes of the records and part counts for a batch shape.
size_t sample_rec_bytes(int rows, int parts);
// Copies rows of vocab < 4 logits into dst[rows][4], NaN past vocab.
hipError_t launch_pad_rows(const float *src, int64_t stride, int vocab, int rows, float *dst, hipStream_t stream);

// --------------------------------------------------------------- lm head --
// sas_lm_head_sample: one block per part of kLmhSpan ids computes the
// part's logits for every row (the hidden states staged in LDS, each lane
// two ids' whole dot products) and writes the part's records as the parts
// kernel does; a group launch folds kLmhGroup consecutive parts into one
// part of the merge kernel's records, which then samples as for sas_sample.
constexpr int kLmhSpan = 512;   // ids per part: two per thread
constexpr int kLmhGroup = 8;    // parts per merge part (4,096 ids)

struct LmhArgs {
  SampleArgs s;          // the sampling descriptor; s.rec/mrec/pinfo: the parts' records, s.parts = parts
  const float *hidden;
  int64_t hidden_stride;
  const void *weight;    // bf16 bits, or GGUF blocks (format)
  int64_t weight_stride; // elements (bf16) or bytes (GGUF) between rows
  int32_t format;        // SAS_HEAD_*
  int32_t dim;
  float *out_logits;     // [rows][vocab] or null
  // the merge's records: kLmhGroup parts each (laid out as SampleArgs' records)
  uint64_t *g_rec;
  uint4 *g_mrec;
  uint64_t *g_pinfo;
  int32_t gparts;
};

// Scratch bytes of both record levels for a batch shape.
size_t lmh_scratch_bytes(int rows, int vocab);
// Fills the record pointers of `a` from `scratch` (lmh_scratch_bytes bytes).
void lmh_layout(LmhArgs *a, void *scratch);
// The three launches (parts with the head, groups, merge), in stream order.
hipError_t launch_lm_head_sample(const LmhArgs &a, bool softcap, hipStream_t stream);

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
  double inv_t;              // 1 / temperature: the weights of the sums use x * inv_t
  uint32_t *out_tokens;      // [seqs][L + 1]
  int32_t *out_accepted;     // [seqs]
  // Scratch, each written before it is read within one call:
  double *stats;   // [positions][chunks][4]: target max, target sum, draft max, draft sum
  double *part;    // [seqs][chunks][2]: residual mass, target mass of the decided position
  double *seqrec;  // [seqs][8]: decided position, its target max / sum, draft max / sum
  float *dtok;     // [positions][2]: target and draft logit of the position's draft token (NaN: masked)
  uint32_t *pk_n;  // [positions][chunks][4 waves]: how the statistics pass packed the wave's allowed values
  float *pk_v;     // [positions][chunks][4 waves][2][256]: those values, target then draft
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

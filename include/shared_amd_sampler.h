/*
 * shared_amd_sampler.h - C ABI of the MI355X logit-processing and sampling
 * library (libshared_amd_sampler.so).
 *
 * One call turns a batch of fp32 logit rows that already sit in HBM into
 * one token id per row: history penalties, the packed grammar bitmask,
 * temperature, top-k, top-p and the categorical draw with a host-supplied
 * uniform (or greedy argmax).  A second call runs speculative verification
 * (accept/resample of draft tokens).  Everything is stream-ordered on the
 * caller's HIP stream; no call blocks unless its name says so.  A call
 * whose scratch is already sized (by sas_reserve, or by an earlier call of
 * the same shape on the handle) issues kernel launches on `stream` and
 * nothing else: no allocation, memset or synchronisation, so it can be
 * recorded into a hipGraph by stream capture and replayed.
 *
 * Reference interfaces replaced (paths relative to the reference repo):
 *   sas_sample        <- sample()            lib/webgpu-llm/tokenizer.js:151-178
 *                        topk WGSL kernel    lib/webgpu-llm/kernels.js:1389-1449
 *                        sampler WGSL kernel lib/webgpu-llm/kernels.js:65-201
 *   sas_verify        <- acceptSpec kernel   lib/webgpu-llm/kernels.js:211-369
 *                        argmaxMerge kernel  lib/webgpu-llm/kernels.js:373-401
 *   sas_mask_from_ids <- TokenMask + isListed()
 *                        lib/webgpu-llm/tool-constraint.ts:39-42,
 *                        lib/webgpu-llm/kernels.js:1401-1412,
 *                        lib/webgpu-llm/token-mask-state.js:8-31
 *   sas_clamp_params  <- #packSamplerParams  lib/webgpu-llm/model.js:401-426,
 *                        lib/webgpu-llm/gemma-model.js:900-919
 *   sas_pcg_uniform   <- pcg() + draw        lib/webgpu-llm/kernels.js:91-95, 181, 320
 *
 * Token ids are uint32 (the reference's Uint32Array).  All floating-point
 * parameters are IEEE doubles, as JS numbers are.
 */
#ifndef SHARED_AMD_SAMPLER_H
#define SHARED_AMD_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SAS_ABI_VERSION 3

/* Largest top_k honoured; the request API accepts 1..128
 * (lib/completions.ts:271).  The reference GPU path caps at 20
 * (lib/webgpu-llm/config.js:48); this library does not. */
#define SAS_MAX_TOP_K 128
/* Largest vocabulary a row may have (ids must fit in 24 bits). */
#define SAS_MAX_VOCAB (1 << 22)
/* Largest history (penalty window) per row. */
#define SAS_MAX_HISTORY 65535
/* Largest number of draft tokens per sequence for sas_verify. */
#define SAS_MAX_DRAFT 16

/* Written to out_ids for a row in which no token is allowed. */
#define SAS_NO_TOKEN 0xFFFFFFFFu

/* Return codes. */
#define SAS_OK 0
#define SAS_ERR_INVALID 1     /* bad argument; see sas_last_error() */
#define SAS_ERR_HIP 2         /* a HIP runtime call failed */
#define SAS_ERR_NOMEM 3       /* device allocation failed */

/* Per-row flags (out_flags). */
#define SAS_FLAG_EMPTY_ROW 1u      /* no allowed, non-NaN token in the row */
#define SAS_FLAG_TOPP_EDGE 2u      /* a running top-p mass was within 1e-6 of top_p */
#define SAS_FLAG_DRAW_EDGE 4u      /* the draw residual was within 1e-12*mass of 0 */
#define SAS_FLAG_SLOW_SELECT 8u    /* exact tie-safe fallback selection ran */

/* sas_rows.row_hints bits: facts about row_params the caller vouches for,
 * so the library can pick a cheaper kernel variant.  0 assumes nothing. */
#define SAS_HINT_NO_SOFTCAP 1u     /* no row of row_params has softcap > 0 */

/* TokenMask kinds (lib/webgpu-llm/tool-constraint.ts:39-42). */
#define SAS_MASK_ALL 0
#define SAS_MASK_ALLOW 1
#define SAS_MASK_DENY 2

/*
 * Sampling parameters of one row.  Semantics follow sample()
 * (lib/webgpu-llm/tokenizer.js:151-178) on the full vocabulary:
 *   v = logit                                   (fp32 value, promoted to double)
 *   v = softcap > 0 ? softcap*tanh(v/softcap) : v   (fp32, kernels.js:1393-1395)
 *   if the id occurs c > 0 times in the row history:
 *       v = v > 0 ? v / repetition_penalty : v * repetition_penalty
 *       v = v - frequency_penalty * c - presence_penalty
 *   candidates = allowed, non-NaN ids ordered by (v desc, id asc)
 *   temperature <= 0 (or NaN): the first candidate (greedy)
 *   otherwise softmax over the first top_k, top-p cut, draw with U.
 * Presence alone with the 512-token window reproduces tokenizer.js:157.
 */
typedef struct sas_params {
  double temperature;
  double top_p;
  double repetition_penalty; /* 1 = off */
  double presence_penalty;   /* 0 = off */
  double frequency_penalty;  /* 0 = off */
  float softcap;             /* 0 = off; Gemma uses 30 (gemma-config.js:47) */
  int32_t top_k;             /* clamped to [1, SAS_MAX_TOP_K] */
} sas_params;

/*
 * One batch of rows for sas_sample.  Pointers marked "device" are HBM
 * addresses; the call only reads inputs and writes the outputs.
 */
typedef struct sas_rows {
  const float *logits;         /* device [rows][logits_stride] fp32 */
  int64_t logits_stride;       /* elements between rows, >= vocab */
  int32_t vocab;               /* 1..SAS_MAX_VOCAB */
  int32_t rows;                /* >= 0 */
  const uint32_t *mask;        /* device [rows][mask_stride] or NULL (all allowed);
                                  bit (id & 31) of word id >> 5 set = id allowed */
  int64_t mask_stride;         /* words between rows, >= ceil(vocab / 32); 0 = every
                                  row uses the same words (one grammar state) */
  const uint32_t *hist_ids;    /* device, all rows' histories back to back, or NULL */
  const int32_t *hist_offsets; /* device [rows + 1]: row r owns
                                  hist_ids[hist_offsets[r] .. hist_offsets[r+1]);
                                  non-decreasing, each row at most SAS_MAX_HISTORY ids
                                  (the kernels clamp: a row's range is cut to
                                  [0, hist_count] and to SAS_MAX_HISTORY ids) */
  const double *uniforms;      /* device [rows], U in [0, 1); may be NULL when every
                                  row is greedy */
  sas_params params;           /* used for every row unless row_params is set */
  const sas_params *row_params;/* device [rows] or NULL */
  uint32_t *out_ids;           /* device [rows] (required) */
  double *out_probs;           /* device [rows][SAS_MAX_TOP_K] or NULL: softmax
                                  probability of each top-k candidate */
  uint32_t *out_cand_ids;      /* device [rows][SAS_MAX_TOP_K] or NULL: the ranked
                                  top-k candidate ids */
  int32_t *out_counts;         /* device [rows][2] or NULL: {k, cut} (0,0 greedy) */
  uint32_t *out_flags;         /* device [rows] or NULL: SAS_FLAG_* bits */
  int64_t hist_count;          /* ids in hist_ids, >= 1 when hist_ids is set: no row
                                  reads past it */
  uint32_t row_hints;          /* SAS_HINT_* bits about row_params (0 = none) */
} sas_rows;

/*
 * Speculative verification (rejection sampling, Leviathan et al. 2023 /
 * Chen et al. 2023).  Sequence s has draft_len draft tokens d_j sampled
 * from q_j = softmax(draft logits row j / T) over allowed ids, and
 * draft_len + 1 target rows p_j = softmax(target logits row j / T).
 * Position j accepts d_j iff U1 * q_j(d_j) <= p_j(d_j); the first
 * rejected position draws from normalize(max(0, p_j - q_j)) with U2; if
 * all drafts are accepted, the bonus token is drawn from p_{draft_len}
 * with its U2.  Draws are inverse-CDF over ids in ascending order.
 */
typedef struct sas_verify_rows {
  const float *target_logits;  /* device [seqs * (draft_len + 1)][logits_stride] */
  const float *draft_logits;   /* device [seqs * draft_len][logits_stride] */
  int64_t logits_stride;
  int32_t vocab;
  int32_t seqs;
  int32_t draft_len;           /* 1..SAS_MAX_DRAFT */
  const uint32_t *draft_ids;   /* device [seqs][draft_len] */
  const uint32_t *mask;        /* device [seqs * (draft_len + 1)][mask_stride] or NULL;
                                  row j of a sequence applies to target row j and
                                  draft row j */
  int64_t mask_stride;         /* as in sas_rows (0 = one mask for every position) */
  const double *uniforms;      /* device [seqs][draft_len + 1][2] = {U1, U2} */
  double temperature;          /* > 0 */
  uint32_t *out_tokens;        /* device [seqs][draft_len + 1]: accepted drafts then
                                  the correction or bonus token; unused tail slots
                                  are SAS_NO_TOKEN */
  int32_t *out_accepted;       /* device [seqs]: number of accepted drafts */
} sas_verify_rows;

/*
 * The reference's speculative acceptance (kernels.js:211-369, driven by
 * model.js:867-1008): drafts are the argmax of the draft head
 * (argmaxMerge, kernels.js:373-401), every verify row is sampled on its own
 * and a draft is accepted iff the verify row before it sampled exactly it
 * (the cascade, kernels.js:328-339).  Sequence s has draft_len drafts and
 * draft_len + 1 verify rows; verify row j is sampled as sas_sample samples a
 * row (the sequence's params, its history, mask row s * (draft_len + 1) + j)
 * with the uniform (pcg(seed ^ round * 0x9E3779B9 ^ j * 0x85EBCA6B) &
 * 0xFFFFFF) / 2^24 (kernels.js:320).  Then a = 1 and next = pick[0]; while
 * a <= draft_len, pick[a - 1] equals draft a - 1 and is not a stop id,
 * a grows by one and next = pick[a - 1].  The sequence commits pick[0 .. a).
 */
typedef struct sas_spec_rows {
  const float *target_logits;   /* device [seqs * (draft_len + 1)][logits_stride]: verify rows */
  const float *draft_logits;    /* device [seqs * draft_len][logits_stride] (the draft head's
                                   logits), or NULL when draft_ids are given */
  int64_t logits_stride;
  int32_t vocab;
  int32_t seqs;
  int32_t draft_len;            /* 1..SAS_MAX_DRAFT (the reference uses 2) */
  uint32_t *draft_ids;          /* device [seqs][draft_len]: written with the argmax of each
                                   draft row (lowest id among equals) when draft_logits is
                                   set, else read */
  const uint32_t *mask;         /* device [seqs * (draft_len + 1)][mask_stride] or NULL: the
                                   verify rows' masks, laid out as in sas_rows */
  int64_t mask_stride;
  const uint32_t *hist_ids;     /* each sequence's history, as in sas_rows with one range */
  const int32_t *hist_offsets;  /* per sequence: device [seqs + 1] */
  int64_t hist_count;
  sas_params params;            /* every sequence, unless seq_params */
  const sas_params *seq_params; /* device [seqs] or NULL */
  const uint32_t *seeds;        /* device [seqs] */
  uint32_t round;               /* the round number the draws use */
  uint32_t row_hints;           /* SAS_HINT_* (with seq_params) */
  const uint32_t *stop_ids;     /* device [seqs][4], SAS_STOP_PAD padded, or NULL */
  uint32_t *out_picks;          /* device [seqs][draft_len + 1]: each verify row's token */
  int32_t *out_accepted;        /* device [seqs]: a, the tokens committed (1..draft_len + 1) */
  uint32_t *out_next;           /* device [seqs]: pick[a - 1], the next input token, or NULL */
} sas_spec_rows;

typedef struct sas_sampler sas_sampler;

/* Library version string ("shared_amd_sampler <abi> gfx950"). */
const char *sas_version(void);

/* Create a sampler bound to HIP device `device`.  Owns device scratch. */
int sas_create(int device, sas_sampler **out);
void sas_destroy(sas_sampler *s);

/* Message of the last failed call on `s` (or of the last failed
 * sas_create / handle-free call on this thread when s is NULL). */
const char *sas_last_error(const sas_sampler *s);

/*
 * Scratch.  A handle owns device scratch and grows it when a call needs
 * more; a call whose scratch is already big enough allocates nothing (see
 * the top of this file).  A growth never frees the buffer it replaces:
 * launches already queued on any stream, and HIP graphs that recorded
 * them, keep valid addresses until sas_destroy, which synchronises the
 * device and frees every buffer.  (A graph replayed after sas_destroy of
 * its handle reads freed memory.)  A call that would grow scratch while
 * its stream is being captured fails with SAS_ERR_INVALID instead.
 */

/* Pre-size scratch for sas_sample / sas_sample_step calls of at most
 * `rows` rows at `vocab` with histories shorter than 1,024 ids per row:
 * sas_reserve_for with only rows and vocab set. */
int sas_reserve(sas_sampler *s, int32_t rows, int32_t vocab);

/* The largest calls a handle must run without allocating.  Zero fields
 * reserve nothing for that entry point. */
typedef struct sas_reserve_desc {
  int32_t rows;              /* sampling rows of one call: sas_sample, sas_sample_step,
                                sas_spec_exact's seqs * (draft_len + 1) verify rows */
  int32_t vocab;             /* 1..SAS_MAX_VOCAB, the vocabulary of every call below */
  int64_t hist_ids;          /* the most history ids of one call (hist_count, or
                                rows * ring_len for sas_sample_step): long histories
                                (>= 1,024 ids per row) are bucketed in scratch */
  int32_t lm_head_rows;      /* 0, or the rows of sas_lm_head_sample (<= SAS_LMH_MAX_ROWS;
                                vocab <= SAS_LMH_MAX_VOCAB) */
  int32_t verify_seqs;       /* 0, or the sequences of sas_verify ... */
  int32_t verify_draft_len;  /* ... with this many drafts (1..SAS_MAX_DRAFT) */
} sas_reserve_desc;

/* Pre-size every scratch buffer for calls of at most the shapes of `d`,
 * so that those calls allocate nothing (and can be captured into a HIP
 * graph with no eager call first).  No reference counterpart: the
 * reference allocates its buffers once per model (gemma-model.js:123-178). */
int sas_reserve_for(sas_sampler *s, const sas_reserve_desc *d);

/* Sample one token per row, stream-ordered on `stream` (a hipStream_t; NULL
 * is HIP's null stream, as everywhere in HIP).  A handle must not run two
 * calls concurrently. */
int sas_sample(sas_sampler *s, const sas_rows *rows, void *stream);

/*
 * In-graph token feedback for consecutive decode steps with no host round
 * trip (the reference's sampler tail, lib/webgpu-llm/kernels.js:184-199, and
 * the penalty window it appends to, lib/webgpu-llm/model.js:386-399,
 * 649-742).  Each sas_sample_step call is one step of every row:
 *   - a row whose state says it already sampled a stop id emits its first
 *     stop id (SAS_STOP_PAD when it has none) and reads no logits;
 *   - any other row samples as sas_sample does, its history being its ring
 *     (the last ring_len tokens it generated), its uniform uniforms[row] or,
 *     with seeds, the reference's (pcg(seed ^ it * 0x9E3779B9) & 0xFFFFFF) / 2^24;
 *   - the token goes to out_ids[row], sampled[row][it] and next_tokens[row]
 *     (the next step's input token), and the iteration advances;
 *   - a stop id (or SAS_NO_TOKEN, an empty row) freezes the row; any other
 *     token of a live row is appended to its ring.
 * All arrays are device memory owned by the caller and persist across calls;
 * a batch of steps starts from zeroed state and a ring seeded by the caller
 * (count = ids in it, which may exceed ring_len: the last ring_len are kept).
 */
#define SAS_STOP_PAD 0xFFFFFFFFu   /* stop_ids padding: never matches a token */

typedef struct sas_step {
  uint32_t *state;            /* device [rows][2] = {stopped, iteration} */
  uint32_t *sampled;          /* device [rows][max_steps] or NULL */
  int32_t max_steps;          /* columns of sampled (steps past it are not recorded) */
  uint32_t *next_tokens;      /* device [rows] or NULL */
  uint32_t *ring;             /* device [rows][1 + ring_len] = {count, ids[ring_len]}:
                                 id i of the window at ids[i % ring_len] */
  int32_t ring_len;           /* 1..SAS_MAX_HISTORY (the reference uses 512) */
  const uint32_t *stop_ids;   /* device [rows][4], SAS_STOP_PAD padded, or NULL (no stops) */
  const uint32_t *seeds;      /* device [rows] or NULL (then rows->uniforms) */
} sas_step;

/* One decode step with in-graph feedback.  rows->hist_ids must be NULL
 * (the ring is the history); everything else as sas_sample. */
int sas_sample_step(sas_sampler *s, const sas_rows *rows, const sas_step *step, void *stream);

/* Bytes of the static scratch of sas_sample_noalloc on each device. */
#define SAS_NOALLOC_SCRATCH_BYTES (48u << 20)

/*
 * sas_sample without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory during the call (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The same kernels and results as sas_sample, on HIP device `device`, with
 * their scratch in a static device array of SAS_NOALLOC_SCRATCH_BYTES per
 * device, held until the process ends (its address is resolved by sas_create
 * on that device, or by the first call).  A batch whose records need more
 * (rows x parts x 10 KiB; 128 rows of 262,144 ids take 40 MiB) fails with
 * SAS_ERR_INVALID.  Every call on one device shares that device's array:
 * calls that overlap on one GPU (other streams, other threads) race.
 * Errors: sas_last_error(NULL) on the calling thread.
 */
int sas_sample_noalloc(int device, const sas_rows *rows, void *stream);

/* Speculative accept/resample, stream-ordered like sas_sample. */
int sas_verify(sas_sampler *s, const sas_verify_rows *v, void *stream);

/* The reference's exact-match speculative round (kernels.js:211-401),
 * stream-ordered like sas_sample. */
int sas_spec_exact(sas_sampler *s, const sas_spec_rows *r, void *stream);

/*
 * acceptSpec's on-device commit (kernels.js:340-367), so that rounds chain
 * with no host work between them (specChain runs R rounds per submit,
 * model.js:867-1008).  Each sas_spec_step call is one round of every
 * sequence, as sas_spec_exact runs it, except:
 *   - a sequence's history is its ring as of the round's start, and its
 *     round number is its state's (rows->round and rows->hist_* are unused);
 *   - a frozen sequence (one that committed a stop id) reads no logits: its
 *     picks are SAS_STOP_PAD, its accepted count 0, its next token its first
 *     stop id, and its log entry {0, first stop id, 0, ...} (kernels.js:358-362);
 *   - any other sequence, after the cascade (a tokens accepted, next =
 *     pick[a - 1]): its log entry {a, next, draft_0 .. draft_{L-1}}, pos += a,
 *     accepted = a, pick[0 .. a) minus stop ids appended to its ring, and it
 *     freezes when next is a stop id (kernels.js:341-357);
 *   - every sequence's round advances by one and next_tokens receives next
 *     (tokens[0] = next, kernels.js:364-365).
 * The state persists across calls in caller-owned device memory; a chain
 * starts from state {0, first round, pos, 0} and a ring seeded by the caller.
 * previous pos = pos - accepted and "partial accept" = accepted < L + 1 are
 * the reference's posBuf[2] and posBuf[3].
 */
typedef struct sas_spec_state {
  uint32_t *state;          /* device [seqs][4] = {frozen, round, pos, accepted}
                               (the reference's ctl[0], posBuf[4], posBuf[0], posBuf[1]) */
  uint32_t *ring;           /* device [seqs][1 + ring_len] = {count, ids} or NULL (no history) */
  int32_t ring_len;         /* 1..SAS_MAX_HISTORY with ring (the reference uses 512) */
  uint32_t *log;            /* device [seqs][max_rounds][2 + draft_len] or NULL: per round
                               {a, next, drafts}; rounds >= max_rounds are not logged */
  int32_t max_rounds;
  uint32_t *next_tokens;    /* device [seqs] or NULL */
} sas_spec_state;

/* One chained round: `r` as for sas_spec_exact (hist_ids must be NULL,
 * round is ignored), `st` the sequences' persistent state. */
int sas_spec_step(sas_sampler *s, const sas_spec_rows *r, const sas_spec_state *st, void *stream);

/* ---- the LM head with the sampling step fused into its epilogue ----
 *
 * Replaces the decode head's final projection and the topk pass that reads
 * its logits: lib/webgpu-llm/model.js:466-471 (Qwen: rms -> lm per
 * embedding shard -> topk) and gemma-model.js:786-799 (Gemma: finalNorm ->
 * lmRuns -> topk with the softcap fused), over a BF16 head as
 * ggml/kernels.js:31-33 reads it (f32 weight = bf16 bits << 16) and
 * gemvGGML (ggml/kernels.js:84-110) computes it (f32 products of the
 * widened weight and the f32 activation, summed in f32).
 *
 * logit[row][id] = sum over k of weight[id][k] * hidden[row][k] in f32, in
 * this order exactly (the reference's WGSL order is its driver's): eight
 * partial sums, partial g a fused multiply-add chain from 0 over
 * k = 64 c + 8 g + j (c ascending, then j = 0 .. 7), added as
 * ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)).  The logits
 * are consumed on chip: no [rows][vocab] array is written unless
 * out_logits asks for it.  Then the sas_sample semantics over them
 * (softcap, mask, penalties, top-k / top-p, draw). */
#define SAS_LMH_MAX_ROWS 4        /* rows per call: decode (1) and verify rounds (3) */
#define SAS_LMH_MAX_LDS_FLOATS 12288  /* rows * dim: the hidden states staged on chip */
#define SAS_LMH_MAX_VOCAB 262144      /* vocabularies of the fused head */

/*
 * Head formats.  SAS_HEAD_BF16: the order above.  The GGUF formats are
 * ggml's block layouts (the reference loads them, gguf/parser.js:29-36, and
 * its GEMVs read them, ggml/kernels.js:64-80, 291-315, ggml/q8.js:202-240):
 *   SAS_HEAD_Q8_0: 34-byte blocks of 32 values: f16 d, int8 q[32]; w = d q
 *   SAS_HEAD_Q4_0: 18-byte blocks of 32: f16 d, 16 bytes; value i < 16 is the
 *                  low nibble of byte i, i >= 16 the high nibble of byte i - 16;
 *                  w = d (nibble - 8)
 *   SAS_HEAD_Q6_K: 210-byte super-blocks of 256: ql[128], qh[64], int8
 *                  scales[16], f16 d; w = d scale (q - 32), q six bits
 *                  (the Qwen head's format, gguf/sources.js:122)
 * For them the hidden states are quantized on chip as the reference's
 * Q8_1 operand (ggml/q8.js:27-42): per 32 values, amax = max |x|,
 * d8 = amax / 127, q8 = round-half-even(x / d8) (x times the f32 reciprocal),
 * and the f16 fields d8 and d8 * sum(q8).  Each block's integer dot product
 * is exact; its term is, in f32 left to right (the reference's Q8_1 GEMV
 * terms, q8.js:202-240):
 *   Q8_0: (dot * d) * d8      Q4_0: (dot * d) * d8 - (8 d) * s8 (nibble dot)
 *   Q6_K: ((d * scale) * d8) * dot, per 16 values (dot over q - 32)
 * and the logit is eight partial sums: partial g adds the terms of blocks
 * g, g + 8, ... (Q6_K: of 64-value units g, g + 8, ..., unit u being
 * super-block u / 4, half (u / 2) % 2 and 16-value half u % 2, its four
 * terms in ascending order), then ((p0 + p1) + (p2 + p3)) + ((p4 + p5) +
 * (p6 + p7)).
 */
#define SAS_HEAD_BF16 0
#define SAS_HEAD_Q8_0 1
#define SAS_HEAD_Q4_0 2
#define SAS_HEAD_Q6_K 3

typedef struct sas_lm_head {
  const float *hidden;        /* device [rows][hidden_stride] fp32: final-normed hidden states */
  int64_t hidden_stride;      /* >= dim */
  const void *weight;         /* device [vocab] rows, 16-byte aligned: bf16 bits, or GGUF blocks */
  int64_t weight_stride;      /* between rows: elements (bf16: >= dim, a multiple of 8) or bytes
                                 (GGUF: >= the row's bytes; Q8_0 / Q4_0 a multiple of 4,
                                 Q6_K of 2) */
  int32_t dim;                /* a multiple of 256; rows * dim <= SAS_LMH_MAX_LDS_FLOATS */
  float *out_logits;          /* device [rows][vocab] or NULL: also write the logits */
  int32_t format;             /* SAS_HEAD_* (0: bf16) */
} sas_lm_head;

/* Samples rows->rows rows (<= SAS_LMH_MAX_ROWS, vocab <= SAS_LMH_MAX_VOCAB)
 * from the logits of `head`:
 * rows->logits must be NULL and rows->logits_stride is ignored; every
 * other field of `rows` means what it means for sas_sample.
 * Stream-ordered; no host synchronisation. */
int sas_lm_head_sample(sas_sampler *s, const sas_lm_head *head, const sas_rows *rows, void *stream);

/* The fused head as one step of the in-graph decode loop: the LM head,
 * then the step of sas_sample_step (ring history, seeded draws, stop
 * freeze, feedback) over its logits; the reference's per-iteration
 * lm -> topk -> sampler with tokens[0] fed back (model.js:711-717,
 * kernels.js:189-199).  rows->hist_ids must be NULL. */
int sas_lm_head_sample_step(sas_sampler *s, const sas_lm_head *head, const sas_rows *rows, const sas_step *step,
                            void *stream);

/* Host: clamp parameters with the reference packer's rules
 * (model.js:418-423): non-finite or negative temperature -> 0 (greedy),
 * top_p -> [0, 1] (non-finite -> 1), presence -> [0, 10] (non-finite -> 0),
 * top_k -> [1, SAS_MAX_TOP_K] (non-finite handled by the caller), softcap
 * non-finite or negative -> 0, repetition non-finite or <= 0 -> 1,
 * frequency non-finite -> 0. */
int sas_clamp_params(const sas_params *in, sas_params *out);

/* Host: build the packed bitmask for a TokenMask.  kind = SAS_MASK_*;
 * ids need not be sorted; ids >= vocab are ignored.  nwords >= ceil(vocab/32);
 * bits at ids >= vocab are left clear.  Returns the number of allowed ids
 * (>= 0) or -SAS_ERR_INVALID. */
int64_t sas_mask_from_ids(int32_t kind, const uint32_t *ids, size_t count,
                          int32_t vocab, uint32_t *words, int64_t nwords);

/* Host: the reference GPU sampler's uniform,
 * (pcg(seed ^ it*0x9E3779B9 ^ row*0x85EBCA6B) & 0xFFFFFF) / 2^24. */
double sas_pcg_uniform(uint32_t seed, uint32_t it, uint32_t row);

/* Device memory plumbing for hosts that have no HIP binding (N-API, ctypes). */
int sas_alloc(sas_sampler *s, size_t bytes, void **out);
int sas_free(sas_sampler *s, void *p);
/* kind: 0 host->device, 1 device->host, 2 device->device.  Asynchronous on
 * `stream` for device->device; host copies complete before returning. */
int sas_memcpy(sas_sampler *s, void *dst, const void *src, size_t bytes,
               int kind, void *stream);
int sas_synchronize(sas_sampler *s, void *stream);
/* The handle's own non-blocking hipStream_t, for hosts that have no HIP
 * binding of their own (the N-API addon passes it to every call). */
void *sas_stream(sas_sampler *s);

#ifdef __cplusplus
}
#endif

#endif /* SHARED_AMD_SAMPLER_H */

/*
 * sampler_oracle.h - CPU oracle for the logit-processing / sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker.
 * The product library (shared_amd/) never links or calls it.
 *
 * The oracle restates, in plain C with IEEE doubles and no FMA contraction,
 * the reference's sampling semantics (lib/webgpu-llm/tokenizer.js:151-178)
 * applied to the full vocabulary, plus the extensions the reference lacks
 * (repetition / frequency penalties, packed bitmask, rejection-sampling
 * verify).  Parity status of each function is listed in sampler_oracle.c.
 */
#ifndef SAMPLER_ORACLE_H
#define SAMPLER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORC_MAX_TOP_K 128
#define ORC_NO_TOKEN 0xFFFFFFFFu

#define ORC_FLAG_EMPTY_ROW 1u
#define ORC_FLAG_TOPP_EDGE 2u
#define ORC_FLAG_DRAW_EDGE 4u

/* Same layout as sas_params (include/shared_amd_sampler.h). */
typedef struct orc_params {
  double temperature;
  double top_p;
  double repetition_penalty;
  double presence_penalty;
  double frequency_penalty;
  float softcap;
  int32_t top_k;
} orc_params;

typedef struct orc_result {
  uint32_t id;
  int32_t k;       /* candidates in the softmax (0 when greedy) */
  int32_t cut;     /* top-p cut (0 when greedy) */
  uint32_t flags;
  uint32_t cand_ids[ORC_MAX_TOP_K];
  double probs[ORC_MAX_TOP_K];
} orc_result;

double orc_exp(double x);
uint32_t orc_pcg(uint32_t x);
double orc_pcg_uniform(uint32_t seed, uint32_t it, uint32_t row);
float orc_tanhf(float x);
float orc_softcap(float x, float cap);
double orc_penalize(double v, uint32_t count, const orc_params *p);

/* One row.  mask: ceil(V/32) words or NULL; hist: H ids or NULL.
 * select_mode 0 = bounded heap, 1 = full qsort (slow, obviously ordered). */
void orc_sample_row(const float *logits, int32_t vocab, const uint32_t *mask,
                    const uint32_t *hist, int32_t hist_len,
                    const orc_params *p, double uniform, int select_mode,
                    orc_result *out);

/* Batch form mirroring sas_sample: strides in elements / words, CSR history,
 * params per row (row_params) or shared (params).  Outputs may be NULL except
 * out_ids.  Rows are processed on `threads` pthreads (<= 0: one). */
void orc_sample_rows(const float *logits, int64_t logits_stride, int32_t vocab,
                     int32_t rows, const uint32_t *mask, int64_t mask_stride,
                     const uint32_t *hist_ids, const int32_t *hist_offsets,
                     const double *uniforms, const orc_params *params,
                     const orc_params *row_params, uint32_t *out_ids,
                     double *out_probs, uint32_t *out_cand_ids,
                     int32_t *out_counts, uint32_t *out_flags, int threads);

/* TokenMask -> packed words (kind 0 all, 1 allow, 2 deny).  Returns the
 * number of allowed ids. */
int64_t orc_mask_from_ids(int32_t kind, const uint32_t *ids, size_t count,
                          int32_t vocab, uint32_t *words, int64_t nwords);

/* Rejection-sampling verify for `seqs` sequences (layout as sas_verify_rows). */
void orc_verify(const float *target, const float *draft, int64_t stride,
                int32_t vocab, int32_t seqs, int32_t draft_len,
                const uint32_t *draft_ids, const uint32_t *mask,
                int64_t mask_stride, const double *uniforms,
                double temperature, uint32_t *out_tokens,
                int32_t *out_accepted, double *out_ratio);

/* The reference's exact-match speculative round for `seqs` sequences
 * (layout as sas_spec_rows): argmax drafts when `draft` is set (written to
 * draft_ids), verify row j of sequence s sampled by orc_sample_row with the
 * sequence's params and history and uniform orc_pcg_uniform(seed, round,
 * j), then the cascade.  stop_ids: [seqs][4] or NULL; out_next may be NULL. */
void orc_spec_exact(const float *target, const float *draft, int64_t stride,
                    int32_t vocab, int32_t seqs, int32_t draft_len,
                    uint32_t *draft_ids, const uint32_t *mask,
                    int64_t mask_stride, const uint32_t *hist_ids,
                    const int32_t *hist_offsets, const orc_params *params,
                    const orc_params *seq_params, const uint32_t *seeds,
                    uint32_t round, const uint32_t *stop_ids,
                    uint32_t *out_picks, int32_t *out_accepted,
                    uint32_t *out_next);

/* acceptSpec's commit (kernels.js:340-367) after one round of
 * orc_spec_exact, for chained rounds (layout as sas_spec_state):
 * state [seqs][4] = {frozen, round, pos, accepted}, ring [seqs][1 +
 * ring_len] or NULL, log [seqs][max_rounds][2 + draft_len] or NULL,
 * next_tokens [seqs] or NULL.  A frozen sequence logs {0, first stop id,
 * 0, ...} and its next token is its first stop id; any other logs {a, next,
 * drafts}, advances pos by a, appends picks[0 .. a) that are not stop ids
 * to its ring and freezes when next is a stop id.  accepted_out (may be
 * NULL) receives a (0 when frozen).  Every round advances. */
void orc_spec_commit(int32_t seqs, int32_t draft_len, const uint32_t *picks, const uint32_t *draft_ids,
                     const int32_t *accepted, const uint32_t *stop_ids, uint32_t *state, uint32_t *ring,
                     int32_t ring_len, uint32_t *log, int32_t max_rounds, uint32_t *next_tokens,
                     int32_t *accepted_out);

/* The LM head's logits (sas_lm_head_sample): the bf16 weight widened to
 * f32 (bits << 16) times the f32 hidden value, summed as eight partials,
 * partial g a fused multiply-add chain from 0 over k = 64 c + 8 g + j
 * (c ascending, then j = 0 .. 7, k < dim), then
 * ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)).  weight:
 * [vocab][weight_stride] bf16 bits; hidden: [rows][hidden_stride]. */
void orc_lm_head_logits(const float *hidden, int64_t hidden_stride, const uint16_t *weight,
                        int64_t weight_stride, int32_t dim, int32_t rows, int32_t vocab,
                        float *logits);

/* ---- the quantized LM head (sas_lm_head_sample with a GGUF head) ----
 *
 * Weight formats (ggml's published block layouts, as gguf/parser.js:29-36
 * sizes them): ORC_HEAD_Q8_0 (34-byte blocks of 32: f16 d, 32 int8),
 * ORC_HEAD_Q4_0 (18-byte blocks of 32: f16 d, 16 bytes, element i < 16 the
 * low nibble of byte i, i >= 16 the high nibble of byte i - 16), ORC_HEAD_Q6_K
 * (210-byte super-blocks of 256: ql[128], qh[64], int8 scales[16], f16 d). */
#define ORC_HEAD_BF16 0
#define ORC_HEAD_Q8_0 1
#define ORC_HEAD_Q4_0 2
#define ORC_HEAD_Q6_K 3

/* f32 -> nearest f16 (ties to even) -> f32; and f16 bits -> f32. */
float orc_f16_round(float x);
float orc_f16_to_f32(uint16_t h);

/* The Q8_1 quantization of one activation row (q8.js:27-42): per block of
 * 32 values, amax = max |x|, d = amax / 127, inv = d > 0 ? 1 / d : 0,
 * q = round-half-even(x * inv) (0 when not a number), sum = sum of q;
 * d8 = f16(d), s8 = f16(d * sum), each read back as f32.  dim % 32 == 0. */
void orc_q81_quantize(const float *x, int32_t dim, int8_t *q, float *d8, float *s8);

/* The quantized head's logits in the order sas_lm_head_sample sums them:
 * the hidden row quantized by orc_q81_quantize, exact integer dot products
 * per weight block, then per block (f32, left to right, no fused ops):
 *   Q8_0: (dot * d) * d8
 *   Q4_0: (dot * d) * d8 - (8 * d) * s8                 (dot over the nibbles)
 *   Q6_K: ((d * scale) * d8) * dot, per 16 values        (dot over q6 - 32)
 * (the reference's Q8_1 GEMV terms, q8.js:202-240).  Eight partial sums:
 * partial g adds, in ascending order, the terms of blocks b = g, g + 8, ...
 * (Q8_0, Q4_0) or of 64-value units u = g, g + 8, ... (Q6_K; unit u is
 * super-block u / 4, half (u / 2) % 2, 16-value half u % 2, its four
 * 16-value pieces in ascending order); then
 * ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)).
 * weight: [vocab] rows of row_bytes bytes; dim % 256 == 0. */
void orc_lm_head_q_logits(int32_t format, const float *hidden, int64_t hidden_stride, const uint8_t *weight,
                          int64_t row_bytes, int32_t dim, int32_t rows, int32_t vocab, float *logits);

#endif

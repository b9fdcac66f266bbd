// capi.hip - the extern "C" boundary of libshared_amd_sampler.so.
//
// Validation, scratch ownership and launches.  No compute happens on the
// host; a missing device is an error, never a fallback.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "sas_device.h"
#include "sas_launch.h"
#include "shared_amd_sampler.h"

struct sas_sampler {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  void *recs = nullptr;        // candidate record slots of every (row, part)
  size_t recs_cap = 0;
  void *vscratch = nullptr;   // sas_verify partials
  size_t vscratch_cap = 0;
  void *pad = nullptr;        // rows of fewer than 4 logits, padded to 4
  size_t pad_cap = 0;
  void *hb = nullptr;         // long histories bucketed by part
  size_t hb_cap = 0;
  int cus = 0;                 // compute units of the device
  // Buffers a growth replaced.  Work already queued (or recorded into a
  // HIP graph) may still use them, so they are freed by sas_destroy only.
  std::vector<void *> retired;
};

namespace {

thread_local std::string g_err;

int fail(sas_sampler *s, int code, const std::string &msg) {
  if (s) s->err = msg;
  else g_err = msg;
  return code;
}

int hip_fail(sas_sampler *s, hipError_t e, const char *what) {
  return fail(s, SAS_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

hipStream_t pick_stream(sas_sampler *, void *stream) { return reinterpret_cast<hipStream_t>(stream); }

// Grow a scratch buffer to at least `need` bytes.  The buffer it replaces
// is retired, not freed: launches queued on any stream, and graphs that
// recorded them, keep a valid address; sas_destroy frees it.  Capacities
// at least double, so retired buffers hold less than the live one.  Under
// stream capture nothing is allocated: the call fails and names the fix.
int grow(sas_sampler *s, void **buf, size_t *cap, size_t need, void *stream, const char *who) {
  if (need <= *cap) return SAS_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &cs) == hipSuccess &&
      cs != hipStreamCaptureStatusNone)
    return fail(s, SAS_ERR_INVALID,
                std::string(who) + ": the handle's scratch is too small for this call and the stream is being "
                                   "captured: size it before the capture (sas_reserve_for, or one eager call "
                                   "of this shape)");
  size_t bytes = (need + 255) & ~size_t(255);
  if (*cap && bytes < 2 * *cap) bytes = 2 * *cap;
  void *fresh = nullptr;
  hipError_t e = hipMalloc(&fresh, bytes);
  if (e != hipSuccess) return fail(s, SAS_ERR_NOMEM, std::string(who) + ": hipMalloc scratch: " + hipGetErrorString(e));
  if (*buf) s->retired.push_back(*buf);
  *buf = fresh;
  *cap = bytes;
  return SAS_OK;
}

// Scratch bytes of each buffer for a call shape (the same sizes the calls
// ask for).
size_t hb_bytes(int64_t hist_ids, int hrows, int parts) {
  return (((size_t)hist_ids * 4 + 255) & ~size_t(255)) + (size_t)hrows * (parts + 1) * 4;
}

int ensure_sample_scratch(sas_sampler *s, int rows, int parts, void *stream, const char *who) {
  return grow(s, &s->recs, &s->recs_cap, sas::sample_rec_bytes(rows, parts), stream, who);
}

int set_device(sas_sampler *s) {
  hipError_t e = hipSetDevice(s->device);
  return e == hipSuccess ? SAS_OK : hip_fail(s, e, "hipSetDevice");
}

// The checks of a sas_rows descriptor shared by sas_sample and
// sas_sample_noalloc: nullptr when it is valid, else the message (after
// `who`).  rows == 0 is valid (nothing to do).
const char *check_rows(const sas_rows *r, bool seeded = false) {
  if (!r) return "rows descriptor is NULL";
  if (r->rows < 0) return "rows must be >= 0";
  if (r->vocab < 1 || r->vocab > SAS_MAX_VOCAB) return "vocab must be in [1, SAS_MAX_VOCAB]";
  if (r->rows == 0) return nullptr;
  if (!r->logits || !r->out_ids) return "logits and out_ids are required";
  if (r->logits_stride < r->vocab) return "logits_stride < vocab";
  if (r->mask && r->mask_stride != 0 && r->mask_stride < ((int64_t)r->vocab + 31) / 32)
    return "mask_stride must be 0 or >= ceil(vocab / 32)";
  if (r->hist_ids && !r->hist_offsets) return "hist_ids requires hist_offsets";
  if (r->hist_ids && r->hist_count < 1) return "hist_count must be >= 1 with hist_ids";
  const bool all_greedy = !r->row_params && !(r->params.temperature > 0.0);
  if (!r->uniforms && !all_greedy && !seeded) return "uniforms are required unless every row is greedy";
  return nullptr;
}

// The softcap kernel variants (fewer waves per SIMD) only when some row may
// have a softcap.
bool any_softcap(const sas_rows *r) {
  return r->row_params ? (r->row_hints & SAS_HINT_NO_SOFTCAP) == 0u : r->params.softcap > 0.0f;
}

// Kernel arguments for a valid descriptor whose record scratch is `recs`
// (sas::sample_rec_bytes(rows, parts) bytes) and whose logits have already
// been padded when vocab < 4.
void fill_args(const sas_rows *r, const float *logits, int64_t logits_stride, int parts, int span, void *recs,
               sas::SampleArgs *a) {
  a->logits = logits;
  a->logits_stride = logits_stride;
  a->mask = r->mask;
  a->mask_stride = r->mask_stride;
  a->hist_ids = r->hist_ids;
  a->hist_offsets = r->hist_ids ? r->hist_offsets : nullptr;
  a->hist_count = r->hist_ids ? r->hist_count : 0;
  a->uniforms = r->uniforms;
  a->row_params = r->row_params;
  a->params = r->params;
  a->out_ids = r->out_ids;
  a->out_probs = r->out_probs;
  a->out_cand_ids = r->out_cand_ids;
  a->out_counts = r->out_counts;
  a->out_flags = r->out_flags;
  a->rec = reinterpret_cast<uint64_t *>(recs);
  a->mrec = reinterpret_cast<uint4 *>(a->rec + (size_t)r->rows * parts * sas::kListCap);
  a->pinfo = reinterpret_cast<uint64_t *>(a->mrec + (size_t)r->rows * parts * (sas::kListCap / 2));
  a->vocab = r->vocab;
  a->rows = r->rows;
  a->parts = parts;
  a->span = span;
}

// ---- the scratch of sas_sample_noalloc: one array per device, for the
// life of the process.  Host code never uses the array's name as an
// address: its device address comes from hipGetSymbolAddress, once per
// device, with that device current.
constexpr size_t kStaticScratch = SAS_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratch];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];
int g_scratch_cus[kMaxDevices];

// The device address of `device`'s scratch (the device must be current).
hipError_t static_scratch(int device, void **ptr, int *cus) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 1) n = 256;
    g_scratch_ptr[device] = p;
    g_scratch_cus[device] = n;
  }
  *ptr = g_scratch_ptr[device];
  *cus = g_scratch_cus[device];
  return hipSuccess;
}

// The checks of a sas_step: nullptr when it is valid, else the message.
const char *check_step(const sas_rows *r, const sas_step *st) {
  if (!st->state) return "state is required";
  if (r->hist_ids) return "hist_ids must be NULL: the step's ring is the history";
  if (st->ring && (st->ring_len < 1 || st->ring_len > SAS_MAX_HISTORY))
    return "ring_len must be in [1, SAS_MAX_HISTORY]";
  if (st->sampled && st->max_steps < 1) return "max_steps must be >= 1 with sampled";
  return nullptr;
}

// sas_sample and sas_sample_step: `st` (checked) or nullptr.
// The verify rows of an exact-match speculative round: groups of `group`
// rows share a sequence's history, params and seed.
struct SpecDraw {
  const uint32_t *seeds;
  uint32_t round;
  int group;
  const sas_spec_state *state;  // chained rounds (sas_spec_step), or null
};

// sas_sample, sas_sample_step (st) and the sampling of sas_spec_exact (sp):
// one checked descriptor's launches.
int sample_on(sas_sampler *s, const sas_rows *r, const sas_step *st, const char *who, void *stream,
              const SpecDraw *sp = nullptr) {
  if (int rc = set_device(s)) return rc;
  // at least two blocks per CU: small batches take shorter parts
  int parts = 0, span = 0;
  sas::choose_parts(r->rows, r->vocab, 2 * s->cus, &parts, &span);
  if (int rc = ensure_sample_scratch(s, r->rows, parts, stream, who)) return rc;
  const float *logits = r->logits;
  int64_t stride = r->logits_stride;
  if (r->vocab < 4) {
    // the kernel loads 16 bytes at a time from inside a row: copy rows of
    // fewer than 4 logits into rows of 4, NaN (never selected) past vocab
    if (int rc = grow(s, &s->pad, &s->pad_cap, (size_t)r->rows * 16, stream, who)) return rc;
    hipError_t e = sas::launch_pad_rows(r->logits, r->logits_stride, r->vocab, r->rows,
                                        reinterpret_cast<float *>(s->pad), pick_stream(s, stream));
    if (e != hipSuccess) return hip_fail(s, e, "sas_sample pad launch");
    logits = reinterpret_cast<const float *>(s->pad);
    stride = 4;
  }
  sas::SampleArgs a{};
  fill_args(r, logits, stride, parts, span, s->recs, &a);
  if (st) {
    a.st_state = st->state;
    a.st_sampled = st->sampled;
    a.st_max_steps = st->sampled ? st->max_steps : 0;
    a.st_next = st->next_tokens;
    a.ring = st->ring;
    a.ring_len = st->ring ? st->ring_len : 0;
    a.stop_ids = st->stop_ids;
    a.seeds = st->seeds;
  }
  if (sp) {
    a.spec_seeds = sp->seeds;
    a.spec_round = sp->round;
    a.group = sp->group;
    if (sp->state) {
      // a chained round: each sequence's ring is its history, its state
      // holds its round and whether it is frozen
      a.sp_state = sp->state->state;
      a.ring = sp->state->ring;
      a.ring_len = sp->state->ring ? sp->state->ring_len : 0;
    }
  }
  // long histories: bucket them by part first, so a part reads its own ids
  const int hrows = sp && sp->group > 1 ? r->rows / sp->group : r->rows;
  const bool ring = a.ring != nullptr;
  const int64_t hist_ids = ring ? (int64_t)hrows * a.ring_len : (r->hist_ids ? r->hist_count : 0);
  if (hist_ids >= sas::kBucketMinIds * hrows && hist_ids > 0) {
    const size_t ids_bytes = ((size_t)hist_ids * 4 + 255) & ~size_t(255);
    if (int rc = grow(s, &s->hb, &s->hb_cap, hb_bytes(hist_ids, hrows, parts), stream, who)) return rc;
    a.hb_ids = reinterpret_cast<uint32_t *>(s->hb);
    a.hb_offs = reinterpret_cast<int32_t *>(static_cast<char *>(s->hb) + ids_bytes);
  }
  hipError_t e = sas::launch_sample(a, any_softcap(r), pick_stream(s, stream));
  if (e != hipSuccess) return hip_fail(s, e, (std::string(who) + " launch").c_str());
  return SAS_OK;
}

// Bytes of one row of a GGUF head of `dim` values (0 for bf16).
int64_t head_row_bytes(int32_t format, int32_t dim) {
  switch (format) {
    case SAS_HEAD_Q8_0: return (int64_t)dim / 32 * 34;
    case SAS_HEAD_Q4_0: return (int64_t)dim / 32 * 18;
    case SAS_HEAD_Q6_K: return (int64_t)dim / 256 * 210;
    default: return 0;
  }
}

// sas_lm_head_sample and sas_lm_head_sample_step (st).
int lm_head_on(sas_sampler *s, const sas_lm_head *h, const sas_rows *r, const sas_step *st, const char *who,
               void *stream) {
  const std::string w(who);
  if (!s) return fail(nullptr, SAS_ERR_INVALID, w + ": handle is NULL");
  if (!h || !r) return fail(s, SAS_ERR_INVALID, w + ": head and rows are required");
  if (r->logits) return fail(s, SAS_ERR_INVALID, w + ": rows->logits must be NULL (the head computes them)");
  // the sampling fields are checked as for sas_sample (sas_sample_step)
  sas_rows chk = *r;
  chk.logits = reinterpret_cast<const float *>(h->hidden ? static_cast<const void *>(h->hidden) : "");
  chk.logits_stride = r->vocab;
  if (const char *m = check_rows(&chk, st && st->seeds)) return fail(s, SAS_ERR_INVALID, w + ": " + m);
  if (st)
    if (const char *m = check_step(r, st)) return fail(s, SAS_ERR_INVALID, w + ": " + m);
  if (r->rows > SAS_LMH_MAX_ROWS) return fail(s, SAS_ERR_INVALID, w + ": rows must be <= SAS_LMH_MAX_ROWS");
  if (r->vocab > SAS_LMH_MAX_VOCAB) return fail(s, SAS_ERR_INVALID, w + ": vocab must be <= SAS_LMH_MAX_VOCAB");
  if (h->format < SAS_HEAD_BF16 || h->format > SAS_HEAD_Q6_K)
    return fail(s, SAS_ERR_INVALID, w + ": format must be one of SAS_HEAD_*");
  if (r->rows == 0) return SAS_OK;
  if (!h->hidden || !h->weight) return fail(s, SAS_ERR_INVALID, w + ": hidden and weight are required");
  if (h->dim < 256 || h->dim % 256 != 0) return fail(s, SAS_ERR_INVALID, w + ": dim must be a positive multiple of 256");
  if ((int64_t)r->rows * h->dim > SAS_LMH_MAX_LDS_FLOATS)
    return fail(s, SAS_ERR_INVALID, w + ": rows * dim must be <= SAS_LMH_MAX_LDS_FLOATS");
  if (h->hidden_stride < h->dim) return fail(s, SAS_ERR_INVALID, w + ": hidden_stride < dim");
  if (h->format == SAS_HEAD_BF16) {
    if (h->weight_stride < h->dim || h->weight_stride % 8 != 0)
      return fail(s, SAS_ERR_INVALID, w + ": weight_stride must be >= dim and a multiple of 8");
  } else {
    const int64_t rb = head_row_bytes(h->format, h->dim);
    if (h->weight_stride < rb || h->weight_stride % (h->format == SAS_HEAD_Q6_K ? 2 : 4) != 0)
      return fail(s, SAS_ERR_INVALID,
                  w + ": weight_stride must be >= the row's " + std::to_string(rb) +
                      " bytes and a multiple of 4 (Q8_0, Q4_0) or 2 (Q6_K)");
    // the kernels address a GGUF head by 32-bit byte offsets (whole 16-byte
    // chunks: up to 15 bytes past the last row)
    if ((int64_t)(r->vocab - 1) * h->weight_stride + rb + 16 > (int64_t)UINT32_MAX)
      return fail(s, SAS_ERR_INVALID, w + ": a GGUF head must span less than 4 GiB");
  }
  if (reinterpret_cast<uintptr_t>(h->weight) % 16 != 0)
    return fail(s, SAS_ERR_INVALID, w + ": weight must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(h->hidden) % 4 != 0)
    return fail(s, SAS_ERR_INVALID, w + ": hidden must be 4-byte aligned");
  if (int rc = set_device(s)) return rc;
  if (int rc = grow(s, &s->recs, &s->recs_cap, sas::lmh_scratch_bytes(r->rows, r->vocab), stream, who)) return rc;
  sas::LmhArgs a{};
  fill_args(r, nullptr, 0, 1, sas::kLmhSpan, s->recs, &a.s);
  sas::lmh_layout(&a, s->recs);
  if (st) {
    a.s.st_state = st->state;
    a.s.st_sampled = st->sampled;
    a.s.st_max_steps = st->sampled ? st->max_steps : 0;
    a.s.st_next = st->next_tokens;
    a.s.ring = st->ring;
    a.s.ring_len = st->ring ? st->ring_len : 0;
    a.s.stop_ids = st->stop_ids;
    a.s.seeds = st->seeds;
  }
  a.hidden = h->hidden;
  a.hidden_stride = h->hidden_stride;
  a.weight = h->weight;
  a.weight_stride = h->weight_stride;
  a.format = h->format;
  a.dim = h->dim;
  a.out_logits = h->out_logits;
  hipError_t e = sas::launch_lm_head_sample(a, any_softcap(r), pick_stream(s, stream));
  if (e != hipSuccess) return hip_fail(s, e, (w + " launch").c_str());
  return SAS_OK;
}

}  // namespace

extern "C" {

const char *sas_version(void) { return "shared_amd_sampler 3 gfx950"; }

int sas_create(int device, sas_sampler **out) {
  if (!out) return fail(nullptr, SAS_ERR_INVALID, "sas_create: out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(nullptr, SAS_ERR_HIP, "sas_create: no HIP device is available");
  if (device < 0 || device >= count)
    return fail(nullptr, SAS_ERR_INVALID, "sas_create: device index out of range");
  if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
  sas_sampler *s = new sas_sampler();
  s->device = device;
  if ((e = hipDeviceGetAttribute(&s->cus, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess || s->cus < 1)
    s->cus = 256;
  if ((e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking)) != hipSuccess) {
    delete s;
    return hip_fail(nullptr, e, "hipStreamCreate");
  }
  // sas_sample_noalloc's scratch address on this device, while it is
  // current (a failure is reported by sas_sample_noalloc itself)
  if (device < kMaxDevices) {
    void *p = nullptr;
    int n = 0;
    (void)static_scratch(device, &p, &n);
  }
  *out = s;
  return SAS_OK;
}

void sas_destroy(sas_sampler *s) {
  if (!s) return;
  (void)hipSetDevice(s->device);
  // the scratch may still be in use by queued work on any stream
  (void)hipDeviceSynchronize();
  for (void *p : s->retired) (void)hipFree(p);
  if (s->recs) (void)hipFree(s->recs);
  if (s->hb) (void)hipFree(s->hb);
  if (s->vscratch) (void)hipFree(s->vscratch);
  if (s->pad) (void)hipFree(s->pad);
  if (s->stream) (void)hipStreamDestroy(s->stream);
  delete s;
}

const char *sas_last_error(const sas_sampler *s) { return s ? s->err.c_str() : g_err.c_str(); }

int sas_reserve(sas_sampler *s, int32_t rows, int32_t vocab) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_reserve: handle is NULL");
  sas_reserve_desc d{};
  d.rows = rows;
  d.vocab = vocab;
  return sas_reserve_for(s, &d);
}

int sas_reserve_for(sas_sampler *s, const sas_reserve_desc *d) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_reserve_for: handle is NULL");
  if (!d) return fail(s, SAS_ERR_INVALID, "sas_reserve_for: descriptor is NULL");
  if (d->rows < 0 || d->vocab < 1 || d->vocab > SAS_MAX_VOCAB || d->hist_ids < 0 || d->lm_head_rows < 0 ||
      d->lm_head_rows > SAS_LMH_MAX_ROWS || d->verify_seqs < 0 || d->verify_draft_len < 0 ||
      d->verify_draft_len > SAS_MAX_DRAFT || (d->verify_seqs > 0 && d->verify_draft_len < 1) ||
      (d->lm_head_rows > 0 && d->vocab > SAS_LMH_MAX_VOCAB))
    return fail(s, SAS_ERR_INVALID,
                "sas_reserve_for: rows, hist_ids, lm_head_rows (<= SAS_LMH_MAX_ROWS, vocab <= SAS_LMH_MAX_VOCAB) "
                "and verify_seqs must be >= 0, vocab in [1, SAS_MAX_VOCAB], verify_draft_len in "
                "[1, SAS_MAX_DRAFT] with verify_seqs");
  if (int rc = set_device(s)) return rc;
  const char *who = "sas_reserve_for";
  // the most parts any batch of <= rows rows may pick (a single row)
  int parts = 0, span = 0;
  sas::choose_parts(1, d->vocab, 2 * s->cus, &parts, &span);
  size_t recs = sas::sample_rec_bytes(d->rows, parts);
  if (d->lm_head_rows > 0) recs = std::max(recs, sas::lmh_scratch_bytes(d->lm_head_rows, d->vocab));
  if (int rc = grow(s, &s->recs, &s->recs_cap, recs, nullptr, who)) return rc;
  if (d->vocab < 4 && d->rows > 0)
    if (int rc = grow(s, &s->pad, &s->pad_cap, (size_t)d->rows * 16, nullptr, who)) return rc;
  if (d->hist_ids >= sas::kBucketMinIds && d->rows > 0)
    if (int rc = grow(s, &s->hb, &s->hb_cap, hb_bytes(d->hist_ids, d->rows, parts), nullptr, who)) return rc;
  if (d->verify_seqs > 0)
    if (int rc = grow(s, &s->vscratch, &s->vscratch_cap,
                      sas::verify_scratch_bytes(d->verify_seqs, d->verify_draft_len, d->vocab), nullptr, who))
      return rc;
  return SAS_OK;
}

int sas_sample(sas_sampler *s, const sas_rows *r, void *stream) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_sample: handle is NULL");
  if (const char *m = check_rows(r)) return fail(s, SAS_ERR_INVALID, std::string("sas_sample: ") + m);
  if (r->rows == 0) return SAS_OK;
  return sample_on(s, r, nullptr, "sas_sample", stream);
}

int sas_sample_step(sas_sampler *s, const sas_rows *r, const sas_step *st, void *stream) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_sample_step: handle is NULL");
  if (!st) return fail(s, SAS_ERR_INVALID, "sas_sample_step: step descriptor is NULL");
  if (const char *m = check_rows(r, st->seeds != nullptr)) return fail(s, SAS_ERR_INVALID, std::string("sas_sample_step: ") + m);
  if (const char *m = check_step(r, st)) return fail(s, SAS_ERR_INVALID, std::string("sas_sample_step: ") + m);
  if (r->rows == 0) return SAS_OK;
  return sample_on(s, r, st, "sas_sample_step", stream);
}

int sas_sample_noalloc(int device, const sas_rows *r, void *stream) {
  if (const char *m = check_rows(r)) return fail(nullptr, SAS_ERR_INVALID, std::string("sas_sample_noalloc: ") + m);
  if (r->rows == 0) return SAS_OK;
  if (device < 0 || device >= kMaxDevices)
    return fail(nullptr, SAS_ERR_INVALID, "sas_sample_noalloc: device index out of range");
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(nullptr, e, "sas_sample_noalloc: hipSetDevice");
  void *base = nullptr;
  int cus = 0;
  if ((e = static_scratch(device, &base, &cus)) != hipSuccess)
    return hip_fail(nullptr, e, "sas_sample_noalloc: hipGetSymbolAddress of the static scratch");
  int parts = 0, span = 0;
  sas::choose_parts(r->rows, r->vocab, 2 * cus, &parts, &span);
  const size_t recs = (sas::sample_rec_bytes(r->rows, parts) + 255) & ~size_t(255);
  const size_t pad = r->vocab < 4 ? (size_t)r->rows * 16 : 0;
  if (recs + pad > kStaticScratch)
    return fail(nullptr, SAS_ERR_INVALID,
                "sas_sample_noalloc: this batch needs " + std::to_string(recs + pad) +
                    " bytes of scratch; the static scratch holds " + std::to_string(kStaticScratch) +
                    " (SAS_NOALLOC_SCRATCH_BYTES): use sas_sample");
  const float *logits = r->logits;
  int64_t stride = r->logits_stride;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (pad) {
    float *dst = reinterpret_cast<float *>(static_cast<unsigned char *>(base) + recs);
    e = sas::launch_pad_rows(r->logits, r->logits_stride, r->vocab, r->rows, dst, st);
    if (e != hipSuccess) return hip_fail(nullptr, e, "sas_sample_noalloc pad launch");
    logits = dst;
    stride = 4;
  }
  sas::SampleArgs a{};
  fill_args(r, logits, stride, parts, span, base, &a);
  e = sas::launch_sample(a, any_softcap(r), st);
  if (e != hipSuccess) return hip_fail(nullptr, e, "sas_sample_noalloc launch");
  return SAS_OK;
}

int sas_lm_head_sample(sas_sampler *s, const sas_lm_head *h, const sas_rows *r, void *stream) {
  return lm_head_on(s, h, r, nullptr, "sas_lm_head_sample", stream);
}

int sas_lm_head_sample_step(sas_sampler *s, const sas_lm_head *h, const sas_rows *r, const sas_step *st,
                            void *stream) {
  if (s && !st) return fail(s, SAS_ERR_INVALID, "sas_lm_head_sample_step: step descriptor is NULL");
  return lm_head_on(s, h, r, st, "sas_lm_head_sample_step", stream);
}

}  // extern "C"

namespace {

// sas_spec_exact (st null) and sas_spec_step: one speculative round.
int spec_on(sas_sampler *s, const sas_spec_rows *r, const sas_spec_state *st, const char *who, void *stream) {
  const std::string w(who);
  if (!s) return fail(nullptr, SAS_ERR_INVALID, w + ": handle is NULL");
  if (!r) return fail(s, SAS_ERR_INVALID, w + ": descriptor is NULL");
  if (r->seqs < 0) return fail(s, SAS_ERR_INVALID, w + ": seqs must be >= 0");
  if (r->draft_len < 1 || r->draft_len > SAS_MAX_DRAFT)
    return fail(s, SAS_ERR_INVALID, w + ": draft_len must be in [1, SAS_MAX_DRAFT]");
  if (st) {
    if (!st->state) return fail(s, SAS_ERR_INVALID, w + ": state is required");
    if (r->hist_ids) return fail(s, SAS_ERR_INVALID, w + ": hist_ids must be NULL: the ring is the history");
    if (st->ring && (st->ring_len < 1 || st->ring_len > SAS_MAX_HISTORY))
      return fail(s, SAS_ERR_INVALID, w + ": ring_len must be in [1, SAS_MAX_HISTORY]");
    if (st->log && st->max_rounds < 1) return fail(s, SAS_ERR_INVALID, w + ": max_rounds must be >= 1 with log");
  }
  if (r->seqs == 0) return SAS_OK;
  if ((int64_t)r->seqs * (r->draft_len + 1) > INT32_MAX)
    return fail(s, SAS_ERR_INVALID, w + ": too many verify rows");
  if (!r->draft_ids || !r->seeds || !r->out_picks || !r->out_accepted)
    return fail(s, SAS_ERR_INVALID, w + ": draft_ids, seeds, out_picks and out_accepted are required");
  hipStream_t stream_h = pick_stream(s, stream);
  const int L = r->draft_len;
  // the drafts: the argmax of every draft row (argmaxMerge, kernels.js:373-401)
  if (r->draft_logits) {
    sas_rows d{};
    d.logits = r->draft_logits;
    d.logits_stride = r->logits_stride;
    d.vocab = r->vocab;
    d.rows = r->seqs * L;
    d.params.temperature = 0.0;
    d.params.top_p = 1.0;
    d.params.repetition_penalty = 1.0;
    d.params.top_k = 1;
    d.out_ids = r->draft_ids;
    if (const char *m = check_rows(&d)) return fail(s, SAS_ERR_INVALID, w + ": drafts: " + m);
    if (int rc = sample_on(s, &d, nullptr, (w + " drafts").c_str(), stream)) return rc;
  }
  // every verify row, sampled on its own (kernels.js:255-327)
  sas_rows v{};
  v.logits = r->target_logits;
  v.logits_stride = r->logits_stride;
  v.vocab = r->vocab;
  v.rows = r->seqs * (L + 1);
  v.mask = r->mask;
  v.mask_stride = r->mask_stride;
  if (!st) {
    v.hist_ids = r->hist_ids;
    v.hist_offsets = r->hist_offsets;
    v.hist_count = r->hist_count;
  }
  v.params = r->params;
  v.row_params = r->seq_params;
  v.row_hints = r->row_hints;
  v.out_ids = r->out_picks;
  if (const char *m = check_rows(&v, true)) return fail(s, SAS_ERR_INVALID, w + ": " + m);
  const SpecDraw sp{r->seeds, r->round, L + 1, st};
  if (int rc = sample_on(s, &v, nullptr, who, stream, &sp)) return rc;
  // the cascade (kernels.js:328-339), and a chained round's commit
  // (kernels.js:340-367)
  sas::SpecCommit c{};
  if (st) {
    c.state = st->state;
    c.ring = st->ring;
    c.ring_len = st->ring ? st->ring_len : 0;
    c.log = st->log;
    c.max_rounds = st->log ? st->max_rounds : 0;
    c.next_tokens = st->next_tokens;
  }
  hipError_t e = sas::launch_spec_cascade(r->out_picks, r->draft_ids, r->stop_ids, r->seqs, L, r->out_accepted,
                                          r->out_next, c, stream_h);
  if (e != hipSuccess) return hip_fail(s, e, (w + " cascade launch").c_str());
  return SAS_OK;
}

}  // namespace

extern "C" {

int sas_spec_exact(sas_sampler *s, const sas_spec_rows *r, void *stream) {
  return spec_on(s, r, nullptr, "sas_spec_exact", stream);
}

int sas_spec_step(sas_sampler *s, const sas_spec_rows *r, const sas_spec_state *st, void *stream) {
  if (s && !st) return fail(s, SAS_ERR_INVALID, "sas_spec_step: state descriptor is NULL");
  return spec_on(s, r, st, "sas_spec_step", stream);
}

int sas_verify(sas_sampler *s, const sas_verify_rows *v, void *stream) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_verify: handle is NULL");
  if (!v) return fail(s, SAS_ERR_INVALID, "sas_verify: descriptor is NULL");
  if (v->seqs < 0) return fail(s, SAS_ERR_INVALID, "sas_verify: seqs must be >= 0");
  if (v->vocab < 1 || v->vocab > SAS_MAX_VOCAB)
    return fail(s, SAS_ERR_INVALID, "sas_verify: vocab must be in [1, SAS_MAX_VOCAB]");
  if (v->draft_len < 1 || v->draft_len > SAS_MAX_DRAFT)
    return fail(s, SAS_ERR_INVALID, "sas_verify: draft_len must be in [1, SAS_MAX_DRAFT]");
  if (!(v->temperature > 0.0) || !std::isfinite(v->temperature))
    return fail(s, SAS_ERR_INVALID, "sas_verify: temperature must be finite and > 0");
  if (v->seqs == 0) return SAS_OK;
  if (!v->target_logits || !v->draft_logits || !v->draft_ids || !v->uniforms || !v->out_tokens ||
      !v->out_accepted)
    return fail(s, SAS_ERR_INVALID,
                "sas_verify: target_logits, draft_logits, draft_ids, uniforms, out_tokens and out_accepted "
                "are required");
  if (v->logits_stride < v->vocab) return fail(s, SAS_ERR_INVALID, "sas_verify: logits_stride < vocab");
  if (v->mask && v->mask_stride != 0 && v->mask_stride < ((int64_t)v->vocab + 31) / 32)
    return fail(s, SAS_ERR_INVALID, "sas_verify: mask_stride must be 0 or >= ceil(vocab / 32)");
  if ((int64_t)v->seqs * (v->draft_len + 1) > 65535)
    return fail(s, SAS_ERR_INVALID, "sas_verify: seqs * (draft_len + 1) must be <= 65535");
  if (int rc = set_device(s)) return rc;
  if (int rc = grow(s, &s->vscratch, &s->vscratch_cap, sas::verify_scratch_bytes(v->seqs, v->draft_len, v->vocab),
                    stream, "sas_verify"))
    return rc;
  sas::VerifyArgs a;
  a.target = v->target_logits;
  a.draft = v->draft_logits;
  a.stride = v->logits_stride;
  a.mask = v->mask;
  a.mask_stride = v->mask_stride;
  a.draft_ids = v->draft_ids;
  a.uniforms = v->uniforms;
  a.temperature = v->temperature;
  a.inv_t = 1.0 / v->temperature;
  a.out_tokens = v->out_tokens;
  a.out_accepted = v->out_accepted;
  a.vocab = v->vocab;
  a.seqs = v->seqs;
  a.L = v->draft_len;
  a.chunks = (v->vocab + sas::kVChunk - 1) / sas::kVChunk;
  const size_t positions = (size_t)v->seqs * (v->draft_len + 1);
  a.stats = reinterpret_cast<double *>(s->vscratch);
  a.part = a.stats + positions * a.chunks * 4;
  a.seqrec = a.part + (size_t)v->seqs * a.chunks * 2;
  a.dtok = reinterpret_cast<float *>(a.seqrec + (size_t)v->seqs * 8);
  a.pk_n = reinterpret_cast<uint32_t *>(a.dtok + positions * 2);
  a.pk_v = reinterpret_cast<float *>(a.pk_n + positions * a.chunks * sas::kWaves);
  a.aligned = (reinterpret_cast<uintptr_t>(v->target_logits) & 15u) == 0 &&
              (reinterpret_cast<uintptr_t>(v->draft_logits) & 15u) == 0 && (v->logits_stride & 3) == 0;
  hipError_t e = sas::launch_verify(a, pick_stream(s, stream));
  if (e != hipSuccess) return hip_fail(s, e, "sas_verify launch");
  return SAS_OK;
}

int sas_clamp_params(const sas_params *in, sas_params *out) {
  if (!in || !out) return fail(nullptr, SAS_ERR_INVALID, "sas_clamp_params: NULL argument");
  sas_params p = *in;
  p.temperature = std::isfinite(in->temperature) && in->temperature > 0.0 ? in->temperature : 0.0;
  p.top_p = std::isfinite(in->top_p) ? std::fmin(1.0, std::fmax(0.0, in->top_p)) : 1.0;
  p.presence_penalty =
      std::isfinite(in->presence_penalty) ? std::fmin(10.0, std::fmax(0.0, in->presence_penalty)) : 0.0;
  p.repetition_penalty =
      std::isfinite(in->repetition_penalty) && in->repetition_penalty > 0.0 ? in->repetition_penalty : 1.0;
  p.frequency_penalty = std::isfinite(in->frequency_penalty) ? in->frequency_penalty : 0.0;
  p.softcap = std::isfinite(in->softcap) && in->softcap > 0.0f ? in->softcap : 0.0f;
  p.top_k = in->top_k < 1 ? 1 : (in->top_k > SAS_MAX_TOP_K ? SAS_MAX_TOP_K : in->top_k);
  *out = p;
  return SAS_OK;
}

int64_t sas_mask_from_ids(int32_t kind, const uint32_t *ids, size_t count, int32_t vocab, uint32_t *words,
                          int64_t nwords) {
  if (vocab < 1 || vocab > SAS_MAX_VOCAB || !words || nwords < ((int64_t)vocab + 31) / 32 ||
      (kind != SAS_MASK_ALL && kind != SAS_MASK_ALLOW && kind != SAS_MASK_DENY) || (count && !ids)) {
    fail(nullptr, SAS_ERR_INVALID, "sas_mask_from_ids: invalid argument");
    return -SAS_ERR_INVALID;
  }
  const int64_t used = ((int64_t)vocab + 31) / 32;
  const uint32_t fill = kind == SAS_MASK_ALLOW ? 0u : ~0u;
  for (int64_t w = 0; w < nwords; ++w) words[w] = w < used ? fill : 0u;
  if (kind != SAS_MASK_ALLOW && (vocab & 31)) words[used - 1] = (1u << (vocab & 31)) - 1u;
  for (size_t i = 0; i < count; ++i) {
    const uint32_t id = ids[i];
    if (id >= (uint32_t)vocab) continue;
    if (kind == SAS_MASK_ALLOW) words[id >> 5] |= 1u << (id & 31);
    else if (kind == SAS_MASK_DENY) words[id >> 5] &= ~(1u << (id & 31));
  }
  int64_t allowed = 0;
  for (int64_t w = 0; w < used; ++w) allowed += __builtin_popcount(words[w]);
  return allowed;
}

double sas_pcg_uniform(uint32_t seed, uint32_t it, uint32_t row) {
  uint32_t h = (seed ^ (it * 0x9E3779B9u) ^ (row * 0x85EBCA6Bu)) * 747796405u + 2891336453u;
  h = ((h >> ((h >> 28u) + 4u)) ^ h) * 277803737u;
  h = (h >> 22u) ^ h;
  return (double)(h & 0xFFFFFFu) / 16777216.0;
}

int sas_alloc(sas_sampler *s, size_t bytes, void **out) {
  if (!s || !out) return fail(s, SAS_ERR_INVALID, "sas_alloc: NULL argument");
  if (int rc = set_device(s)) return rc;
  hipError_t e = hipMalloc(out, bytes ? bytes : 1);
  if (e != hipSuccess) {
    *out = nullptr;
    return fail(s, SAS_ERR_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
  }
  return SAS_OK;
}

int sas_free(sas_sampler *s, void *p) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_free: handle is NULL");
  if (!p) return SAS_OK;
  if (int rc = set_device(s)) return rc;
  hipError_t e = hipFree(p);
  return e == hipSuccess ? SAS_OK : hip_fail(s, e, "hipFree");
}

int sas_memcpy(sas_sampler *s, void *dst, const void *src, size_t bytes, int kind, void *stream) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_memcpy: handle is NULL");
  if (bytes == 0) return SAS_OK;
  if (!dst || !src) return fail(s, SAS_ERR_INVALID, "sas_memcpy: NULL pointer");
  if (int rc = set_device(s)) return rc;
  hipStream_t st = pick_stream(s, stream);
  hipError_t e;
  switch (kind) {
    case 0:
      e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
      if (e == hipSuccess) e = hipStreamSynchronize(st);
      break;
    case 1:
      e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st);
      if (e == hipSuccess) e = hipStreamSynchronize(st);
      break;
    case 2:
      e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st);
      break;
    default:
      return fail(s, SAS_ERR_INVALID, "sas_memcpy: kind must be 0, 1 or 2");
  }
  return e == hipSuccess ? SAS_OK : hip_fail(s, e, "hipMemcpyAsync");
}

int sas_synchronize(sas_sampler *s, void *stream) {
  if (!s) return fail(nullptr, SAS_ERR_INVALID, "sas_synchronize: handle is NULL");
  if (int rc = set_device(s)) return rc;
  hipError_t e = hipStreamSynchronize(pick_stream(s, stream));
  return e == hipSuccess ? SAS_OK : hip_fail(s, e, "hipStreamSynchronize");
}

void *sas_stream(sas_sampler *s) { return s ? reinterpret_cast<void *>(s->stream) : nullptr; }

}  // extern "C"

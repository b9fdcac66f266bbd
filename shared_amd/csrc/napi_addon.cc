// napi_addon.cc - Node-API binding of libshared_amd_sampler.so (sas_napi.node).
//
// A thin, synchronous-by-default mirror of the C ABI for a Node host: device
// pointers cross as BigInt, descriptors as plain objects whose keys are the
// C fields in camelCase.  Every call runs on the handle's own HIP stream
// (sas_stream).  sampleAsync / verifyAsync run the launch and the stream
// synchronisation on a libuv worker and resolve a Promise, so the JS thread
// is free while the GPU works (the reference awaits mapAsync the same way,
// lib/webgpu-llm/model.js:724).  Errors throw a JS Error carrying
// sas_last_error().  Host code only: no HIP header is needed here.
//
// A handle is not re-entrant, so every call on it holds the handle's mutex
// for the whole C call, the async ones on their worker thread included: a
// synchronous call made while a worker runs waits for it instead of racing
// it.  destroy() takes the mutex too, marks the handle closed (later calls
// throw "sampler is closed") and frees the C handle; the wrapper itself
// lives until the JS external is collected, and queued async work holds a
// reference to that external, so no worker ever sees freed memory.
#define NAPI_VERSION 8
#include <node_api.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>

#include "shared_amd_sampler.h"

namespace {

#define NAPI_OK(call)                                    \
  do {                                                   \
    if ((call) != napi_ok) return throw_napi(env, #call); \
  } while (0)

napi_value throw_napi(napi_env env, const char *what) {
  const napi_extended_error_info *info = nullptr;
  napi_get_last_error_info(env, &info);
  bool pending = false;
  napi_is_exception_pending(env, &pending);
  if (!pending) {
    std::string msg = std::string("sas_napi: ") + what;
    if (info && info->error_message) msg += std::string(": ") + info->error_message;
    napi_throw_error(env, nullptr, msg.c_str());
  }
  return nullptr;
}

napi_value throw_sas(napi_env env, const sas_sampler *s, int rc) {
  const char *m = sas_last_error(s);
  std::string msg = (m && *m) ? m : "shared_amd_sampler call failed";
  napi_value err, code, text;
  napi_create_string_utf8(env, msg.c_str(), NAPI_AUTO_LENGTH, &text);
  napi_create_error(env, nullptr, text, &err);
  napi_create_int32(env, rc, &code);
  napi_set_named_property(env, err, "code", code);
  napi_throw(env, err);
  return nullptr;
}

napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

// ---------------------------------------------------------------- values --

bool has(napi_env env, napi_value obj, const char *key, napi_value *out) {
  bool present = false;
  if (napi_has_named_property(env, obj, key, &present) != napi_ok || !present) return false;
  if (napi_get_named_property(env, obj, key, out) != napi_ok) return false;
  napi_valuetype t;
  napi_typeof(env, *out, &t);
  return t != napi_undefined && t != napi_null;
}

bool get_f64(napi_env env, napi_value obj, const char *key, double *v) {
  napi_value x;
  if (!has(env, obj, key, &x)) return true;
  return napi_get_value_double(env, x, v) == napi_ok;
}

bool get_i64(napi_env env, napi_value obj, const char *key, int64_t *v) {
  napi_value x;
  if (!has(env, obj, key, &x)) return true;
  napi_valuetype t;
  napi_typeof(env, x, &t);
  if (t == napi_bigint) {
    bool lossless;
    return napi_get_value_bigint_int64(env, x, v, &lossless) == napi_ok;
  }
  double d;
  if (napi_get_value_double(env, x, &d) != napi_ok || !std::isfinite(d) || d != std::floor(d)) return false;
  *v = (int64_t)d;
  return true;
}

// A device address: BigInt, or null / undefined for "none".
bool get_ptr(napi_env env, napi_value obj, const char *key, void **p) {
  napi_value x;
  *p = nullptr;
  if (!has(env, obj, key, &x)) return true;
  uint64_t u;
  bool lossless;
  if (napi_get_value_bigint_uint64(env, x, &u, &lossless) != napi_ok || !lossless) return false;
  *p = reinterpret_cast<void *>((uintptr_t)u);
  return true;
}

napi_value make_ptr(napi_env env, const void *p) {
  napi_value v;
  napi_create_bigint_uint64(env, (uint64_t)(uintptr_t)p, &v);
  return v;
}

// What the JS external holds: the C handle and its call lock.
struct Handle {
  sas_sampler *s = nullptr;
  std::mutex mu;
  bool closed = false;
};

Handle *get_wrapper(napi_env env, napi_value v) {
  void *p = nullptr;
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) return nullptr;
  napi_get_value_external(env, v, &p);
  return reinterpret_cast<Handle *>(p);
}

void finalize_handle(napi_env, void *data, void *) {
  Handle *h = static_cast<Handle *>(data);
  {
    std::lock_guard<std::mutex> g(h->mu);
    if (!h->closed && h->s) sas_destroy(h->s);
    h->s = nullptr;
    h->closed = true;
  }
  delete h;
}

bool read_params(napi_env env, napi_value obj, sas_params *p) {
  std::memset(p, 0, sizeof *p);
  p->top_p = 1.0;
  p->repetition_penalty = 1.0;
  p->top_k = 1;
  double softcap = 0.0;
  int64_t top_k = 1;
  bool ok = get_f64(env, obj, "temperature", &p->temperature) && get_f64(env, obj, "topP", &p->top_p) &&
            get_f64(env, obj, "repetitionPenalty", &p->repetition_penalty) &&
            get_f64(env, obj, "presencePenalty", &p->presence_penalty) &&
            get_f64(env, obj, "frequencyPenalty", &p->frequency_penalty) && get_f64(env, obj, "softcap", &softcap) &&
            get_i64(env, obj, "topK", &top_k);
  p->softcap = (float)softcap;
  p->top_k = top_k > INT32_MAX ? INT32_MAX : (top_k < INT32_MIN ? INT32_MIN : (int32_t)top_k);
  return ok;
}

napi_value params_object(napi_env env, const sas_params &p) {
  napi_value o, v;
  napi_create_object(env, &o);
  napi_create_double(env, p.temperature, &v);
  napi_set_named_property(env, o, "temperature", v);
  napi_create_double(env, p.top_p, &v);
  napi_set_named_property(env, o, "topP", v);
  napi_create_int32(env, p.top_k, &v);
  napi_set_named_property(env, o, "topK", v);
  napi_create_double(env, p.repetition_penalty, &v);
  napi_set_named_property(env, o, "repetitionPenalty", v);
  napi_create_double(env, p.presence_penalty, &v);
  napi_set_named_property(env, o, "presencePenalty", v);
  napi_create_double(env, p.frequency_penalty, &v);
  napi_set_named_property(env, o, "frequencyPenalty", v);
  napi_create_double(env, (double)p.softcap, &v);
  napi_set_named_property(env, o, "softcap", v);
  return o;
}

bool read_rows(napi_env env, napi_value d, sas_rows *r) {
  std::memset(r, 0, sizeof *r);
  int64_t vocab = 0, rows = 0;
  napi_value pv;
  bool ok = get_ptr(env, d, "logits", (void **)&r->logits) && get_i64(env, d, "logitsStride", &r->logits_stride) &&
            get_i64(env, d, "vocab", &vocab) && get_i64(env, d, "rows", &rows) &&
            get_ptr(env, d, "mask", (void **)&r->mask) && get_i64(env, d, "maskStride", &r->mask_stride) &&
            get_ptr(env, d, "histIds", (void **)&r->hist_ids) &&
            get_ptr(env, d, "histOffsets", (void **)&r->hist_offsets) &&
            get_ptr(env, d, "uniforms", (void **)&r->uniforms) &&
            get_ptr(env, d, "rowParams", (void **)&r->row_params) && get_ptr(env, d, "outIds", (void **)&r->out_ids) &&
            get_ptr(env, d, "outProbs", (void **)&r->out_probs) &&
            get_ptr(env, d, "outCandIds", (void **)&r->out_cand_ids) &&
            get_ptr(env, d, "outCounts", (void **)&r->out_counts) &&
            get_ptr(env, d, "outFlags", (void **)&r->out_flags) && get_i64(env, d, "histCount", &r->hist_count);
  int64_t hints = 0;
  ok = ok && get_i64(env, d, "rowHints", &hints);
  r->row_hints = (uint32_t)hints;
  if (!ok || vocab < INT32_MIN || vocab > INT32_MAX || rows < INT32_MIN || rows > INT32_MAX) return false;
  r->vocab = (int32_t)vocab;
  r->rows = (int32_t)rows;
  if (has(env, d, "params", &pv) && !read_params(env, pv, &r->params)) return false;
  return true;
}

bool read_verify(napi_env env, napi_value d, sas_verify_rows *v) {
  std::memset(v, 0, sizeof *v);
  int64_t vocab = 0, seqs = 0, L = 0;
  bool ok = get_ptr(env, d, "targetLogits", (void **)&v->target_logits) &&
            get_ptr(env, d, "draftLogits", (void **)&v->draft_logits) &&
            get_i64(env, d, "logitsStride", &v->logits_stride) && get_i64(env, d, "vocab", &vocab) &&
            get_i64(env, d, "seqs", &seqs) && get_i64(env, d, "draftLen", &L) &&
            get_ptr(env, d, "draftIds", (void **)&v->draft_ids) && get_ptr(env, d, "mask", (void **)&v->mask) &&
            get_i64(env, d, "maskStride", &v->mask_stride) && get_ptr(env, d, "uniforms", (void **)&v->uniforms) &&
            get_f64(env, d, "temperature", &v->temperature) &&
            get_ptr(env, d, "outTokens", (void **)&v->out_tokens) &&
            get_ptr(env, d, "outAccepted", (void **)&v->out_accepted);
  if (!ok || vocab < INT32_MIN || vocab > INT32_MAX || seqs < INT32_MIN || seqs > INT32_MAX || L < INT32_MIN ||
      L > INT32_MAX)
    return false;
  v->vocab = (int32_t)vocab;
  v->seqs = (int32_t)seqs;
  v->draft_len = (int32_t)L;
  return true;
}

bool read_spec(napi_env env, napi_value d, sas_spec_rows *r) {
  std::memset(r, 0, sizeof *r);
  int64_t vocab = 0, seqs = 0, L = 0, round = 0, hints = 0;
  napi_value pv;
  bool ok = get_ptr(env, d, "targetLogits", (void **)&r->target_logits) &&
            get_ptr(env, d, "draftLogits", (void **)&r->draft_logits) &&
            get_i64(env, d, "logitsStride", &r->logits_stride) && get_i64(env, d, "vocab", &vocab) &&
            get_i64(env, d, "seqs", &seqs) && get_i64(env, d, "draftLen", &L) &&
            get_ptr(env, d, "draftIds", (void **)&r->draft_ids) && get_ptr(env, d, "mask", (void **)&r->mask) &&
            get_i64(env, d, "maskStride", &r->mask_stride) && get_ptr(env, d, "histIds", (void **)&r->hist_ids) &&
            get_ptr(env, d, "histOffsets", (void **)&r->hist_offsets) &&
            get_i64(env, d, "histCount", &r->hist_count) &&
            get_ptr(env, d, "seqParams", (void **)&r->seq_params) && get_ptr(env, d, "seeds", (void **)&r->seeds) &&
            get_i64(env, d, "round", &round) && get_i64(env, d, "rowHints", &hints) &&
            get_ptr(env, d, "stopIds", (void **)&r->stop_ids) && get_ptr(env, d, "outPicks", (void **)&r->out_picks) &&
            get_ptr(env, d, "outAccepted", (void **)&r->out_accepted) &&
            get_ptr(env, d, "outNext", (void **)&r->out_next);
  if (!ok || vocab < INT32_MIN || vocab > INT32_MAX || seqs < INT32_MIN || seqs > INT32_MAX || L < INT32_MIN ||
      L > INT32_MAX || round < 0 || round > UINT32_MAX)
    return false;
  r->vocab = (int32_t)vocab;
  r->seqs = (int32_t)seqs;
  r->draft_len = (int32_t)L;
  r->round = (uint32_t)round;
  r->row_hints = (uint32_t)hints;
  if (has(env, d, "params", &pv) && !read_params(env, pv, &r->params)) return false;
  return true;
}

bool args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr) != napi_ok) return false;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return true;
}

// ----------------------------------------------------------- functions --

napi_value Version(napi_env env, napi_callback_info) {
  napi_value v;
  napi_create_string_utf8(env, sas_version(), NAPI_AUTO_LENGTH, &v);
  return v;
}

napi_value Create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args(env, info, 1, argv)) return throw_napi(env, "arguments");
  int32_t device = 0;
  napi_valuetype t;
  napi_typeof(env, argv[0], &t);
  if (t == napi_number) napi_get_value_int32(env, argv[0], &device);
  sas_sampler *s = nullptr;
  int rc = sas_create(device, &s);
  if (rc != SAS_OK) return throw_sas(env, nullptr, rc);
  Handle *h = new Handle();
  h->s = s;
  napi_value ext;
  if (napi_create_external(env, h, finalize_handle, nullptr, &ext) != napi_ok) {
    sas_destroy(s);
    delete h;
    return throw_napi(env, "napi_create_external");
  }
  return ext;
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args(env, info, 1, argv)) return throw_napi(env, "arguments");
  Handle *h = get_wrapper(env, argv[0]);
  if (!h) {
    napi_throw_type_error(env, nullptr, "sas_napi: expected a sampler handle");
    return nullptr;
  }
  std::lock_guard<std::mutex> g(h->mu);
  if (!h->closed && h->s) sas_destroy(h->s);
  h->s = nullptr;
  h->closed = true;
  return undefined(env);
}

// Binds `s` to the handle's C sampler with its mutex held until the end of
// the enclosing scope; throws when the value is no handle or it is closed.
#define HANDLE_OR_THROW(v, s)                                                   \
  Handle *s##_w = get_wrapper(env, v);                                          \
  if (!s##_w) {                                                                 \
    napi_throw_type_error(env, nullptr, "sas_napi: expected a sampler handle"); \
    return nullptr;                                                             \
  }                                                                             \
  std::lock_guard<std::mutex> s##_lock(s##_w->mu);                              \
  if (s##_w->closed) {                                                          \
    napi_throw_error(env, nullptr, "sampler is closed");                        \
    return nullptr;                                                             \
  }                                                                             \
  sas_sampler *s = s##_w->s;

// reserve(handle, rows, vocab[, histIds, lmHeadRows, verifySeqs, verifyDraftLen])
napi_value Reserve(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  size_t argc = 7;
  NAPI_OK(napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  if (argc != 3 && argc != 7) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_reserve_desc d{};
  NAPI_OK(napi_get_value_int32(env, argv[1], &d.rows));
  NAPI_OK(napi_get_value_int32(env, argv[2], &d.vocab));
  if (argc == 7) {
    NAPI_OK(napi_get_value_int64(env, argv[3], &d.hist_ids));
    NAPI_OK(napi_get_value_int32(env, argv[4], &d.lm_head_rows));
    NAPI_OK(napi_get_value_int32(env, argv[5], &d.verify_seqs));
    NAPI_OK(napi_get_value_int32(env, argv[6], &d.verify_draft_len));
  }
  int rc = sas_reserve_for(s, &d);
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

napi_value Alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  double bytes = 0;
  NAPI_OK(napi_get_value_double(env, argv[1], &bytes));
  if (!(bytes >= 0) || bytes > 9.0e15) {
    napi_throw_range_error(env, nullptr, "sas_napi: alloc size out of range");
    return nullptr;
  }
  void *p = nullptr;
  int rc = sas_alloc(s, (size_t)bytes, &p);
  return rc == SAS_OK ? make_ptr(env, p) : throw_sas(env, s, rc);
}

napi_value Free(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  uint64_t u = 0;
  bool lossless;
  NAPI_OK(napi_get_value_bigint_uint64(env, argv[1], &u, &lossless));
  int rc = sas_free(s, reinterpret_cast<void *>((uintptr_t)u));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

// copy(handle, devicePtr: BigInt, typedArray, direction 0 = to device, 1 = to host)
napi_value Copy(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!args(env, info, 4, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  uint64_t u = 0;
  bool lossless;
  NAPI_OK(napi_get_value_bigint_uint64(env, argv[1], &u, &lossless));
  bool is_ta = false;
  NAPI_OK(napi_is_typedarray(env, argv[2], &is_ta));
  if (!is_ta) {
    napi_throw_type_error(env, nullptr, "sas_napi: copy needs a TypedArray");
    return nullptr;
  }
  napi_typedarray_type type;
  size_t length = 0, offset = 0;
  void *data = nullptr;
  napi_value ab;
  NAPI_OK(napi_get_typedarray_info(env, argv[2], &type, &length, &data, &ab, &offset));
  size_t elem = 1;
  switch (type) {
    case napi_int16_array:
    case napi_uint16_array: elem = 2; break;
    case napi_int32_array:
    case napi_uint32_array:
    case napi_float32_array: elem = 4; break;
    case napi_float64_array:
    case napi_bigint64_array:
    case napi_biguint64_array: elem = 8; break;
    default: elem = 1;
  }
  int32_t dir = 0;
  NAPI_OK(napi_get_value_int32(env, argv[3], &dir));
  void *dev = reinterpret_cast<void *>((uintptr_t)u);
  int rc = dir == 0 ? sas_memcpy(s, dev, data, length * elem, 0, sas_stream(s))
                    : sas_memcpy(s, data, dev, length * elem, 1, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

napi_value Synchronize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args(env, info, 1, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  int rc = sas_synchronize(s, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

napi_value Sample(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_rows r;
  if (!read_rows(env, argv[1], &r)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad sample descriptor");
    return nullptr;
  }
  int rc = sas_sample(s, &r, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

// A sas_step descriptor: {state, sampled?, maxSteps?, nextTokens?, ring?,
// ringLen?, stopIds?, seeds?} of device addresses (BigInt) and sizes.
bool read_step(napi_env env, napi_value d, sas_step *st) {
  std::memset(st, 0, sizeof *st);
  int64_t max_steps = 0, ring_len = 0;
  const bool ok = get_ptr(env, d, "state", (void **)&st->state) && get_ptr(env, d, "sampled", (void **)&st->sampled) &&
                  get_i64(env, d, "maxSteps", &max_steps) &&
                  get_ptr(env, d, "nextTokens", (void **)&st->next_tokens) &&
                  get_ptr(env, d, "ring", (void **)&st->ring) && get_i64(env, d, "ringLen", &ring_len) &&
                  get_ptr(env, d, "stopIds", (void **)&st->stop_ids) && get_ptr(env, d, "seeds", (void **)&st->seeds);
  if (!ok || max_steps < 0 || max_steps > INT32_MAX || ring_len < 0 || ring_len > INT32_MAX) return false;
  st->max_steps = (int32_t)max_steps;
  st->ring_len = (int32_t)ring_len;
  return true;
}

napi_value SampleStep(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_rows r;
  sas_step st;
  if (!read_rows(env, argv[1], &r) || !read_step(env, argv[2], &st)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad sample step descriptor");
    return nullptr;
  }
  int rc = sas_sample_step(s, &r, &st, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

// A sas_lm_head descriptor: {hidden, hiddenStride, weight, weightStride,
// dim, outLogits?, format?} of device addresses (BigInt) and sizes.
bool read_head(napi_env env, napi_value d, sas_lm_head *hd) {
  std::memset(hd, 0, sizeof *hd);
  int64_t dim = 0;
  int64_t format = SAS_HEAD_BF16;
  const bool ok = get_ptr(env, d, "hidden", (void **)&hd->hidden) &&
                  get_i64(env, d, "hiddenStride", &hd->hidden_stride) &&
                  get_ptr(env, d, "weight", (void **)&hd->weight) &&
                  get_i64(env, d, "weightStride", &hd->weight_stride) && get_i64(env, d, "dim", &dim) &&
                  get_ptr(env, d, "outLogits", (void **)&hd->out_logits) && get_i64(env, d, "format", &format);
  if (!ok || dim < INT32_MIN || dim > INT32_MAX || format < INT32_MIN || format > INT32_MAX) return false;
  hd->dim = (int32_t)dim;
  hd->format = (int32_t)format;
  return true;
}

napi_value LmHeadSample(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_rows r;
  sas_lm_head hd;
  if (!read_rows(env, argv[1], &r) || !read_head(env, argv[2], &hd)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad lm head descriptor");
    return nullptr;
  }
  int rc = sas_lm_head_sample(s, &hd, &r, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

// The fused head as a step of the in-graph decode loop.
napi_value LmHeadStep(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!args(env, info, 4, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_rows r;
  sas_lm_head hd;
  sas_step st;
  if (!read_rows(env, argv[1], &r) || !read_head(env, argv[2], &hd) || !read_step(env, argv[3], &st)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad lm head step descriptor");
    return nullptr;
  }
  int rc = sas_lm_head_sample_step(s, &hd, &r, &st, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

napi_value Verify(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_verify_rows v;
  if (!read_verify(env, argv[1], &v)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad verify descriptor");
    return nullptr;
  }
  int rc = sas_verify(s, &v, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

napi_value SpecExact(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_spec_rows r;
  if (!read_spec(env, argv[1], &r)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad spec descriptor");
    return nullptr;
  }
  int rc = sas_spec_exact(s, &r, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

// A sas_spec_state descriptor: {state, ring?, ringLen?, log?, maxRounds?,
// nextTokens?} of device addresses (BigInt) and sizes.
bool read_spec_state(napi_env env, napi_value d, sas_spec_state *st) {
  std::memset(st, 0, sizeof *st);
  int64_t ring_len = 0, max_rounds = 0;
  const bool ok = get_ptr(env, d, "state", (void **)&st->state) && get_ptr(env, d, "ring", (void **)&st->ring) &&
                  get_i64(env, d, "ringLen", &ring_len) && get_ptr(env, d, "log", (void **)&st->log) &&
                  get_i64(env, d, "maxRounds", &max_rounds) &&
                  get_ptr(env, d, "nextTokens", (void **)&st->next_tokens);
  if (!ok || ring_len < 0 || ring_len > INT32_MAX || max_rounds < 0 || max_rounds > INT32_MAX) return false;
  st->ring_len = (int32_t)ring_len;
  st->max_rounds = (int32_t)max_rounds;
  return true;
}

// One chained speculative round with the on-device commit.
napi_value SpecStep(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  HANDLE_OR_THROW(argv[0], s);
  sas_spec_rows r;
  sas_spec_state st;
  if (!read_spec(env, argv[1], &r) || !read_spec_state(env, argv[2], &st)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad spec step descriptor");
    return nullptr;
  }
  int rc = sas_spec_step(s, &r, &st, sas_stream(s));
  return rc == SAS_OK ? undefined(env) : throw_sas(env, s, rc);
}

// --------------------------------------------------------------- async --

struct AsyncCall {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  napi_ref handle_ref = nullptr;  // keeps the handle's external alive until completion
  Handle *h = nullptr;
  bool verify = false;
  bool step = false;
  bool spec = false;
  bool head = false;
  bool head_step = false;
  bool spec_step = false;
  sas_lm_head hd;
  sas_spec_state sst;
  sas_spec_rows srows;
  sas_rows rows;
  sas_step srow;
  sas_verify_rows vrows;
  int rc = SAS_OK;
  std::string err;
};

void async_execute(napi_env, void *data) {
  AsyncCall *c = static_cast<AsyncCall *>(data);
  std::lock_guard<std::mutex> g(c->h->mu);
  if (c->h->closed) {
    c->rc = SAS_ERR_INVALID;
    c->err = "sampler is closed";
    return;
  }
  sas_sampler *s = c->h->s;
  c->rc = c->verify      ? sas_verify(s, &c->vrows, sas_stream(s))
          : c->head_step ? sas_lm_head_sample_step(s, &c->hd, &c->rows, &c->srow, sas_stream(s))
          : c->spec_step ? sas_spec_step(s, &c->srows, &c->sst, sas_stream(s))
          : c->step      ? sas_sample_step(s, &c->rows, &c->srow, sas_stream(s))
          : c->spec      ? sas_spec_exact(s, &c->srows, sas_stream(s))
          : c->head      ? sas_lm_head_sample(s, &c->hd, &c->rows, sas_stream(s))
                         : sas_sample(s, &c->rows, sas_stream(s));
  if (c->rc == SAS_OK) c->rc = sas_synchronize(s, sas_stream(s));
  if (c->rc != SAS_OK) c->err = sas_last_error(s);
}

void async_complete(napi_env env, napi_status, void *data) {
  AsyncCall *c = static_cast<AsyncCall *>(data);
  if (c->handle_ref) napi_delete_reference(env, c->handle_ref);
  if (c->rc == SAS_OK) {
    napi_resolve_deferred(env, c->deferred, undefined(env));
  } else {
    napi_value err, text, code;
    napi_create_string_utf8(env, c->err.c_str(), NAPI_AUTO_LENGTH, &text);
    napi_create_error(env, nullptr, text, &err);
    napi_create_int32(env, c->rc, &code);
    napi_set_named_property(env, err, "code", code);
    napi_reject_deferred(env, c->deferred, err);
  }
  napi_delete_async_work(env, c->work);
  delete c;
}

napi_value start_async(napi_env env, AsyncCall *c, napi_value handle, const char *name) {
  napi_value promise, rname;
  if (napi_create_reference(env, handle, 1, &c->handle_ref) != napi_ok) {
    delete c;
    return throw_napi(env, "napi_create_reference");
  }
  if (napi_create_promise(env, &c->deferred, &promise) != napi_ok) {
    napi_delete_reference(env, c->handle_ref);
    delete c;
    return throw_napi(env, "napi_create_promise");
  }
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &rname);
  if (napi_create_async_work(env, nullptr, rname, async_execute, async_complete, c, &c->work) != napi_ok ||
      napi_queue_async_work(env, c->work) != napi_ok) {
    napi_delete_reference(env, c->handle_ref);
    delete c;
    return throw_napi(env, "napi_queue_async_work");
  }
  return promise;
}

// The wrapper of an async call's handle, checked open; the worker takes the
// mutex itself.
Handle *open_wrapper(napi_env env, napi_value v) {
  Handle *h = get_wrapper(env, v);
  if (!h) {
    napi_throw_type_error(env, nullptr, "sas_napi: expected a sampler handle");
    return nullptr;
  }
  std::lock_guard<std::mutex> g(h->mu);
  if (h->closed) {
    napi_throw_error(env, nullptr, "sampler is closed");
    return nullptr;
  }
  return h;
}

napi_value SampleAsync(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  if (!read_rows(env, argv[1], &c->rows)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad sample descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_sample");
}

napi_value SampleStepAsync(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  c->step = true;
  if (!read_rows(env, argv[1], &c->rows) || !read_step(env, argv[2], &c->srow)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad sample step descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_sample_step");
}

napi_value LmHeadSampleAsync(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  c->head = true;
  if (!read_rows(env, argv[1], &c->rows) || !read_head(env, argv[2], &c->hd)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad lm head descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_lm_head_sample");
}

napi_value SpecExactAsync(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  c->spec = true;
  if (!read_spec(env, argv[1], &c->srows)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad spec descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_spec_exact");
}

napi_value LmHeadStepAsync(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!args(env, info, 4, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  c->head_step = true;
  if (!read_rows(env, argv[1], &c->rows) || !read_head(env, argv[2], &c->hd) || !read_step(env, argv[3], &c->srow)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad lm head step descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_lm_head_sample_step");
}

napi_value SpecStepAsync(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  c->spec_step = true;
  if (!read_spec(env, argv[1], &c->srows) || !read_spec_state(env, argv[2], &c->sst)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad spec step descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_spec_step");
}

napi_value VerifyAsync(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  Handle *h = open_wrapper(env, argv[0]);
  if (!h) return nullptr;
  AsyncCall *c = new AsyncCall();
  c->h = h;
  c->verify = true;
  if (!read_verify(env, argv[1], &c->vrows)) {
    delete c;
    napi_throw_type_error(env, nullptr, "sas_napi: bad verify descriptor");
    return nullptr;
  }
  return start_async(env, c, argv[0], "sas_verify");
}

// --------------------------------------------------------- host helpers --

napi_value ClampParams(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args(env, info, 1, argv)) return throw_napi(env, "arguments");
  sas_params in, out;
  if (!read_params(env, argv[0], &in)) {
    napi_throw_type_error(env, nullptr, "sas_napi: bad params object");
    return nullptr;
  }
  int rc = sas_clamp_params(&in, &out);
  if (rc != SAS_OK) return throw_sas(env, nullptr, rc);
  return params_object(env, out);
}

// maskFromIds(kind, Uint32Array ids, vocab) -> {words: Uint32Array, allowed: number}
// A content key of a Uint32Array (id list or mask words): FNV-1a style
// 64-bit hashes of its 32-bit values in four interleaved chains, folded
// with its length, as 16 hex digits.
// Equal contents give equal keys; the mask cache confirms a hit by
// comparing the contents.
napi_value IdsKey(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!args(env, info, 1, argv)) return throw_napi(env, "arguments");
  bool is_ta = false;
  napi_is_typedarray(env, argv[0], &is_ta);
  napi_typedarray_type type = napi_int8_array;
  size_t count = 0, off = 0;
  void *data = nullptr;
  napi_value ab;
  if (is_ta) napi_get_typedarray_info(env, argv[0], &type, &count, &data, &ab, &off);
  if (!is_ta || type != napi_uint32_array) {
    napi_throw_type_error(env, nullptr, "sas_napi: expected a Uint32Array");
    return nullptr;
  }
  const uint32_t *v = static_cast<const uint32_t *>(data);
  // four independent chains (the multiplies overlap), folded at the end
  uint64_t c[4] = {0xcbf29ce484222325ull, 0x84222325cbf29ce4ull, 0x9e3779b97f4a7c15ull, 0xbf58476d1ce4e5b9ull};
  size_t i = 0;
  for (; i + 4 <= count; i += 4)
    for (int k = 0; k < 4; ++k) c[k] = (c[k] ^ v[i + k]) * 0x100000001b3ull;
  for (; i < count; ++i) c[0] = (c[0] ^ v[i]) * 0x100000001b3ull;
  uint64_t h = (uint64_t)count * 0x9e3779b97f4a7c15ull;
  for (int k = 0; k < 4; ++k) {
    h ^= c[k] ^ (c[k] >> 29);
    h *= 0x100000001b3ull;
  }
  char buf[17];
  static const char hex[] = "0123456789abcdef";
  for (int i = 15; i >= 0; --i) {
    buf[i] = hex[h & 0xF];
    h >>= 4;
  }
  buf[16] = 0;
  napi_value out;
  napi_create_string_utf8(env, buf, 16, &out);
  return out;
}

// Whether two Uint32Arrays hold the same values.
napi_value U32Equal(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!args(env, info, 2, argv)) return throw_napi(env, "arguments");
  const uint32_t *p[2] = {nullptr, nullptr};
  size_t n[2] = {0, 0};
  for (int k = 0; k < 2; ++k) {
    bool is_ta = false;
    napi_is_typedarray(env, argv[k], &is_ta);
    napi_typedarray_type type = napi_int8_array;
    size_t off = 0;
    void *data = nullptr;
    napi_value ab;
    if (is_ta) napi_get_typedarray_info(env, argv[k], &type, &n[k], &data, &ab, &off);
    if (!is_ta || type != napi_uint32_array) {
      napi_throw_type_error(env, nullptr, "sas_napi: expected two Uint32Arrays");
      return nullptr;
    }
    p[k] = static_cast<const uint32_t *>(data);
  }
  napi_value out;
  napi_get_boolean(env, n[0] == n[1] && (n[0] == 0 || std::memcmp(p[0], p[1], n[0] * 4) == 0), &out);
  return out;
}

napi_value MaskFromIds(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  int32_t kind = 0, vocab = 0;
  NAPI_OK(napi_get_value_int32(env, argv[0], &kind));
  NAPI_OK(napi_get_value_int32(env, argv[2], &vocab));
  const uint32_t *ids = nullptr;
  size_t count = 0;
  napi_valuetype t;
  napi_typeof(env, argv[1], &t);
  if (t != napi_undefined && t != napi_null) {
    bool is_ta = false;
    napi_is_typedarray(env, argv[1], &is_ta);
    napi_typedarray_type type = napi_int8_array;
    void *data = nullptr;
    napi_value ab;
    size_t off;
    if (is_ta) napi_get_typedarray_info(env, argv[1], &type, &count, &data, &ab, &off);
    if (!is_ta || type != napi_uint32_array) {
      napi_throw_type_error(env, nullptr, "sas_napi: ids must be a Uint32Array");
      return nullptr;
    }
    ids = static_cast<const uint32_t *>(data);
  }
  if (vocab < 1 || vocab > SAS_MAX_VOCAB) {
    napi_throw_range_error(env, nullptr, "sas_napi: vocab must be in [1, SAS_MAX_VOCAB]");
    return nullptr;
  }
  const size_t nwords = ((size_t)vocab + 31) / 32;
  napi_value ab, words, result, allowed_v;
  void *wdata = nullptr;
  NAPI_OK(napi_create_arraybuffer(env, nwords * 4, &wdata, &ab));
  NAPI_OK(napi_create_typedarray(env, napi_uint32_array, nwords, ab, 0, &words));
  int64_t allowed = sas_mask_from_ids(kind, ids, count, vocab, static_cast<uint32_t *>(wdata), (int64_t)nwords);
  if (allowed < 0) return throw_sas(env, nullptr, (int)-allowed);
  napi_create_object(env, &result);
  napi_set_named_property(env, result, "words", words);
  napi_create_double(env, (double)allowed, &allowed_v);
  napi_set_named_property(env, result, "allowed", allowed_v);
  return result;
}

napi_value PcgUniform(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!args(env, info, 3, argv)) return throw_napi(env, "arguments");
  uint32_t seed = 0, it = 0, row = 0;
  NAPI_OK(napi_get_value_uint32(env, argv[0], &seed));
  NAPI_OK(napi_get_value_uint32(env, argv[1], &it));
  NAPI_OK(napi_get_value_uint32(env, argv[2], &row));
  napi_value v;
  napi_create_double(env, sas_pcg_uniform(seed, it, row), &v);
  return v;
}

napi_value Init(napi_env env, napi_value exports) {
  const napi_property_descriptor fns[] = {
      {"version", nullptr, Version, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"create", nullptr, Create, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"destroy", nullptr, Destroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"reserve", nullptr, Reserve, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"alloc", nullptr, Alloc, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"free", nullptr, Free, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"copy", nullptr, Copy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"synchronize", nullptr, Synchronize, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sample", nullptr, Sample, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sampleAsync", nullptr, SampleAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sampleStep", nullptr, SampleStep, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sampleStepAsync", nullptr, SampleStepAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHeadSample", nullptr, LmHeadSample, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHeadSampleAsync", nullptr, LmHeadSampleAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHeadStep", nullptr, LmHeadStep, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHeadStepAsync", nullptr, LmHeadStepAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"specStep", nullptr, SpecStep, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"specStepAsync", nullptr, SpecStepAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"verify", nullptr, Verify, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"verifyAsync", nullptr, VerifyAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"specExact", nullptr, SpecExact, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"specExactAsync", nullptr, SpecExactAsync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"clampParams", nullptr, ClampParams, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"maskFromIds", nullptr, MaskFromIds, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"idsKey", nullptr, IdsKey, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"u32Equal", nullptr, U32Equal, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"pcgUniform", nullptr, PcgUniform, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
  };
  napi_define_properties(env, exports, sizeof fns / sizeof fns[0], fns);
  napi_value c;
  const struct {
    const char *name;
    double value;
  } consts[] = {{"MAX_TOP_K", SAS_MAX_TOP_K},       {"MAX_VOCAB", SAS_MAX_VOCAB},
                {"MAX_HISTORY", SAS_MAX_HISTORY},   {"MAX_DRAFT", SAS_MAX_DRAFT},
                {"NO_TOKEN", (double)SAS_NO_TOKEN}, {"MASK_ALL", SAS_MASK_ALL},
                {"MASK_ALLOW", SAS_MASK_ALLOW},     {"MASK_DENY", SAS_MASK_DENY},
                {"FLAG_EMPTY_ROW", SAS_FLAG_EMPTY_ROW}, {"FLAG_TOPP_EDGE", SAS_FLAG_TOPP_EDGE},
                {"FLAG_DRAW_EDGE", SAS_FLAG_DRAW_EDGE}, {"FLAG_SLOW_SELECT", SAS_FLAG_SLOW_SELECT},
                {"HINT_NO_SOFTCAP", SAS_HINT_NO_SOFTCAP}, {"STOP_PAD", (double)SAS_STOP_PAD},
                {"PARAMS_BYTES", (double)sizeof(sas_params)},
                {"LMH_MAX_ROWS", SAS_LMH_MAX_ROWS}, {"LMH_MAX_LDS_FLOATS", SAS_LMH_MAX_LDS_FLOATS},
                {"LMH_MAX_VOCAB", SAS_LMH_MAX_VOCAB}};
  for (const auto &k : consts) {
    napi_create_double(env, k.value, &c);
    napi_set_named_property(env, exports, k.name, c);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(sas_napi, Init)

// host_check.cc - drives every entry point of the C ABI through its host
// paths (argument checks, error messages, host helpers) and, when a HIP
// device exists, through one small call of each device entry point.  Built
// with AddressSanitizer and UndefinedBehaviorSanitizer over the library's
// host code (tests/sanitize/Makefile); any report aborts the run.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>
#include <string>
#include <vector>

#include "shared_amd_sampler.h"

static int g_fail = 0;
#define EXPECT(c)                                                              \
  do {                                                                         \
    if (!(c)) {                                                                \
      std::fprintf(stderr, "host_check: %s:%d: %s\n", __FILE__, __LINE__, #c); \
      ++g_fail;                                                                \
    }                                                                          \
  } while (0)

static bool last_error_has(const sas_sampler *s, const char *what) {
  const char *m = sas_last_error(s);
  return m && std::strstr(m, what) != nullptr;
}

static void host_helpers() {
  EXPECT(std::strstr(sas_version(), "gfx950") != nullptr);
  // clamps: every non-finite and out-of-range input lands in range
  const double nan = std::numeric_limits<double>::quiet_NaN(), inf = std::numeric_limits<double>::infinity();
  const double odd[] = {nan, inf, -inf, -1.0, 0.0, 0.5, 1.0, 3.0, 1e300, -1e-300};
  for (double t : odd)
    for (double q : odd) {
      sas_params in{}, out{};
      in.temperature = t;
      in.top_p = q;
      in.repetition_penalty = t;
      in.presence_penalty = q;
      in.frequency_penalty = t;
      in.softcap = (float)q;
      in.top_k = (int32_t)(std::isfinite(q) ? (int)std::fmin(std::fmax(q, -1e6), 1e6) : 7);
      EXPECT(sas_clamp_params(&in, &out) == SAS_OK);
      EXPECT(out.temperature >= 0.0 && std::isfinite(out.temperature));
      EXPECT(out.top_p >= 0.0 && out.top_p <= 1.0);
      EXPECT(out.presence_penalty >= 0.0 && out.presence_penalty <= 10.0);
      EXPECT(out.top_k >= 1 && out.top_k <= SAS_MAX_TOP_K);
      EXPECT(out.repetition_penalty > 0.0 && std::isfinite(out.repetition_penalty));
      EXPECT(std::isfinite(out.frequency_penalty));
      EXPECT(out.softcap >= 0.0f && std::isfinite(out.softcap));
    }
  EXPECT(sas_clamp_params(nullptr, nullptr) != SAS_OK);
  // masks: every kind, ids past the vocabulary, word counts at the edges
  const int32_t vocabs[] = {1, 31, 32, 33, 1000, 151936};
  for (int32_t v : vocabs) {
    const int64_t nw = (v + 31) / 32;
    std::vector<uint32_t> words(nw + 3, 0xA5A5A5A5u);
    std::vector<uint32_t> ids = {0u, (uint32_t)v - 1, (uint32_t)v, 0xFFFFFFFFu, (uint32_t)v / 2, 0u};
    EXPECT(sas_mask_from_ids(SAS_MASK_ALL, nullptr, 0, v, words.data(), nw) == v);
    const int64_t a = sas_mask_from_ids(SAS_MASK_ALLOW, ids.data(), ids.size(), v, words.data(), nw + 3);
    EXPECT(a >= 1 && a <= 3);
    EXPECT(words[nw] == 0u && words[nw + 2] == 0u);
    const int64_t d = sas_mask_from_ids(SAS_MASK_DENY, ids.data(), ids.size(), v, words.data(), nw);
    EXPECT(d == v - a);
    EXPECT(sas_mask_from_ids(SAS_MASK_ALLOW, ids.data(), ids.size(), v, words.data(), nw - 1) < 0);
    EXPECT(sas_mask_from_ids(7, ids.data(), ids.size(), v, words.data(), nw) < 0);
    EXPECT(sas_mask_from_ids(SAS_MASK_ALLOW, nullptr, 3, v, words.data(), nw) < 0);
    EXPECT(last_error_has(nullptr, "sas_mask_from_ids"));
  }
  EXPECT(sas_mask_from_ids(SAS_MASK_ALL, nullptr, 0, 0, nullptr, 0) < 0);
  EXPECT(sas_mask_from_ids(SAS_MASK_ALL, nullptr, 0, SAS_MAX_VOCAB + 1, nullptr, 0) < 0);
  for (uint32_t s = 0; s < 64; ++s) {
    const double u = sas_pcg_uniform(s * 2654435761u, s, s & 3);
    EXPECT(u >= 0.0 && u < 1.0);
  }
}

static void null_handle_paths() {
  sas_rows r{};
  sas_step st{};
  sas_spec_rows sp{};
  sas_verify_rows v{};
  void *p = nullptr;
  EXPECT(sas_sample(nullptr, &r, nullptr) == SAS_ERR_INVALID);
  EXPECT(last_error_has(nullptr, "handle is NULL"));
  EXPECT(sas_sample_step(nullptr, &r, &st, nullptr) == SAS_ERR_INVALID);
  EXPECT(sas_spec_exact(nullptr, &sp, nullptr) == SAS_ERR_INVALID);
  sas_spec_state sst{};
  EXPECT(sas_spec_step(nullptr, &sp, &sst, nullptr) == SAS_ERR_INVALID);
  EXPECT(sas_verify(nullptr, &v, nullptr) == SAS_ERR_INVALID);
  sas_lm_head lh{};
  EXPECT(sas_lm_head_sample(nullptr, &lh, &r, nullptr) == SAS_ERR_INVALID);
  EXPECT(sas_reserve(nullptr, 1, 1) == SAS_ERR_INVALID);
  sas_reserve_desc rd{};
  rd.rows = 1;
  rd.vocab = 1;
  EXPECT(sas_reserve_for(nullptr, &rd) == SAS_ERR_INVALID);
  EXPECT(sas_alloc(nullptr, 16, &p) == SAS_ERR_INVALID);
  EXPECT(sas_free(nullptr, p) == SAS_ERR_INVALID);
  EXPECT(sas_memcpy(nullptr, &p, &p, 8, 0, nullptr) == SAS_ERR_INVALID);
  EXPECT(sas_synchronize(nullptr, nullptr) == SAS_ERR_INVALID);
  EXPECT(sas_stream(nullptr) == nullptr);
  sas_destroy(nullptr);
  // the handle-free entry point checks its descriptor before any device call
  EXPECT(sas_sample_noalloc(0, nullptr, nullptr) == SAS_ERR_INVALID);
  r.rows = 1;
  r.vocab = 0;
  EXPECT(sas_sample_noalloc(0, &r, nullptr) == SAS_ERR_INVALID);
  EXPECT(last_error_has(nullptr, "vocab"));
  r.vocab = 10;
  r.rows = -1;
  EXPECT(sas_sample_noalloc(0, &r, nullptr) == SAS_ERR_INVALID);
  r.rows = 0;
  EXPECT(sas_sample_noalloc(0, &r, nullptr) == SAS_OK);  // nothing to do
  r.rows = 2;
  EXPECT(sas_sample_noalloc(-1, &r, nullptr) == SAS_ERR_INVALID);  // logits missing
}

// A device buffer owned by the handle, filled from the host.
template <typename T>
static T *upload(sas_sampler *s, const std::vector<T> &h) {
  void *d = nullptr;
  if (sas_alloc(s, h.size() * sizeof(T), &d) != SAS_OK) return nullptr;
  if (sas_memcpy(s, d, h.data(), h.size() * sizeof(T), 0, nullptr) != SAS_OK) return nullptr;
  return static_cast<T *>(d);
}

template <typename T>
static std::vector<T> download(sas_sampler *s, const T *d, size_t n) {
  std::vector<T> h(n);
  EXPECT(sas_memcpy(s, h.data(), d, n * sizeof(T), 1, nullptr) == SAS_OK);
  return h;
}

static void device_paths(sas_sampler *s) {
  const int rows = 6, vocab = 3000, L = 2, seqs = 2;
  std::mt19937 g(7);
  std::normal_distribution<float> nd(0.0f, 3.0f);
  std::vector<float> x((size_t)rows * vocab);
  for (auto &v : x) v = nd(g);
  std::vector<uint32_t> mask((size_t)rows * ((vocab + 31) / 32), 0xFFFFFFFFu);
  for (size_t i = 0; i < mask.size(); i += 3) mask[i] = 0x0F0F0F0Fu;
  std::vector<uint32_t> hist = {1, 2, 3, 40, 40, 41, 2999};
  std::vector<int32_t> offs = {0, 2, 2, 5, 7, 7, 7};
  std::vector<double> u(rows);
  for (int r = 0; r < rows; ++r) u[r] = (r + 0.5) / rows;
  std::vector<sas_params> rp(rows);
  for (int r = 0; r < rows; ++r) {
    sas_params in{};
    in.temperature = r % 3 ? 0.8 : 0.0;
    in.top_p = 0.9;
    in.top_k = 5 + r;
    in.repetition_penalty = 1.2;
    in.presence_penalty = 0.5;
    in.frequency_penalty = 0.1;
    sas_clamp_params(&in, &rp[r]);
  }
  float *dx = upload(s, x);
  uint32_t *dm = upload(s, mask), *dh = upload(s, hist);
  int32_t *doff = upload(s, offs);
  double *du = upload(s, u);
  sas_params *drp = upload(s, rp);
  void *ids = nullptr, *probs = nullptr, *cand = nullptr, *cnt = nullptr, *flg = nullptr;
  EXPECT(sas_alloc(s, rows * 4, &ids) == SAS_OK && sas_alloc(s, rows * SAS_MAX_TOP_K * 8, &probs) == SAS_OK &&
         sas_alloc(s, rows * SAS_MAX_TOP_K * 4, &cand) == SAS_OK && sas_alloc(s, rows * 8, &cnt) == SAS_OK &&
         sas_alloc(s, rows * 4, &flg) == SAS_OK);
  if (!dx || !dm || !dh || !doff || !du || !drp || !ids) {
    ++g_fail;
    return;
  }
  sas_rows r{};
  r.logits = dx;
  r.logits_stride = vocab;
  r.vocab = vocab;
  r.rows = rows;
  r.mask = dm;
  r.mask_stride = (vocab + 31) / 32;
  r.hist_ids = dh;
  r.hist_offsets = doff;
  r.hist_count = (int64_t)hist.size();
  r.uniforms = du;
  r.row_params = drp;
  r.out_ids = (uint32_t *)ids;
  r.out_probs = (double *)probs;
  r.out_cand_ids = (uint32_t *)cand;
  r.out_counts = (int32_t *)cnt;
  r.out_flags = (uint32_t *)flg;
  EXPECT(sas_reserve(s, rows, vocab) == SAS_OK);
  {
    // every shape field of the reserve descriptor, then its range checks
    sas_reserve_desc d{};
    d.rows = rows;
    d.vocab = vocab;
    d.hist_ids = 2048 * (int64_t)rows;
    d.lm_head_rows = 2;
    d.verify_seqs = 3;
    d.verify_draft_len = 4;
    EXPECT(sas_reserve_for(s, &d) == SAS_OK);
    EXPECT(sas_reserve_for(s, nullptr) == SAS_ERR_INVALID);
    sas_reserve_desc b = d;
    b.lm_head_rows = SAS_LMH_MAX_ROWS + 1;
    EXPECT(sas_reserve_for(s, &b) == SAS_ERR_INVALID);
    b = d;
    b.verify_draft_len = 0;
    EXPECT(sas_reserve_for(s, &b) == SAS_ERR_INVALID);
    b = d;
    b.hist_ids = -1;
    EXPECT(sas_reserve_for(s, &b) == SAS_ERR_INVALID);
  }
  EXPECT(sas_sample(s, &r, sas_stream(s)) == SAS_OK);
  EXPECT(sas_synchronize(s, sas_stream(s)) == SAS_OK);
  std::vector<uint32_t> out = download(s, (uint32_t *)ids, rows);
  for (uint32_t t : out) EXPECT(t < (uint32_t)vocab);
  EXPECT(sas_sample_noalloc(0, &r, nullptr) == SAS_OK);
  EXPECT(sas_synchronize(s, nullptr) == SAS_OK);
  EXPECT(download(s, (uint32_t *)ids, rows) == out);
  // every descriptor check, with a live handle
  sas_rows bad = r;
  bad.logits_stride = vocab - 1;
  EXPECT(sas_sample(s, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "logits_stride"));
  bad = r;
  bad.hist_offsets = nullptr;
  EXPECT(sas_sample(s, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "hist_offsets"));
  bad = r;
  bad.uniforms = nullptr;
  EXPECT(sas_sample(s, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "uniforms"));
  bad = r;
  bad.mask_stride = 1;
  EXPECT(sas_sample(s, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "mask_stride"));
  // three decode steps with the token fed back
  std::vector<uint32_t> zeros(rows * 2, 0u), ring(rows * 9, 0u), seeds(rows), stops(rows * 4, SAS_STOP_PAD);
  for (int i = 0; i < rows; ++i) seeds[i] = 11u * i + 1u;
  uint32_t *dst = upload(s, zeros), *dring = upload(s, ring), *dseed = upload(s, seeds), *dstop = upload(s, stops);
  void *sampled = nullptr, *next = nullptr;
  EXPECT(sas_alloc(s, rows * 3 * 4, &sampled) == SAS_OK && sas_alloc(s, rows * 4, &next) == SAS_OK);
  sas_step st{};
  st.state = dst;
  st.sampled = (uint32_t *)sampled;
  st.max_steps = 3;
  st.next_tokens = (uint32_t *)next;
  st.ring = dring;
  st.ring_len = 8;
  st.stop_ids = dstop;
  st.seeds = dseed;
  sas_rows sr = r;
  sr.hist_ids = nullptr;
  sr.hist_offsets = nullptr;
  sr.hist_count = 0;
  sr.uniforms = nullptr;
  for (int i = 0; i < 3; ++i) EXPECT(sas_sample_step(s, &sr, &st, nullptr) == SAS_OK);
  EXPECT(sas_synchronize(s, nullptr) == SAS_OK);
  std::vector<uint32_t> state = download(s, dst, rows * 2);
  for (int i = 0; i < rows; ++i) EXPECT(state[2 * i + 1] == 3u);
  sas_step bst = st;
  bst.ring_len = 0;
  EXPECT(sas_sample_step(s, &sr, &bst, nullptr) == SAS_ERR_INVALID && last_error_has(s, "ring_len"));
  EXPECT(sas_sample_step(s, &r, &st, nullptr) == SAS_ERR_INVALID && last_error_has(s, "hist_ids"));
  // one exact-match speculative round: rows 0..5 are 2 sequences x 3 verify rows
  std::vector<float> dr((size_t)seqs * L * vocab);
  for (auto &v : dr) v = nd(g);
  float *ddr = upload(s, dr);
  void *dids = nullptr, *picks = nullptr, *acc = nullptr;
  EXPECT(sas_alloc(s, seqs * L * 4, &dids) == SAS_OK && sas_alloc(s, seqs * (L + 1) * 4, &picks) == SAS_OK &&
         sas_alloc(s, seqs * 4, &acc) == SAS_OK);
  sas_spec_rows sp{};
  sp.target_logits = dx;
  sp.draft_logits = ddr;
  sp.logits_stride = vocab;
  sp.vocab = vocab;
  sp.seqs = seqs;
  sp.draft_len = L;
  sp.draft_ids = (uint32_t *)dids;
  sp.hist_ids = dh;
  sp.hist_offsets = doff;
  sp.hist_count = (int64_t)hist.size();
  sp.params = rp[1];
  sp.seeds = dseed;
  sp.round = 3;
  sp.stop_ids = dstop;
  sp.out_picks = (uint32_t *)picks;
  sp.out_accepted = (int32_t *)acc;
  EXPECT(sas_spec_exact(s, &sp, nullptr) == SAS_OK);
  EXPECT(sas_synchronize(s, nullptr) == SAS_OK);
  for (int32_t a : download(s, (int32_t *)acc, seqs)) EXPECT(a >= 1 && a <= L + 1);
  sas_spec_rows bsp = sp;
  bsp.draft_len = SAS_MAX_DRAFT + 1;
  EXPECT(sas_spec_exact(s, &bsp, nullptr) == SAS_ERR_INVALID && last_error_has(s, "draft_len"));
  bsp = sp;
  bsp.seeds = nullptr;
  EXPECT(sas_spec_exact(s, &bsp, nullptr) == SAS_ERR_INVALID && last_error_has(s, "required"));
  {
    // a chained round over the same rows: state, ring, log and next tokens
    // in device memory, then its argument checks
    std::vector<uint32_t> st0((size_t)seqs * 4, 0u), ring0((size_t)seqs * 9, 0u);
    uint32_t *cst = upload(s, st0), *dring = upload(s, ring0);
    void *dlog = nullptr, *dnext = nullptr;
    EXPECT(sas_alloc(s, (size_t)seqs * 2 * (L + 2) * 4, &dlog) == SAS_OK && sas_alloc(s, seqs * 4, &dnext) == SAS_OK);
    sas_spec_state cs{};
    cs.state = cst;
    cs.ring = dring;
    cs.ring_len = 8;
    cs.log = (uint32_t *)dlog;
    cs.max_rounds = 2;
    cs.next_tokens = (uint32_t *)dnext;
    sas_spec_rows csp = sp;
    csp.hist_ids = nullptr;
    csp.hist_offsets = nullptr;
    csp.hist_count = 0;
    EXPECT(sas_spec_step(s, &csp, &cs, nullptr) == SAS_OK);
    EXPECT(sas_spec_step(s, &csp, &cs, nullptr) == SAS_OK);
    EXPECT(sas_synchronize(s, nullptr) == SAS_OK);
    std::vector<uint32_t> st1 = download(s, cst, (size_t)seqs * 4);
    for (int32_t q = 0; q < seqs; ++q) EXPECT(st1[4 * q + 1] == 2u);  // two rounds
    EXPECT(sas_spec_step(s, &csp, nullptr, nullptr) == SAS_ERR_INVALID && last_error_has(s, "state"));
    EXPECT(sas_spec_step(s, &sp, &cs, nullptr) == SAS_ERR_INVALID && last_error_has(s, "ring is the history"));
    sas_spec_state bad = cs;
    bad.ring_len = 0;
    EXPECT(sas_spec_step(s, &csp, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "ring_len"));
    bad = cs;
    bad.max_rounds = 0;
    EXPECT(sas_spec_step(s, &csp, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "max_rounds"));
    bad = cs;
    bad.state = nullptr;
    EXPECT(sas_spec_step(s, &csp, &bad, nullptr) == SAS_ERR_INVALID && last_error_has(s, "state is required"));
    EXPECT(sas_free(s, cst) == SAS_OK && sas_free(s, dring) == SAS_OK && sas_free(s, dlog) == SAS_OK &&
           sas_free(s, dnext) == SAS_OK);
  }
  // rejection-sampling verify over the same rows
  std::vector<double> vu((size_t)seqs * (L + 1) * 2);
  for (size_t i = 0; i < vu.size(); ++i) vu[i] = (i + 0.25) / vu.size();
  double *dvu = upload(s, vu);
  void *vtok = nullptr, *vacc = nullptr;
  EXPECT(sas_alloc(s, seqs * (L + 1) * 4, &vtok) == SAS_OK && sas_alloc(s, seqs * 4, &vacc) == SAS_OK);
  sas_verify_rows v{};
  v.target_logits = dx;
  v.draft_logits = ddr;
  v.logits_stride = vocab;
  v.vocab = vocab;
  v.seqs = seqs;
  v.draft_len = L;
  v.draft_ids = (uint32_t *)dids;
  v.uniforms = dvu;
  v.temperature = 1.0;
  v.out_tokens = (uint32_t *)vtok;
  v.out_accepted = (int32_t *)vacc;
  EXPECT(sas_verify(s, &v, nullptr) == SAS_OK);
  EXPECT(sas_synchronize(s, nullptr) == SAS_OK);
  for (int32_t a : download(s, (int32_t *)vacc, seqs)) EXPECT(a >= 0 && a <= L);
  v.temperature = 0.0;
  EXPECT(sas_verify(s, &v, nullptr) == SAS_ERR_INVALID);
  // the LM head with the sampling step fused: the first 3 rows over a
  // 64-wide head (bf16 bits of small values)
  const int lrows = 3, dim = 256;
  std::vector<float> hid((size_t)lrows * dim);
  for (auto &e : hid) e = nd(g) * 0.1f;
  std::vector<uint16_t> wt((size_t)vocab * dim);
  for (auto &e : wt) {
    const float f = nd(g) * 0.05f;
    uint32_t b;
    std::memcpy(&b, &f, 4);
    e = (uint16_t)(b >> 16);
  }
  float *dhid = upload(s, hid);
  uint16_t *dwt = upload(s, wt);
  void *lgt = nullptr;
  EXPECT(sas_alloc(s, (size_t)lrows * vocab * 4, &lgt) == SAS_OK);
  sas_lm_head lh{};
  lh.hidden = dhid;
  lh.hidden_stride = dim;
  lh.weight = dwt;
  lh.weight_stride = dim;
  lh.dim = dim;
  lh.out_logits = (float *)lgt;
  sas_rows lr = r;
  lr.logits = nullptr;
  lr.rows = lrows;
  EXPECT(sas_lm_head_sample(s, &lh, &lr, nullptr) == SAS_OK);
  EXPECT(sas_synchronize(s, nullptr) == SAS_OK);
  for (uint32_t t : download(s, (uint32_t *)ids, lrows)) EXPECT(t < (uint32_t)vocab);
  sas_rows blr = lr;
  blr.logits = dx;
  EXPECT(sas_lm_head_sample(s, &lh, &blr, nullptr) == SAS_ERR_INVALID && last_error_has(s, "NULL"));
  blr = lr;
  blr.rows = SAS_LMH_MAX_ROWS + 1;
  EXPECT(sas_lm_head_sample(s, &lh, &blr, nullptr) == SAS_ERR_INVALID && last_error_has(s, "rows"));
  sas_lm_head blh = lh;
  blh.dim = 320;
  EXPECT(sas_lm_head_sample(s, &blh, &lr, nullptr) == SAS_ERR_INVALID && last_error_has(s, "dim"));
  blh = lh;
  blh.weight_stride = 258;
  EXPECT(sas_lm_head_sample(s, &blh, &lr, nullptr) == SAS_ERR_INVALID && last_error_has(s, "weight_stride"));
  for (void *q : {(void *)dhid, (void *)dwt, lgt}) EXPECT(sas_free(s, q) == SAS_OK);
  for (void *q : {(void *)dx, (void *)dm, (void *)dh, (void *)doff, (void *)du, (void *)drp, ids, probs, cand, cnt,
                  flg, (void *)dst, (void *)dring, (void *)dseed, (void *)dstop, sampled, next, (void *)ddr, dids, picks,
                  acc, (void *)dvu, vtok, vacc})
    EXPECT(sas_free(s, q) == SAS_OK);
}

int main() {
  host_helpers();
  std::printf("[host_check] host helpers done\n");
  null_handle_paths();
  std::printf("[host_check] handle-free error paths done\n");
  sas_sampler *s = nullptr;
  if (sas_create(0, &s) != SAS_OK) {
    EXPECT(s == nullptr && sas_last_error(nullptr) != nullptr);
    std::printf("[host_check] no HIP device (%s): device paths skipped\n", sas_last_error(nullptr));
  } else {
    device_paths(s);
    sas_destroy(s);
    std::printf("[host_check] device paths done\n");
  }
  std::printf("[host_check] %s (%d failed expectations)\n", g_fail ? "FAILED" : "ok", g_fail);
  return g_fail ? 1 : 0;
}

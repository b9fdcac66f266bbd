"""CPU tests that pin the oracle (oracle/sampler_oracle.c) before it is
trusted as the GPU path's checker.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign or index, a transposed comparison, a different rounding
order) fails it:

* exp against V8's own Math.exp outputs (tests/golden/v8_math_exp.json,
  written by tests/golden/make_v8_exp.js) - the engine the reference's
  sample() (lib/webgpu-llm/tokenizer.js:165) runs on;
* sample() semantics (tokenizer.js:151-178) against answers derived by hand
  from the closed forms (logistic weights, the top-p cut, the draw bound);
* the bounded-heap selection against a full sort (brute force);
* the draw against its exact distribution over a fine grid of uniforms;
* the whole row pipeline against the independent Node restatement
  (oracle/sample_js.js, a different two-stage structure) run on V8;
* rejection-sampling verify against the properties that fix it.
"""
import json
import math
import os
import struct

import numpy as np
import pytest

import oracle as O
from shared_amd import Params
from shared_amd import workloads as W

HERE = os.path.dirname(os.path.abspath(__file__))


def _bits(x: float) -> bytes:
    return struct.pack(">d", x)


# -------------------------------------------------------------------- exp --

def test_exp_matches_v8_math_exp_bit_for_bit():
    with open(os.path.join(HERE, "golden", "v8_math_exp.json")) as f:
        cases = json.load(f)["cases"]
    assert len(cases) > 5000
    exp = O.lib().orc_exp
    bad = []
    for xin, yout in cases:
        x = struct.unpack(">d", bytes.fromhex(xin))[0]
        y = struct.unpack(">d", bytes.fromhex(yout))[0]
        z = exp(x)
        if math.isnan(y):
            ok = math.isnan(z)
        else:
            ok = _bits(z) == _bits(y)
        if not ok:
            bad.append((x, y, z))
    assert not bad, f"{len(bad)} mismatches, first {bad[:3]}"


def test_exp_against_libm_within_one_ulp():
    rng = np.random.default_rng(0)
    exp = O.lib().orc_exp
    for x in np.concatenate([rng.uniform(-700, 700, 2000), -rng.exponential(3.0, 2000)]):
        y, z = math.exp(x), exp(float(x))
        assert abs(z - y) <= math.ulp(y), (x, y, z)
    assert exp(0.0) == 1.0 and exp(-math.inf) == 0.0 and exp(math.inf) == math.inf
    assert math.isnan(exp(math.nan))


# ------------------------------------------------------- sample() by hand --

def _row(logits, p, *, mask_ids=None, hist=None, u=0.0, mode=0):
    x = np.asarray(logits, np.float32)
    mask = None
    if mask_ids is not None:
        bits = np.zeros((1, x.size), bool)
        bits[0, list(mask_ids)] = True
        mask = W.pack_bits(bits)[0]
    h = None if hist is None else np.asarray(hist, np.uint32)
    return O.sample_row(x, p, mask=mask, hist=h, uniform=u, select_mode=mode)


LOG4 = [1.0, 3.0, 2.0, -1.0]          # ranked: id1 (3), id2 (2), id0 (1), id3 (-1)


def test_softmax_weights_and_topp_cut_closed_form():
    r = _row(LOG4, Params(temperature=1.0, top_k=3, top_p=0.9), u=0.5)
    w = [1.0, math.exp(-1.0), math.exp(-2.0)]
    s = sum(w)
    assert (r.k, r.cut) == (3, 2)          # 0.665 < 0.9 <= 0.665 + 0.245
    assert list(r.cand_ids[:3]) == [1, 2, 0]
    for i in range(3):
        assert abs(r.probs[i] - w[i] / s) <= 2e-16
    # temperature divides the logit gaps
    r = _row(LOG4, Params(temperature=0.5, top_k=4, top_p=1.0))
    w = [1.0, math.exp(-2.0), math.exp(-4.0), math.exp(-8.0)]
    for i in range(4):
        assert abs(r.probs[i] - w[i] / sum(w)) <= 2e-16


def test_draw_boundary_is_the_logistic_of_the_gap():
    # with cut = 2 the draw picks id1 iff U * (1 + e^-1) - 1 <= 0, i.e.
    # U <= 1 / (1 + e^-1) = 0.7310585...
    p = Params(temperature=1.0, top_k=3, top_p=0.9)
    edge = 1.0 / (1.0 + math.exp(-1.0))
    assert _row(LOG4, p, u=0.0).id == 1
    assert _row(LOG4, p, u=edge - 1e-9).id == 1
    assert _row(LOG4, p, u=edge + 1e-9).id == 2
    assert _row(LOG4, p, u=0.999999).id == 2


def test_greedy_topk1_and_topp0_take_the_best():
    for p in [Params(temperature=0.0), Params(temperature=-1.0), Params(temperature=1.0, top_k=1),
              Params(temperature=1.0, top_k=4, top_p=0.0)]:
        for u in (0.0, 0.5, 0.99):
            assert _row(LOG4, p, u=u).id == 1


def test_ties_take_the_lowest_id():
    assert _row([2.0, 2.0, 1.0], Params(temperature=0.0)).id == 0
    r = _row([5.0, 7.0, 7.0, 7.0, 1.0], Params(temperature=1.0, top_k=2, top_p=1.0))
    assert list(r.cand_ids[:2]) == [1, 2]
    assert r.probs[0] == r.probs[1] == 0.5


def test_mask_excludes_ids_and_empty_row_has_no_token():
    assert _row(LOG4, Params(temperature=0.0), mask_ids=[0, 3]).id == 0
    assert _row(LOG4, Params(temperature=0.0), mask_ids=[3]).id == 3
    r = _row(LOG4, Params(temperature=1.0, top_k=5), mask_ids=[])
    assert r.id == O.NO_TOKEN and r.flags & 1
    # fewer allowed ids than top_k: k shrinks to the allowed count
    r = _row(LOG4, Params(temperature=1.0, top_k=20), mask_ids=[0, 2])
    assert r.k == 2 and list(r.cand_ids[:2]) == [2, 0]


def test_presence_penalty_as_tokenizer_js_157():
    # v -= pp for ids in the recent set: 3 - 2.5 = 0.5 drops below id2 and id0
    assert _row(LOG4, Params(temperature=0.0, presence_penalty=2.5), hist=[1]).id == 2
    # a repeated id is penalised once by presence
    assert _row(LOG4, Params(temperature=0.0, presence_penalty=0.9), hist=[1, 1, 1]).id == 1


def test_repetition_and_frequency_penalties():
    # CTRL repetition: positive logits divide, negative multiply
    assert _row(LOG4, Params(temperature=0.0, repetition_penalty=2.0), hist=[1]).id == 2   # 1.5 < 2
    assert _row(LOG4, Params(temperature=0.0, repetition_penalty=1.4), hist=[1]).id == 1   # 2.14 > 2
    r = _row([-1.0, -2.0], Params(temperature=1.0, top_k=2, repetition_penalty=3.0), hist=[0])
    assert list(r.cand_ids[:2]) == [1, 0]                    # -3 < -2
    # frequency: count 3 * 0.4 = 1.2 -> 1.8 < 2
    assert _row(LOG4, Params(temperature=0.0, frequency_penalty=0.4), hist=[1, 1, 1]).id == 2
    assert _row(LOG4, Params(temperature=0.0, frequency_penalty=0.4), hist=[1, 1]).id == 1


def test_penalty_order_closed_form():
    # repetition first, then frequency, then presence, for positive, negative
    # and zero logits; operands exact in binary so every result is exact.
    # Another order gives another value: e.g. v=3 with frequency and
    # presence first is (3 - 1 - 0.25) / 2 = 0.875, not 0.25.
    pen = O.lib().orc_penalize
    p = O.params(Params(repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25))
    assert pen(3.0, 2, p) == 0.25          # 3 / 2 - 0.5 * 2 - 0.25
    assert pen(-3.0, 2, p) == -7.25        # -3 * 2 - 1 - 0.25
    assert pen(0.0, 2, p) == -1.25         # 0 is not > 0: 0 * 2 - 1 - 0.25
    assert pen(3.0, 1, p) == 0.75          # 1.5 - 0.5 - 0.25
    q = O.params(Params(repetition_penalty=4.0, frequency_penalty=0.25, presence_penalty=0.5))
    assert pen(4.0, 4, q) == -0.5          # 4 / 4 - 1 - 0.5
    assert pen(-0.5, 4, q) == -3.5         # -0.5 * 4 - 1 - 0.5
    # through a whole row: the penalized id drops below 0.26 but stays above 0.24
    pp = Params(temperature=0.0, repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25)
    assert _row([3.0, 0.26, 0.1], pp, hist=[0, 0]).id == 1
    assert _row([3.0, 0.24, 0.1], pp, hist=[0, 0]).id == 0
    assert _row([-3.0, -7.2, -9.0], pp, hist=[0, 0]).id == 1
    assert _row([-3.0, -7.3, -9.0], pp, hist=[0, 0]).id == 0


def test_penalty_invariants():
    pen = O.lib().orc_penalize
    rng = np.random.default_rng(1)
    ident = O.params(Params())
    for v in rng.standard_normal(200) * 5:
        for c in (1, 2, 7):
            assert pen(float(v), c, ident) == float(v)     # r=1, f=0, p=0 is the identity
    p = O.params(Params(repetition_penalty=1.3, frequency_penalty=0.2, presence_penalty=0.5))
    for v in rng.standard_normal(200) * 5:
        assert pen(float(v), 0, p) == float(v)            # ids outside the history are untouched
        a, b = pen(float(v), 1, p), pen(float(v), 2, p)
        assert b < a < float(v) + 1e-12                    # more occurrences, lower value
    lo = O.params(Params(repetition_penalty=1.1))
    hi = O.params(Params(repetition_penalty=1.5))
    for v in rng.standard_normal(200) * 5:
        assert pen(float(v), 1, hi) <= pen(float(v), 1, lo)  # monotone in r


def test_tanh_is_correctly_rounded_fp32():
    # the double evaluation rounded once to fp32 equals the correctly rounded
    # tanh (math.tanh in double, rounded to fp32) except within double
    # rounding error of an fp32 rounding boundary
    rng = np.random.default_rng(2)
    xs = np.concatenate([rng.standard_normal(20000) * 2, rng.standard_normal(2000) * 1e-3,
                         [0.0, -0.0, 1e-30, -1e-30, 9.4, 9.6, 20.0, -20.0, np.inf, -np.inf]]).astype(np.float32)
    tanhf = O.lib().orc_tanhf
    off = 0
    for x in xs:
        want = np.float32(math.tanh(float(x)))
        got = np.float32(tanhf(float(x)))
        d = abs(int(got.view(np.int32)) - int(want.view(np.int32)))
        assert d <= 1, (x, got, want)
        off += d
    assert off <= 2
    assert math.copysign(1.0, tanhf(-0.0)) == -1.0 and math.isnan(tanhf(math.nan))


def test_softcap_is_cap_tanh_of_the_fp32_quotient():
    cap = np.float32(30.0)
    xs = np.random.default_rng(3).standard_normal(3000).astype(np.float32) * np.float32(40)
    for x in xs:
        q = np.float32(x / cap)
        want = np.float32(cap * np.float32(O.lib().orc_tanhf(float(q))))
        assert np.float32(O.lib().orc_softcap(float(x), 30.0)) == want
        assert abs(float(want) - 30.0 * math.tanh(float(x) / 30.0)) <= 4e-6 * 30.0


# --------------------------------------------------- selection and draws --

def test_heap_selection_equals_full_sort_with_ties():
    rng = np.random.default_rng(3)
    for trial in range(60):
        vocab = int(rng.integers(1, 3000))
        x = rng.integers(-3, 4, vocab).astype(np.float32) * np.float32(0.5)   # heavy ties
        x[rng.random(vocab) < 0.05] = np.nan
        p = Params(temperature=float(rng.choice([0.0, 0.7, 1.3])), top_k=int(rng.integers(1, 129)),
                   top_p=float(rng.choice([0.5, 0.9, 1.0])), presence_penalty=float(rng.choice([0.0, 0.5])),
                   repetition_penalty=float(rng.choice([1.0, 1.2])))
        mask = None
        if trial % 2:
            mask = W.pack_bits((rng.random((1, vocab)) < 0.3))[0]
        hist = rng.integers(0, vocab, int(rng.integers(0, 40))).astype(np.uint32)
        u = float(rng.random())
        a = O.sample_row(x, p, mask=mask, hist=hist, uniform=u, select_mode=0)
        b = O.sample_row(x, p, mask=mask, hist=hist, uniform=u, select_mode=1)
        assert (a.id, a.k, a.cut, a.flags) == (b.id, b.k, b.cut, b.flags)
        assert list(a.cand_ids[:a.k]) == list(b.cand_ids[:b.k])
        assert list(a.probs[:a.k]) == list(b.probs[:b.k])


def test_draw_frequencies_match_the_cut_distribution():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(64) * 2).astype(np.float32)
    p = Params(temperature=0.8, top_k=10, top_p=0.8)
    n = 20000
    counts = {}
    for i in range(n):
        r = O.sample_row(x, p, uniform=(i + 0.5) / n)
        counts[r.id] = counts.get(r.id, 0) + 1
    ref = O.sample_row(x, p, uniform=0.5)
    q = np.array(ref.probs[:ref.cut]) / sum(ref.probs[:ref.cut])
    ids = list(ref.cand_ids[:ref.cut])
    assert set(counts) <= set(ids)
    for i, t in zip(ids, q):
        assert abs(counts.get(i, 0) / n - t) <= 2.0 / n


# ------------------------------------------------ Node restatement on V8 --

@pytest.mark.skipif(O.node_binary() is None, reason="node is not installed")
@pytest.mark.parametrize("case", range(4))
def test_node_restatement_agrees_bit_for_bit(case):
    rng = np.random.default_rng(10 + case)
    rows, vocab = 6, int(rng.choice([1000, 2049, 5000, 7777]))
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    x[:, rng.integers(0, vocab, 5)] += np.float32(8)
    params = [Params(temperature=0.7, top_k=40, top_p=0.95),
              Params(temperature=1.0, top_k=50, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.5,
                     frequency_penalty=0.3),
              Params(temperature=0.0, repetition_penalty=1.15),
              Params(temperature=1.3, top_k=128, top_p=1.0, softcap=30.0)][case]
    mask = W.random_mask(rng, rows, vocab, 0.05, 0.6) if case in (1, 3) else None
    hi, ho = W._csr([rng.integers(0, vocab, 300) for _ in range(rows)]) if case in (1, 2) else (None, None)
    b = W.Batch("node", x, params, mask=mask, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
    js, _ = O.run_node(b)
    c = O.sample_rows(b)
    assert np.array_equal(js["ids"], c["ids"])
    assert np.array_equal(js["counts"], c["counts"])
    assert np.array_equal(js["cand_ids"], c["cand_ids"])
    assert np.array_equal(js["probs"].view(np.uint64), c["probs"].view(np.uint64))


# ------------------------------------------------------------------- mask --

def test_mask_from_ids_brute_force():
    rng = np.random.default_rng(5)
    for vocab in (1, 31, 32, 33, 1000, 4099):
        ids = rng.integers(0, vocab + 40, 50).astype(np.uint32)   # includes ids >= vocab
        for kind in (0, 1, 2):
            w = O.mask_from_ids(kind, ids, vocab)
            bits = np.unpackbits(w.view(np.uint8), bitorder="little")
            want = np.zeros(w.size * 32, np.uint8)
            listed = ids[ids < vocab]
            if kind == 0:
                want[:vocab] = 1
            elif kind == 1:
                want[listed] = 1
            else:
                want[:vocab] = 1
                want[listed] = 0
            assert np.array_equal(bits, want), (vocab, kind)


# ----------------------------------------------------------------- verify --

def _verify_inp(target, draft, draft_ids, u, mask=None, T=1.0):
    t = np.asarray(target, np.float32)
    L = len(draft_ids)
    return {"target": t.reshape(L + 1, -1), "draft": np.asarray(draft, np.float32).reshape(L, -1),
            "mask": mask, "draft_ids": np.asarray([draft_ids], np.uint32),
            "uniforms": np.asarray(u, np.float64).reshape(1, L + 1, 2), "temperature": T,
            "vocab": t.size // (L + 1), "seqs": 1, "drafts": L}


def test_verify_accepts_always_when_draft_equals_target():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((3, 50)) * 2).astype(np.float32)
    for trial in range(50):
        d = [int(i) for i in rng.integers(0, 50, 2)]
        u = rng.random((3, 2))
        out = O.verify(_verify_inp(x, x[:2], d, u))
        assert out["accepted"][0] == 2 and list(out["tokens"][0, :2]) == d


def test_verify_one_hot_draft_accepts_with_target_probability():
    rng = np.random.default_rng(7)
    V = 16
    t = (rng.standard_normal((2, V))).astype(np.float32)
    d = 5
    q = np.full((1, V), -1000.0, np.float32)
    q[0, d] = 10.0                                   # q(d) = 1 in double
    w = np.exp(t[0].astype(np.float64) - t[0].max())
    pd = w[d] / w.sum()
    n = 4000
    acc = sum(O.verify(_verify_inp(t, q, [d], [[(i + 0.5) / n, 0.5], [0.5, 0.5]]))["accepted"][0]
              for i in range(n))
    assert abs(acc / n - pd) <= 1.5 / n


def test_verify_output_marginal_equals_target():
    # P(token at position 0) = sum_d q(d) [a_d 1{d} + (1 - a_d) residual_d] = p,
    # with the acceptance a_d and the residual draw measured on uniform grids
    rng = np.random.default_rng(8)
    V = 6
    t = (rng.standard_normal((2, V)) * 1.5).astype(np.float32)
    dl = (rng.standard_normal((1, V)) * 1.5).astype(np.float32)
    p = np.exp(t[0].astype(np.float64) - t[0].max()); p /= p.sum()
    q = np.exp(dl[0].astype(np.float64) - dl[0].max()); q /= q.sum()
    g = 400
    grid = (np.arange(g) + 0.5) / g
    marg = np.zeros(V)
    for d in range(V):
        acc = np.mean([O.verify(_verify_inp(t, dl, [d], [[u, 0.5], [0.5, 0.5]]))["accepted"][0] for u in grid])
        marg[d] += q[d] * acc
        if acc < 1.0:
            for u2 in grid:
                tok = O.verify(_verify_inp(t, dl, [d], [[1.0 - 1e-12, u2], [0.5, 0.5]]))["tokens"][0, 0]
                marg[tok] += q[d] * (1.0 - acc) / g
    assert np.abs(marg - p).max() < 4.0 / g


# ------------------------------------------ exact-match speculative round --

def _spec_inp(target, L, *, draft=None, draft_ids=None, stop=None, seeds=None, rnd=0, params=None, hist=None):
    seqs = target.shape[0] // (L + 1)
    inp = {"target": target, "draft": draft, "draft_ids": draft_ids, "vocab": target.shape[1], "seqs": seqs,
           "drafts": L, "seeds": np.zeros(seqs, np.uint32) if seeds is None else np.asarray(seeds, np.uint32),
           "round": rnd, "params": params or Params()}
    if stop is not None:
        st = np.full((seqs, 4), 0xFFFFFFFF, np.uint32)
        for s, ids in enumerate(stop):
            st[s, :len(ids)] = ids
        inp["stop_ids"] = st
    if hist is not None:
        inp["hist_ids"], inp["hist_offsets"] = W._csr(hist)
    return inp


def test_spec_drafts_are_the_first_argmax():
    """argmaxMerge (kernels.js:373-401): the draft is the largest value of
    the draft row, the lowest id among equal maxima, NaNs never chosen."""
    rng = np.random.default_rng(3)
    L, V = 3, 700
    draft = rng.standard_normal((L, V)).astype(np.float32)
    draft[0, [9, 4, 600]] = 8.0           # a three-way tie: id 4
    draft[1, 17] = np.nan
    draft[1, 30] = 9.0
    draft[2, :] = np.nan
    draft[2, [650, 651]] = [-1.0, 2.0]    # only two real values
    target = rng.standard_normal((L + 1, V)).astype(np.float32)
    o = O.spec_exact(_spec_inp(target, L, draft=draft))
    want = []
    for j in range(L):
        z = np.where(np.isnan(draft[j]), -np.inf, draft[j])
        want.append(int(np.argmax(z)))  # numpy returns the first maximum
    assert o["draft_ids"][0].tolist() == want == [4, 30, 651]


def test_spec_cascade_closed_form():
    """kernels.js:328-339: a = 1, next = pick 0; each draft equal to the
    pick before it (and not a stop id) accepts the next pick."""
    L, V = 3, 256
    picks = [5, 6, 7, 8]
    target = np.zeros(((L + 1) * 4, V), np.float32)
    for s in range(4):
        for j, t in enumerate(picks):
            target[s * (L + 1) + j, t] = 50.0   # every draw takes this id
    drafts = np.array([[5, 6, 9], [1, 6, 7], [5, 6, 7], [5, 6, 7]], np.uint32)
    stop = [[], [], [], [6]]
    p = Params(temperature=1.0, top_k=10, top_p=0.9)
    o = O.spec_exact(_spec_inp(target, L, draft_ids=drafts, stop=stop, params=p, seeds=[1, 2, 3, 4], rnd=7))
    assert o["picks"].tolist() == [picks] * 4
    # accepted drafts 5, 6 then 9 != 7; none; all three (bonus 8); 6 is a stop id
    assert o["accepted"].tolist() == [3, 1, 4, 2]
    assert o["next"].tolist() == [7, 5, 8, 6]


def test_spec_draws_use_the_row_uniform():
    """Verify row j draws with (pcg(seed ^ round 0x9E3779B9 ^ j 0x85EBCA6B)
    & 0xFFFFFF) / 2^24 (kernels.js:320): between two equal logits at
    T = 1 the lower id is drawn iff U <= 1/2."""
    def pcg(x):
        h = (x * 747796405 + 2891336453) & 0xFFFFFFFF
        h = (((h >> ((h >> 28) + 4)) ^ h) * 277803737) & 0xFFFFFFFF
        return ((h >> 22) ^ h) & 0xFFFFFFFF

    L, V, seqs = 2, 64, 40
    target = np.full((seqs * (L + 1), V), -30.0, np.float32)
    target[:, [10, 20]] = 1.0
    seeds = (np.arange(seqs, dtype=np.uint64) * 2654435761 % (2**32)).astype(np.uint32)
    rnd = 11
    o = O.spec_exact(_spec_inp(target, L, draft_ids=np.zeros((seqs, L), np.uint32), seeds=seeds, rnd=rnd,
                               params=Params(temperature=1.0, top_k=2, top_p=1.0)))
    for s in range(seqs):
        for j in range(L + 1):
            x = (int(seeds[s]) ^ ((rnd * 0x9E3779B9) & 0xFFFFFFFF) ^ ((j * 0x85EBCA6B) & 0xFFFFFFFF)) & 0xFFFFFFFF
            u = (pcg(x) & 0xFFFFFF) / 16777216.0
            assert o["picks"][s, j] == (10 if u <= 0.5 else 20), (s, j, u)


def test_spec_history_is_the_rounds_start_for_every_row():
    """Every verify row is penalized by the sequence's history as it was at
    the round's start (kernels.js:279-290): a presence penalty moves all
    three rows off the history id alike."""
    L, V = 2, 128
    target = np.zeros((L + 1, V), np.float32)
    target[:, 3] = 5.0
    target[:, 4] = 4.5
    p = Params(temperature=0.0, presence_penalty=1.0)
    o = O.spec_exact(_spec_inp(target, L, draft_ids=np.array([[4, 4]], np.uint32), params=p, hist=[[3, 3, 9]]))
    assert o["picks"].tolist() == [[4, 4, 4]]
    assert o["accepted"].tolist() == [3]


def test_spec_commit_hand_derived_chain():
    """acceptSpec's commit (kernels.js:340-367) over planted rounds whose
    results are worked out by hand: the log entry {a, next, d0, d1}, pos += a,
    accepted = a, pick[0 .. a) appended to a ring of 3 that wraps, a stop id
    that ends the cascade is not appended and freezes the sequence, a frozen
    round logs {0, first stop id, 0, 0} and changes nothing else, and a round
    past max_rounds is not logged."""
    pad = 0xFFFFFFFF
    stops = np.array([[99, pad, pad, pad], [pad] * 4, [77, pad, pad, pad]], np.uint32)
    state = np.array([[0, 0, 10, 0], [0, 0, 0, 0], [1, 5, 20, 2]], np.uint32)
    ring = np.array([[2, 1, 2, 0], [0, 0, 0, 0], [1, 55, 0, 0]], np.uint32)
    log = np.full((3, 4, 4), 7, np.uint32)
    # round 0: seq 0 accepts both drafts (a = 3), seq 1 misses its first (a = 1)
    nxt, acc = O.spec_commit([[5, 6, 7], [4, 9, 9], [1, 2, 3]], [[5, 6], [3, 9], [1, 2]], [3, 1, 3], stops, state,
                             ring, log)
    assert nxt.tolist() == [7, 4, 77] and acc.tolist() == [3, 1, 0]
    assert log[0, 0].tolist() == [3, 7, 5, 6] and log[1, 0].tolist() == [1, 4, 3, 9]
    assert (log[2] == 7).all()                       # round 5 of seq 2: past max_rounds, not logged
    # ring of seq 0: count 2 -> slots 2, 0, 1 take 5, 6, 7
    assert ring[0].tolist() == [5, 6, 7, 5] and ring[1].tolist() == [1, 4, 0, 0]
    assert ring[2].tolist() == [1, 55, 0, 0]
    assert state.tolist() == [[0, 1, 13, 3], [0, 1, 1, 1], [1, 6, 20, 2]]
    # round 1: seq 0's first pick is its stop id 99 (the cascade stopped at a = 1)
    nxt, acc = O.spec_commit([[99, 8, 8], [4, 4, 4], [0, 0, 0]], [[99, 8], [4, 4], [0, 0]], [1, 3, 3], stops,
                             state, ring, log)
    assert nxt.tolist() == [99, 4, 77] and acc.tolist() == [1, 3, 0]
    assert log[0, 1].tolist() == [1, 99, 99, 8] and log[1, 1].tolist() == [3, 4, 4, 4]
    assert ring[0].tolist() == [5, 6, 7, 5]          # the stop id is not appended
    assert ring[1].tolist() == [4, 4, 4, 4]          # count 1 -> 4: slots 1, 2, 0
    assert state.tolist() == [[1, 2, 14, 1], [0, 2, 4, 3], [1, 7, 20, 2]]
    # round 2: seq 0 is frozen now
    nxt, acc = O.spec_commit([[1, 1, 1], [5, 6, 6], [0, 0, 0]], [[1, 1], [5, 7], [0, 0]], [3, 2, 3], stops, state,
                             ring, log)
    assert nxt.tolist() == [99, 6, 77] and acc.tolist() == [0, 2, 0]
    assert log[0, 2].tolist() == [0, 99, 0, 0] and log[1, 2].tolist() == [2, 6, 5, 7]
    assert state.tolist() == [[1, 3, 14, 1], [0, 3, 6, 2], [1, 8, 20, 2]]
    assert ring[0].tolist() == [5, 6, 7, 5] and ring[1].tolist() == [6, 4, 5, 6]  # count 4: slots 1, 2 take 5, 6


def test_spec_commit_stop_among_the_accepted_picks():
    """A stop id drawn as the second pick when it equals the second draft
    ends the cascade there (a = 2, next = the stop id): the first pick is
    appended, the stop is not, and the sequence freezes."""
    pad = 0xFFFFFFFF
    state = np.zeros((1, 4), np.uint32)
    ring = np.zeros((1, 9), np.uint32)
    target = np.zeros((3, 64), np.float32)
    for j, t in enumerate([3, 4, 5]):
        target[j, t] = 5.0                            # greedy picks 3, 4, 5
    o = O.spec_exact(_spec_inp(target, 2, draft_ids=np.array([[3, 4]], np.uint32), params=Params(temperature=0.0),
                               stop=[[4]]))
    assert o["picks"].tolist() == [[3, 4, 5]] and o["accepted"].tolist() == [2] and o["next"].tolist() == [4]
    nxt, acc = O.spec_commit(o["picks"], [[3, 4]], o["accepted"], np.array([[4, pad, pad, pad]], np.uint32), state,
                             ring)
    assert nxt.tolist() == [4] and acc.tolist() == [2]
    assert ring[0, :3].tolist() == [1, 3, 0]
    assert state.tolist() == [[1, 1, 2, 2]]


# ---------------------------------------------------------------- lm head --

def _bf16(x: float) -> int:
    """bf16 bits of a float that bf16 holds exactly."""
    b = struct.unpack("<I", struct.pack("<f", x))[0]
    assert b & 0xFFFF == 0, x
    return b >> 16


def test_lm_head_one_hot_hidden_reads_a_weight_column():
    """hidden = e_k gives logit[id] = weight[id][k] widened (bits << 16):
    pins the widening and which index is the vocabulary."""
    rng = np.random.default_rng(21)
    w = W.bf16_bits(rng, (37, 64), -6, 2)
    for k in (0, 5, 63):
        h = np.zeros((1, 64), np.float32)
        h[0, k] = 1.0
        got = O.lm_head_logits(h, w)[0]
        want = (w[:, k].astype(np.uint32) << 16).view(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_lm_head_lane_partial_is_one_fma_chain():
    """w = [-1, 1 + 2^-7], x = [1, 1 + 2^-23] (both in partial 0): the fused
    chain over k = 0, 1 keeps the product's 2^-30 bit (exact result
    2^-7 + 2^-23 + 2^-30); a separately rounded product, or the chain run
    k = 1, 0, loses it."""
    w = np.array([[_bf16(-1.0), _bf16(1.0 + 2.0 ** -7)]], np.uint16)
    h = np.array([[1.0, 1.0 + 2.0 ** -23]], np.float32)
    got = float(O.lm_head_logits(h, w, dim=2)[0, 0])
    assert got == 2.0 ** -7 + 2.0 ** -23 + 2.0 ** -30
    reversed_order = float(np.float32(np.float32(1.0 + 2.0 ** -7) * np.float32(1.0 + 2.0 ** -23)) - np.float32(1.0))
    assert reversed_order == 2.0 ** -7 + 2.0 ** -23 and got != reversed_order


def test_lm_head_partials_add_in_a_pairwise_tree():
    """Terms at k = 0, 8, 16, 24 fall in partials 0, 1, 2, 3 (lane g takes
    k = 8 g .. 8 g + 7 of every 64): 1, 2^-24, 2^-24, 2^-24 add as
    (1 + 2^-24) + (2^-24 + 2^-24) = 1 + 2^-23.  One chain over k, or the
    four terms in one partial, rounds each 1 + 2^-24 back to 1."""
    dim = 256
    w = np.zeros((1, dim), np.uint16)
    h = np.zeros((1, dim), np.float32)
    for k, v in ((0, 1.0), (8, 2.0 ** -24), (16, 2.0 ** -24), (24, 2.0 ** -24)):
        w[0, k] = _bf16(v)
        h[0, k] = 1.0
    assert float(O.lm_head_logits(h, w)[0, 0]) == 1.0 + 2.0 ** -23
    seq = np.float32(0.0)
    for v in (1.0, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24):
        seq = np.float32(seq + np.float32(v))
    assert float(seq) == 1.0


def test_lm_head_within_the_chain_bound_of_the_exact_dot():
    """Against the float64 dot product: an f32 fma chain of n terms errs by
    at most n * 2^-24 * sum |w x| (each step rounds once)."""
    rng = np.random.default_rng(22)
    h = rng.standard_normal((3, 512)).astype(np.float32)
    w = W.bf16_bits(rng, (200, 512), -7, -4)
    got = O.lm_head_logits(h, w).astype(np.float64)
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    exact = h.astype(np.float64) @ wf.T
    bound = 512 * 2.0 ** -24 * (np.abs(h.astype(np.float64)) @ np.abs(wf).T)
    assert np.all(np.abs(got - exact) <= bound)
    assert np.any(got != exact)  # the f32 chain does round


# ------------------------------------------------------ quantized LM head --

def test_f16_round_is_numpys_float16():
    """orc_f16_round (the Q8_1 operand's f16 fields) rounds to nearest, ties
    to even, with subnormals and overflow, as numpy's float16 does."""
    rng = np.random.default_rng(31)
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
                         np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                                   1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf], np.float32)])
    want = xs.astype(np.float16).astype(np.float32)
    got = np.array([O.f16_round(float(x)) for x in xs], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q81_quantize_hand_blocks():
    """q8.js:27-42 on blocks worked out by hand: amax 127 gives d = 1 and
    q = round-half-even(x); amax 63.5 gives d = 0.5 and q = rint(2 x); an
    all-zero block has d = 0 and q = 0; d8 and s8 are the f16 d and d * sum."""
    x = np.zeros(96, np.float32)
    x[0:8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.49, -126.5]
    x[32:36] = [63.5, 0.25, -0.75, 10.0]
    q, d8, s8 = O.q81_quantize(x)
    assert q[0:8].tolist() == [127, 0, 2, 2, 0, -2, 3, -126]
    assert (q[8:32] == 0).all()
    assert q[32:36].tolist() == [127, 0, -2, 20] and (q[36:64] == 0).all()
    assert (q[64:] == 0).all()
    assert d8.tolist() == [1.0, 0.5, 0.0]
    assert s8.tolist() == [float(np.float16(127 + 2 + 2 - 2 + 3 - 126)), float(np.float16(0.5 * 145)), 0.0]


def _ref_weight(fmt, row: np.ndarray, k: int) -> float:
    """The reference's per-element dequantization (ggml/kernels.js:64-80,
    loadWeight) of value k of one GGUF row, exactly (float64)."""
    def f16(off):
        return float(row[off:off + 2].copy().view(np.float16)[0])
    if fmt == O.HEAD_Q8_0:
        base = (k >> 5) * 34
        return f16(base) * float(np.int8(row[base + 2 + (k & 31)]))
    if fmt == O.HEAD_Q4_0:
        base, i = (k >> 5) * 18, k & 31
        qb = int(row[base + 2 + (i & 15)])
        return f16(base) * ((qb >> 4 if i >= 16 else qb & 15) - 8.0)
    base, i = (k >> 8) * 210, k & 255
    half, p = i >> 7, i & 127
    quarter, l = p >> 5, p & 31
    packed = int(row[base + half * 64 + (32 if quarter & 1 else 0) + l])
    nib = packed >> 4 if quarter >= 2 else packed & 15
    high = (int(row[base + 128 + half * 32 + l]) >> (quarter * 2)) & 3
    sc = float(np.int8(row[base + 192 + half * 8 + (l >> 4) + quarter * 2]))
    return f16(base + 208) * sc * ((nib | (high << 4)) - 32.0)


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_gguf_head_one_hot_reads_the_reference_weight(fmt):
    """hidden = 127 e_k (its Q8_1 block has d = 1, q = 127 at k, every other
    block d = 0) makes each logit the term of the one block holding k, which
    equals 127 times the reference's dequantized weight rounded once to f32
    (the exact products have at most 32 significant bits): pins every byte,
    nibble, two-bit field and scale index of the three layouts."""
    from shared_amd import workloads as W
    rng = np.random.default_rng(40 + fmt)
    dim, vocab = 512, 40
    w = W.gguf_head(rng, fmt, vocab, dim)
    ks = list(range(0, dim, 7)) + [1, 15, 16, 17, 31, 32, 63, 64, 127, 128, 129, 255, 256, 300, 511]
    hid = np.zeros((len(ks), dim), np.float32)
    for r, k in enumerate(ks):
        hid[r, k] = 127.0
    got = O.lm_head_q_logits(fmt, hid, w)
    for r, k in enumerate(ks):
        want = np.array([127.0 * _ref_weight(fmt, w[i], k) for i in range(vocab)]).astype(np.float32)
        # values equal (a zero weight under a negative scale is -0 in the
        # formula, +0 once added to the partial sums)
        assert np.array_equal(got[r], want), (fmt, k)


def test_gguf_head_partials_add_in_the_fixed_tree():
    """Q8_0 rows whose block terms are planted (hidden 127 at the first value
    of every block: each block's term is 127 q d rounded once): the logit is
    the eight lane chains (blocks g, g + 8) added in the pairwise tree, and a
    left-to-right sum of the same terms differs for the planted rows."""
    from shared_amd import workloads as W
    dim = 512
    hid = np.zeros((1, dim), np.float32)
    hid[0, ::32] = 127.0
    found = 0
    for seed in range(200):
        rng = np.random.default_rng(seed)
        w = W.gguf_head(rng, O.HEAD_Q8_0, 8, dim)
        got = O.lm_head_q_logits(O.HEAD_Q8_0, hid, w)[0]
        for i in range(8):
            t = [np.float32(np.float32(127.0 * float(np.int8(w[i, 34 * b + 2]))) *
                            np.float32(w[i, 34 * b:34 * b + 2].copy().view(np.float16)[0])) for b in range(16)]
            p = [np.float32(np.float32(np.float32(0.0) + t[g]) + t[g + 8]) for g in range(8)]
            tree = np.float32(np.float32(np.float32(p[0] + p[1]) + np.float32(p[2] + p[3])) +
                              np.float32(np.float32(p[4] + p[5]) + np.float32(p[6] + p[7])))
            seq = np.float32(0.0)
            for x in t:
                seq = np.float32(seq + x)
            assert got[i] == tree
            found += int(tree != seq)
        if found >= 3:
            break
    assert found >= 3

"""The Node host layer on the GPU: tests/node/host_gpu.js samples a C3P-shaped
batch through every entry of the JS API (host and device-resident logits,
async, per-row params, TokenMask state, the reference's sample(cands, opts)
signature, verify), and every result is compared with the oracle."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle as O
from shared_amd import Params
from shared_amd import workloads as W
from shared_amd._capi import MASK_ALLOW

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _u32(d, name):
    return np.fromfile(os.path.join(d, name), np.uint32)


def test_node_api_end_to_end(tmp_path):
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    d = str(tmp_path)
    b = W.c3p(rows=12, seed=91)
    O.write_case(d, b)
    rng = np.random.default_rng(5)
    allow = np.unique(rng.integers(0, b.vocab, 3000)).astype(np.uint32)
    allow.tofile(os.path.join(d, "tokmask_allow.u32"))
    # a candidate list as the reference's GPU top-k hands it to sample()
    cand_ids = rng.choice(b.vocab, 20, replace=False).astype(np.uint32)
    cand_vals = (rng.standard_normal(20) * 3).astype(np.float32)
    recent = [int(cand_ids[3]), int(cand_ids[7]), 5]
    us = [0.0, 0.1, 0.37, 0.5, 0.9, 0.999]
    cc = {"ids": cand_ids.tolist(), "vals": cand_vals.astype(float).tolist(), "temperature": 0.8, "topK": 12,
          "topP": 0.9, "presencePenalty": 1.2, "recent": recent, "uniforms": us}
    with open(os.path.join(d, "cands.json"), "w") as f:
        json.dump(cc, f)
    v = W.c5(seqs=4, seed=17)
    v["target"].tofile(os.path.join(d, "v_target.f32"))
    v["draft"].tofile(os.path.join(d, "v_draft.f32"))
    np.ascontiguousarray(v["draft_ids"], np.uint32).tofile(os.path.join(d, "v_ids.u32"))
    np.ascontiguousarray(v["uniforms"], np.float64).tofile(os.path.join(d, "v_u.f64"))
    np.ascontiguousarray(v["mask"], np.uint32).tofile(os.path.join(d, "v_mask.u32"))
    with open(os.path.join(d, "verify.json"), "w") as f:
        json.dump({"vocab": v["vocab"], "seqs": v["seqs"], "drafts": v["drafts"],
                   "temperature": v["temperature"]}, f)

    want = O.sample_rows(b)
    want["ids"].astype(np.uint32).tofile(os.path.join(d, "want_ids.u32"))

    print("[gpu] node host_gpu.js", d, flush=True)
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "host_gpu.js"), d], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:]

    got = _u32(d, "js_sync_ids.u32")
    assert np.array_equal(got, want["ids"])
    probs = np.fromfile(os.path.join(d, "js_sync_probs.f64")).reshape(b.rows, -1)
    assert np.array_equal(probs, want["probs"])
    assert np.array_equal(_u32(d, "js_sync_cand.u32").reshape(b.rows, -1), want["cand_ids"])
    for name in ("js_async_ids.u32", "js_dev_ids.u32", "js_rowparams_ids.u32", "js_conc1_ids.u32",
                 "js_conc2_ids.u32"):
        assert np.array_equal(_u32(d, name), want["ids"]), name

    m1 = O.mask_from_ids(MASK_ALLOW, allow, b.vocab)
    bt = W.Batch("tokmask", b.logits, b.params, mask=np.repeat(m1[None, :], b.rows, axis=0),
                 hist_ids=b.hist_ids, hist_offsets=b.hist_offsets, uniforms=b.uniforms)
    wt = O.sample_rows(bt)["ids"]
    assert np.array_equal(_u32(d, "js_tokmask_ids.u32"), wt)
    assert np.array_equal(_u32(d, "js_tokmask2_ids.u32"), wt)
    # MaskBuilder words: the allow list minus its first 100 ids; packedToolMask
    # over the allow list itself
    mw = O.mask_from_ids(MASK_ALLOW, allow[100:], b.vocab)
    bw = W.Batch("words", b.logits, b.params, mask=np.repeat(mw[None, :], b.rows, axis=0),
                 hist_ids=b.hist_ids, hist_offsets=b.hist_offsets, uniforms=b.uniforms)
    assert np.array_equal(_u32(d, "js_words_ids.u32"), O.sample_rows(bw)["ids"])
    assert np.array_equal(_u32(d, "js_tool_ids.u32"), wt)

    # allowedTokenIds: every row, then the even rows only
    ba = W.Batch("allowed", b.logits, b.params, mask=np.repeat(m1[None, :], b.rows, axis=0),
                 hist_ids=b.hist_ids, hist_offsets=b.hist_offsets, uniforms=b.uniforms)
    assert np.array_equal(_u32(d, "js_allowed_ids.u32"), O.sample_rows(ba)["ids"])
    full = O.mask_from_ids(0, np.zeros(0, np.uint32), b.vocab)
    mixed = np.stack([full if r % 2 else m1 for r in range(b.rows)])
    bm = W.Batch("allowed_mixed", b.logits, b.params, mask=mixed, hist_ids=b.hist_ids,
                 hist_offsets=b.hist_offsets, uniforms=b.uniforms)
    assert np.array_equal(_u32(d, "js_allowed_mixed_ids.u32"), O.sample_rows(bm)["ids"])

    # decodeBatch's per-row result: {ids, fed, eos, stopped, stopId}; stops
    # are the tokens of rows 0 and 1, the first of them the eos id
    with open(os.path.join(d, "js_decode.json")) as f:
        dec = json.load(f)
    stops = [int(want["ids"][0]), int(want["ids"][1])]
    for r, res in enumerate(dec["results"]):
        tok = int(want["ids"][r])
        hit = tok in stops
        assert res == {"ids": [tok], "fed": 1, "eos": hit and tok == stops[0], "stopped": hit,
                       "stopId": tok if hit else None}, (r, res)
        n0 = int(b.hist_offsets[r + 1] - b.hist_offsets[r])
        assert dec["lens"][r] == n0 + (0 if hit else 1), r
        if not hit:
            assert dec["last"][r] == tok

    cv = int(cand_ids.max()) + 1
    row = np.full(cv, np.nan, np.float32)
    row[cand_ids] = cand_vals
    bits = np.zeros(cv, bool)
    bits[cand_ids] = True
    n = len(us)
    hi, ho = W._csr([np.unique(np.array(recent, np.uint32))] * n)
    bc = W.Batch("compat", np.repeat(row[None, :], n, axis=0),
                 Params(temperature=0.8, top_k=12, top_p=0.9, presence_penalty=1.2),
                 mask=np.repeat(W.pack_bits(bits[None, :]), n, axis=0), hist_ids=hi, hist_offsets=ho,
                 uniforms=np.array(us))
    with open(os.path.join(d, "js_compat.json")) as f:
        compat = json.load(f)
    assert compat == O.sample_rows(bc)["ids"].tolist()

    ov = O.verify(v)
    L = v["drafts"]
    assert np.array_equal(_u32(d, "js_v_tokens.u32").reshape(v["seqs"], L + 1), ov["tokens"])
    assert np.array_equal(np.fromfile(os.path.join(d, "js_v_acc.i32"), np.int32), ov["accepted"])
    assert np.array_equal(_u32(d, "js_v2_tokens.u32"), _u32(d, "js_v_tokens.u32"))


def test_node_decode_steps(tmp_path):
    """decodeSteps / decodeStepsAsync against the oracle stepped the same way
    (kernels.js:174-199 per row; decodeBatch's result, model.js:727-741)."""
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    from gpu_helpers import oracle_steps
    d = str(tmp_path)
    rows, vocab, k, wsize = 6, 60_000, 6, 4
    rng = np.random.default_rng(23)
    xs = (rng.standard_normal((k, rows, vocab)) * 1.5).astype(np.float32)
    for j, sid in enumerate([17, 2_049, 40_000]):
        xs[:, :, sid] += np.float32(6.0 - 0.3 * j)
    js = [dict(temperature=0.9, topK=30, topP=0.9, repetitionPenalty=1.3, presencePenalty=0.8, frequencyPenalty=0.2,
               softcap=0, seed=int(rng.integers(1, 2**31))) for _ in range(rows)]
    js[1].update(temperature=0)  # greedy: the penalties alone move it off the spikes
    prm = [Params(temperature=p["temperature"], top_k=p["topK"], top_p=p["topP"],
                  repetition_penalty=p["repetitionPenalty"], presence_penalty=p["presencePenalty"],
                  frequency_penalty=p["frequencyPenalty"]) for p in js]
    seeds = np.array([p["seed"] for p in js], np.uint32)
    hist = [[17, 17, 5, 2_049, 9], [], [40_000], [], [1, 2, 3], [17]]
    free, _, _, _ = oracle_steps(xs, prm, seeds=seeds, history=hist, ring_len=wsize)
    # stops: row 0 at its third token (also its eos), row 2 on its first
    # token as a second stop id, row 4 on an id it never draws
    stops = [[int(free[2]["ids"][0])], [], [3, int(free[0]["ids"][2])], [], [7], []]
    for r, st in enumerate(stops):
        if st:
            js[r]["stopIds"] = st
    want, _, _, window = oracle_steps(xs, prm, seeds=seeds, stop_ids=stops, history=hist, ring_len=wsize)
    xs.tofile(os.path.join(d, "step_logits.f32"))
    first = np.arange(rows, dtype=np.uint32) + 1000
    first.tofile(os.path.join(d, "first.u32"))
    with open(os.path.join(d, "steps.json"), "w") as f:
        json.dump({"rows": rows, "vocab": vocab, "k": k, "params": js, "windows": hist, "windowSize": wsize}, f)
    print("[gpu] node steps_gpu.js", d, flush=True)
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "steps_gpu.js"), d], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:]
    seqs = [[int(w["ids"][r]) for w in want] for r in range(rows)]
    expect = []
    for r in range(rows):
        ids = seqs[r]
        at = next((i for i, t in enumerate(ids) if t in stops[r]), -1)
        hit = at >= 0
        expect.append({"ids": ids[:at + 1] if hit else ids, "fed": at + 1 if hit else k,
                       "eos": hit and ids[at] == stops[r][0], "stopped": hit, "stopId": ids[at] if hit else None})
    assert expect[0]["stopped"] and expect[0]["eos"] and expect[2]["stopped"] and not expect[2]["eos"]
    for name in ("js_steps.json", "js_steps_async.json"):
        with open(os.path.join(d, name)) as f:
            got = json.load(f)
        assert got["results"] == expect, name
        assert got["windows"] == window, name
    with open(os.path.join(d, "js_steps.json")) as f:
        fed = json.load(f)["fed"]
    assert fed[0] == first.tolist()
    for i in range(1, k):
        assert fed[i] == [int(x) for x in want[i - 1]["ids"]], i


def test_node_spec_exact(tmp_path):
    """specExact / specExactAsync against the oracle's exact-match round
    (kernels.js:211-401), with the windows mirroring the commits
    (model.js:994-996)."""
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    d = str(tmp_path)
    c = W.spec_case(seqs=10, vocab=W.QWEN_VOCAB, drafts=2, hist=40, seed=8)
    hist = [c["hist_ids"][c["hist_offsets"][q]:c["hist_offsets"][q + 1]].tolist() for q in range(c["seqs"])]
    js = []
    for q, p in enumerate(c["seq_params"]):
        stops = [int(x) for x in c["stop_ids"][q] if x != 0xFFFFFFFF]
        js.append(dict(temperature=p.temperature, topK=p.top_k, topP=p.top_p, presencePenalty=p.presence_penalty,
                       repetitionPenalty=p.repetition_penalty, frequencyPenalty=p.frequency_penalty, softcap=0,
                       seed=int(c["seeds"][q]), stopIds=stops))
    c["target"].tofile(os.path.join(d, "spec_target.f32"))
    c["draft"].tofile(os.path.join(d, "spec_draft.f32"))
    with open(os.path.join(d, "spec.json"), "w") as f:
        json.dump({"vocab": c["vocab"], "seqs": c["seqs"], "drafts": c["drafts"], "round": c["round"],
                   "params": js, "history": hist}, f)
    print("[gpu] node spec_gpu.js", d, flush=True)
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "spec_gpu.js"), d], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:]
    o = O.spec_exact(c)
    stops = [set(int(x) for x in c["stop_ids"][q]) for q in range(c["seqs"])]
    for name in ("js_spec.json", "js_spec_async.json"):
        with open(os.path.join(d, name)) as f:
            got = json.load(f)
        for q, r in enumerate(got["results"]):
            a = int(o["accepted"][q])
            assert r["a"] == a and r["next"] == int(o["next"][q]), (name, q, r)
            assert r["picks"] == o["picks"][q].tolist() and r["drafts"] == o["draft_ids"][q].tolist(), (name, q)
            assert r["stopped"] == (r["next"] in stops[q]), (name, q)
        if "windows" in got:
            for q in range(c["seqs"]):
                kept = [t for t in o["picks"][q][:int(o["accepted"][q])].tolist() if t not in stops[q]]
                assert got["windows"][q] == hist[q] + kept, q


def test_node_lm_head_sample(tmp_path):
    """Sampler#lmHeadSample / lmHeadSampleAsync: the fused head's ids,
    candidates and probabilities bit-exact with the oracle over the oracle's
    head logits, and the logits it writes bit-exact with orc_lm_head_logits."""
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    d = str(tmp_path)
    b = W.lmh(rows=3, vocab=W.QWEN_VOCAB, dim=1024, seed=44, softcap=0.0)
    lo = O.lm_head_logits(b.hidden, b.weight_bits)
    bl = b.with_logits(lo)
    O.write_case(d, bl)
    with open(os.path.join(d, "meta.json")) as f:
        meta = json.load(f)
    meta["dim"] = b.dim
    with open(os.path.join(d, "meta.json"), "w") as f:
        json.dump(meta, f)
    np.ascontiguousarray(b.hidden, np.float32).tofile(os.path.join(d, "hidden.f32"))
    np.ascontiguousarray(b.weight_bits, np.uint16).tofile(os.path.join(d, "weight.u16"))
    want = O.sample_rows(bl)
    # the same rows over a GGUF Q6_K head
    wq = W.gguf_head(np.random.default_rng(45), W.HEAD_Q6_K, b.vocab, b.dim)
    wq.tofile(os.path.join(d, "q6k.u8"))
    lq = O.lm_head_q_logits(W.HEAD_Q6_K, b.hidden, wq)
    want_q = O.sample_rows(b.with_logits(lq))

    print("[gpu] node lmhead_gpu.js", d, flush=True)
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "lmhead_gpu.js"), d], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:]

    got = np.fromfile(os.path.join(d, "lmh_logits.f32"), np.float32).reshape(b.rows, b.vocab)
    assert np.array_equal(got.view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(_u32(d, "lmh_sync_ids.u32"), want["ids"])
    probs = np.fromfile(os.path.join(d, "lmh_sync_probs.f64")).reshape(b.rows, -1)
    assert np.array_equal(probs, want["probs"])
    assert np.array_equal(_u32(d, "lmh_sync_cand.u32").reshape(b.rows, -1), want["cand_ids"])
    for name in ("lmh_async_ids.u32", "lmh_unfused_ids.u32"):
        assert np.array_equal(_u32(d, name), want["ids"]), name
    gq = np.fromfile(os.path.join(d, "lmh_q6k_logits.f32"), np.float32).reshape(b.rows, b.vocab)
    assert np.array_equal(gq.view(np.uint32), lq.view(np.uint32))
    assert np.array_equal(_u32(d, "lmh_q6k_ids.u32"), want_q["ids"])
    assert np.array_equal(np.fromfile(os.path.join(d, "lmh_q6k_probs.f64")).reshape(b.rows, -1), want_q["probs"])


def _step_expectations(want, stops, k):
    """decodeBatch's per-row result (model.js:727-741) of oracle steps."""
    rows = len(stops)
    seqs = [[int(w["ids"][r]) for w in want] for r in range(rows)]
    expect = []
    for r in range(rows):
        ids = seqs[r]
        at = next((i for i, t in enumerate(ids) if t in stops[r]), -1)
        hit = at >= 0
        expect.append({"ids": ids[:at + 1] if hit else ids, "fed": at + 1 if hit else k,
                       "eos": hit and ids[at] == stops[r][0], "stopped": hit, "stopId": ids[at] if hit else None})
    return expect


def test_node_decode_steps_with_head(tmp_path):
    """decodeStepsWithHead / decodeStepsWithHeadAsync over Qwen's head format
    (Q6_K): each step's logits are the oracle's head logits of that step's
    hidden states, sampled and fed back as the reference's per-iteration
    lm -> topk -> sampler does (model.js:711-717, kernels.js:174-199); a
    planted stop freezes one row mid-loop."""
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    from gpu_helpers import oracle_steps
    d = str(tmp_path)
    rows, vocab, dim, k, wsize = 3, 20_000, 512, 5, 16
    rng = np.random.default_rng(61)
    head = W.gguf_head(rng, W.HEAD_Q6_K, vocab, dim)
    hs = rng.standard_normal((k, rows, dim)).astype(np.float32)
    xs = np.stack([O.lm_head_q_logits(W.HEAD_Q6_K, hs[t], head) for t in range(k)])
    mask = W.random_mask(rng, rows, vocab, 0.05, 0.3)
    js = [dict(temperature=0.9, topK=40, topP=0.9, repetitionPenalty=1.2, presencePenalty=0.4, frequencyPenalty=0.0,
               softcap=0, seed=int(rng.integers(1, 2**31))) for _ in range(rows)]
    prm = [Params(temperature=p["temperature"], top_k=p["topK"], top_p=p["topP"],
                  repetition_penalty=p["repetitionPenalty"], presence_penalty=p["presencePenalty"]) for p in js]
    seeds = np.array([p["seed"] for p in js], np.uint32)
    hist = [[5, 17, 19_999], [], [1_000, 1_000]]
    free, _, _, _ = oracle_steps(xs, prm, mask=mask, seeds=seeds, history=hist, ring_len=wsize)
    stops = [[], [int(free[2]["ids"][1])], []]
    js[1]["stopIds"] = stops[1]
    want, stopped, _, window = oracle_steps(xs, prm, mask=mask, seeds=seeds, stop_ids=stops, history=hist,
                                            ring_len=wsize)
    assert stopped[1], "the planted stop must freeze row 1"
    hs.tofile(os.path.join(d, "hs.f32"))
    head.tofile(os.path.join(d, "head.u8"))
    mask.tofile(os.path.join(d, "mask.u32"))
    first = np.arange(rows, dtype=np.uint32) + 7
    first.tofile(os.path.join(d, "first.u32"))
    with open(os.path.join(d, "headsteps.json"), "w") as f:
        json.dump({"rows": rows, "vocab": vocab, "k": k, "dim": dim, "params": js, "windows": hist,
                   "windowSize": wsize}, f)
    print("[gpu] node headsteps_gpu.js", d, flush=True)
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "headsteps_gpu.js"), d], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:]
    expect = _step_expectations(want, stops, k)
    for name in ("js_headsteps.json", "js_headsteps_async.json"):
        with open(os.path.join(d, name)) as f:
            got = json.load(f)
        assert got["results"] == expect, name
        assert got["windows"] == window, name
    with open(os.path.join(d, "js_headsteps.json")) as f:
        fed = json.load(f)["fed"]
    assert fed[0] == first.tolist()
    for i in range(1, k):
        assert fed[i] == [int(x) for x in want[i - 1]["ids"]], i


def test_node_spec_steps(tmp_path):
    """specSteps / specStepsAsync: four chained rounds with acceptSpec's
    commit on the device (kernels.js:340-367, model.js:867-1008) against the
    oracle stepped round by round (orc_spec_exact, then orc_spec_commit):
    the round log, the positions, the stop state, and the windows mirroring
    the device rings; one sequence draws its stop id mid-chain."""
    if shutil.which("node") is None:
        pytest.skip("node is not installed")
    from gpu_helpers import oracle_chain
    from shared_amd.sampler import ring_rows
    d = str(tmp_path)
    seqs, L, vocab, rounds, ring_len = 6, 2, 32_000, 4, 48
    cases = [W.spec_case(seqs=seqs, vocab=vocab, drafts=L, hist=0, seed=400 + r) for r in range(rounds)]
    for c in cases[1:]:
        c["seq_params"] = cases[0]["seq_params"]
    rng = np.random.default_rng(19)
    seeds = rng.integers(1, 2**31, seqs, dtype=np.int64).astype(np.uint32)
    hist = [[int(i) for i in rng.integers(0, vocab, 5 + 11 * q)] for q in range(seqs)]
    ring0 = ring_rows(seqs, ring_len, hist)
    pad = 0xFFFFFFFF
    stops = np.full((seqs, 4), pad, np.uint32)
    stops[:, 0] = 151645
    per0, _, _, _ = oracle_chain(cases, seeds, stops, rounds, ring0, 0)
    stops[2, 1] = per0[1]["next"][2]
    _, want_state, _, want_log = oracle_chain(cases, seeds, stops, rounds, ring0, 0)
    assert want_state[2, 0] == 1, "the plant must freeze sequence 2 mid-chain"
    js = []
    for q, p in enumerate(cases[0]["seq_params"]):
        js.append(dict(temperature=p.temperature, topK=p.top_k, topP=p.top_p, presencePenalty=p.presence_penalty,
                       repetitionPenalty=p.repetition_penalty, frequencyPenalty=p.frequency_penalty, softcap=0,
                       seed=int(seeds[q]), stopIds=[int(x) for x in stops[q] if x != pad]))
    for r, c in enumerate(cases):
        c["target"].tofile(os.path.join(d, f"target_{r}.f32"))
        c["draft"].tofile(os.path.join(d, f"draft_{r}.f32"))
    with open(os.path.join(d, "specsteps.json"), "w") as f:
        json.dump({"vocab": vocab, "seqs": seqs, "drafts": L, "rounds": rounds, "params": js, "windows": hist,
                   "windowSize": ring_len}, f)
    print("[gpu] node specsteps_gpu.js", d, flush=True)
    proc = subprocess.run(["node", os.path.join(ROOT, "tests", "node", "specsteps_gpu.js"), d], stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout[-3000:]
    stop_sets = [set(int(x) for x in stops[q] if x != pad) for q in range(seqs)]
    want_windows = [list(h) for h in hist]
    for r in range(rounds):
        for q in range(seqs):
            a, nxt = int(want_log[q, r, 0]), int(want_log[q, r, 1])
            if a > 0:
                committed = [int(x) for x in want_log[q, r, 2:2 + a - 1]] + [nxt]
                want_windows[q] += [t for t in committed if t not in stop_sets[q]]
    for name in ("js_specsteps.json", "js_specsteps_async.json"):
        with open(os.path.join(d, name)) as f:
            got = json.load(f)
        for r in range(rounds):
            for q in range(seqs):
                e = got["rounds"][r][q]
                a = int(want_log[q, r, 0])
                assert e["a"] == a and e["next"] == int(want_log[q, r, 1]), (name, r, q, e)
                assert e["drafts"] == [int(x) for x in want_log[q, r, 2:]], (name, r, q)
                assert e["frozen"] == (a == 0), (name, r, q)
        assert got["pos"] == [int(x) for x in want_state[:, 2]], name
        assert got["stopped"] == [bool(x) for x in want_state[:, 0]], name
        assert got["windows"] == want_windows, name

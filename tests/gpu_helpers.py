"""Helpers shared by the GPU parity tests: run a Batch through the HIP path
and the oracle on the same inputs and compare."""
from __future__ import annotations

import numpy as np

import oracle as O
from shared_amd import Sampler
from shared_amd import workloads as W
from shared_amd._capi import FLAG_DRAW_EDGE, FLAG_EMPTY_ROW, FLAG_TOPP_EDGE, MAX_TOP_K, NO_TOKEN, STOP_PAD

ORACLE_FLAGS = FLAG_EMPTY_ROW | FLAG_TOPP_EDGE | FLAG_DRAW_EDGE


def to_dev(a, dtype=None):
    import torch
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def run_gpu(s: Sampler, b, *, logits_dev=None, row_params=None, full=True):
    import torch
    lg = logits_dev if logits_dev is not None else to_dev(b.logits)
    mask = to_dev(b.mask, torch.int32) if b.mask is not None else None
    hi = to_dev(b.hist_ids, torch.int32) if b.hist_ids is not None else None
    ho = to_dev(b.hist_offsets) if b.hist_offsets is not None else None
    u = to_dev(b.uniforms) if b.uniforms is not None else None
    rp = None
    hints = 0
    if row_params is not None:
        from shared_amd import pack_params
        from shared_amd.sampler import row_hints
        rp = to_dev(pack_params(row_params).view(np.uint8))
        hints = row_hints(row_params)
    out = s.sample(lg, vocab=b.vocab, mask=mask, hist_ids=hi, hist_offsets=ho, uniforms=u, params=b.params,
                   row_params=rp, row_hints=hints, full=full)
    torch.cuda.synchronize()
    if not full:
        return {"ids": out.cpu().numpy().view(np.uint32)}
    return {"ids": out["ids"].cpu().numpy().view(np.uint32), "probs": out["probs"].cpu().numpy(),
            "cand_ids": out["cand_ids"].cpu().numpy().view(np.uint32), "counts": out["counts"].cpu().numpy(),
            "flags": out["flags"].cpu().numpy().view(np.uint32)}


def assert_parity(g: dict, o: dict, label: str = "") -> None:
    """Bit-exact ids, ranked candidates, counts and probabilities."""
    bad = np.nonzero(g["ids"] != o["ids"])[0]
    assert bad.size == 0, f"{label}: id mismatch rows {bad[:8]} gpu {g['ids'][bad[:8]]} oracle {o['ids'][bad[:8]]}"
    if "counts" in g:
        assert np.array_equal(g["counts"], o["counts"]), f"{label}: k/cut differ"
        assert np.array_equal(g["cand_ids"], o["cand_ids"]), f"{label}: ranked candidates differ"
        # probabilities: identical double arithmetic, so bitwise equal
        assert np.array_equal(g["probs"].view(np.uint64), o["probs"].view(np.uint64)), f"{label}: probs differ"
        assert np.array_equal(g["flags"] & ORACLE_FLAGS, o["flags"] & ORACLE_FLAGS), f"{label}: flags differ"


def oracle_steps(xs, prm, *, mask=None, stop_ids=None, seeds=None, uniforms=None, history=None, ring_len=512):
    """The reference's loop (kernels.js:174-199) for each row on the CPU."""
    steps, rows, _ = xs.shape
    stop_ids = stop_ids or [[] for _ in range(rows)]
    window = [list(h) for h in (history or [[] for _ in range(rows)])]
    stopped = [False] * rows
    it = [0] * rows
    outs = []
    for t in range(steps):
        step = {"ids": np.zeros(rows, np.uint32), "counts": np.zeros((rows, 2), np.int32),
                "probs": np.zeros((rows, MAX_TOP_K)), "cand_ids": np.full((rows, MAX_TOP_K), NO_TOKEN, np.uint32)}
        for r in range(rows):
            frozen = stopped[r]
            if frozen:
                tok = stop_ids[r][0] if stop_ids[r] else STOP_PAD
            else:
                u = O.lib().orc_pcg_uniform(int(seeds[r]), it[r], 0) if seeds is not None else uniforms[t][r]
                h = window[r][-ring_len:] if ring_len else []
                res = O.sample_row(xs[t, r], prm[r], mask=None if mask is None else mask[r],
                                   hist=np.array(h, np.uint32) if h else None, uniform=u)
                tok = res.id
                n = res.k  # the ranked candidates (0 for a greedy row)
                step["counts"][r] = (res.k, res.cut)
                step["probs"][r, :n] = np.array(res.probs)[:n]
                step["cand_ids"][r, :n] = np.array(res.cand_ids, np.uint32)[:n]
            step["ids"][r] = tok
            it[r] += 1
            if tok == NO_TOKEN or tok in stop_ids[r]:
                stopped[r] = True
            elif not frozen:
                window[r].append(tok)
        outs.append(step)
    return outs, stopped, it, window


def ring_of(window, ring_len):
    ring = np.zeros(1 + ring_len, np.uint32)
    for i in range(max(0, len(window) - ring_len), len(window)):
        ring[1 + i % ring_len] = window[i]
    ring[0] = len(window)
    return ring


def oracle_chain(cases, seeds, stop_ids, rounds, ring0, first_round):
    """orc_spec_exact then orc_spec_commit, round by round, every sequence's
    history being its ring as of the round's start."""
    seqs, L = cases[0]["seqs"], cases[0]["drafts"]
    ring = ring0.copy()
    ring_len = ring.shape[1] - 1
    state = np.zeros((seqs, 4), np.uint32)
    state[:, 1] = first_round
    log = np.zeros((seqs, rounds, L + 2), np.uint32)
    per = []
    for r in range(rounds):
        c = dict(cases[r])
        hist = [ring[s, 1:1 + min(int(ring[s, 0]), ring_len)] for s in range(seqs)]
        c["hist_ids"], c["hist_offsets"] = W._csr(hist)
        c["seeds"], c["stop_ids"], c["round"] = seeds, stop_ids, int(state[0, 1])
        frozen = state[:, 0].copy()
        o = O.spec_exact(c)
        nxt, acc = O.spec_commit(o["picks"], o["draft_ids"], o["accepted"], stop_ids, state, ring, log)
        per.append({"frozen": frozen, "draft_ids": o["draft_ids"], "picks": o["picks"], "accepted": acc,
                    "next": nxt})
    return per, state, ring, log

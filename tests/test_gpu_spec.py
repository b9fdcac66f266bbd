"""GPU parity of sas_spec_exact, the reference's exact-match speculative
round (argmax drafts, kernels.js:373-401; every verify row sampled on its
own, kernels.js:255-327; the cascade, kernels.js:328-339), against the C
oracle: drafts, picks, accepted counts and next tokens bit-exact."""
import numpy as np
import pytest

import oracle as O
from shared_amd import Params, SasError
from shared_amd import workloads as W
from shared_amd.sampler import pack_params, row_hints
from gpu_helpers import oracle_chain

pytestmark = pytest.mark.gpu


def dev(a, view=None):
    import torch
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t.view(view) if view is not None else t).cuda()


def run_spec(sampler, c, *, drafts_given=False):
    import torch
    seqs, L = c["seqs"], c["drafts"]
    ids = dev(np.ascontiguousarray(c["draft_ids"], np.uint32), torch.int32) if drafts_given else \
        torch.zeros((seqs, L), dtype=torch.int32, device="cuda")
    picks = torch.empty((seqs, L + 1), dtype=torch.int32, device="cuda")
    acc = torch.empty(seqs, dtype=torch.int32, device="cuda")
    nxt = torch.empty(seqs, dtype=torch.int32, device="cuda")
    sp = c.get("seq_params")
    sampler.spec_exact_into(
        dev(c["target"]), ids, dev(c["seeds"], torch.int32), picks, acc,
        draft_logits=None if drafts_given else dev(c["draft"]), out_next=nxt, round=c["round"],
        mask=dev(c.get("mask"), torch.int32), hist_ids=dev(c.get("hist_ids"), torch.int32),
        hist_offsets=dev(c.get("hist_offsets")), params=c.get("params"),
        seq_params=None if sp is None else dev(pack_params(sp).view(np.uint8)),
        row_hints=0 if sp is None else row_hints(sp), stop_ids=dev(c.get("stop_ids"), torch.int32))
    torch.cuda.synchronize()
    u32 = lambda t: t.cpu().numpy().view(np.uint32)  # noqa: E731
    return {"draft_ids": u32(ids), "picks": u32(picks), "accepted": acc.cpu().numpy(), "next": u32(nxt)}


def check(g, o, label):
    for k in ("draft_ids", "picks", "accepted", "next"):
        assert np.array_equal(g[k], o[k]), f"{label}: {k} differ\n gpu {g[k][:4]}\n oracle {o[k][:4]}"


@pytest.mark.parametrize("seqs,vocab,L,mask,hist", [
    (32, W.QWEN_VOCAB, 2, False, 512),   # the reference's round: 2 drafts, Qwen vocabulary
    (16, 32_000, 4, True, 64),
    (9, 50_000, 1, False, 0),
])
def test_spec_round_matches_oracle(sampler, seqs, vocab, L, mask, hist):
    print(f"[gpu] spec_exact seqs={seqs} vocab={vocab} L={L}", flush=True)
    c = W.spec_case(seqs=seqs, vocab=vocab, drafts=L, hist=hist, mask=mask, seed=seqs + L)
    g = run_spec(sampler, c)
    o = O.spec_exact(c)
    check(g, o, f"spec {seqs}x{vocab} L{L}")
    # the case exercises both outcomes of the cascade
    assert (o["accepted"] > 1).any() and (o["accepted"] == 1).any()


def test_spec_round_with_given_drafts_and_stops(sampler):
    """Drafts handed in (no draft head), one shared sas_params, and stop ids
    that are drawn: a stop-id draft ends the cascade."""
    c = W.spec_case(seqs=12, vocab=40_000, drafts=3, hist=0, seed=77, greedy_every=1)
    o0 = O.spec_exact(c)
    c["draft_ids"] = o0["draft_ids"].copy()
    c["draft_ids"][::2, 1] = 7          # every other sequence misses its second draft
    c["draft"] = None                   # the oracle takes the drafts as given too
    c["seq_params"] = None
    c["params"] = Params(temperature=0.0)
    st = np.full((12, 4), 0xFFFFFFFF, np.uint32)
    st[3, 2] = o0["picks"][3, 0]        # sequence 3's first pick is one of its stop ids
    c["stop_ids"] = st
    g = run_spec(sampler, c, drafts_given=True)
    o = O.spec_exact(c)
    check(g, o, "given drafts")
    if c["draft_ids"][3, 0] == o["picks"][3, 0]:
        assert o["accepted"][3] == 1


def test_spec_rejects_bad_descriptors(sampler):
    import torch
    c = W.spec_case(seqs=2, vocab=1000, drafts=2, hist=0, seed=1)
    t = dev(c["target"])
    ids = torch.zeros((2, 2), dtype=torch.int32, device="cuda")
    picks = torch.empty((2, 3), dtype=torch.int32, device="cuda")
    acc = torch.empty(2, dtype=torch.int32, device="cuda")
    with pytest.raises(SasError, match="required"):
        sampler.spec_exact_into(t, ids, None, picks, acc)
    with pytest.raises(ValueError):
        sampler.spec_exact_into(t[:5], ids, dev(c["seeds"], torch.int32), picks, acc)
    big = torch.zeros((2, 20), dtype=torch.int32, device="cuda")
    with pytest.raises(SasError, match="draft_len"):
        sampler.spec_exact_into(torch.zeros((42, 1000), device="cuda"), big, dev(c["seeds"], torch.int32),
                                torch.empty((2, 21), dtype=torch.int32, device="cuda"), acc)


def test_random_sweep(sampler):
    # 30 seeded random rounds: 1-16 sequences, 1-16 drafts, vocabularies 300
    # to 151,936, masks, histories up to 1,500 ids, greedy and sampled
    # sequences, drafts from the draft head or handed in, stop ids among the
    # target's own picks
    for case in range(30):
        rng = np.random.default_rng(80000 + case)
        seqs, L = int(rng.integers(1, 17)), int(rng.choice([1, 2, 3, 4, 8, 16]))
        vocab = int(rng.choice([300, 5000, 40_000, W.QWEN_VOCAB]))
        c = W.spec_case(seqs=seqs, vocab=vocab, drafts=L, hist=int(rng.choice([0, 64, 1500])),
                        mask=bool(rng.random() < 0.4), greedy_every=int(rng.integers(0, 4)), seed=80000 + case)
        given = bool(rng.random() < 0.3)
        if given:
            o0 = O.spec_exact(c)
            c["draft_ids"] = o0["draft_ids"].copy()
            miss = rng.random(c["draft_ids"].shape) < 0.3
            c["draft_ids"][miss] = rng.integers(0, vocab, int(miss.sum()))
            c["draft"] = None
            if rng.random() < 0.5:
                c["stop_ids"][:, 1] = o0["picks"][:, 0]
        label = f"sweep {case}: seqs={seqs} L={L} vocab={vocab} given={given}"
        print(f"[gpu] spec {label}", flush=True)
        check(run_spec(sampler, c, drafts_given=given), O.spec_exact(c), label)


def test_spec_chain_of_rounds_in_a_graph(sampler):
    """sas_spec_step: four chained rounds recorded into one HIP graph (the
    reference's specChain submits R rounds at once, model.js:867-1008), every
    replay bit-exact with the oracle stepped round by round: drafts, picks and
    accepted counts of the live sequences, the round log, the state {frozen,
    round, pos, accepted}, the rings and the next tokens; one sequence draws
    its stop id mid-chain and freezes, one ring wraps."""
    import torch
    from shared_amd import SpecState
    from shared_amd.sampler import ring_rows
    seqs, L, vocab, rounds, ring_len, first = 8, 2, 32_000, 4, 48, 0  # a chain starts at round 0 (posBuf[4])
    cases = [W.spec_case(seqs=seqs, vocab=vocab, drafts=L, hist=0, seed=300 + r) for r in range(rounds)]
    for c in cases[1:]:
        c["seq_params"] = cases[0]["seq_params"]
    rng = np.random.default_rng(9)
    seeds = rng.integers(0, 2**32, seqs, dtype=np.uint64).astype(np.uint32)
    hist = [[int(i) for i in rng.integers(0, vocab, 10 + 9 * s)] for s in range(seqs)]  # seq 5 on wrap past 48
    ring0 = ring_rows(seqs, ring_len, hist)
    pad = 0xFFFFFFFF
    stops = np.full((seqs, 4), pad, np.uint32)
    stops[:, 0] = 151645
    # plant: sequence 2's round-1 next token becomes one of its stop ids
    per0, _, _, _ = oracle_chain(cases, seeds, stops, rounds, ring0, first)
    stops[2, 1] = per0[1]["next"][2]
    per, want_state, want_ring, want_log = oracle_chain(cases, seeds, stops, rounds, ring0, first)
    assert want_state[2, 0] == 1 and (want_log[2, 2:, 0] == 0).all(), "the plant must freeze seq 2 mid-chain"
    print(f"[gpu] spec chain: {rounds} rounds x {seqs} seqs, L={L}, vocab={vocab}, ring {ring_len}", flush=True)
    sp = dev(pack_params(cases[0]["seq_params"]).view(np.uint8))
    hints = row_hints(cases[0]["seq_params"])
    tg = [dev(c["target"]) for c in cases]
    dr = [dev(c["draft"]) for c in cases]
    ids = [torch.zeros((seqs, L), dtype=torch.int32, device="cuda") for _ in range(rounds)]
    picks = [torch.empty((seqs, L + 1), dtype=torch.int32, device="cuda") for _ in range(rounds)]
    acc = [torch.empty(seqs, dtype=torch.int32, device="cuda") for _ in range(rounds)]
    sd, st_d = dev(seeds, torch.int32), dev(stops, torch.int32)
    state = SpecState(seqs, L, max_rounds=rounds, ring_len=ring_len, first_round=first, history=hist)
    init = {k: getattr(state, k).clone() for k in ("state", "ring", "log", "next_tokens")}

    def run(stream=None):
        for r in range(rounds):
            sampler.spec_step_into(tg[r], ids[r], sd, picks[r], acc[r], state, draft_logits=dr[r], seq_params=sp,
                                   row_hints=hints, stop_ids=st_d, stream=stream)

    def reset():
        for k, v in init.items():
            getattr(state, k).copy_(v)

    def check(label):
        u32 = lambda t: t.cpu().numpy().view(np.uint32)  # noqa: E731
        for r in range(rounds):
            live = per[r]["frozen"] == 0
            assert np.array_equal(u32(ids[r]), per[r]["draft_ids"]), f"{label} round {r}: drafts"
            assert np.array_equal(u32(picks[r])[live], per[r]["picks"][live]), f"{label} round {r}: picks"
            assert (u32(picks[r])[~live] == pad).all(), f"{label} round {r}: frozen picks"
            assert np.array_equal(acc[r].cpu().numpy(), per[r]["accepted"]), f"{label} round {r}: accepted"
        assert np.array_equal(u32(state.state), want_state), f"{label}: state"
        assert np.array_equal(u32(state.ring), want_ring), f"{label}: rings"
        assert np.array_equal(u32(state.log), want_log), f"{label}: log"
        assert np.array_equal(u32(state.next_tokens), per[-1]["next"]), f"{label}: next tokens"

    run()
    torch.cuda.synchronize()
    check("eager")
    reset()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(torch.cuda.current_stream())
    torch.cuda.synchronize()
    for rep in range(3):
        for t in picks + acc + ids:
            t.fill_(-7)
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(f"replay {rep}")


def test_spec_step_argument_errors(sampler):
    import torch
    from shared_amd import SpecState
    seqs, L, vocab = 2, 2, 1000
    state = SpecState(seqs, L, max_rounds=1, ring_len=8)
    t = torch.zeros((seqs * (L + 1), vocab), dtype=torch.float32, device="cuda")
    ids = torch.zeros((seqs, L), dtype=torch.int32, device="cuda")
    seeds = torch.zeros(seqs, dtype=torch.int32, device="cuda")
    picks = torch.empty((seqs, L + 1), dtype=torch.int32, device="cuda")
    acc = torch.empty(seqs, dtype=torch.int32, device="cuda")
    h = torch.zeros(4, dtype=torch.int32, device="cuda")
    ho = torch.tensor([0, 2, 4], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="ring"):
        sampler.spec_step_into(t, ids, seeds, picks, acc, state, hist_ids=h, hist_offsets=ho)
    state.ring_len = 0
    with pytest.raises(SasError, match="ring_len"):
        sampler.spec_step_into(t, ids, seeds, picks, acc, state)

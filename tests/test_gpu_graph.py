"""HIP graph capture of the library's entry points.  The reference submits up
to eight decode steps as one command buffer (lib/webgpu-llm/model.js:649-742);
here a caller records its loop into a hipGraph (torch.cuda.graph) and replays
it.  Once a handle's scratch is sized (one eager call of the same shape), a
call issues only kernel launches on the caller's stream: no allocation, no
memset node, no synchronization.  Every replay must equal the same calls run
eagerly, bit for bit, with the program's own eager work and synchronizations
between the replays; a graph over persistent buffers follows their contents."""
import numpy as np
import pytest

from gpu_helpers import to_dev
from shared_amd import DecodeState, Params, Sampler
from shared_amd import workloads as W
from shared_amd._capi import MAX_TOP_K
from shared_amd.sampler import pack_params, row_hints

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _outs(rows):
    import torch
    dev = torch.device("cuda", 0)
    return {"ids": torch.empty(rows, dtype=torch.int32, device=dev),
            "probs": torch.empty((rows, MAX_TOP_K), dtype=torch.float64, device=dev),
            "cand_ids": torch.empty((rows, MAX_TOP_K), dtype=torch.int32, device=dev),
            "counts": torch.empty((rows, 2), dtype=torch.int32, device=dev)}


def _host(d):
    return {k: v.cpu().numpy().copy() for k, v in d.items()}


def _scrub(d):
    # eager work between replays: overwrite what the graph writes
    for v in d.values():
        v.fill_(-7)


def _equal(got, want, label):
    for k in want:
        assert np.array_equal(got[k].view(np.uint8), want[k].view(np.uint8)), f"{label}: {k} differs"


def _capture(fn):
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("ring_len", [64, 2048])  # 2048: the rows' rings are bucketed first (three launches)
def test_decode_steps_in_a_graph(ring_len):
    import torch
    rows, vocab, steps = 8, 50_000, 6
    print(f"[gpu] graph: {steps} decode steps, rows={rows} vocab={vocab} ring_len={ring_len}", flush=True)
    rng = np.random.default_rng(ring_len)
    xs = (rng.standard_normal((steps, rows, vocab)) * 2.0).astype(np.float32)
    xs[:, :, [11, 4_097, 20_011]] += np.float32(6.0)  # tall ids: the ring's penalties decide among them
    xs[2, 3, 77] = np.float32(60.0)                   # row 3 meets its stop id at step 2
    xd = to_dev(xs)
    prm = [Params(temperature=0.8, top_k=40, top_p=0.95, repetition_penalty=1.3, presence_penalty=0.7),
           Params(repetition_penalty=1.5, presence_penalty=2.0),  # greedy with penalties
           Params(temperature=1.1, top_k=64, top_p=0.9, frequency_penalty=0.6)] * 3
    prm = prm[:rows]
    rp = to_dev(pack_params(prm).view(np.uint8))
    hints = row_hints(prm)
    seeds = rng.integers(0, 2**32, rows, dtype=np.uint64).astype(np.uint32)
    history = [[11, 11, 4_097] + [int(i) for i in rng.integers(0, vocab, 40 * r)] for r in range(rows)]
    stop_ids = [[77] if r == 3 else [] for r in range(rows)]
    with Sampler(0) as s:
        st = DecodeState(rows, max_steps=steps, ring_len=ring_len, stop_ids=stop_ids, seeds=seeds, history=history)
        keep = ("state", "sampled", "next_tokens", "ring")
        init = {k: getattr(st, k).clone() for k in keep}
        outs = [_outs(rows) for _ in range(steps)]

        def run():
            for t in range(steps):
                o = outs[t]
                s.sample_step_into(xd[t], o["ids"], st, row_params=rp, row_hints=hints, out_probs=o["probs"],
                                   out_cand_ids=o["cand_ids"], out_counts=o["counts"])

        def reset():
            for k in keep:
                getattr(st, k).copy_(init[k])

        run()
        torch.cuda.synchronize()
        eager = [_host(o) for o in outs]
        eager_state = _host({k: getattr(st, k) for k in keep})
        assert eager_state["state"][3, 0] == 1 and eager[2]["ids"][3] == 77  # the stop froze row 3
        reset()
        g = _capture(run)
        for rep in range(REPLAYS):
            for o in outs:
                _scrub(o)
            reset()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for t in range(steps):
                _equal(_host(outs[t]), eager[t], f"ring {ring_len} replay {rep} step {t}")
            _equal(_host({k: getattr(st, k) for k in keep}), eager_state, f"ring {ring_len} replay {rep} state")


def test_lm_head_in_a_graph():
    import torch
    b = W.lmh(rows=2, vocab=20_000, dim=512, seed=31, hist=300)
    print(f"[gpu] graph: lm head rows={b.rows} vocab={b.vocab} dim={b.dim}", flush=True)
    other = np.random.default_rng(32).standard_normal(b.hidden.shape).astype(np.float32)
    with Sampler(0) as s:
        hid = to_dev(b.hidden)
        wt = to_dev(b.weight_bits.view(np.int16))
        mask = to_dev(b.mask, torch.int32)
        hist = to_dev(b.hist_ids, torch.int32)
        offs = to_dev(b.hist_offsets)
        uni = to_dev(b.uniforms)
        o = _outs(b.rows)
        logits = torch.empty((b.rows, b.vocab), dtype=torch.float32, device=hid.device)

        def run():
            s.lm_head_sample_into(hid, wt, o["ids"], out_logits=logits, mask=mask, hist_ids=hist, hist_offsets=offs,
                                  uniforms=uni, params=b.params, out_probs=o["probs"], out_cand_ids=o["cand_ids"],
                                  out_counts=o["counts"])

        def eager_on(h):
            hid.copy_(torch.from_numpy(h))
            run()
            torch.cuda.synchronize()
            return {**_host(o), "logits": logits.cpu().numpy().copy()}

        want = [eager_on(b.hidden), eager_on(other)]
        assert not np.array_equal(want[0]["logits"], want[1]["logits"])
        g = _capture(run)
        for rep, which in enumerate([0, 1, 0, 1][:REPLAYS + 1]):
            _scrub(o)
            logits.fill_(0.0)
            hid.copy_(torch.from_numpy(b.hidden if which == 0 else other))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            _equal({**_host(o), "logits": logits.cpu().numpy()}, want[which], f"lm head replay {rep} (hidden {which})")


def test_verify_in_a_graph():
    import torch
    inp = W.c5(seqs=8, vocab=30_000, seed=33, drafts=3, density=0.3)
    seqs, L = inp["seqs"], inp["drafts"]
    print(f"[gpu] graph: verify seqs={seqs} drafts={L} vocab={inp['vocab']}", flush=True)
    with Sampler(0) as s:
        t, d = to_dev(inp["target"]), to_dev(inp["draft"])
        m = to_dev(inp["mask"].view(np.int32))
        ids = to_dev(np.ascontiguousarray(inp["draft_ids"], np.uint32).view(np.int32))
        u = to_dev(np.ascontiguousarray(inp["uniforms"], np.float64))
        o = {"tokens": torch.empty((seqs, L + 1), dtype=torch.int32, device=t.device),
             "accepted": torch.empty(seqs, dtype=torch.int32, device=t.device)}

        def run():
            s.verify_into(t, d, ids, u, o["tokens"], o["accepted"], temperature=inp["temperature"], mask=m,
                          vocab=inp["vocab"])

        run()
        torch.cuda.synchronize()
        want = _host(o)
        u2 = np.random.default_rng(34).random(inp["uniforms"].shape)
        u.copy_(torch.from_numpy(u2))
        run()
        torch.cuda.synchronize()
        want2 = _host(o)
        g = _capture(run)
        for rep in range(REPLAYS):
            uu, ww = (inp["uniforms"], want) if rep % 2 == 0 else (u2, want2)
            _scrub(o)
            u.copy_(torch.from_numpy(np.ascontiguousarray(uu, np.float64)))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            _equal(_host(o), ww, f"verify replay {rep}")


def test_reserved_handle_captures_with_no_eager_call():
    """sas_reserve_for sizes every buffer, so a fresh handle's first calls can
    be captured: a decode step whose ring (2,048 ids) is bucketed, the LM
    head and a verify round, in one graph, each replay equal to the same
    calls run eagerly on another handle."""
    import torch
    from shared_amd._capi import SasError
    rows, vocab, ring_len = 4, 20_000, 2048
    print(f"[gpu] graph: reserved handle, step rows={rows} ring={ring_len}, lm head, verify; vocab={vocab}", flush=True)
    rng = np.random.default_rng(41)
    x = to_dev((rng.standard_normal((rows, vocab)) * 2.0).astype(np.float32))
    seeds = rng.integers(0, 2**32, rows, dtype=np.uint64).astype(np.uint32)
    history = [[int(i) for i in rng.integers(0, vocab, 3000)] for _ in range(rows)]
    prm = Params(temperature=0.9, top_k=40, top_p=0.9, repetition_penalty=1.2, frequency_penalty=0.2)
    b = W.lmh(rows=2, vocab=vocab, dim=512, seed=42, hist=300)
    inp = W.c5(seqs=4, vocab=vocab, seed=43, drafts=3, density=0.3)
    seqs, L = inp["seqs"], inp["drafts"]

    def make(s):
        st = DecodeState(rows, max_steps=2, ring_len=ring_len, seeds=seeds, history=history)
        bufs = {"st": st, "init": {k: getattr(st, k).clone() for k in ("state", "sampled", "next_tokens", "ring")},
                "step": _outs(rows), "lmh": _outs(b.rows),
                "hid": to_dev(b.hidden), "wt": to_dev(b.weight_bits.view(np.int16)),
                "mask": to_dev(b.mask, torch.int32), "hist": to_dev(b.hist_ids, torch.int32),
                "offs": to_dev(b.hist_offsets), "uni": to_dev(b.uniforms),
                "t": to_dev(inp["target"]), "d": to_dev(inp["draft"]), "m": to_dev(inp["mask"].view(np.int32)),
                "ids": to_dev(np.ascontiguousarray(inp["draft_ids"], np.uint32).view(np.int32)),
                "u": to_dev(np.ascontiguousarray(inp["uniforms"], np.float64)),
                "tok": torch.empty((seqs, L + 1), dtype=torch.int32, device="cuda"),
                "acc": torch.empty(seqs, dtype=torch.int32, device="cuda")}

        def run():
            o = bufs["step"]
            s.sample_step_into(x, o["ids"], bufs["st"], params=prm, out_probs=o["probs"], out_cand_ids=o["cand_ids"],
                               out_counts=o["counts"])
            o = bufs["lmh"]
            s.lm_head_sample_into(bufs["hid"], bufs["wt"], o["ids"], mask=bufs["mask"], hist_ids=bufs["hist"],
                                  hist_offsets=bufs["offs"], uniforms=bufs["uni"], params=b.params,
                                  out_probs=o["probs"], out_cand_ids=o["cand_ids"], out_counts=o["counts"])
            s.verify_into(bufs["t"], bufs["d"], bufs["ids"], bufs["u"], bufs["tok"], bufs["acc"],
                          temperature=inp["temperature"], mask=bufs["m"], vocab=vocab)

        def reset():
            for k, v in bufs["init"].items():
                getattr(bufs["st"], k).copy_(v)

        def host():
            st = bufs["st"]
            return {**{"step_" + k: v for k, v in _host(bufs["step"]).items()},
                    **{"lmh_" + k: v for k, v in _host(bufs["lmh"]).items()},
                    "tok": bufs["tok"].cpu().numpy().copy(), "acc": bufs["acc"].cpu().numpy().copy(),
                    **_host({k: getattr(st, k) for k in ("state", "sampled", "next_tokens", "ring")})}

        def scrub():
            for d in (bufs["step"], bufs["lmh"]):
                _scrub(d)
            bufs["tok"].fill_(-7)
            bufs["acc"].fill_(-7)
        return run, reset, host, scrub

    with Sampler(0) as e:
        run, reset, host, _ = make(e)
        run()
        torch.cuda.synchronize()
        want = host()
    with Sampler(0) as s:
        s.reserve(rows, vocab, hist_ids=rows * ring_len, lm_head_rows=b.rows, verify_seqs=seqs, verify_draft_len=L)
        run, reset, host, scrub = make(s)
        g = _capture(run)
        for rep in range(REPLAYS):
            scrub()
            reset()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            _equal(host(), want, f"reserved handle replay {rep}")
        # a shape past the reservation cannot grow scratch under capture: the
        # call fails with the reason and records nothing
        big = to_dev(np.zeros((64, vocab), np.float32))
        big_ids = torch.empty(64, dtype=torch.int32, device="cuda")
        g2 = torch.cuda.CUDAGraph()
        err = None
        with torch.cuda.graph(g2):
            try:
                s.sample_into(big, big_ids, vocab=vocab, params=Params())
            except SasError as ex:
                err = str(ex)
        torch.cuda.synchronize()
        assert err is not None and "being captured" in err, err

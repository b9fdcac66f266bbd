"""GPU parity of sas_lm_head_sample (the LM head with the sampling step fused
into its epilogue) through the C ABI:
  - the head's logits (out_logits) bit-exact with the oracle's summation
    order (orc_lm_head_logits: eight fused multiply-add chains, a fixed tree);
  - ids, ranked candidates, {k, cut}, probabilities and flags bit-exact with
    the sampling oracle over those logits;
  - the fused call without out_logits gives the same ids, and so does
    sas_sample over the logits the head wrote (the unfused path)."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import assert_parity, run_gpu, to_dev
from shared_amd import Params, pack_params
from shared_amd import workloads as W
from shared_amd._capi import FLAG_EMPTY_ROW, FLAG_SLOW_SELECT, NO_TOKEN
from shared_amd.sampler import row_hints

pytestmark = pytest.mark.gpu


def run_lmh(s, b: W.LmhBatch, *, logits=True, row_params=None):
    import torch
    kw = {}
    if row_params is not None:
        kw["row_params"] = to_dev(pack_params(row_params).view(np.uint8))
        kw["row_hints"] = row_hints(row_params)
    wt = to_dev(b.weight_bits.view(np.int16)) if b.fmt == W.HEAD_BF16 else to_dev(b.weight_q)
    out = s.lm_head_sample(to_dev(b.hidden), wt, full=True, logits=logits, fmt=b.fmt,
                           mask=to_dev(b.mask, torch.int32) if b.mask is not None else None,
                           hist_ids=to_dev(b.hist_ids, torch.int32) if b.hist_ids is not None else None,
                           hist_offsets=to_dev(b.hist_offsets) if b.hist_offsets is not None else None,
                           uniforms=to_dev(b.uniforms) if b.uniforms is not None else None, params=b.params, **kw)
    torch.cuda.synchronize()
    g = {"ids": out["ids"].cpu().numpy().view(np.uint32), "probs": out["probs"].cpu().numpy(),
         "cand_ids": out["cand_ids"].cpu().numpy().view(np.uint32), "counts": out["counts"].cpu().numpy(),
         "flags": out["flags"].cpu().numpy().view(np.uint32)}
    if logits:
        g["logits"] = out["logits"].cpu().numpy()
        g["logits_dev"] = out["logits"]
    return g


def check(s, b: W.LmhBatch, label: str, row_params=None):
    print(f"[gpu] lm head {label}: rows={b.rows} vocab={b.vocab} dim={b.dim}", flush=True)
    g = run_lmh(s, b, row_params=row_params)
    lo = O.lm_head_logits(b.hidden, b.weight_bits) if b.fmt == W.HEAD_BF16 else \
        O.lm_head_q_logits(b.fmt, b.hidden, b.weight_q)
    bad = np.nonzero(g["logits"].view(np.uint32) != lo.view(np.uint32))
    assert bad[0].size == 0, f"{label}: logits differ at {list(zip(*bad))[:4]}"
    o = O.sample_rows(b.with_logits(lo), row_params=row_params)
    assert_parity(g, o, label)
    # the fused call alone, and the unfused path over the head's own logits
    f = run_lmh(s, b, logits=False, row_params=row_params)
    assert np.array_equal(f["ids"], g["ids"]), f"{label}: fused ids differ from the logits-writing call"
    u = run_gpu(s, b.with_logits(lo), logits_dev=g["logits_dev"], row_params=row_params)
    assert_parity(u, o, label + " (unfused)")
    return g, o


def test_gemma_decode_full_size(sampler):
    # Gemma-4 E4B shape: one decode row, vocab 262,144, hidden 2,560, softcap 30
    check(sampler, W.lmh(rows=1), "gemma decode")


def test_gemma_verify_rows(sampler):
    # a speculative round's three verify rows over the same head
    check(sampler, W.lmh(rows=3, vocab=W.GEMMA_VOCAB, dim=1024, seed=8), "gemma verify rows")


def test_qwen_rows_with_row_params(sampler):
    b = W.lmh(rows=4, vocab=W.QWEN_VOCAB, dim=768, seed=9, softcap=0.0)
    rp = [Params(temperature=0.0, top_k=1),
          Params(temperature=0.7, top_k=40, top_p=0.95, presence_penalty=0.5),
          Params(temperature=1.3, top_k=128, top_p=1.0, repetition_penalty=1.3, frequency_penalty=0.2),
          Params(temperature=1.0, top_k=5, top_p=0.5, softcap=30.0)]
    check(sampler, b, "qwen row params", row_params=rp)


@pytest.mark.parametrize("vocab,dim,rows", [(1, 256, 1), (300, 256, 2), (4097, 256, 4), (20000, 3072, 2)])
def test_shapes(sampler, vocab, dim, rows):
    check(sampler, W.lmh(rows=rows, vocab=vocab, dim=dim, seed=vocab + dim, hist=min(512, vocab)),
          f"shape v{vocab} d{dim}")


def test_long_history_and_unmasked(sampler):
    b = W.lmh(rows=2, vocab=30000, dim=256, seed=11, hist=4096, mask=False)
    check(sampler, b, "long history")


def test_members_fill_a_part(sampler):
    # every id of the first 1,024 is in the history with identity penalties:
    # parts 0 and 1 hold only members (more than a part's member slots), so
    # their exact slow selection runs
    b = W.lmh(rows=1, vocab=4096, dim=256, seed=12, hist=0, mask=False)
    ids = np.arange(1024, dtype=np.uint32)
    b.hist_ids, b.hist_offsets = ids, np.array([0, ids.size], np.int32)
    b.params = Params(temperature=1.0, top_k=50, top_p=0.9)
    g, _ = check(sampler, b, "members fill a part")
    b.hidden[:] = 0.0
    b.hidden[0, 0] = 1.0  # logits = the heads' first column: ids 0..1023 lead
    b.weight_bits[:, 0] = 0x3F80          # 1.0 everywhere
    b.weight_bits[1024:, 0] = 0x3F00      # 0.5 past the history
    g, _ = check(sampler, b, "members lead")
    assert g["flags"][0] & FLAG_SLOW_SELECT


def test_ties_rank_by_id(sampler):
    # identical head rows give identical logits: the lowest ids rank first
    b = W.lmh(rows=2, vocab=2048, dim=256, seed=13, hist=0, mask=False)
    b.weight_bits[:] = b.weight_bits[7]
    b.params = Params(temperature=0.0, top_k=1)
    g, _ = check(sampler, b, "ties greedy")
    assert list(g["ids"]) == [0, 0]
    b.params = Params(temperature=1.0, top_k=20, top_p=1.0)
    g, _ = check(sampler, b, "ties sampled")
    assert list(g["cand_ids"][0, :20]) == list(range(20))


def test_empty_rows(sampler):
    b = W.lmh(rows=2, vocab=5000, dim=256, seed=14, hist=0)
    b.mask[1, :] = 0
    g, _ = check(sampler, b, "empty row")
    assert g["ids"][1] == NO_TOKEN and g["flags"][1] & FLAG_EMPTY_ROW


def test_strided_head_and_broadcast_mask(sampler):
    # hidden rows and head rows wider than dim (hidden_stride 544, weight
    # stride 520), one mask row for every row (mask_stride 0)
    import torch
    b = W.lmh(rows=3, vocab=70000, dim=512, seed=15, hist=300)
    rng = np.random.default_rng(15)
    hid_w = np.zeros((3, 544), np.float32)
    hid_w[:, :512] = b.hidden
    hid_w[:, 512:] = rng.standard_normal((3, 32)).astype(np.float32)  # never read
    w_w = np.zeros((b.vocab, 520), np.uint16)
    w_w[:, :512] = b.weight_bits
    w_w[:, 512:] = 0x7FC0  # NaN bits: a read past dim would show
    b.mask[:] = b.mask[0]
    b.params = Params(temperature=0.8, top_k=20, top_p=0.9, repetition_penalty=1.2, presence_penalty=0.3)
    print(f"[gpu] lm head strided: rows={b.rows} vocab={b.vocab} dim={b.dim}", flush=True)
    hid = to_dev(hid_w)[:, :512]
    wt = to_dev(w_w.view(np.int16))[:, :512]
    mask_row = to_dev(b.mask[:1], torch.int32)
    out = sampler.lm_head_sample(hid, wt, full=True, logits=True, dim=512,
                                 mask=mask_row.expand(b.rows, -1),
                                 hist_ids=to_dev(b.hist_ids, torch.int32), hist_offsets=to_dev(b.hist_offsets),
                                 uniforms=to_dev(b.uniforms), params=b.params)
    torch.cuda.synchronize()
    lo = O.lm_head_logits(b.hidden, b.weight_bits)
    got = out["logits"].cpu().numpy()
    assert np.array_equal(got.view(np.uint32), lo.view(np.uint32))
    g = {"ids": out["ids"].cpu().numpy().view(np.uint32), "probs": out["probs"].cpu().numpy(),
         "cand_ids": out["cand_ids"].cpu().numpy().view(np.uint32), "counts": out["counts"].cpu().numpy(),
         "flags": out["flags"].cpu().numpy().view(np.uint32)}
    assert_parity(g, O.sample_rows(b.with_logits(lo)), "lm head strided")


def test_greedy_rows(sampler):
    # temperature 0: the best penalized (value, id) of every row
    b = W.lmh(rows=4, vocab=W.QWEN_VOCAB, dim=256, seed=16, softcap=0.0)
    b.params = Params(temperature=0.0, top_k=1, repetition_penalty=1.3, frequency_penalty=0.5)
    g, o = check(sampler, b, "greedy rows")
    assert np.array_equal(g["ids"], o["ids"])


def test_random_sweep(sampler):
    # 40 seeded random cases: 1-4 rows, dim 256-3072 within the LDS limit,
    # vocabularies from 1 to 50,000, masks, histories, softcap, greedy rows,
    # penalties that lower or raise values, per-row params
    for case in range(40):
        rng = np.random.default_rng(90000 + case)
        rows = int(rng.integers(1, 5))
        dim = int(rng.choice([d for d in range(256, 3073, 256) if rows * d <= 12288]))
        vocab = int(rng.choice([1, 5, 300, 513, 4097, 20000, 50000]))
        b = W.lmh(rows=rows, vocab=vocab, dim=dim, seed=90000 + case,
                  hist=int(rng.choice([0, 16, 600])) if vocab > 16 else 0, softcap=float(rng.choice([0.0, 30.0])),
                  mask=bool(rng.random() < 0.6))

        def params():
            return Params(temperature=float(rng.choice([0.0, 0.7, 1.0])), top_k=int(rng.integers(1, 129)),
                          top_p=float(rng.choice([1.0, 0.9])), repetition_penalty=float(rng.choice([1.0, 1.2, 0.8])),
                          presence_penalty=float(rng.choice([0.0, 0.5])),
                          frequency_penalty=float(rng.choice([0.0, 0.3])), softcap=float(rng.choice([0.0, 30.0])))
        b.params = params()
        rp = [params() for _ in range(rows)] if rng.random() < 0.3 else None
        check(sampler, b, f"sweep {case}: rows={rows} dim={dim} vocab={vocab}", row_params=rp)


# ---------------------------------------------------------------- GGUF heads --

def test_qwen_q6k_head_full_size(sampler):
    """Qwen3.5-4B's tied Q6_K head (gguf/sources.js:122): vocabulary 248,320,
    hidden 2,560, one decode row."""
    check(sampler, W.lmhq(W.HEAD_Q6_K, rows=1), "qwen q6_k decode")


def test_qwen_q6k_verify_rows(sampler):
    check(sampler, W.lmhq(W.HEAD_Q6_K, rows=3, seed=12), "qwen q6_k verify rows")


@pytest.mark.parametrize("fmt", [W.HEAD_Q8_0, W.HEAD_Q4_0])
def test_gemma_shape_q8_0_q4_0(sampler, fmt):
    check(sampler, W.lmhq(fmt, rows=1, vocab=W.GEMMA_VOCAB, dim=2560, seed=13 + fmt, softcap=30.0),
          f"gemma-shaped {W.HEAD_NAMES[fmt]}")


@pytest.mark.parametrize("fmt,vocab,dim,rows", [(W.HEAD_Q6_K, 300, 256, 2), (W.HEAD_Q6_K, 4097, 768, 4),
                                                (W.HEAD_Q6_K, 20000, 1280, 3), (W.HEAD_Q8_0, 777, 256, 4),
                                                (W.HEAD_Q4_0, 5000, 512, 2), (W.HEAD_Q8_0, 1, 256, 1),
                                                (W.HEAD_Q6_K, 6000, 2304, 1), (W.HEAD_Q6_K, 5000, 2304, 2),
                                                (W.HEAD_Q8_0, 2000, 1280, 3), (W.HEAD_Q4_0, 3000, 768, 3),
                                                (W.HEAD_Q4_0, 999, 256, 4), (W.HEAD_Q8_0, 333, 2560, 2)])
def test_gguf_shapes(sampler, fmt, vocab, dim, rows):
    # dims of 256, 768 and 2304 leave lanes with fewer Q6_K units than
    # others; at 2304 a row is 9 super-blocks (1,890 bytes), so consecutive
    # rows alternate between 4-byte and 2-byte alignment
    check(sampler, W.lmhq(fmt, rows=rows, vocab=vocab, dim=dim, seed=vocab + dim + fmt, hist=min(300, vocab)),
          f"{W.HEAD_NAMES[fmt]} {rows}x{vocab}x{dim}")


def test_gguf_head_with_a_row_stride(sampler):
    """Rows further apart than their blocks (a stride of the row's bytes plus
    padding), one Q6_K row length odd in super-blocks (2-byte aligned rows)."""
    import torch
    b = W.lmhq(W.HEAD_Q6_K, rows=2, vocab=3000, dim=768, seed=21)
    rb = b.weight_q.shape[1]
    padded = np.zeros((b.vocab, rb + 6), np.uint8)
    padded[:, :rb] = b.weight_q
    dev_w = to_dev(padded)[:, :rb]
    print(f"[gpu] lm head q6_k strided rows: stride {rb + 6} bytes, row {rb}", flush=True)
    out = sampler.lm_head_sample(to_dev(b.hidden), dev_w, full=True, logits=True, fmt=W.HEAD_Q6_K,
                                 mask=to_dev(b.mask, torch.int32), hist_ids=to_dev(b.hist_ids, torch.int32),
                                 hist_offsets=to_dev(b.hist_offsets), uniforms=to_dev(b.uniforms), params=b.params)
    torch.cuda.synchronize()
    lo = O.lm_head_q_logits(W.HEAD_Q6_K, b.hidden, b.weight_q)
    assert np.array_equal(out["logits"].cpu().numpy().view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(out["ids"].cpu().numpy().view(np.uint32), O.sample_rows(b.with_logits(lo))["ids"])


def test_gguf_head_argument_errors(sampler):
    import torch
    from shared_amd import SasError
    hid = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    w = torch.zeros((10, 210), dtype=torch.uint8, device="cuda")
    short = torch.zeros((10, 200), dtype=torch.uint8, device="cuda")  # rows of 200 < 210 bytes
    with pytest.raises(SasError, match="weight_stride"):
        sampler.lm_head_sample(hid, short, fmt=W.HEAD_Q6_K, params=Params())
    with pytest.raises(SasError, match="format"):
        sampler.lm_head_sample(hid, w, fmt=7, params=Params())
    with pytest.raises(SasError, match="aligned"):
        sampler.lm_head_sample(hid, w.view(-1)[2:2 + 9 * 210].view(9, 210), fmt=W.HEAD_Q6_K, params=Params())
    # rows 2^31 bytes apart: three rows span more than 4 GiB (rejected
    # before anything is read)
    import ctypes
    from shared_amd import _capi
    from shared_amd.sampler import rows_descriptor
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    h = sampler._head(hid, w, None, None, W.HEAD_Q6_K)
    h.weight_stride = 1 << 31
    d = rows_descriptor(hid, out, vocab=3, params=Params())
    d.logits = None
    d.logits_stride = 0
    lib = _capi.load()
    rc = lib.sas_lm_head_sample(sampler._h, ctypes.byref(h), ctypes.byref(d), None)
    assert rc == _capi.ERR_INVALID
    assert b"4 GiB" in lib.sas_last_error(sampler._h)


@pytest.mark.parametrize("fmt", [W.HEAD_BF16, W.HEAD_Q6_K])
def test_fused_head_decode_steps(sampler, fmt):
    """sas_lm_head_sample_step: k steps of the in-graph decode loop with the
    head fused (the reference's per-iteration lm -> topk -> sampler with
    tokens[0] fed back, model.js:711-717): every step's token, candidates and
    probabilities, and the state (stop flags, iterations, sampled, next
    tokens, rings) equal the oracle's head logits stepped with the sampling
    oracle; a planted stop freezes one row mid-loop."""
    import torch
    from gpu_helpers import oracle_steps, ring_of
    from shared_amd import DecodeState
    from shared_amd._capi import MAX_TOP_K
    rows, steps, vocab, dim, ring_len = 3, 5, 20_000, 512, 64
    rng = np.random.default_rng(50 + fmt)
    if fmt == W.HEAD_BF16:
        b = W.lmh(rows=rows, vocab=vocab, dim=dim, seed=51, hist=0, softcap=30.0, mask=True)
        wt = to_dev(b.weight_bits.view(np.int16))
        logits_of = lambda h: O.lm_head_logits(h, b.weight_bits)  # noqa: E731
    else:
        b = W.lmhq(fmt, rows=rows, vocab=vocab, dim=dim, seed=52, hist=0, mask=True)
        wt = to_dev(b.weight_q)
        logits_of = lambda h: O.lm_head_q_logits(fmt, h, b.weight_q)  # noqa: E731
    hs = rng.standard_normal((steps, rows, dim)).astype(np.float32)
    xs = np.stack([logits_of(hs[t]) for t in range(steps)])
    # row 1's step-2 token is its stop id
    prm = [Params(temperature=0.9, top_k=40, top_p=0.9, repetition_penalty=1.2, presence_penalty=0.4,
                  softcap=b.params.softcap)] * rows
    seeds = rng.integers(0, 2**32, rows, dtype=np.uint64).astype(np.uint32)
    history = [[int(i) for i in rng.integers(0, vocab, 20)] for _ in range(rows)]
    free, _, _, _ = oracle_steps(xs, prm, mask=b.mask, seeds=seeds, history=history, ring_len=ring_len)
    stop_ids = [[], [int(free[2]["ids"][1])], []]
    want, stopped, it, window = oracle_steps(xs, prm, mask=b.mask, seeds=seeds, history=history, ring_len=ring_len,
                                             stop_ids=stop_ids)
    assert stopped[1], "the planted stop must freeze row 1"
    print(f"[gpu] fused head decode steps {W.HEAD_NAMES[fmt]}: {steps} x {rows} rows, vocab {vocab}", flush=True)
    st = DecodeState(rows, max_steps=steps, ring_len=ring_len, stop_ids=stop_ids, seeds=seeds, history=history)
    rp = to_dev(pack_params(prm).view(np.uint8))
    mask = to_dev(b.mask, torch.int32)
    ids = torch.empty(rows, dtype=torch.int32, device="cuda")
    probs = torch.empty((rows, MAX_TOP_K), dtype=torch.float64, device="cuda")
    cand = torch.empty((rows, MAX_TOP_K), dtype=torch.int32, device="cuda")
    for t in range(steps):
        sampler.lm_head_step_into(to_dev(hs[t]), wt, ids, st, fmt=fmt, mask=mask, row_params=rp,
                                  row_hints=row_hints(prm), out_probs=probs, out_cand_ids=cand)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy().view(np.uint32), want[t]["ids"]), f"step {t}: ids"
        assert np.array_equal(cand.cpu().numpy().view(np.uint32), want[t]["cand_ids"]), f"step {t}: candidates"
        assert np.array_equal(probs.cpu().numpy().view(np.uint64), want[t]["probs"].view(np.uint64)), f"step {t}: probs"
    sv = st.state.cpu().numpy()
    assert sv[:, 0].tolist() == [int(x) for x in stopped] and sv[:, 1].tolist() == it
    sampled = st.sampled.cpu().numpy().view(np.uint32)
    ring = st.ring.cpu().numpy().view(np.uint32)
    for r in range(rows):
        assert sampled[r].tolist() == [int(w["ids"][r]) for w in want], f"sampled row {r}"
        assert np.array_equal(ring[r], ring_of(window[r], ring_len)), f"ring row {r}"
    assert np.array_equal(st.next_tokens.cpu().numpy().view(np.uint32), want[-1]["ids"])

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
    out = s.lm_head_sample(to_dev(b.hidden), to_dev(b.weight_bits.view(np.int16)), full=True, logits=logits,
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
    lo = O.lm_head_logits(b.hidden, b.weight_bits)
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

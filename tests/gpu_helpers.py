"""Helpers shared by the GPU parity tests: run a Batch through the HIP path
and the oracle on the same inputs and compare."""
from __future__ import annotations

import numpy as np

import oracle as O
from shared_amd import Sampler
from shared_amd._capi import FLAG_DRAW_EDGE, FLAG_EMPTY_ROW, FLAG_TOPP_EDGE

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

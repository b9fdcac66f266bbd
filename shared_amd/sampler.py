"""Python handle over the C ABI, for tests and benchmarks.

Device buffers are torch CUDA tensors (plumbing only): every computation
runs in the HIP kernels of libshared_amd_sampler.so, on torch's current
stream unless another is given.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _capi
from ._capi import SasLmHead, SasParams, SasRows, SasSpecRows, SasVerifyRows, check, load


@dataclass
class Params:
    """One row's sampling parameters (sas_params)."""

    temperature: float = 0.0
    top_k: int = 1
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    softcap: float = 0.0

    def to_c(self) -> SasParams:
        return SasParams(float(self.temperature), float(self.top_p), float(self.repetition_penalty),
                         float(self.presence_penalty), float(self.frequency_penalty), float(self.softcap),
                         int(self.top_k))

    def as_dict(self) -> dict:
        return {"temperature": self.temperature, "top_k": self.top_k, "top_p": self.top_p,
                "repetition_penalty": self.repetition_penalty, "presence_penalty": self.presence_penalty,
                "frequency_penalty": self.frequency_penalty, "softcap": self.softcap}


PARAMS_DTYPE = np.dtype([("temperature", "<f8"), ("top_p", "<f8"), ("repetition_penalty", "<f8"),
                         ("presence_penalty", "<f8"), ("frequency_penalty", "<f8"), ("softcap", "<f4"),
                         ("top_k", "<i4")])
assert PARAMS_DTYPE.itemsize == ctypes.sizeof(SasParams)


def pack_params(rows: Sequence[Params]) -> np.ndarray:
    """Array of sas_params (for row_params)."""
    out = np.zeros(len(rows), dtype=PARAMS_DTYPE)
    for i, p in enumerate(rows):
        out[i] = (p.temperature, p.top_p, p.repetition_penalty, p.presence_penalty, p.frequency_penalty,
                  p.softcap, p.top_k)
    return out


def clamp_params(p: Params) -> Params:
    """The reference packer's clamps (sas_clamp_params)."""
    out = SasParams()
    check(load().sas_clamp_params(ctypes.byref(p.to_c()), ctypes.byref(out)))
    return Params(out.temperature, out.top_k, out.top_p, out.repetition_penalty, out.presence_penalty,
                  out.frequency_penalty, out.softcap)


def mask_from_ids(kind: int, ids, vocab: int) -> np.ndarray:
    """Packed uint32 bitmask of a TokenMask (sas_mask_from_ids)."""
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
    words = np.zeros((vocab + 31) // 32, dtype=np.uint32)
    n = load().sas_mask_from_ids(int(kind), ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size,
                                 int(vocab), words.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), words.size)
    if n < 0:
        check(-n)
    return words


def check_history(offsets, count: int) -> None:
    """Validate CSR history offsets on the host: int32 [rows + 1], starting
    at >= 0, non-decreasing, ending at <= count ids, each row at most
    MAX_HISTORY ids.  Raises ValueError naming the first bad row."""
    o = np.asarray(offsets)
    if o.ndim != 1 or o.size < 1:
        raise ValueError("hist_offsets must be a 1-D array of rows + 1 offsets")
    o = o.astype(np.int64)
    if o[0] < 0:
        raise ValueError(f"hist_offsets[0] = {o[0]} is negative")
    d = np.diff(o)
    bad = np.nonzero(d < 0)[0]
    if bad.size:
        raise ValueError(f"hist_offsets decrease at row {int(bad[0])}")
    big = np.nonzero(d > _capi.MAX_HISTORY)[0]
    if big.size:
        raise ValueError(f"row {int(big[0])} holds {int(d[big[0]])} history ids; at most {_capi.MAX_HISTORY}")
    if o[-1] > count:
        raise ValueError(f"hist_offsets end at {int(o[-1])} but hist_ids holds {count} ids")


def row_hints(rows: Sequence[Params]) -> int:
    """SAS_HINT_* bits that hold for every row of a per-row parameter list."""
    return _capi.HINT_NO_SOFTCAP if all(not (p.softcap > 0) for p in rows) else 0


# Element types the C ABI reads: 4-byte integers (ids, offsets, mask words,
# seeds, counts, flags; int32 or uint32), float64 (uniforms, probabilities)
# and float32 (logits).  A tensor of another width would be read as the
# wrong values, so it is refused here.
_KINDS = {"i32": (4, False), "f64": (8, True), "f32": (4, True)}


def _ptr(t, kind: Optional[str] = None, name: str = "tensor") -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("device tensors are required")
    if not t.is_contiguous() and t.dim() == 1:
        raise ValueError("1-D inputs must be contiguous")
    if kind is not None:
        size, fp = _KINDS[kind]
        if t.element_size() != size or t.dtype.is_floating_point != fp:
            want = f"float{8 * size}" if fp else f"{8 * size}-bit integer"
            raise ValueError(f"{name} must hold {want} elements (got {t.dtype})")
    return t.data_ptr()


def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def rows_descriptor(logits, out_ids, *, vocab: Optional[int] = None, mask=None, hist_ids=None, hist_offsets=None,
                    uniforms=None, params: Optional[Params] = None, row_params=None, out_probs=None,
                    out_cand_ids=None, out_counts=None, out_flags=None, row_hints: int = 0) -> SasRows:
    """The sas_rows descriptor of torch device tensors."""
    rows = logits.shape[0]
    vocab = int(vocab if vocab is not None else logits.shape[1])
    if logits.dtype.itemsize != 4 or logits.stride(1) != 1:
        raise ValueError("logits must be fp32 with unit element stride")
    d = SasRows()
    d.logits = logits.data_ptr()
    d.logits_stride = logits.stride(0)
    d.vocab = vocab
    d.rows = rows
    if mask is not None:
        d.mask = _ptr(mask, "i32", "mask")
        d.mask_stride = mask.stride(0)
    d.hist_ids = _ptr(hist_ids, "i32", "hist_ids")
    d.hist_offsets = _ptr(hist_offsets, "i32", "hist_offsets")
    d.hist_count = hist_ids.numel() if hist_ids is not None else 0
    d.row_hints = int(row_hints)
    d.uniforms = _ptr(uniforms, "f64", "uniforms")
    d.params = (params or Params()).to_c()
    d.row_params = _ptr(row_params)
    d.out_ids = _ptr(out_ids, "i32", "out_ids")
    d.out_probs = _ptr(out_probs, "f64", "out_probs")
    d.out_cand_ids = _ptr(out_cand_ids, "i32", "out_cand_ids")
    d.out_counts = _ptr(out_counts, "i32", "out_counts")
    d.out_flags = _ptr(out_flags, "i32", "out_flags")
    return d


def sample_noalloc_into(device: int, logits, out_ids, *, stream=None, **kw) -> None:
    """sas_sample_noalloc on caller-provided device buffers: no allocation
    at all (the scratch is the library's static device array)."""
    d = rows_descriptor(logits, out_ids, **kw)
    check(load().sas_sample_noalloc(int(device), ctypes.byref(d), _stream(stream)), None)


class SpecState:
    """The caller-owned device state of sas_spec_step for `seqs` sequences
    with `draft_len` drafts: {frozen, round, pos, accepted} per sequence (the
    reference's ctl[0], posBuf[4], posBuf[0], posBuf[1]), the penalty ring,
    the per-round log {a, next, drafts} and the next input tokens
    (kernels.js:340-367 keeps the same state for one sequence)."""

    def __init__(self, seqs: int, draft_len: int, *, max_rounds: int, ring_len: int = 512, first_round: int = 0,
                 pos=None, history=None, device=0):
        import torch
        if not 1 <= ring_len <= _capi.MAX_HISTORY:
            raise ValueError("ring_len must be in [1, SAS_MAX_HISTORY]")
        dev = torch.device("cuda", device) if isinstance(device, int) else device
        self.seqs, self.draft_len, self.max_rounds, self.ring_len = seqs, draft_len, max_rounds, ring_len
        st = np.zeros((seqs, 4), dtype=np.uint32)
        st[:, 1] = first_round
        if pos is not None:
            st[:, 2] = np.asarray(pos, dtype=np.uint32)
        self.state = torch.from_numpy(st.view(np.int32)).to(dev)
        self.ring = torch.from_numpy(ring_rows(seqs, ring_len, history).view(np.int32)).to(dev)
        self.log = torch.zeros((seqs, max_rounds, draft_len + 2), dtype=torch.int32, device=dev)
        self.next_tokens = torch.full((seqs,), -1, dtype=torch.int32, device=dev)

    def descriptor(self):
        from ._capi import SasSpecState
        d = SasSpecState()
        d.state = self.state.data_ptr()
        d.ring = self.ring.data_ptr()
        d.ring_len = self.ring_len
        d.log = self.log.data_ptr()
        d.max_rounds = self.max_rounds
        d.next_tokens = self.next_tokens.data_ptr()
        return d


def ring_rows(rows: int, ring_len: int, history=None) -> np.ndarray:
    """uint32 [rows][1 + ring_len] rings {count, ids}: the last ring_len ids
    of each row's window, id i of the window at slot i % ring_len."""
    ring = np.zeros((rows, 1 + ring_len), dtype=np.uint32)
    for r, h in enumerate(history or []):
        h = [int(x) for x in h]
        for i in range(max(0, len(h) - ring_len), len(h)):
            ring[r, 1 + i % ring_len] = h[i]
        ring[r, 0] = len(h)
    return ring


class DecodeState:
    """The caller-owned device state of sas_sample_step for `rows` sequences:
    {stopped, iteration} per row, the sampled tokens, the next input token,
    the penalty ring, the stop ids and the seeds (kernels.js:63-200 keeps the
    same state for one sequence)."""

    def __init__(self, rows: int, *, max_steps: int, ring_len: int = 512, stop_ids=None, seeds=None,
                 history=None, device=0):
        import torch
        if not 1 <= ring_len <= _capi.MAX_HISTORY:
            raise ValueError("ring_len must be in [1, SAS_MAX_HISTORY]")
        dev = torch.device("cuda", device) if isinstance(device, int) else device
        self.rows, self.max_steps, self.ring_len = rows, max_steps, ring_len
        self.state = torch.zeros((rows, 2), dtype=torch.int32, device=dev)
        self.sampled = torch.full((rows, max_steps), -1, dtype=torch.int32, device=dev)
        self.next_tokens = torch.full((rows,), -1, dtype=torch.int32, device=dev)
        self.ring = torch.from_numpy(ring_rows(rows, ring_len, history).view(np.int32)).to(dev)
        self.stop_ids = None
        if stop_ids is not None:
            st = np.full((rows, 4), _capi.STOP_PAD, dtype=np.uint32)
            for r, ids in enumerate(stop_ids):
                ids = list(ids)[:4]
                st[r, :len(ids)] = ids
            self.stop_ids = torch.from_numpy(st.view(np.int32)).to(dev)
        self.seeds = None
        if seeds is not None:
            self.seeds = torch.from_numpy(np.asarray(seeds, dtype=np.uint32).view(np.int32)).to(dev)

    def descriptor(self):
        from ._capi import SasStep
        d = SasStep()
        d.state = self.state.data_ptr()
        d.sampled = self.sampled.data_ptr()
        d.max_steps = self.max_steps
        d.next_tokens = self.next_tokens.data_ptr()
        d.ring = self.ring.data_ptr()
        d.ring_len = self.ring_len
        d.stop_ids = _ptr(self.stop_ids)
        d.seeds = _ptr(self.seeds)
        return d


class Sampler:
    """A sas_sampler handle bound to one device."""

    def __init__(self, device: int = 0):
        self._lib = load()
        h = ctypes.c_void_p()
        rc = self._lib.sas_create(int(device), ctypes.byref(h))
        check(rc, None)
        self._h = h
        self.device = device

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.sas_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reserve(self, rows: int, vocab: int, *, hist_ids: int = 0, lm_head_rows: int = 0, verify_seqs: int = 0,
                verify_draft_len: int = 0) -> None:
        """Pre-size the handle's scratch (sas_reserve_for): calls of at most
        these shapes then allocate nothing and can be captured directly."""
        from ._capi import SasReserveDesc
        d = SasReserveDesc(int(rows), int(vocab), int(hist_ids), int(lm_head_rows), int(verify_seqs),
                           int(verify_draft_len))
        check(self._lib.sas_reserve_for(self._h, ctypes.byref(d)), self._h)

    def sample_into(self, logits, out_ids, *, stream=None, **kw) -> None:
        """Launch sas_sample on caller-provided device buffers (no allocation,
        no synchronisation: the history offsets are not checked here, the
        kernels clamp them to hist_ids' length)."""
        d = rows_descriptor(logits, out_ids, **kw)
        check(self._lib.sas_sample(self._h, ctypes.byref(d), _stream(stream)), self._h)

    def sample(self, logits, *, full: bool = False, **kw):
        """Allocate outputs and sample; returns ids (and the extras if full).
        The history offsets are checked on the host first."""
        import torch
        if kw.get("hist_ids") is not None:
            if kw.get("hist_offsets") is None:
                raise ValueError("hist_ids requires hist_offsets")
            check_history(kw["hist_offsets"].cpu().numpy(), kw["hist_ids"].numel())
        rows = logits.shape[0]
        dev = logits.device
        out = {"ids": torch.empty(rows, dtype=torch.int32, device=dev)}
        if full:
            out["probs"] = torch.empty((rows, _capi.MAX_TOP_K), dtype=torch.float64, device=dev)
            out["cand_ids"] = torch.empty((rows, _capi.MAX_TOP_K), dtype=torch.int32, device=dev)
            out["counts"] = torch.empty((rows, 2), dtype=torch.int32, device=dev)
            out["flags"] = torch.empty(rows, dtype=torch.int32, device=dev)
        self.sample_into(logits, out["ids"], out_probs=out.get("probs"), out_cand_ids=out.get("cand_ids"),
                         out_counts=out.get("counts"), out_flags=out.get("flags"), **kw)
        return out if full else out["ids"]

    @staticmethod
    def _head(hidden, weight, dim, out_logits, fmt):
        if hidden.dtype.itemsize != 4 or hidden.stride(1) != 1:
            raise ValueError("hidden must be fp32 with unit element stride")
        if fmt == _capi.HEAD_BF16:
            if weight.dtype.itemsize != 2 or weight.stride(1) != 1:
                raise ValueError("a bf16 head holds bf16 bits (2 bytes) with unit element stride")
        elif weight.dtype.itemsize != 1 or weight.stride(1) != 1:
            raise ValueError("a GGUF head holds its blocks as bytes (uint8 / int8), one row per id")
        h = SasLmHead()
        h.hidden = hidden.data_ptr()
        h.hidden_stride = hidden.stride(0)
        h.weight = weight.data_ptr()
        h.weight_stride = weight.stride(0)
        h.dim = int(dim if dim is not None else hidden.shape[1])
        h.out_logits = _ptr(out_logits, "f32", "out_logits")
        h.format = int(fmt)
        return h

    def lm_head_sample_into(self, hidden, weight, out_ids, *, dim: Optional[int] = None, out_logits=None,
                            vocab: Optional[int] = None, fmt: int = _capi.HEAD_BF16, stream=None, **kw) -> None:
        """sas_lm_head_sample: the LM head (hidden [rows][>= dim] fp32 times
        weight: [vocab][>= dim] bf16 bits as an int16/uint16 tensor, or with
        fmt = HEAD_Q8_0 / HEAD_Q4_0 / HEAD_Q6_K the GGUF blocks as a
        [vocab][row bytes] uint8 tensor) with the sampling step fused into its
        epilogue; kw as for sample_into."""
        vocab = int(vocab if vocab is not None else weight.shape[0])
        h = self._head(hidden, weight, dim, out_logits, fmt)
        d = rows_descriptor(hidden, out_ids, vocab=vocab, **kw)
        d.logits = None
        d.logits_stride = 0
        check(self._lib.sas_lm_head_sample(self._h, ctypes.byref(h), ctypes.byref(d), _stream(stream)), self._h)

    def lm_head_step_into(self, hidden, weight, out_ids, state: "DecodeState", *, dim: Optional[int] = None,
                          out_logits=None, vocab: Optional[int] = None, fmt: int = _capi.HEAD_BF16, stream=None,
                          **kw) -> None:
        """sas_lm_head_sample_step: the fused head as one step of the in-graph
        decode loop (the rows' history is `state`'s ring, their draws its
        seeds, and the token is written back into `state`)."""
        if kw.get("hist_ids") is not None:
            raise ValueError("a decode step's history is its ring")
        vocab = int(vocab if vocab is not None else weight.shape[0])
        h = self._head(hidden, weight, dim, out_logits, fmt)
        d = rows_descriptor(hidden, out_ids, vocab=vocab, **kw)
        d.logits = None
        d.logits_stride = 0
        st = state.descriptor()
        check(self._lib.sas_lm_head_sample_step(self._h, ctypes.byref(h), ctypes.byref(d), ctypes.byref(st),
                                                _stream(stream)), self._h)

    def lm_head_sample(self, hidden, weight, *, full: bool = False, logits: bool = False, **kw):
        """Allocate outputs and run lm_head_sample_into; returns ids, or a
        dict with the extras (and the head's logits when `logits`)."""
        import torch
        rows = hidden.shape[0]
        vocab = int(kw.get("vocab") or weight.shape[0])
        dev = hidden.device
        out = {"ids": torch.empty(rows, dtype=torch.int32, device=dev)}
        if full:
            out["probs"] = torch.empty((rows, _capi.MAX_TOP_K), dtype=torch.float64, device=dev)
            out["cand_ids"] = torch.empty((rows, _capi.MAX_TOP_K), dtype=torch.int32, device=dev)
            out["counts"] = torch.empty((rows, 2), dtype=torch.int32, device=dev)
            out["flags"] = torch.empty(rows, dtype=torch.int32, device=dev)
        if logits:
            out["logits"] = torch.empty((rows, vocab), dtype=torch.float32, device=dev)
        self.lm_head_sample_into(hidden, weight, out["ids"], out_logits=out.get("logits"),
                                 out_probs=out.get("probs"), out_cand_ids=out.get("cand_ids"),
                                 out_counts=out.get("counts"), out_flags=out.get("flags"), **kw)
        return out if (full or logits) else out["ids"]

    def sample_step_into(self, logits, out_ids, state: DecodeState, *, stream=None, **kw) -> None:
        """One decode step with in-graph feedback (sas_sample_step): the
        rows' history is `state`'s ring, their uniforms come from its seeds
        (or `uniforms`), and the token is written back into `state`."""
        if kw.get("hist_ids") is not None:
            raise ValueError("sample_step_into takes its history from the state's ring")
        d = rows_descriptor(logits, out_ids, **kw)
        st = state.descriptor()
        check(self._lib.sas_sample_step(self._h, ctypes.byref(d), ctypes.byref(st), _stream(stream)), self._h)

    @staticmethod
    def _spec_rows(target, draft_ids, seeds, out_picks, out_accepted, *, draft_logits=None, out_next=None,
                   round: int = 0, vocab: Optional[int] = None, mask=None, hist_ids=None, hist_offsets=None,
                   params: Optional[Params] = None, seq_params=None, row_hints: int = 0, stop_ids=None):
        seqs, L = draft_ids.shape
        if target.shape[0] != seqs * (L + 1):
            raise ValueError("target must hold seqs * (draft_len + 1) rows")
        if target.dtype.itemsize != 4 or target.stride(1) != 1:
            raise ValueError("target logits must be fp32 with unit element stride")
        d = SasSpecRows()
        d.target_logits = target.data_ptr()
        d.logits_stride = target.stride(0)
        if draft_logits is not None:
            if draft_logits.shape[0] != seqs * L or draft_logits.stride(0) != target.stride(0):
                raise ValueError("draft_logits must hold seqs * draft_len rows of the target's stride")
            d.draft_logits = draft_logits.data_ptr()
        d.vocab = int(vocab if vocab is not None else target.shape[1])
        d.seqs = seqs
        d.draft_len = L
        d.draft_ids = _ptr(draft_ids, "i32", "draft_ids")
        if mask is not None:
            d.mask = _ptr(mask, "i32", "mask")
            d.mask_stride = mask.stride(0)
        d.hist_ids = _ptr(hist_ids, "i32", "hist_ids")
        d.hist_offsets = _ptr(hist_offsets, "i32", "hist_offsets")
        d.hist_count = hist_ids.numel() if hist_ids is not None else 0
        d.params = (params or Params()).to_c()
        d.seq_params = _ptr(seq_params)
        d.seeds = _ptr(seeds, "i32", "seeds")
        d.round = int(round) & 0xFFFFFFFF
        d.row_hints = int(row_hints)
        d.stop_ids = _ptr(stop_ids, "i32", "stop_ids")
        d.out_picks = _ptr(out_picks, "i32", "out_picks")
        d.out_accepted = _ptr(out_accepted, "i32", "out_accepted")
        d.out_next = _ptr(out_next, "i32", "out_next")
        return d

    def spec_exact_into(self, target, draft_ids, seeds, out_picks, out_accepted, *, stream=None, **kw) -> None:
        """sas_spec_exact: the reference's exact-match speculative round
        (argmax drafts when draft_logits is given, every verify row sampled
        on its own, the cascade) on caller-provided device buffers."""
        d = self._spec_rows(target, draft_ids, seeds, out_picks, out_accepted, **kw)
        check(self._lib.sas_spec_exact(self._h, ctypes.byref(d), _stream(stream)), self._h)

    def spec_step_into(self, target, draft_ids, seeds, out_picks, out_accepted, state: "SpecState", *, stream=None,
                       **kw) -> None:
        """sas_spec_step: one chained round; the history is `state`'s ring,
        the round number its own, and the commit (log, pos, ring, stop
        freeze, next token) is written back into `state`."""
        if kw.get("hist_ids") is not None:
            raise ValueError("a chained round's history is its ring")
        if draft_ids.shape != (state.seqs, state.draft_len):
            raise ValueError("draft_ids must be [seqs][draft_len] of the state's shape")
        d = self._spec_rows(target, draft_ids, seeds, out_picks, out_accepted, **kw)
        st = state.descriptor()
        check(self._lib.sas_spec_step(self._h, ctypes.byref(d), ctypes.byref(st), _stream(stream)), self._h)

    def verify_into(self, target, draft, draft_ids, uniforms, out_tokens, out_accepted, *, temperature=1.0,
                    mask=None, vocab: Optional[int] = None, stream=None) -> None:
        seqs, L = draft_ids.shape
        d = SasVerifyRows()
        d.target_logits = target.data_ptr()
        d.draft_logits = draft.data_ptr()
        d.logits_stride = target.stride(0)
        if draft.stride(0) != target.stride(0):
            raise ValueError("target and draft rows must share a stride")
        d.vocab = int(vocab if vocab is not None else target.shape[1])
        d.seqs = seqs
        d.draft_len = L
        d.draft_ids = _ptr(draft_ids, "i32", "draft_ids")
        if mask is not None:
            d.mask = _ptr(mask, "i32", "mask")
            d.mask_stride = mask.stride(0)
        d.uniforms = _ptr(uniforms, "f64", "uniforms")
        d.temperature = float(temperature)
        d.out_tokens = _ptr(out_tokens, "i32", "out_tokens")
        d.out_accepted = _ptr(out_accepted, "i32", "out_accepted")
        check(self._lib.sas_verify(self._h, ctypes.byref(d), _stream(stream)), self._h)

    def verify(self, target, draft, draft_ids, uniforms, **kw):
        import torch
        seqs, L = draft_ids.shape
        toks = torch.empty((seqs, L + 1), dtype=torch.int32, device=target.device)
        acc = torch.empty(seqs, dtype=torch.int32, device=target.device)
        self.verify_into(target, draft, draft_ids, uniforms, toks, acc, **kw)
        return toks, acc

"""ctypes wrapper of the C oracle and a driver for the Node restatement.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  Never on the product path.
"""
from __future__ import annotations

import ctypes
import json
import os
import shutil
import subprocess
import tempfile
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
JS_PATH = os.path.join(HERE, "sample_js.js")
MAX_TOP_K = 128
NO_TOKEN = 0xFFFFFFFF


class OrcParams(ctypes.Structure):
    _fields_ = [("temperature", c_double), ("top_p", c_double), ("repetition_penalty", c_double),
                ("presence_penalty", c_double), ("frequency_penalty", c_double), ("softcap", c_float),
                ("top_k", c_int32)]


class OrcResult(ctypes.Structure):
    _fields_ = [("id", c_uint32), ("k", c_int32), ("cut", c_int32), ("flags", c_uint32),
                ("cand_ids", c_uint32 * MAX_TOP_K), ("probs", c_double * MAX_TOP_K)]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_exp.restype = c_double
        L.orc_exp.argtypes = [c_double]
        L.orc_pcg_uniform.restype = c_double
        L.orc_pcg_uniform.argtypes = [c_uint32, c_uint32, c_uint32]
        L.orc_softcap.restype = c_float
        L.orc_softcap.argtypes = [c_float, c_float]
        L.orc_tanhf.restype = c_float
        L.orc_tanhf.argtypes = [c_float]
        L.orc_penalize.restype = c_double
        L.orc_penalize.argtypes = [c_double, c_uint32, POINTER(OrcParams)]
        L.orc_sample_row.restype = None
        L.orc_sample_row.argtypes = [c_void_p, c_int32, c_void_p, c_void_p, c_int32, POINTER(OrcParams), c_double,
                                     c_int, POINTER(OrcResult)]
        L.orc_sample_rows.restype = None
        L.orc_sample_rows.argtypes = [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_void_p, c_void_p,
                                      c_void_p, POINTER(OrcParams), c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_int]
        L.orc_mask_from_ids.restype = c_int64
        L.orc_mask_from_ids.argtypes = [c_int32, c_void_p, c_size_t, c_int32, c_void_p, c_int64]
        L.orc_verify.restype = None
        L.orc_verify.argtypes = [c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_int64,
                                 c_void_p, c_double, c_void_p, c_void_p, c_void_p]
        L.orc_spec_exact.restype = None
        L.orc_spec_exact.argtypes = [c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                     c_int64, c_void_p, c_void_p, POINTER(OrcParams), c_void_p, c_void_p, c_uint32,
                                     c_void_p, c_void_p, c_void_p, c_void_p]
        L.orc_spec_commit.restype = None
        L.orc_spec_commit.argtypes = [c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_int32, c_void_p, c_int32, c_void_p, c_void_p]
        L.orc_f16_round.restype = ctypes.c_float
        L.orc_f16_round.argtypes = [ctypes.c_float]
        L.orc_q81_quantize.restype = None
        L.orc_q81_quantize.argtypes = [c_void_p, c_int32, c_void_p, c_void_p, c_void_p]
        L.orc_lm_head_q_logits.restype = None
        L.orc_lm_head_q_logits.argtypes = [c_int32, c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                           c_void_p]
        L.orc_lm_head_logits.restype = None
        L.orc_lm_head_logits.argtypes = [c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p]
        _lib = L
    return _lib


HEAD_BF16, HEAD_Q8_0, HEAD_Q4_0, HEAD_Q6_K = 0, 1, 2, 3
HEAD_BLOCK = {HEAD_Q8_0: (32, 34), HEAD_Q4_0: (32, 18), HEAD_Q6_K: (256, 210)}  # values, bytes per block


def f16_round(x: float) -> float:
    return float(lib().orc_f16_round(float(x)))


def q81_quantize(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """orc_q81_quantize of one row: (int8 q [dim], f32 d8 [dim/32], f32 s8)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    dim = x.shape[0]
    q = np.empty(dim, np.int8)
    d8 = np.empty(dim // 32, np.float32)
    s8 = np.empty(dim // 32, np.float32)
    lib().orc_q81_quantize(x.ctypes.data, dim, q.ctypes.data, d8.ctypes.data, s8.ctypes.data)
    return q, d8, s8


def lm_head_q_logits(fmt: int, hidden, weight, dim: int | None = None) -> np.ndarray:
    """The quantized head's f32 logits in the order sas_lm_head_sample sums
    them (hidden [rows][>= dim] f32, weight [vocab][row_bytes] uint8 GGUF
    blocks)."""
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    weight = np.ascontiguousarray(weight, dtype=np.uint8)
    rows, vocab = hidden.shape[0], weight.shape[0]
    dim = int(dim if dim is not None else hidden.shape[1])
    out = np.empty((rows, vocab), dtype=np.float32)
    lib().orc_lm_head_q_logits(fmt, hidden.ctypes.data, hidden.shape[1], weight.ctypes.data, weight.shape[1], dim,
                               rows, vocab, out.ctypes.data)
    return out


def lm_head_logits(hidden, weight_bits, dim: int | None = None) -> np.ndarray:
    """The LM head's f32 logits in the order sas_lm_head_sample sums them
    (hidden [rows][>= dim] f32, weight_bits [vocab][>= dim] uint16 bf16)."""
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    weight_bits = np.ascontiguousarray(weight_bits, dtype=np.uint16)
    rows, vocab = hidden.shape[0], weight_bits.shape[0]
    dim = int(dim if dim is not None else hidden.shape[1])
    out = np.empty((rows, vocab), dtype=np.float32)
    lib().orc_lm_head_logits(hidden.ctypes.data, hidden.shape[1], weight_bits.ctypes.data, weight_bits.shape[1],
                             dim, rows, vocab, out.ctypes.data)
    return out


def params(p) -> OrcParams:
    """OrcParams from shared_amd.Params or a dict with the same fields."""
    d = p.as_dict() if hasattr(p, "as_dict") else dict(p)
    return OrcParams(d.get("temperature", 0.0), d.get("top_p", 1.0), d.get("repetition_penalty", 1.0),
                     d.get("presence_penalty", 0.0), d.get("frequency_penalty", 0.0), d.get("softcap", 0.0),
                     int(d.get("top_k", 1)))


def _p(a):
    return None if a is None else a.ctypes.data


def sample_row(logits, p, *, mask=None, hist=None, uniform=0.0, select_mode=0) -> OrcResult:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    mask = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    hist = None if hist is None else np.ascontiguousarray(hist, dtype=np.uint32)
    res = OrcResult()
    lib().orc_sample_row(_p(logits), logits.size, _p(mask), _p(hist), 0 if hist is None else hist.size,
                         ctypes.byref(params(p)), float(uniform), int(select_mode), ctypes.byref(res))
    return res


def sample_rows(batch, threads: int = 8, row_params=None) -> dict:
    """Oracle outputs for a shared_amd.workloads.Batch (or same-named fields)."""
    x = np.ascontiguousarray(batch.logits, dtype=np.float32)
    rows, vocab = x.shape
    mask = None if batch.mask is None else np.ascontiguousarray(batch.mask, dtype=np.uint32)
    hi = None if batch.hist_ids is None else np.ascontiguousarray(batch.hist_ids, dtype=np.uint32)
    ho = None if batch.hist_offsets is None else np.ascontiguousarray(batch.hist_offsets, dtype=np.int32)
    u = None if batch.uniforms is None else np.ascontiguousarray(batch.uniforms, dtype=np.float64)
    rp = None
    if row_params is not None:
        rp = (OrcParams * rows)(*[params(q) for q in row_params])
    out = {"ids": np.zeros(rows, np.uint32), "probs": np.zeros((rows, MAX_TOP_K)),
           "cand_ids": np.zeros((rows, MAX_TOP_K), np.uint32), "counts": np.zeros((rows, 2), np.int32),
           "flags": np.zeros(rows, np.uint32)}
    lib().orc_sample_rows(_p(x), vocab, vocab, rows, _p(mask), 0 if mask is None else mask.shape[1], _p(hi),
                          _p(ho), _p(u), ctypes.byref(params(batch.params)),
                          None if rp is None else ctypes.cast(rp, c_void_p), _p(out["ids"]), _p(out["probs"]),
                          _p(out["cand_ids"]), _p(out["counts"]), _p(out["flags"]), int(threads))
    return out


def mask_from_ids(kind: int, ids, vocab: int) -> np.ndarray:
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
    words = np.zeros((vocab + 31) // 32, np.uint32)
    lib().orc_mask_from_ids(int(kind), _p(ids), ids.size, int(vocab), _p(words), words.size)
    return words


def verify(inp: dict) -> dict:
    L, seqs, vocab = inp["drafts"], inp["seqs"], inp["vocab"]
    t = np.ascontiguousarray(inp["target"], np.float32)
    d = np.ascontiguousarray(inp["draft"], np.float32)
    m = None if inp.get("mask") is None else np.ascontiguousarray(inp["mask"], np.uint32)
    ids = np.ascontiguousarray(inp["draft_ids"], np.uint32)
    u = np.ascontiguousarray(inp["uniforms"], np.float64)
    toks = np.zeros((seqs, L + 1), np.uint32)
    acc = np.zeros(seqs, np.int32)
    ratio = np.zeros((seqs, L + 1))
    lib().orc_verify(_p(t), _p(d), vocab, vocab, seqs, L, _p(ids), _p(m), 0 if m is None else m.shape[1], _p(u),
                     float(inp["temperature"]), _p(toks), _p(acc), _p(ratio))
    return {"tokens": toks, "accepted": acc, "ratio": ratio}


def spec_exact(inp: dict) -> dict:
    """The exact-match speculative round (orc_spec_exact) for the fields of
    shared_amd.workloads.spec_case: target [seqs*(L+1)][V], draft [seqs*L][V]
    or None (then draft_ids), mask, CSR history per sequence, params or
    seq_params, seeds, round, stop_ids."""
    seqs, L, vocab = inp["seqs"], inp["drafts"], inp["vocab"]
    t = np.ascontiguousarray(inp["target"], np.float32)
    d = inp.get("draft")
    d = None if d is None else np.ascontiguousarray(d, np.float32)
    ids = (np.zeros((seqs, L), np.uint32) if d is not None
           else np.ascontiguousarray(inp["draft_ids"], np.uint32).copy())
    m = None if inp.get("mask") is None else np.ascontiguousarray(inp["mask"], np.uint32)
    hi = None if inp.get("hist_ids") is None else np.ascontiguousarray(inp["hist_ids"], np.uint32)
    ho = None if inp.get("hist_offsets") is None else np.ascontiguousarray(inp["hist_offsets"], np.int32)
    sp = None
    if inp.get("seq_params") is not None:
        sp = (OrcParams * seqs)(*[params(q) for q in inp["seq_params"]])
    seeds = np.ascontiguousarray(inp["seeds"], np.uint32)
    st = None if inp.get("stop_ids") is None else np.ascontiguousarray(inp["stop_ids"], np.uint32)
    picks = np.zeros((seqs, L + 1), np.uint32)
    acc = np.zeros(seqs, np.int32)
    nxt = np.zeros(seqs, np.uint32)
    lib().orc_spec_exact(_p(t), _p(d), vocab, vocab, seqs, L, _p(ids), _p(m), 0 if m is None else m.shape[1],
                         _p(hi), _p(ho), ctypes.byref(params(inp.get("params") or {})),
                         None if sp is None else ctypes.cast(sp, c_void_p), _p(seeds), int(inp.get("round", 0)),
                         _p(st), _p(picks), _p(acc), _p(nxt))
    return {"draft_ids": ids, "picks": picks, "accepted": acc, "next": nxt}


def spec_commit(picks, draft_ids, accepted, stop_ids, state, ring=None, log=None):
    """acceptSpec's commit (orc_spec_commit) in place on `state` ([seqs][4]
    uint32), `ring` ([seqs][1 + ring_len] uint32 or None) and `log`
    ([seqs][max_rounds][2 + L] uint32 or None); returns (next tokens,
    accepted counts) of the round."""
    picks = np.ascontiguousarray(picks, np.uint32)
    seqs, L1 = picks.shape
    ids = np.ascontiguousarray(draft_ids, np.uint32)
    acc = np.ascontiguousarray(accepted, np.int32)
    st = None if stop_ids is None else np.ascontiguousarray(stop_ids, np.uint32)
    assert state.dtype == np.uint32 and state.flags.c_contiguous
    ring_len = 0
    if ring is not None:
        assert ring.dtype == np.uint32 and ring.flags.c_contiguous
        ring_len = ring.shape[1] - 1
    max_rounds = 0
    if log is not None:
        assert log.dtype == np.uint32 and log.flags.c_contiguous and log.shape[2] == L1 + 1
        max_rounds = log.shape[1]
    nxt = np.zeros(seqs, np.uint32)
    out_acc = np.zeros(seqs, np.int32)
    lib().orc_spec_commit(seqs, L1 - 1, _p(picks), _p(ids), _p(acc), _p(st), state.ctypes.data, _p(ring), ring_len,
                          _p(log), max_rounds, nxt.ctypes.data, out_acc.ctypes.data)
    return nxt, out_acc


# ------------------------------------------------------------ Node driver --

def node_binary():
    return shutil.which("node")


def write_case(dirpath: str, batch) -> None:
    os.makedirs(dirpath, exist_ok=True)
    x = np.ascontiguousarray(batch.logits, dtype=np.float32)
    meta = {"rows": int(x.shape[0]), "vocab": int(x.shape[1]), "stride": int(x.shape[1]),
            "params": batch.params.as_dict()}
    x.tofile(os.path.join(dirpath, "logits.f32"))
    if batch.mask is not None:
        np.ascontiguousarray(batch.mask, np.uint32).tofile(os.path.join(dirpath, "mask.u32"))
        meta["mask_stride"] = int(batch.mask.shape[1])
    if batch.hist_ids is not None:
        np.ascontiguousarray(batch.hist_ids, np.uint32).tofile(os.path.join(dirpath, "hist.u32"))
        np.ascontiguousarray(batch.hist_offsets, np.int32).tofile(os.path.join(dirpath, "hist_off.i32"))
    if batch.uniforms is not None:
        np.ascontiguousarray(batch.uniforms, np.float64).tofile(os.path.join(dirpath, "uniforms.f64"))
    with open(os.path.join(dirpath, "meta.json"), "w") as f:
        json.dump(meta, f)


def run_node(batch, threads: int = 1, repeat: int = 1, workdir: str | None = None, timeout: float = 600):
    """Run sample_js.js on a batch; returns (outputs, timing dict)."""
    node = node_binary()
    if node is None:
        raise RuntimeError("node is not installed")
    tmp = workdir or tempfile.mkdtemp(prefix="sas_js_")
    try:
        write_case(tmp, batch)
        proc = subprocess.run([node, JS_PATH, tmp, "--threads", str(threads), "--repeat", str(repeat)],
                              stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=timeout)
        if proc.returncode != 0:
            raise RuntimeError(f"node failed: {proc.stderr[-2000:]}")
        timing = json.loads(proc.stdout.strip().splitlines()[-1])
        rows = batch.logits.shape[0]
        out = {"ids": np.fromfile(os.path.join(tmp, "out_ids.u32"), np.uint32),
               "counts": np.fromfile(os.path.join(tmp, "out_counts.i32"), np.int32).reshape(rows, 2),
               "probs": np.fromfile(os.path.join(tmp, "out_probs.f64"), np.float64).reshape(rows, MAX_TOP_K),
               "cand_ids": np.fromfile(os.path.join(tmp, "out_cand.u32"), np.uint32).reshape(rows, MAX_TOP_K)}
        return out, timing
    finally:
        if workdir is None:
            shutil.rmtree(tmp, ignore_errors=True)

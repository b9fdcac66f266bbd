"""ctypes view of include/shared_amd_sampler.h.

The structures mirror the C layout field for field; the library is the
in-tree ``libshared_amd_sampler.so``.  Loading fails loudly when it has not
been built: there is no Python fallback for any computation.
"""
from __future__ import annotations

import ctypes
import os
import re
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_void_p

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libshared_amd_sampler.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "shared_amd_sampler.h")


def _header_define(name: str) -> int:
    """Integer value of `#define NAME <int>` or `#define NAME (<int> << <int>)`."""
    with open(HEADER) as f:
        for line in f:
            m = re.match(r"#define\s+" + name + r"\s+\(?\s*(\d+)u?\s*(?:<<\s*(\d+))?\s*\)?\s*(?:/\*.*)?$", line)
            if m:
                return int(m.group(1)) << int(m.group(2) or 0)
    raise KeyError(name)


MAX_TOP_K = _header_define("SAS_MAX_TOP_K")
MAX_VOCAB = _header_define("SAS_MAX_VOCAB")
MAX_HISTORY = _header_define("SAS_MAX_HISTORY")
MAX_DRAFT = _header_define("SAS_MAX_DRAFT")
NOALLOC_SCRATCH_BYTES = _header_define("SAS_NOALLOC_SCRATCH_BYTES")
LMH_MAX_ROWS = _header_define("SAS_LMH_MAX_ROWS")
LMH_MAX_LDS_FLOATS = _header_define("SAS_LMH_MAX_LDS_FLOATS")
LMH_MAX_VOCAB = _header_define("SAS_LMH_MAX_VOCAB")
NO_TOKEN = 0xFFFFFFFF
STOP_PAD = 0xFFFFFFFF
OK, ERR_INVALID, ERR_HIP, ERR_NOMEM = 0, 1, 2, 3
FLAG_EMPTY_ROW, FLAG_TOPP_EDGE, FLAG_DRAW_EDGE, FLAG_SLOW_SELECT = 1, 2, 4, 8
HINT_NO_SOFTCAP = 1
HEAD_BF16, HEAD_Q8_0, HEAD_Q4_0, HEAD_Q6_K = 0, 1, 2, 3
MASK_ALL, MASK_ALLOW, MASK_DENY = 0, 1, 2


class SasParams(ctypes.Structure):
    _fields_ = [
        ("temperature", c_double),
        ("top_p", c_double),
        ("repetition_penalty", c_double),
        ("presence_penalty", c_double),
        ("frequency_penalty", c_double),
        ("softcap", c_float),
        ("top_k", c_int32),
    ]


class SasRows(ctypes.Structure):
    _fields_ = [
        ("logits", c_void_p),
        ("logits_stride", c_int64),
        ("vocab", c_int32),
        ("rows", c_int32),
        ("mask", c_void_p),
        ("mask_stride", c_int64),
        ("hist_ids", c_void_p),
        ("hist_offsets", c_void_p),
        ("uniforms", c_void_p),
        ("params", SasParams),
        ("row_params", c_void_p),
        ("out_ids", c_void_p),
        ("out_probs", c_void_p),
        ("out_cand_ids", c_void_p),
        ("out_counts", c_void_p),
        ("out_flags", c_void_p),
        ("hist_count", c_int64),
        ("row_hints", c_uint32),
    ]


class SasStep(ctypes.Structure):
    _fields_ = [
        ("state", c_void_p),
        ("sampled", c_void_p),
        ("max_steps", c_int32),
        ("next_tokens", c_void_p),
        ("ring", c_void_p),
        ("ring_len", c_int32),
        ("stop_ids", c_void_p),
        ("seeds", c_void_p),
    ]


class SasVerifyRows(ctypes.Structure):
    _fields_ = [
        ("target_logits", c_void_p),
        ("draft_logits", c_void_p),
        ("logits_stride", c_int64),
        ("vocab", c_int32),
        ("seqs", c_int32),
        ("draft_len", c_int32),
        ("draft_ids", c_void_p),
        ("mask", c_void_p),
        ("mask_stride", c_int64),
        ("uniforms", c_void_p),
        ("temperature", c_double),
        ("out_tokens", c_void_p),
        ("out_accepted", c_void_p),
    ]


class SasSpecRows(ctypes.Structure):
    _fields_ = [
        ("target_logits", c_void_p),
        ("draft_logits", c_void_p),
        ("logits_stride", c_int64),
        ("vocab", c_int32),
        ("seqs", c_int32),
        ("draft_len", c_int32),
        ("draft_ids", c_void_p),
        ("mask", c_void_p),
        ("mask_stride", c_int64),
        ("hist_ids", c_void_p),
        ("hist_offsets", c_void_p),
        ("hist_count", c_int64),
        ("params", SasParams),
        ("seq_params", c_void_p),
        ("seeds", c_void_p),
        ("round", c_uint32),
        ("row_hints", c_uint32),
        ("stop_ids", c_void_p),
        ("out_picks", c_void_p),
        ("out_accepted", c_void_p),
        ("out_next", c_void_p),
    ]


class SasSpecState(ctypes.Structure):
    _fields_ = [
        ("state", c_void_p),
        ("ring", c_void_p),
        ("ring_len", c_int32),
        ("log", c_void_p),
        ("max_rounds", c_int32),
        ("next_tokens", c_void_p),
    ]


class SasReserveDesc(ctypes.Structure):
    _fields_ = [
        ("rows", c_int32),
        ("vocab", c_int32),
        ("hist_ids", c_int64),
        ("lm_head_rows", c_int32),
        ("verify_seqs", c_int32),
        ("verify_draft_len", c_int32),
    ]


class SasLmHead(ctypes.Structure):
    _fields_ = [
        ("hidden", c_void_p),
        ("hidden_stride", c_int64),
        ("weight", c_void_p),
        ("weight_stride", c_int64),
        ("dim", c_int32),
        ("out_logits", c_void_p),
        ("format", c_int32),
    ]


# name -> (restype, argtypes); every function declared in the header.
SIGNATURES = {
    "sas_version": (c_char_p, []),
    "sas_create": (c_int, [c_int, POINTER(c_void_p)]),
    "sas_destroy": (None, [c_void_p]),
    "sas_last_error": (c_char_p, [c_void_p]),
    "sas_reserve": (c_int, [c_void_p, c_int32, c_int32]),
    "sas_reserve_for": (c_int, [c_void_p, POINTER(SasReserveDesc)]),
    "sas_sample": (c_int, [c_void_p, POINTER(SasRows), c_void_p]),
    "sas_sample_noalloc": (c_int, [c_int, POINTER(SasRows), c_void_p]),
    "sas_sample_step": (c_int, [c_void_p, POINTER(SasRows), POINTER(SasStep), c_void_p]),
    "sas_verify": (c_int, [c_void_p, POINTER(SasVerifyRows), c_void_p]),
    "sas_spec_exact": (c_int, [c_void_p, POINTER(SasSpecRows), c_void_p]),
    "sas_spec_step": (c_int, [c_void_p, POINTER(SasSpecRows), POINTER(SasSpecState), c_void_p]),
    "sas_lm_head_sample": (c_int, [c_void_p, POINTER(SasLmHead), POINTER(SasRows), c_void_p]),
    "sas_lm_head_sample_step": (c_int, [c_void_p, POINTER(SasLmHead), POINTER(SasRows), POINTER(SasStep), c_void_p]),
    "sas_clamp_params": (c_int, [POINTER(SasParams), POINTER(SasParams)]),
    "sas_mask_from_ids": (c_int64, [c_int32, POINTER(c_uint32), c_size_t, c_int32, POINTER(c_uint32), c_int64]),
    "sas_pcg_uniform": (c_double, [c_uint32, c_uint32, c_uint32]),
    "sas_alloc": (c_int, [c_void_p, c_size_t, POINTER(c_void_p)]),
    "sas_free": (c_int, [c_void_p, c_void_p]),
    "sas_memcpy": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_int, c_void_p]),
    "sas_synchronize": (c_int, [c_void_p, c_void_p]),
    "sas_stream": (c_void_p, [c_void_p]),
}

_lib = None


def header_functions() -> list[str]:
    """Names of every function the public header declares."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"^[a-z_0-9 \*]*?\b(sas_[a-z_0-9]+)\s*\(", text, flags=re.M)))


def load() -> ctypes.CDLL:
    """Load the in-tree library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run `python -m shared_amd.build` first")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class SasError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check(rc: int, handle=None) -> None:
    if rc != OK:
        msg = load().sas_last_error(handle)
        raise SasError(rc, (msg or b"").decode())

"""The C ABI without a GPU: the library loads, exports every function the
header declares, and its host-only functions follow the reference's rules.
No call here launches a kernel."""
import ctypes
import math
import os

import numpy as np
import pytest

import oracle as O
from shared_amd import Params, clamp_params, mask_from_ids
from shared_amd import _capi


def test_library_exports_every_header_function():
    lib = _capi.load()
    names = _capi.header_functions()
    assert "sas_sample" in names and "sas_verify" in names and "sas_stream" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_capi.SIGNATURES), "ctypes signatures and header differ"


def test_probe_library_exports_its_header():
    """libsas_probe.so (bench.py's measurement probes, outside the sampling
    ABI) exports what include/sas_probe.h declares."""
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    path = os.path.join(root, "shared_amd", "libsas_probe.so")
    if not os.path.exists(path):
        pytest.skip("libsas_probe.so is not built")
    text = open(os.path.join(root, "include", "sas_probe.h")).read()
    names = sorted(set(re.findall(r"^int\s+(sasp_[a-z_0-9]+)\s*\(", text, flags=re.M)))
    assert names == ["sasp_masked_read", "sasp_memset_order", "sasp_read"]
    lib = ctypes.CDLL(path)
    for name in names:
        assert hasattr(lib, name), name
    # the sampling library does not carry the probes
    assert not hasattr(_capi.load(), "sas_probe_read")


def test_reserve_for_rejects_bad_shapes_without_a_handle():
    lib = _capi.load()
    d = _capi.SasReserveDesc(1, 1000, 0, 0, 0, 0)
    assert lib.sas_reserve_for(None, ctypes.byref(d)) == _capi.ERR_INVALID
    assert b"handle is NULL" in lib.sas_last_error(None)


def test_version_names_the_target():
    v = _capi.load().sas_version().decode()
    assert v.startswith("shared_amd_sampler ") and v.endswith("gfx950")


def test_header_constants():
    assert _capi.MAX_TOP_K == 128          # the request API's top_k range (completions.ts:271)
    assert _capi.MAX_VOCAB == 1 << 22


def test_ctypes_layout_matches_the_c_compiler(tmp_path):
    """Every struct the bindings mirror has the offsets gcc gives it."""
    import shutil
    import subprocess
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not installed")
    structs = {"sas_params": _capi.SasParams, "sas_rows": _capi.SasRows, "sas_verify_rows": _capi.SasVerifyRows,
               "sas_spec_rows": _capi.SasSpecRows, "sas_step": _capi.SasStep, "sas_lm_head": _capi.SasLmHead,
               "sas_reserve_desc": _capi.SasReserveDesc, "sas_spec_state": _capi.SasSpecState}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "shared_amd_sampler.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'  printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
    subprocess.run(["gcc", "-std=c11", "-I", inc, str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                  text=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(got[cname]) == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(cls, fname).offset, (cname, fname)


@pytest.mark.parametrize("field,value,want", [
    # model.js:420-423: non-finite or non-positive temperature -> 0 (greedy)
    ("temperature", math.nan, 0.0), ("temperature", -1.0, 0.0), ("temperature", math.inf, 0.0),
    ("temperature", 0.7, 0.7),
    # top_p clamped to [0, 1], non-finite -> 1
    ("top_p", 1.5, 1.0), ("top_p", -0.2, 0.0), ("top_p", math.nan, 1.0), ("top_p", 0.95, 0.95),
    # presence clamped to [0, 10], non-finite -> 0
    ("presence_penalty", 20.0, 10.0), ("presence_penalty", -1.0, 0.0), ("presence_penalty", math.nan, 0.0),
    # build-defined: repetition <= 0 or non-finite -> 1, frequency non-finite -> 0, softcap -> 0
    ("repetition_penalty", 0.0, 1.0), ("repetition_penalty", math.nan, 1.0), ("repetition_penalty", 1.1, 1.1),
    ("frequency_penalty", math.inf, 0.0), ("frequency_penalty", -0.5, -0.5),
    ("softcap", math.nan, 0.0), ("softcap", -3.0, 0.0), ("softcap", 30.0, 30.0),
    # top_k clamped to [1, SAS_MAX_TOP_K] (the reference clamps to 20: config.js:48)
    ("top_k", 0, 1), ("top_k", 500, 128), ("top_k", 50, 50),
])
def test_clamp_params_follows_reference_packer(field, value, want):
    p = Params(temperature=1.0, top_k=10, top_p=0.5)
    setattr(p, field, value)
    got = getattr(clamp_params(p), field)
    assert got == want or (math.isnan(want) and math.isnan(got)), (field, value, got)


def test_mask_from_ids_matches_oracle_and_counts_allowed():
    rng = np.random.default_rng(0)
    for vocab in (1, 31, 32, 33, 151936, 262144):
        ids = rng.integers(0, vocab + 100, 300).astype(np.uint32)
        for kind in (_capi.MASK_ALL, _capi.MASK_ALLOW, _capi.MASK_DENY):
            w = mask_from_ids(kind, ids, vocab)
            assert np.array_equal(w, O.mask_from_ids(kind, ids, vocab)), (vocab, kind)
            bits = np.unpackbits(w.view(np.uint8), bitorder="little")
            assert not bits[vocab:].any()      # no bit beyond the vocabulary
            listed = np.unique(ids[ids < vocab]).size
            want = {_capi.MASK_ALL: vocab, _capi.MASK_ALLOW: listed, _capi.MASK_DENY: vocab - listed}[kind]
            lib = _capi.load()
            out = np.zeros_like(w)
            n = lib.sas_mask_from_ids(kind, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size, vocab,
                                      out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), out.size)
            assert n == want


def test_mask_from_ids_rejects_bad_arguments():
    lib = _capi.load()
    words = np.zeros(4, np.uint32)
    wp = words.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
    assert lib.sas_mask_from_ids(7, None, 0, 100, wp, 4) == -_capi.ERR_INVALID      # unknown kind
    assert lib.sas_mask_from_ids(1, None, 0, 200, wp, 4) == -_capi.ERR_INVALID      # too few words
    assert lib.sas_mask_from_ids(1, None, 5, 100, wp, 4) == -_capi.ERR_INVALID      # ids missing
    assert b"invalid" in lib.sas_last_error(None)


def test_pcg_uniform_is_the_reference_hash():
    # kernels.js:91-95 (pcg) and :181 / :320 (seed ^ it*0x9E3779B9 ^ row*0x85EBCA6B)
    def pcg(x):
        h = (x * 747796405 + 2891336453) & 0xFFFFFFFF
        h = (((h >> ((h >> 28) + 4)) ^ h) * 277803737) & 0xFFFFFFFF
        return ((h >> 22) ^ h) & 0xFFFFFFFF

    lib = _capi.load()
    for seed, it, row in [(1, 0, 0), (0xDEADBEEF, 7, 2), (12345, 99, 1), (0, 0xFFFFFFFF, 0xFFFFFFFF)]:
        x = (seed ^ ((it * 0x9E3779B9) & 0xFFFFFFFF) ^ ((row * 0x85EBCA6B) & 0xFFFFFFFF)) & 0xFFFFFFFF
        want = (pcg(x) & 0xFFFFFF) / 16777216.0
        assert lib.sas_pcg_uniform(seed, it, row) == want == O.lib().orc_pcg_uniform(seed, it, row)
        assert 0.0 <= want < 1.0


def test_handle_calls_fail_loudly_without_a_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    lib = _capi.load()
    h = ctypes.c_void_p()
    assert lib.sas_create(0, ctypes.byref(h)) == _capi.ERR_HIP
    assert not h.value
    assert b"no HIP device" in lib.sas_last_error(None)
    assert lib.sas_sample(None, None, None) == _capi.ERR_INVALID
    assert lib.sas_verify(None, None, None) == _capi.ERR_INVALID
    with pytest.raises(_capi.SasError):
        from shared_amd import Sampler
        Sampler(0)


def test_history_offsets_checked_on_the_host():
    from shared_amd.sampler import check_history
    check_history(np.array([0, 3, 3, 7], np.int32), 7)
    with pytest.raises(ValueError, match="negative"):
        check_history(np.array([-1, 3], np.int32), 7)
    with pytest.raises(ValueError, match="decrease at row 1"):
        check_history(np.array([0, 4, 2], np.int32), 7)
    with pytest.raises(ValueError, match="hist_ids holds 5 ids"):
        check_history(np.array([0, 3, 6], np.int32), 5)
    with pytest.raises(ValueError, match="at most 65535"):
        check_history(np.array([0, 70000], np.int32), 70000)


def test_row_hints_follow_the_rows():
    from shared_amd.sampler import row_hints
    assert row_hints([Params(), Params(temperature=1.0)]) == _capi.HINT_NO_SOFTCAP
    assert row_hints([Params(), Params(softcap=30.0)]) == 0


def test_rows_struct_matches_the_header():
    # the ctypes layout has the fields the header declares, in order
    import re
    text = open(_capi.HEADER).read()
    body = re.search(r"typedef struct sas_rows \{(.*?)\} sas_rows;", text, re.S).group(1)
    names = re.findall(r"\b([a-z_]+);", re.sub(r"/\*.*?\*/", "", body, flags=re.S))
    assert names == [f for f, _ in _capi.SasRows._fields_]


def test_device_pointers_refuse_other_element_types():
    # the Python mirror checks each tensor's element type against the one the
    # C ABI reads (a tensor stand-in: no device is needed for the check)
    import torch
    from shared_amd import sampler as S

    class DeviceTensor:
        is_cuda = True

        def __init__(self, dtype):
            self.dtype = dtype

        def is_contiguous(self):
            return True

        def dim(self):
            return 1

        def element_size(self):
            return self.dtype.itemsize

        def data_ptr(self):
            return 4096

    for dtype, kind in ((torch.int32, "i32"), (torch.uint32, "i32"), (torch.float64, "f64"), (torch.float32, "f32")):
        assert S._ptr(DeviceTensor(dtype), kind, "x") == 4096
    for dtype, kind in ((torch.int64, "i32"), (torch.float32, "i32"), (torch.int16, "i32"), (torch.float32, "f64"),
                        (torch.int64, "f64"), (torch.float16, "f32")):
        with pytest.raises(ValueError, match="x must hold"):
            S._ptr(DeviceTensor(dtype), kind, "x")

"""MI355X-native logit processing and sampling.

The product is the C ABI in include/shared_amd_sampler.h, implemented by
HIP kernels in csrc/ (built into libshared_amd_sampler.so) and exposed to
Node by js/ over an N-API addon.  This Python package is the build and test
harness' handle on the same library.
"""
from ._capi import HEAD_BF16, HEAD_Q4_0, HEAD_Q6_K, HEAD_Q8_0, MAX_TOP_K, NO_TOKEN, SasError  # noqa: F401
from .sampler import DecodeState, Params, Sampler, SpecState, clamp_params, mask_from_ids, pack_params  # noqa: F401

__all__ = ["DecodeState", "Params", "Sampler", "SasError", "SpecState", "clamp_params", "mask_from_ids", "pack_params", "MAX_TOP_K",
           "NO_TOKEN", "HEAD_BF16", "HEAD_Q8_0", "HEAD_Q4_0", "HEAD_Q6_K"]

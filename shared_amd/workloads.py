"""Deterministic synthetic inputs for the benchmark configurations.

Each generator returns host numpy arrays shaped exactly as the C ABI takes
them (fp32 logits [rows][vocab], packed uint32 mask words, CSR history,
float64 uniforms) plus the sampling parameters.  `rows` and `vocab` can be
scaled down for fast tests; the defaults are the configuration's own sizes.

  C1  greedy + repetition 1.1, V=151,936, B=1, N(0,3) + 5 spikes of +12,
      512 uniform history ids
  C2  T 0.7 / top-k 40 / top-p 0.95, V=151,936, B=64, N(0,3) plus a
      Zipf(1.1) rank-ordered bias of up to +10 over a per-row permutation
  C3  V=262,144, B=128, N(0,4), mask density U[0.5%, 20%] per row (>= 1
      allowed), top-k 50 / top-p 0.9 / T 1.0
  C3P C3 plus repetition 1.1, presence 0.5, frequency 0.3 over 512 uniform
      history ids (the headline benchmark)
  C4  V=262,144, B=256, N(0,3), 4,096 history ids Zipf(1.2) over a per-row
      permutation, repetition 1.15 / presence 0.5 / frequency 0.3, greedy
  C5  V=151,936, 32 sequences x (4 drafts + 1 bonus); target N(0,3), draft
      0.8*target + 0.6*N(0,3); drafts drawn from the masked draft softmax;
      5% mask on both; two uniforms per position
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from .sampler import Params

QWEN_VOCAB = 151936
GEMMA_VOCAB = 262144


@dataclass
class Batch:
    name: str
    logits: np.ndarray                      # float32 [rows, vocab]
    params: Params
    mask: Optional[np.ndarray] = None       # uint32 [rows, ceil(vocab/32)]
    hist_ids: Optional[np.ndarray] = None   # uint32 [total]
    hist_offsets: Optional[np.ndarray] = None  # int32 [rows + 1]
    uniforms: Optional[np.ndarray] = None   # float64 [rows]
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def algorithmic_bytes(self) -> int:
        """Compulsory HBM bytes of one step as the C ABI takes it: the fp32
        logits, the mask words, the history ids and their row offsets, the
        float64 uniforms (when some row samples) read once, and the uint32
        ids written once."""
        b = self.logits.nbytes + 4 * self.rows
        if self.mask is not None:
            b += self.rows * ((self.vocab + 31) // 32) * 4
        if self.hist_ids is not None:
            b += self.hist_ids.nbytes + self.hist_offsets.nbytes
        if self.uniforms is not None and self.params.temperature > 0:
            b += self.uniforms.nbytes
        return b


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _normal(rng, rows, vocab, sigma) -> np.ndarray:
    return (rng.standard_normal((rows, vocab), dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def pack_bits(bits: np.ndarray) -> np.ndarray:
    """bool [rows, vocab] -> uint32 [rows, ceil(vocab/32)], bit i of word i/32."""
    rows, vocab = bits.shape
    words = (vocab + 31) // 32
    padded = np.zeros((rows, words * 32), dtype=bool)
    padded[:, :vocab] = bits
    b = np.packbits(padded.reshape(rows, words * 4, 8), axis=-1, bitorder="little").reshape(rows, words * 4)
    return np.ascontiguousarray(b).view("<u4").reshape(rows, words)


def random_mask(rng, rows, vocab, lo, hi) -> np.ndarray:
    dens = rng.uniform(lo, hi, size=(rows, 1))
    bits = rng.random((rows, vocab), dtype=np.float32) < dens
    for r in range(rows):
        if not bits[r].any():
            bits[r, rng.integers(vocab)] = True
    return pack_bits(bits)


def _affine_perm(rng, vocab):
    """A random bijection rank -> id of [0, vocab): id = (a*rank + b) mod vocab."""
    while True:
        a = int(rng.integers(1, vocab)) | 1
        if np.gcd(a, vocab) == 1:
            return a, int(rng.integers(vocab))


def zipf_ranks(rng, n, vocab, s) -> np.ndarray:
    """n draws of a rank in [0, vocab) with P(rank r) proportional to (r+1)^-s."""
    w = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, rng.random(n)), vocab - 1)


def _csr(lists) -> tuple[np.ndarray, np.ndarray]:
    offs = np.zeros(len(lists) + 1, dtype=np.int32)
    offs[1:] = np.cumsum([len(x) for x in lists])
    ids = np.concatenate(lists).astype(np.uint32) if lists else np.zeros(0, np.uint32)
    return ids, offs


def c1(rows: int = 1, vocab: int = QWEN_VOCAB, seed: int = 1, hist: int = 512) -> Batch:
    rng = _rng(seed)
    x = _normal(rng, rows, vocab, 3.0)
    for r in range(rows):
        x[r, rng.integers(0, vocab, 5)] += np.float32(12.0)
    h = [rng.integers(0, vocab, hist) for _ in range(rows)]
    ids, offs = _csr(h)
    return Batch("C1", x, Params(temperature=0.0, repetition_penalty=1.1), hist_ids=ids, hist_offsets=offs)


def c2(rows: int = 64, vocab: int = QWEN_VOCAB, seed: int = 2) -> Batch:
    rng = _rng(seed)
    x = _normal(rng, rows, vocab, 3.0)
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    bias = (10.0 * ranks ** -1.1).astype(np.float32)
    for r in range(rows):
        a, b = _affine_perm(rng, vocab)
        ids = (a * np.arange(vocab, dtype=np.int64) + b) % vocab
        x[r, ids] += bias
    u = rng.random(rows)
    return Batch("C2", x, Params(temperature=0.7, top_k=40, top_p=0.95), uniforms=u)


def c3(rows: int = 128, vocab: int = GEMMA_VOCAB, seed: int = 3, penalties: bool = False,
       hist: int = 512) -> Batch:
    rng = _rng(seed)
    x = _normal(rng, rows, vocab, 4.0)
    mask = random_mask(rng, rows, vocab, 0.005, 0.20)
    u = rng.random(rows)
    p = Params(temperature=1.0, top_k=50, top_p=0.9)
    ids = offs = None
    name = "C3"
    if penalties:
        name = "C3P"
        p = Params(temperature=1.0, top_k=50, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.5,
                   frequency_penalty=0.3)
        ids, offs = _csr([rng.integers(0, vocab, hist) for _ in range(rows)])
    return Batch(name, x, p, mask=mask, hist_ids=ids, hist_offsets=offs, uniforms=u)


def c3p(rows: int = 128, vocab: int = GEMMA_VOCAB, seed: int = 33, hist: int = 512) -> Batch:
    return c3(rows, vocab, seed, penalties=True, hist=hist)


def c4(rows: int = 256, vocab: int = GEMMA_VOCAB, seed: int = 4, hist: int = 4096) -> Batch:
    rng = _rng(seed)
    x = _normal(rng, rows, vocab, 3.0)
    h = []
    for _ in range(rows):
        a, b = _affine_perm(rng, vocab)
        rk = zipf_ranks(rng, hist, vocab, 1.2)
        h.append((a * rk.astype(np.int64) + b) % vocab)
    ids, offs = _csr(h)
    p = Params(temperature=0.0, repetition_penalty=1.15, presence_penalty=0.5, frequency_penalty=0.3)
    return Batch("C4", x, p, hist_ids=ids, hist_offsets=offs)


def c5(seqs: int = 32, vocab: int = QWEN_VOCAB, seed: int = 5, drafts: int = 4, density: float = 0.05):
    """Speculative verify inputs: dict of host arrays (see module docstring)."""
    rng = _rng(seed)
    L = drafts
    target = _normal(rng, seqs * (L + 1), vocab, 3.0)
    tview = target.reshape(seqs, L + 1, vocab)
    # 0.8 * N(0,3) + 0.6 * N(0,3): unit-free correlation 2.4 / sqrt(2.4^2 + 1.8^2) = 0.8
    draft = (np.float32(0.8) * tview[:, :L, :] + _normal(rng, seqs * L, vocab, 1.8).reshape(seqs, L, vocab))
    draft = np.ascontiguousarray(draft.reshape(seqs * L, vocab), dtype=np.float32)
    mask = random_mask(rng, seqs * (L + 1), vocab, density, density)
    bits = np.unpackbits(mask.view(np.uint8), bitorder="little").reshape(seqs * (L + 1), -1)[:, :vocab]
    draft_ids = np.zeros((seqs, L), dtype=np.uint32)
    for s in range(seqs):
        for j in range(L):
            allowed = bits[s * (L + 1) + j].astype(bool)
            z = draft[s * L + j].astype(np.float64)
            z = np.where(allowed, z, -np.inf)
            w = np.exp(z - z.max())
            w /= w.sum()
            draft_ids[s, j] = rng.choice(vocab, p=w)
    u = rng.random((seqs, L + 1, 2))
    return {"target": target, "draft": draft, "mask": mask, "draft_ids": draft_ids, "uniforms": u,
            "temperature": 1.0, "vocab": vocab, "seqs": seqs, "drafts": L}


def spec_case(seqs: int = 32, vocab: int = QWEN_VOCAB, seed: int = 6, drafts: int = 2, hist: int = 512,
              greedy_every: int = 3, mask: bool = False):
    """Exact-match speculative round inputs (the reference's mode: argmax
    drafts, kernels.js:211-401): dict of host arrays.  The draft head's rows
    are the target rows they predict plus noise, so drafts often equal the
    target's argmax; every greedy_every-th sequence is greedy (its verify
    rows then accept every draft that is the target's argmax)."""
    rng = _rng(seed)
    L = drafts
    target = _normal(rng, seqs * (L + 1), vocab, 3.0)
    tview = target.reshape(seqs, L + 1, vocab)
    draft = np.ascontiguousarray(
        (tview[:, :L, :] + _normal(rng, seqs * L, vocab, 0.3).reshape(seqs, L, vocab)).reshape(seqs * L, vocab),
        dtype=np.float32)
    sp = []
    for s in range(seqs):
        if greedy_every and s % greedy_every == 0:
            sp.append(Params(temperature=0.0, presence_penalty=0.5))
        else:
            sp.append(Params(temperature=0.6, top_k=20, top_p=0.95, presence_penalty=1.5,
                             repetition_penalty=1.05))
    ids, offs = _csr([rng.integers(0, vocab, hist) for _ in range(seqs)]) if hist else (None, None)
    m = random_mask(rng, seqs * (L + 1), vocab, 0.3, 0.9) if mask else None
    stop = np.full((seqs, 4), 0xFFFFFFFF, np.uint32)
    stop[:, 0] = 151645  # Qwen's <|im_end|>
    return {"target": target, "draft": draft, "mask": m, "hist_ids": ids, "hist_offsets": offs,
            "seq_params": sp, "seeds": rng.integers(0, 2**32, seqs, dtype=np.uint64).astype(np.uint32),
            "round": int(rng.integers(0, 1000)), "stop_ids": stop, "vocab": vocab, "seqs": seqs, "drafts": L}


def bf16_bits(rng, shape, lo_exp: int = -6, hi_exp: int = -3) -> np.ndarray:
    """Random bf16 bit patterns (uint16): random sign and 7-bit mantissa,
    exponent uniform in [lo_exp, hi_exp] (magnitudes 2^lo_exp .. 2^(hi_exp+1)),
    as one table lookup per uniform 16-bit draw."""
    r = np.arange(1 << 16, dtype=np.uint32)
    span = hi_exp - lo_exp + 1
    e = ((r >> 7) & 0xFF) % span
    table = ((r & 0x8000) | ((e + np.uint32(127 + lo_exp)) << 7) | (r & 0x7F)).astype(np.uint16)
    return table[rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)]


HEAD_BF16, HEAD_Q8_0, HEAD_Q4_0, HEAD_Q6_K = 0, 1, 2, 3
HEAD_NAMES = {HEAD_BF16: "bf16", HEAD_Q8_0: "Q8_0", HEAD_Q4_0: "Q4_0", HEAD_Q6_K: "Q6_K"}


@dataclass
class LmhBatch:
    """Inputs of sas_lm_head_sample: fp32 hidden states, the head (bf16 bits
    [vocab][dim] as uint16, or GGUF blocks [vocab][row bytes] as uint8 with
    fmt set) and the sampling descriptor's host arrays."""
    name: str
    hidden: np.ndarray            # float32 [rows, dim]
    weight_bits: Optional[np.ndarray]  # uint16 [vocab, dim] (bf16) or None
    params: Params
    mask: Optional[np.ndarray] = None
    hist_ids: Optional[np.ndarray] = None
    hist_offsets: Optional[np.ndarray] = None
    uniforms: Optional[np.ndarray] = None
    fmt: int = HEAD_BF16
    weight_q: Optional[np.ndarray] = None  # uint8 [vocab, row bytes] (GGUF formats)

    @property
    def rows(self) -> int:
        return self.hidden.shape[0]

    @property
    def vocab(self) -> int:
        return (self.weight_bits if self.fmt == HEAD_BF16 else self.weight_q).shape[0]

    @property
    def weight(self) -> np.ndarray:
        """The head as the C ABI takes it (bf16 bits or GGUF bytes)."""
        return self.weight_bits if self.fmt == HEAD_BF16 else self.weight_q

    @property
    def dim(self) -> int:
        return self.hidden.shape[1]

    def with_logits(self, logits: np.ndarray) -> Batch:
        """The sampling step over given logits (the unfused path's input)."""
        return Batch(self.name, logits, self.params, mask=self.mask, hist_ids=self.hist_ids,
                     hist_offsets=self.hist_offsets, uniforms=self.uniforms)

    def algorithmic_bytes(self) -> int:
        """Compulsory HBM bytes of one call: the head read once, the hidden
        states, mask words, history ids and offsets, uniforms, ids out."""
        b = self.weight.nbytes + self.hidden.nbytes + 4 * self.rows
        if self.mask is not None:
            b += self.rows * ((self.vocab + 31) // 32) * 4
        if self.hist_ids is not None:
            b += self.hist_ids.nbytes + self.hist_offsets.nbytes
        if self.uniforms is not None and self.params.temperature > 0:
            b += self.uniforms.nbytes
        return b


def lmh(rows: int = 1, vocab: int = GEMMA_VOCAB, dim: int = 2560, seed: int = 7, hist: int = 512,
        softcap: float = 30.0, mask: bool = True) -> LmhBatch:
    """LMH: the decode head with sampling fused (sas_lm_head_sample), Gemma-4
    E4B-shaped: hidden 2560 fp32 rows times a [vocab][2560] bf16 head
    (logits ~ N(0, 3) at dim 2560), softcap 30 (gemma-config.js:47), then
    C3P's sampling: mask density U[0.5 %, 20 %], top-k 50 / top-p 0.9 /
    T 1.0, repetition 1.1 / presence 0.5 / frequency 0.3 over `hist` ids."""
    rng = _rng(seed)
    hidden = rng.standard_normal((rows, dim), dtype=np.float32)
    w = bf16_bits(rng, (vocab, dim), -7, -4)
    m = random_mask(rng, rows, vocab, 0.005, 0.20) if mask else None
    ids, offs = _csr([rng.integers(0, vocab, hist) for _ in range(rows)]) if hist else (None, None)
    p = Params(temperature=1.0, top_k=50, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.5,
               frequency_penalty=0.3, softcap=softcap)
    return LmhBatch("LMH", hidden, w, p, mask=m, hist_ids=ids, hist_offsets=offs, uniforms=rng.random(rows))


def gguf_head(rng, fmt: int, vocab: int, dim: int) -> np.ndarray:
    """A random GGUF head [vocab][row bytes] (uint8) of ggml's block layout,
    scaled so that an N(0, 1) hidden row gives logits of about N(0, 3):
    f16 block scales, random quants; Q6_K scales signed."""
    if fmt == HEAD_Q8_0:
        nb, bs = dim // 32, 34
    elif fmt == HEAD_Q4_0:
        nb, bs = dim // 32, 18
    elif fmt == HEAD_Q6_K:
        nb, bs = dim // 256, 210
    else:
        raise ValueError("not a GGUF format")
    w = rng.integers(0, 256, size=(vocab * nb, bs), dtype=np.uint8)
    if fmt == HEAD_Q8_0:
        d = (rng.uniform(0.5, 1.5, vocab * nb) * 8.1e-4).astype(np.float16)
        w[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    elif fmt == HEAD_Q4_0:
        d = (rng.uniform(0.5, 1.5, vocab * nb) * 1.28e-2).astype(np.float16)
        w[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    else:
        sc = rng.integers(-63, 64, size=(vocab * nb, 16)).astype(np.int8)
        w[:, 192:208] = sc.view(np.uint8)
        d = (rng.uniform(0.5, 1.5, vocab * nb) * 1.0e-4).astype(np.float16)
        w[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return np.ascontiguousarray(w.reshape(vocab, nb * bs))


def lmhq(fmt: int = HEAD_Q6_K, rows: int = 1, vocab: int = 248320, dim: int = 2560, seed: int = 8, hist: int = 512,
         softcap: float = 0.0, mask: bool = True) -> LmhBatch:
    """LMQ: the decode head with sampling fused over a GGUF head, by default
    Qwen3.5-4B's tied Q6_K head (hidden 2560, vocabulary 248,320,
    config.js:6-9, gguf/sources.js:122), then C3P's sampling (mask density
    U[0.5 %, 20 %], top-k 50 / top-p 0.9 / T 1.0, repetition 1.1 / presence
    0.5 / frequency 0.3 over `hist` ids)."""
    rng = _rng(seed)
    hidden = rng.standard_normal((rows, dim), dtype=np.float32)
    w = gguf_head(rng, fmt, vocab, dim)
    m = random_mask(rng, rows, vocab, 0.005, 0.20) if mask else None
    ids, offs = _csr([rng.integers(0, vocab, hist) for _ in range(rows)]) if hist else (None, None)
    p = Params(temperature=1.0, top_k=50, top_p=0.9, repetition_penalty=1.1, presence_penalty=0.5,
               frequency_penalty=0.3, softcap=softcap)
    return LmhBatch("LMQ", hidden, None, p, mask=m, hist_ids=ids, hist_offsets=offs, uniforms=rng.random(rows),
                    fmt=fmt, weight_q=w)


def c3p_shard8(rows: int = 128, seed: int = 38) -> Batch:
    """One GPU's share of C3P split 8 ways over the vocabulary: 32,768 ids
    (a multiple of 32, so the mask words split cleanly) and the history ids
    that fall in the shard (512 / 8 on average)."""
    return c3p(rows, GEMMA_VOCAB // 8, seed, hist=512 // 8)


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C3P": c3p, "C3P8": c3p_shard8, "C4": c4}

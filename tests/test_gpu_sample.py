"""GPU parity of sas_sample against the C oracle (bit-exact ids, ranked
candidates and double probabilities), through the C ABI."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import assert_parity, run_gpu, to_dev
from shared_amd import Params
from shared_amd import workloads as W
from shared_amd._capi import FLAG_EMPTY_ROW, FLAG_SLOW_SELECT, NO_TOKEN

pytestmark = pytest.mark.gpu


def check(s, b, row_params=None, label=""):
    g = run_gpu(s, b, row_params=row_params)
    o = O.sample_rows(b, row_params=row_params)
    assert_parity(g, o, label or b.name)
    return g, o


# ---------------------------------------------------------------- configs --

@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C3P", "C4"])
def test_config_full_size(sampler, name):
    b = W.CONFIGS[name]()
    print(f"[gpu] config {name} rows={b.rows} vocab={b.vocab}", flush=True)
    check(sampler, b)


# ------------------------------------------------------- random small cases --

def _small_batch(seed, rows, vocab, params, mask_density=None, hist=0, sigma=3.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, vocab)) * sigma).astype(np.float32)
    mask = None
    if mask_density is not None:
        mask = W.random_mask(rng, rows, vocab, mask_density, mask_density)
    hi = ho = None
    if hist:
        hi, ho = W._csr([rng.integers(0, vocab, hist) for _ in range(rows)])
    return W.Batch("small", x, params, mask=mask, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("vocab", [1000, 4099, 33333, 151936])
def test_random_params(sampler, seed, vocab):
    rng = np.random.default_rng(100 + seed)
    p = Params(temperature=float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])), top_k=int(rng.integers(1, 129)),
               top_p=float(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0])),
               repetition_penalty=float(rng.choice([1.0, 1.1, 1.3])),
               presence_penalty=float(rng.choice([0.0, 0.5, 1.5])),
               frequency_penalty=float(rng.choice([0.0, 0.3])))
    b = _small_batch(seed, rows=int(rng.integers(1, 40)), vocab=vocab, params=p,
                     mask_density=rng.choice([None, 0.01, 0.3]), hist=int(rng.choice([0, 7, 300])))
    print(f"[gpu] random seed={seed} vocab={vocab} rows={b.rows} {p}", flush=True)
    check(sampler, b)


@pytest.mark.parametrize("tail", [1, 5, 255, 257, 384, 511, 513, 767, 769, 1023])
def test_short_last_part(sampler, tail):
    # 12 rows of 37 * 4,096 + tail ids: on 256 CUs the library splits each row
    # into 38 parts of 4,096 ids, so the last part holds `tail` ids and the
    # lanes of its last waves hold none.  Its bound comes from the waves that
    # hold ids (rank 1, the exact wave maximum, for greedy rows and small k);
    # some rows have their best values in that part.
    vocab = 37 * 4096 + tail
    for p in (Params(temperature=0.0, repetition_penalty=1.1), Params(temperature=1.0, top_k=3, top_p=1.0),
              Params(temperature=0.8, top_k=50, top_p=0.9), Params(temperature=1.0, top_k=128, top_p=1.0)):
        b = _small_batch(7 + tail, rows=12, vocab=vocab, params=p, hist=64)
        b.logits[::3, vocab - tail:] += np.float32(4.0)
        print(f"[gpu] short last part tail={tail} {p}", flush=True)
        check(sampler, b)


def test_row_params_mixed(sampler):
    rng = np.random.default_rng(7)
    rows = 24
    plist = [Params(temperature=float(t), top_k=int(k), top_p=float(pp), presence_penalty=float(pr))
             for t, k, pp, pr in zip(rng.choice([0.0, 0.6, 1.0], rows), rng.integers(1, 129, rows),
                                     rng.choice([0.3, 0.95, 1.0], rows), rng.choice([0.0, 1.5], rows))]
    b = _small_batch(11, rows, 20000, Params(temperature=1.0), mask_density=0.2, hist=64)
    check(sampler, b, row_params=plist, label="row_params")


def test_penalty_order_closed_form_on_gpu(sampler):
    # repetition, then frequency, then presence: id 0 (seen twice) becomes
    # 3 / 2 - 0.5 * 2 - 0.25 = 0.25 and -3 * 2 - 1 - 0.25 = -7.25; the
    # greedy pick flips exactly at those values (another order gives 0.875
    # and -8.5)
    rows = np.array([[3.0, 0.26, 0.1, 0.0], [3.0, 0.24, 0.1, 0.0],
                     [-3.0, -7.2, -9.0, -9.5], [-3.0, -7.3, -9.0, -9.5]], np.float32)
    hi, ho = W._csr([np.array([0, 0], np.uint32)] * 4)
    p = Params(temperature=0.0, repetition_penalty=2.0, frequency_penalty=0.5, presence_penalty=0.25)
    b = W.Batch("penalty_order", rows, p, hist_ids=hi, hist_offsets=ho)
    g, _ = check(sampler, b)
    assert g["ids"].tolist() == [1, 0, 1, 0]


def test_row_params_full_size_mixed(sampler):
    # C3P at full size with per-row params: softcap, repetition, frequency,
    # presence, temperature, top-k and top-p all vary by row
    b = W.c3p()
    rng = np.random.default_rng(21)
    plist = [Params(temperature=float(rng.choice([0.0, 0.7, 1.0, 1.3])), top_k=int(rng.integers(1, 129)),
                    top_p=float(rng.choice([0.5, 0.9, 1.0])), repetition_penalty=float(rng.choice([1.0, 1.1, 1.3])),
                    presence_penalty=float(rng.choice([0.0, 0.5])), frequency_penalty=float(rng.choice([0.0, 0.3])),
                    softcap=float(rng.choice([0.0, 30.0])))
             for _ in range(b.rows)]
    print(f"[gpu] row_params full size rows={b.rows} vocab={b.vocab}", flush=True)
    check(sampler, b, row_params=plist, label="row_params_full")
    # no row with a softcap: the cheaper kernel variant through the hint
    for q in plist:
        q.softcap = 0.0
    check(sampler, b, row_params=plist, label="row_params_full_nocap")


# ------------------------------------------------------------------ edges --

def test_empty_and_single_allowed_rows(sampler):
    vocab, rows = 5000, 4
    b = _small_batch(1, rows, vocab, Params(temperature=1.0, top_k=50, top_p=0.9))
    bits = np.zeros((rows, vocab), bool)
    bits[1, 4321] = True                # exactly one allowed id
    bits[2, [7, 4999]] = True           # two, far apart
    bits[3, :] = True
    b.mask = W.pack_bits(bits)          # row 0: nothing allowed
    g, _ = check(sampler, b, label="empty")
    assert g["ids"][0] == NO_TOKEN and g["flags"][0] & FLAG_EMPTY_ROW
    assert g["ids"][1] == 4321


def test_ties_take_lowest_id(sampler):
    # every logit equal: greedy takes id 0, top-k takes the k lowest ids
    vocab, rows = 70000, 3
    x = np.full((rows, vocab), 1.25, np.float32)
    b = W.Batch("ties", x, Params(temperature=1.0, top_k=64, top_p=1.0), uniforms=np.array([0.0, 0.5, 0.999]))
    g, _ = check(sampler, b, label="ties")
    assert np.array_equal(g["cand_ids"][0, :64], np.arange(64))
    assert g["flags"][0] & FLAG_SLOW_SELECT
    b.params = Params(temperature=0.0)
    g, _ = check(sampler, b, label="ties-greedy")
    assert (g["ids"] == 0).all()


def test_signed_zero_ties(sampler):
    # +0 and -0 are one value: their ties go by id, whatever the sign
    rng = np.random.default_rng(12)
    vocab, rows = 50000, 4
    x = (-1.0 - np.abs(rng.standard_normal((rows, vocab)))).astype(np.float32)
    zeros = rng.choice(vocab, 300, replace=False)
    x[:, zeros] = np.float32(0.0)
    x[:, zeros[::2]] = np.float32(-0.0)
    x[1, zeros.min()] = np.float32(-0.0)       # the lowest zero id negative
    x[2, zeros.min()] = np.float32(0.0)        # the lowest zero id positive
    b = W.Batch("zeros", x, Params(temperature=1.0, top_k=40, top_p=0.5), uniforms=rng.random(rows))
    g, _ = check(sampler, b, label="zeros")
    assert np.array_equal(g["cand_ids"][0, :40], np.sort(zeros)[:40])
    b.params = Params(temperature=0.0)
    g, _ = check(sampler, b, label="zeros-greedy")
    assert (g["ids"] == zeros.min()).all()


def test_penalized_members_of_one_key(sampler):
    # two history members whose penalized doubles differ but round to one
    # float: their ranks need the doubles (the slow select) exactly when
    # the lower one is among the first k + 1 ranks
    a, b_id = 1200, 3400
    xa, xb = np.float32(10.0), np.float32(10.3)
    va = float(xa) - 0.3 * 1
    vb = float(xb) - 0.3 * 2
    assert va < vb and np.float32(va) == np.float32(vb)
    vocab, rows = 5000, 5
    rng = np.random.default_rng(31)
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    x[:, a], x[:, b_id] = xa, xb
    above = rng.choice(np.setdiff1d(np.arange(vocab), [a, b_id]), 20, replace=False)
    # plain values above the pair: the pair takes ranks (n, n + 1)
    n_above = [0, 5, 10, 9, 20]
    for r, n in enumerate(n_above):
        x[r, above[:n]] = np.float32(20.0) + np.arange(n, dtype=np.float32)
    hi, ho = W._csr([np.array([a, b_id, b_id])] * rows)
    b = W.Batch("one_key", x, Params(temperature=1.0, top_k=10, top_p=1.0, frequency_penalty=0.3),
                hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
    g, _ = check(sampler, b, label="one_key")
    for r, n in enumerate(n_above):
        slow = bool(g["flags"][r] & FLAG_SLOW_SELECT)
        assert slow == (n + 1 <= 10), (r, n, g["flags"][r])
        if n + 1 < 10:
            assert g["cand_ids"][r, n] == b_id and g["cand_ids"][r, n + 1] == a


@pytest.mark.parametrize("vocab", [1, 2, 3, 4, 5, 6, 7, 4097, 8191])
def test_small_and_ragged_vocab(sampler, vocab):
    # rows of fewer than 4 logits, and rows whose end cuts a float4
    rng = np.random.default_rng(vocab)
    rows = 5
    x = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    for p in (Params(temperature=0.0), Params(temperature=1.0, top_k=3, top_p=0.9),
              Params(temperature=0.7, top_k=128, top_p=1.0)):
        b = W.Batch("ragged", x, p, uniforms=rng.random(rows))
        print(f"[gpu] ragged vocab={vocab} {p}", flush=True)
        check(sampler, b, label=f"ragged{vocab}")


@pytest.mark.parametrize("vocab,rows", [(524_289, 3), (1_000_003, 3), (2_000_000, 4)])
def test_multi_pass_parts(sampler, vocab, rows):
    # vocabularies past 64 parts of 8,192 ids: every part runs 2 or 4 passes
    # of 8,192 ids (its history bitmap rebuilt per pass, its lists and bound
    # carried across them); 524,289 leaves a last part of one id, and the
    # ragged ends cut the row's last float4
    for i, p in enumerate((Params(temperature=0.8, top_k=100, top_p=0.9, repetition_penalty=1.2,
                                  presence_penalty=0.4, frequency_penalty=0.2),
                           Params(temperature=0.0, repetition_penalty=1.3))):
        b = _small_batch(7 + i, rows=rows, vocab=vocab, params=p, mask_density=[0.3, None][i], hist=2000)
        print(f"[gpu] multi-pass vocab={vocab} rows={rows} {p}", flush=True)
        check(sampler, b, label=f"multipass{vocab}")


def test_many_ties_at_threshold(sampler):
    # a few distinct levels, each shared by thousands of ids
    rng = np.random.default_rng(3)
    vocab, rows = 100000, 6
    x = rng.integers(0, 5, (rows, vocab)).astype(np.float32)
    b = W.Batch("levels", x, Params(temperature=0.8, top_k=100, top_p=0.99), uniforms=rng.random(rows))
    check(sampler, b, label="levels")


def test_nan_inf_logits(sampler):
    rng = np.random.default_rng(4)
    vocab, rows = 9000, 5
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    x[0, ::3] = np.nan
    x[1, 17] = np.inf
    x[2, :] = -np.inf
    x[2, 100] = 0.5
    x[3, :] = np.nan
    x[4, 5] = -np.inf
    b = W.Batch("naninf", x, Params(temperature=1.0, top_k=20, top_p=0.9), uniforms=rng.random(rows))
    check(sampler, b, label="naninf")


def test_stride_and_unaligned(sampler):
    import torch
    rng = np.random.default_rng(5)
    vocab, rows, stride = 30001, 7, 30017
    full = rng.standard_normal((rows, stride + 1)).astype(np.float32)
    b = W.Batch("stride", np.ascontiguousarray(full[:, 1:1 + vocab]), Params(temperature=0.9, top_k=30, top_p=0.8),
                uniforms=rng.random(rows))
    dev = torch.from_numpy(full).cuda()
    view = dev[:, 1:1 + vocab]          # misaligned rows, stride != vocab
    g = run_gpu(sampler, b, logits_dev=view)
    assert_parity(g, O.sample_rows(b), "unaligned")


def test_history_edge_ids(sampler):
    rng = np.random.default_rng(6)
    vocab, rows = 12345, 3
    x = rng.standard_normal((rows, vocab)).astype(np.float32) * 2
    top = np.argsort(-x, axis=1)[:, :5]
    hist = [np.concatenate([top[0], top[0], [vocab + 10, 0xFFFFFFF0]]),  # duplicates + out-of-range ids
            np.zeros(0, np.int64), np.repeat(top[2, :1], 3100)]          # empty; one id many times
    # (over 1,024 ids per row on average: the history is bucketed by part)
    hi, ho = W._csr(hist)
    b = W.Batch("hist", x, Params(temperature=1.0, top_k=10, top_p=1.0, repetition_penalty=1.3,
                                  presence_penalty=0.7, frequency_penalty=0.01),
                hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
    check(sampler, b, label="hist")


def test_dense_and_long_histories(sampler):
    # history members packed into whole float4s and words, members that stay
    # in the top k after their penalties, more distinct members in one part
    # than its exact list holds (the part's exact fallback), and a history
    # longer than the ids a block loads up front
    rng = np.random.default_rng(17)
    vocab, rows = 20000, 5
    x = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    x[1, 2048:2348] += 6.0                                   # members that win despite the penalties
    x[4, :64] = np.float32(9.0)                              # tied members at the top
    hist = [np.arange(0, 600),                               # 600 distinct ids in the row's first ids
            np.arange(2048, 2348),                           # contiguous: every id of whole words
            rng.integers(0, vocab, 5000),                    # long, with repeats
            np.zeros(0, np.int64),
            np.concatenate([np.arange(0, 64), np.arange(0, 64)])]
    hi, ho = W._csr(hist)
    for p in (Params(temperature=1.0, top_k=40, top_p=0.95, repetition_penalty=1.2, presence_penalty=0.3,
                     frequency_penalty=0.1),
              Params(temperature=0.0, repetition_penalty=1.2, presence_penalty=0.3),
              Params(temperature=0.8, top_k=128, top_p=1.0, repetition_penalty=0.8)):  # penalties that raise
        b = W.Batch("dense_hist", x, p, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
        print(f"[gpu] dense/long histories {p}", flush=True)
        check(sampler, b, label="dense_hist")


def test_long_history_members_in_the_lists(sampler):
    # bucketed (long) histories with penalties that only lower values: the
    # members ride in the lists with their raw values.  Row 0's 1,024 members
    # lead its first part (more than a part's member slots: the exact
    # selection restarts its member records); row 1 mixes members and plain
    # values near the top; the third case's repetition < 1 raises values
    # (members collected in the slot loop instead)
    rng = np.random.default_rng(23)
    vocab, rows = 40000, 3
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    x[0, :1024] += np.float32(10.0)
    x[1, 5000:5100] += np.float32(3.0)
    hist = [np.concatenate([np.arange(0, 1024), rng.integers(0, vocab, 176)]),
            np.concatenate([np.arange(5000, 5100, 2), rng.integers(0, vocab, 1150)]),
            rng.integers(0, vocab, 1200)]
    hi, ho = W._csr(hist)
    for p in (Params(temperature=1.0, top_k=128, top_p=1.0, repetition_penalty=1.0001),
              Params(temperature=0.9, top_k=40, top_p=0.9, repetition_penalty=1.3, frequency_penalty=0.4,
                     presence_penalty=0.2),
              Params(temperature=1.0, top_k=64, top_p=0.95, repetition_penalty=0.9),
              Params(temperature=0.0, repetition_penalty=1.2, presence_penalty=0.5)):
        b = W.Batch("members_in_lists", x, p, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
        print(f"[gpu] members in the lists {p}", flush=True)
        g, _ = check(sampler, b, label="members_in_lists")
        if p.repetition_penalty == 1.0001:
            assert g["flags"][0] & FLAG_SLOW_SELECT


@pytest.mark.parametrize("top_k", [65, 100, 128])
@pytest.mark.parametrize("hist_len", [64, 1500])
def test_top_k_above_64_stays_on_the_lists(sampler, top_k, hist_len):
    # top-k above 64: a wave's list passes 64 float4s and each lane cuts a
    # second entry; whole 8192-id parts still emit their records from the
    # lists (no SAS_FLAG_SLOW_SELECT), with short histories (hash) and long
    # ones (bucketed, members riding in the lists)
    rng = np.random.default_rng(top_k + hist_len)
    vocab, rows = 151936, 8
    x = (rng.standard_normal((rows, vocab)) * 3.0).astype(np.float32)
    x[2, 70000:70200] = np.float32(11.0)  # ties across the cut
    hist = [rng.integers(0, vocab, hist_len) for _ in range(rows)]
    hist[3] = np.concatenate([np.arange(70000, 70100), hist[3]])
    hi, ho = W._csr(hist)
    for p in (Params(temperature=1.0, top_k=top_k, top_p=0.95),
              Params(temperature=0.7, top_k=top_k, top_p=0.99, repetition_penalty=1.1, frequency_penalty=0.2,
                     presence_penalty=0.1)):
        b = W.Batch("top_k_lists", x, p, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
        print(f"[gpu] top-k {top_k} hist {hist_len} {p}", flush=True)
        g, _ = check(sampler, b, label="top_k_lists")
        assert not np.any(g["flags"] & FLAG_SLOW_SELECT), g["flags"]


def test_repeated_launches_reset_state(sampler):
    b = W.c3p(rows=32, vocab=50000)
    first = run_gpu(sampler, b)
    for _ in range(3):
        again = run_gpu(sampler, b)
        assert np.array_equal(first["ids"], again["ids"])
        assert np.array_equal(first["probs"].view(np.uint64), again["probs"].view(np.uint64))


def test_pcg_uniform_matches_reference_hash():
    from shared_amd import _capi
    lib = _capi.load()
    for seed, it, row in [(1, 0, 0), (0xDEADBEEF, 7, 2), (12345, 99, 1)]:
        assert lib.sas_pcg_uniform(seed, it, row) == O.lib().orc_pcg_uniform(seed, it, row)


# -------------------------------------------------- softcap, reuse, errors --

@pytest.mark.parametrize("params", [Params(temperature=1.0, top_k=64, top_p=0.95, softcap=30.0),
                                    Params(temperature=0.0, softcap=30.0, presence_penalty=1.5)])
def test_gemma_softcap_rows(sampler, params):
    rng = np.random.default_rng(21)
    rows, vocab = 16, W.GEMMA_VOCAB
    x = (rng.standard_normal((rows, vocab)) * 12).astype(np.float32)      # beyond the cap's linear range
    hi, ho = W._csr([rng.integers(0, vocab, 512) for _ in range(rows)])
    b = W.Batch("softcap", x, params, mask=W.random_mask(rng, rows, vocab, 0.02, 0.5), hist_ids=hi,
                hist_offsets=ho, uniforms=rng.random(rows))
    check(sampler, b, label="softcap")


@pytest.mark.parametrize("sigma,shift", [(0.3, 0.0), (12.0, 0.0), (80.0, 0.0), (20.0, 320.0), (20.0, -320.0)])
def test_softcap_bounds_from_raw_values(sampler, sigma, shift):
    # The parts bound softcap rows on their raw values and cap only the
    # values near the bound.  Spreads where the cap is nearly linear (0.3),
    # curved (12), and flat at the bound (80: bounds beyond 5 cap, where every
    # value is capped first); rows shifted into the flat ends, where many
    # values cap to +-30 exactly and ties go by id.
    rng = np.random.default_rng(int(sigma * 10) + abs(int(shift)))
    rows, vocab = 8, W.GEMMA_VOCAB
    x = (rng.standard_normal((rows, vocab)) * sigma + shift).astype(np.float32)
    hi, ho = W._csr([rng.integers(0, vocab, 64) for _ in range(rows)])
    for p in (Params(temperature=1.0, top_k=50, top_p=0.9, softcap=30.0),
              Params(temperature=0.0, repetition_penalty=1.2, softcap=30.0),
              Params(temperature=0.7, top_k=8, top_p=1.0, presence_penalty=0.5, softcap=30.0)):
        b = W.Batch("softcap_raw", x, p, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
        print(f"[gpu] softcap raw bound sigma={sigma} shift={shift} {p}", flush=True)
        check(sampler, b, label="softcap_raw")


def test_back_to_back_launches_with_different_inputs(sampler):
    # the record area and its counters are reused by every launch: a stale
    # record would change ids or probabilities of the next batch
    import torch
    batches = [W.c3p(rows=24, vocab=70000, seed=s) for s in (40, 41, 42)]
    batches.append(W.c4(rows=24, vocab=70000, seed=43, hist=1000))
    outs = []
    for b in batches:
        dev = {k: to_dev(getattr(b, k), torch.int32 if k in ("mask", "hist_ids") else None)
               for k in ("mask", "hist_ids", "hist_offsets", "uniforms")}
        outs.append(sampler.sample(to_dev(b.logits), vocab=b.vocab, params=b.params, full=True, **dev))
    torch.cuda.synchronize()
    for b, o in zip(batches, outs):
        g = {"ids": o["ids"].cpu().numpy().view(np.uint32), "probs": o["probs"].cpu().numpy(),
             "cand_ids": o["cand_ids"].cpu().numpy().view(np.uint32), "counts": o["counts"].cpu().numpy(),
             "flags": o["flags"].cpu().numpy().view(np.uint32)}
        assert_parity(g, O.sample_rows(b), b.name)


def test_argument_errors_are_reported(sampler):
    import torch
    from shared_amd import SasError
    x = torch.zeros((2, 100), dtype=torch.float32, device="cuda")
    ids = torch.empty(2, dtype=torch.int32, device="cuda")
    with pytest.raises(SasError, match="uniforms are required"):
        sampler.sample_into(x, ids, params=Params(temperature=1.0))
    with pytest.raises(SasError, match="vocab"):
        sampler.sample_into(x, ids, vocab=0, params=Params())
    with pytest.raises(SasError, match="logits_stride"):
        sampler.sample_into(x, ids, vocab=101, params=Params())
    with pytest.raises(SasError, match="mask_stride"):
        sampler.sample_into(x, ids, mask=torch.zeros((2, 2), dtype=torch.int32, device="cuda"), params=Params())
    sampler.sample_into(x[:0], ids, params=Params())          # zero rows is a no-op
    # element types the C ABI would misread are refused before the call
    hid = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="hist_offsets"):
        sampler.sample_into(x, ids, hist_ids=hid, hist_offsets=torch.zeros(3, dtype=torch.int64, device="cuda"),
                            params=Params())
    with pytest.raises(ValueError, match="uniforms"):
        sampler.sample_into(x, ids, uniforms=torch.zeros(2, dtype=torch.float32, device="cuda"),
                            params=Params(temperature=1.0))


def test_one_mask_for_every_row(sampler):
    """mask_stride 0: one grammar state shared by all rows equals the same
    words repeated per row."""
    import torch
    b = _small_batch(77, rows=9, vocab=50000, params=Params(temperature=0.8, top_k=40, top_p=0.9),
                     mask_density=0.05)
    one = b.mask[:1]
    b.mask = np.ascontiguousarray(np.repeat(one, b.rows, axis=0))
    lg = to_dev(b.logits)
    u = to_dev(b.uniforms)
    shared = to_dev(one, torch.int32).expand(b.rows, one.shape[1])
    assert shared.stride(0) == 0
    got = sampler.sample(lg, vocab=b.vocab, mask=shared, uniforms=u, params=b.params).cpu().numpy().view(np.uint32)
    want = O.sample_rows(b)["ids"]
    assert np.array_equal(got, want)


def test_random_sweep(sampler):
    # 200 seeded random cases, each bit-exact with the oracle: shapes from 7
    # to 600,001 ids (multi-pass parts), ties, masks of 0.2-90 % density,
    # short and long (bucketed) uniform or Zipf histories with members near
    # the top, penalties that lower or raise values, softcap, greedy rows,
    # top-k 1-128, top-p, and per-row params
    for case in range(200):
        rng = np.random.default_rng(70000 + case)
        rows = int(rng.choice([1, 2, 3, 5, 8, 16]))
        vocab = int(rng.choice([7, 300, 1024, 4097, 20000, 65536, 151936, 262144, 600001]))
        sigma = float(rng.choice([0.5, 2.0, 4.0]))
        x = (rng.standard_normal((rows, vocab)) * sigma).astype(np.float32)
        if rng.random() < 0.3:
            x = np.round(x * 2) / 2
        mask = None
        if rng.random() < 0.6:
            d = float(rng.choice([0.002, 0.05, 0.3, 0.9]))
            mask = W.random_mask(rng, rows, vocab, d, d)
        hi = ho = None
        hlen = int(rng.choice([0, 16, 512, 1500, 4096]))
        if hlen:
            hs = [rng.integers(0, vocab, hlen) if rng.random() < 0.5 else W.zipf_ranks(rng, hlen, vocab, 1.2) % vocab
                  for _ in range(rows)]
            hi, ho = W._csr(hs)
            if rng.random() < 0.5:
                for r in range(rows):
                    x[r, hs[r][:64]] += np.float32(3 * sigma)

        def params():
            return Params(temperature=float(rng.choice([0.0, 0.7, 1.0, 1.5])), top_k=int(rng.integers(1, 129)),
                          top_p=float(rng.choice([1.0, 0.9, 0.5])),
                          repetition_penalty=float(rng.choice([1.0, 1.1, 1.5, 0.8])),
                          presence_penalty=float(rng.choice([0.0, 0.5, -0.3])),
                          frequency_penalty=float(rng.choice([0.0, 0.3, -0.2])),
                          softcap=float(rng.choice([0.0, 0.0, 30.0])))
        b = W.Batch("sweep", x, params(), mask=mask, hist_ids=hi, hist_offsets=ho, uniforms=rng.random(rows))
        rp = [params() for _ in range(rows)] if rng.random() < 0.3 else None
        if case % 50 == 0:
            print(f"[gpu] random sweep case {case}", flush=True)
        check(sampler, b, row_params=rp,
              label=f"sweep {case}: rows={rows} vocab={vocab} hist={hlen} mask={mask is not None} rp={rp is not None}")

"""CPU pins of the oracle.

Each oracle function is checked against something that does not restate it:
the reference's own known answers and input generators, library routines
(numpy, scipy, Hugging Face's logits processors), closed forms and Monte-Carlo
laws.  Every check is chosen so that a plausible mistake -- a dropped penalty
term, a wrong sign, an inclusive / exclusive cut, a transposed p and q, an
off-by-one in the drafted path -- fails it.
"""
from __future__ import annotations

import numpy as np
import pytest
from scipy import special, stats

from helpers import greedy_reference_patterns, xorshift_topk_case, xorshift_topk_case_fast

BF16, F16, F32 = 0, 1, 2


def decode(bits: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F16:
        return bits.astype(np.uint16).view(np.float16).astype(np.float32)
    if dtype == BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return np.asarray(bits, dtype=np.float32)


def random_bits(rng, shape, dtype, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    if dtype == F32:
        return x
    if dtype == F16:
        return x.astype(np.float16).view(np.uint16)
    import torch
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def chi2_pvalue(counts: np.ndarray, probs: np.ndarray) -> float:
    """Pearson chi-square p-value; bins with expected < 5 are pooled."""
    n = counts.sum()
    exp = probs * n
    keep = exp >= 5
    c = np.append(counts[keep], counts[~keep].sum())
    e = np.append(exp[keep], exp[~keep].sum())
    if e[-1] == 0:
        c, e = c[:-1], e[:-1]
    assert counts[probs == 0].sum() == 0, "a token of probability 0 was drawn"
    return float(stats.chisquare(c, e).pvalue)


# ---------------------------------------------------------------- greedy

def greedy_closed_form(vals: np.ndarray):
    """First maximum over finite values; index V when none is finite."""
    rows, v = vals.shape
    fin = np.isfinite(vals)
    tok = np.where(fin, vals, -np.inf).argmax(axis=1)
    tok[~fin.any(axis=1)] = v
    return tok, (~fin).any(axis=1)


@pytest.mark.parametrize("rows,vocab", [(1, 1), (8, 255), (16, 257), (8, 1025), (1, 248320)])
def test_greedy_reference_device_patterns(orc, rows, vocab):
    for bits in greedy_reference_patterns(rows, vocab):
        got = orc.greedy_rows(bits, F16, vocabulary=vocab, serial=5)
        tok, nf = greedy_closed_form(decode(bits[:, :vocab], F16))
        assert np.array_equal(got["token"], tok)
        assert np.array_equal(got["nonfinite"].astype(bool), nf)
        assert np.all(got["serial"] == 5)


@pytest.mark.parametrize("dtype", [BF16, F16, F32])
def test_greedy_random_rows_with_specials(orc, rng, dtype):
    bits = random_bits(rng, (32, 3001), dtype, 3.0)
    special_vals = {F32: [np.float32(np.nan), np.float32(np.inf), np.float32(-np.inf)],
                    F16: [0x7E00, 0x7C00, 0xFC00], BF16: [0x7FC0, 0x7F80, 0xFF80]}[dtype]
    for r in range(0, 32, 3):
        bits[r, rng.integers(0, 3001, 5)] = special_vals[r % 3]
    bits[31, :] = special_vals[0]                     # no finite value -> index V
    x30 = decode(bits[30], dtype)
    bits[30, 3000] = bits[30, int(np.argmax(np.where(np.isfinite(x30), x30, -np.inf)))]   # tie: first wins
    got = orc.greedy_rows(bits, dtype)
    tok, nf = greedy_closed_form(decode(bits, dtype))
    assert np.array_equal(got["token"], tok)
    assert np.array_equal(got["nonfinite"].astype(bool), nf)
    assert got["token"][31] == 3001


def test_cpu_greedy_is_first_max_element(orc, rng):
    x = rng.standard_normal(151936).astype(np.float32)
    x[[100, 90000]] = x.max() + 1
    assert orc.cpu_greedy(x) == 100
    x[5] = np.inf
    assert orc.cpu_greedy(x) == -1                  # the reference throws on non-finite


# ---------------------------------------------------------------- top-k

def topk_reference_test_ids(vals: np.ndarray, k: int) -> list[int]:
    """The reference test's CPU top-k (test_exl3_dflash2_topk.h:11-37): library
    partial sort (value desc, id asc) for ordered rows, the legacy serial
    insertion for rows holding a NaN."""
    if not np.isnan(vals).any():
        order = np.lexsort((np.arange(vals.size), -vals.astype(np.float64)))
        return order[:k].tolist()
    v = vals.tolist()
    ids: list[int] = []
    for i, x in enumerate(v):
        if len(ids) == k and not (x > v[ids[-1]]):
            continue
        if len(ids) == k:
            ids.pop()
        pos = len(ids)
        while pos > 0 and v[ids[pos - 1]] < x:
            pos -= 1
        ids.insert(pos, i)
    return ids


def _check_topk_rows(orc, bits, dtype, k):
    ids, vals, _, nf = orc.topk_rows(bits, dtype, k)
    x = decode(bits, dtype)
    for r in range(bits.shape[0]):
        want = topk_reference_test_ids(x[r], k)
        assert ids[r].tolist() == want, (r, ids[r][:8], want[:8])
        wv = x[r][want]
        nan = np.isnan(wv)
        assert np.array_equal(np.isnan(vals[r]), nan)    # NaN payloads are not part of the result
        assert np.array_equal(vals[r][~nan].view(np.uint32), wv[~nan].view(np.uint32))
    assert nf == int(not np.isfinite(x).all())


@pytest.mark.parametrize("vocab", [16, 17, 31, 255, 257])
@pytest.mark.parametrize("pattern", range(8))
def test_topk_reference_qualification_small(orc, vocab, pattern):
    for rows in (1, 7):
        _check_topk_rows(orc, xorshift_topk_case(rows, vocab, pattern), F16, 16)


@pytest.mark.parametrize("vocab", [248319, 248320, 248321])
@pytest.mark.parametrize("pattern", range(8))
def test_topk_reference_qualification_full_vocab(orc, vocab, pattern):
    rows = 2 if pattern in (5, 6) else 7 if vocab == 248320 else 1
    _check_topk_rows(orc, xorshift_topk_case_fast(rows, vocab, pattern), F16, 16)


@pytest.mark.parametrize("dtype", [BF16, F16, F32])
@pytest.mark.parametrize("k", [1, 8, 16, 64])
def test_topk_ties_and_logprobs(orc, rng, dtype, k):
    bits = random_bits(rng, (6, 5000), dtype, 2.0)
    if dtype != F32:
        bits[:, ::7] = bits[:, 3:4]                     # many exact ties
    ids, vals, lp, _ = orc.topk_rows(bits, dtype, k)
    x = decode(bits, dtype).astype(np.float64)
    lse = special.logsumexp(x, axis=1)
    for r in range(6):
        want = np.lexsort((np.arange(5000), -x[r]))[:k]
        assert np.array_equal(ids[r], want)
        np.testing.assert_allclose(lp[r], x[r][want] - lse[r], rtol=0, atol=2e-6)


# ---------------------------------------------------------------- coupled packet (cap 20)

def packet_support(vals: np.ndarray, temperature, top_k, top_p, min_p):
    """Sorted candidates, cap and support of sampled_select.cuh:79-116 computed
    with numpy in fp64 (cap = min(top_k or 20, 20, V))."""
    order = np.lexsort((np.arange(vals.size), -vals.astype(np.float64)))
    cap = min(top_k if top_k > 0 else 20, 20, vals.size)
    cand = order[:cap]
    w = np.exp((vals[cand].astype(np.float64) - vals[cand[0]]) / temperature)
    keep = np.ones(cap, bool)
    if min_p > 0:
        keep &= np.cumprod(w >= min_p).astype(bool)
    if top_p < 1:
        before = np.concatenate([[0.0], np.cumsum(w)[:-1]])
        keep &= before < top_p * w.sum()
    n = max(1, int(keep.sum()))
    return cand, n, w[:n] / w[:n].sum()


def test_packet_candidates_follow_presence_and_drafted_path(orc, rng):
    v = 300
    bits = random_bits(rng, (4, v), F16, 1.0)
    base = decode(bits, F16)
    fo = np.full(v, 2**31 - 1, dtype=np.int32)        # absent
    hot = np.argsort(-base[0])[:6]
    fo[hot[0]] = 3                                    # generated at position 3
    fo[hot[1]] = 9                                    # generated after the keys below
    inputs = [int(hot[2]), int(hot[3]), int(hot[4]), int(hot[5])]
    depths = [0, 1, 2, 3]
    first_key = 7
    bits[:] = bits[0]
    out, det = orc.sampled_packet(bits, F16, 0.9, 0, 1.0, 0.0, seed=11, presence_penalty=1.5,
                                  first_occurrence=fo, first_key=first_key, depths=depths, inputs=inputs)
    for r in range(4):
        key = first_key + depths[r]
        path = set(inputs[: depths[r]]) | {inputs[r]}
        seen = (fo < key) | np.isin(np.arange(v), list(path))
        pen = np.where(seen, np.float32(base[0]) - np.float32(1.5), base[0]).astype(np.float32)
        want = np.lexsort((np.arange(v), -pen.astype(np.float64)))[:20]
        assert det["key"][r] == key
        assert det["cap"][r] == 20
        assert np.array_equal(det["cand_idx"][r], want)
        assert np.array_equal(det["cand_val"][r], pen[want])


def test_packet_temperature_zero_is_penalized_argmax(orc, rng):
    bits = random_bits(rng, (3, 1000), F16, 1.0)
    x = decode(bits, F16)
    fo = np.full(1000, 2**31 - 1, dtype=np.int32)
    fo[np.argmax(x, axis=1)] = 0
    out, det = orc.sampled_packet(bits, F16, 0.0, 0, 0.9, 0.1, seed=3, presence_penalty=10.0,
                                  first_occurrence=fo, first_key=1)
    pen = np.where(fo < 1, x - 10.0, x)
    assert np.array_equal(out["token"], np.argmax(pen, axis=1))
    assert np.all(det["support"] == 1)


@pytest.mark.parametrize("params", [(0.8, 0, 0.9, 0.02), (1.3, 12, 1.0, 0.0), (0.5, 5, 0.95, 0.1)])
def test_packet_gumbel_max_law(orc, params):
    """Over seeds, the selected token follows softmax(l/T) over the truncated
    support (the Gumbel-max theorem)."""
    temperature, top_k, top_p, min_p = params
    rng = np.random.default_rng(7)
    bits = random_bits(rng, (1, 64), F16, 1.0)
    x = decode(bits, F16)[0]
    cand, n, probs = packet_support(x, temperature, top_k, top_p, min_p)
    counts = np.zeros(n, dtype=np.int64)
    pos = {int(c): j for j, c in enumerate(cand[:n])}
    for seed in range(1, 6001):
        out, det = orc.sampled_packet(bits, F16, temperature, top_k, top_p, min_p, seed=seed, first_key=seed % 97)
        assert det["support"][0] == n
        counts[pos[int(out["token"][0])]] += 1
    assert chi2_pvalue(counts, probs) > 1e-4


# ---------------------------------------------------------------- batched sampler

def make_params(n, **kw):
    import oracle
    p = np.zeros(n, dtype=oracle.ROW_PARAMS)
    p["temperature"] = 1.0
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    for k, v in kw.items():
        p[k] = v
    return p


def penalized_closed_form(x32: np.ndarray, hist: np.ndarray, rep, pres, freq, dtype):
    """HF repetition penalty (RepetitionPenaltyLogitsProcessor, via the library),
    then OpenAI frequency / presence `l - freq*c - pres*[c>0]`, fp32 per op; the
    result stored back in the row's dtype."""
    import torch
    from transformers.generation.logits_process import RepetitionPenaltyLogitsProcessor
    y = torch.from_numpy(x32.copy()).unsqueeze(0)
    if len(hist) and rep != 1.0:
        y = RepetitionPenaltyLogitsProcessor(float(rep))(torch.from_numpy(hist.astype(np.int64)).unsqueeze(0), y)
    y = y[0].numpy().astype(np.float32)
    c = np.bincount(hist, minlength=x32.size).astype(np.float32)
    m = c > 0
    y[m] = y[m] - np.float32(freq) * c[m]
    y[m] = y[m] - np.float32(pres)
    if dtype == BF16:
        y = torch.from_numpy(y).to(torch.bfloat16).float().numpy()
    elif dtype == F16:
        y = y.astype(np.float16).astype(np.float32)
    return y


def hf_filtered_probs(y32: np.ndarray, temperature, top_k, top_p, min_p) -> np.ndarray:
    """Hugging Face's warper chain in fp64 (temperature, top-k, top-p, min-p)."""
    import torch
    from transformers.generation.logits_process import (MinPLogitsWarper, TemperatureLogitsWarper,
                                                        TopKLogitsWarper, TopPLogitsWarper)
    s = torch.from_numpy(y32.astype(np.float64)).unsqueeze(0)
    ids = torch.zeros((1, 1), dtype=torch.long)
    s = TemperatureLogitsWarper(float(temperature))(ids, s)
    if top_k > 0:
        s = TopKLogitsWarper(int(top_k))(ids, s)
    if top_p < 1.0:
        s = TopPLogitsWarper(float(top_p))(ids, s)
    if min_p > 0.0:
        s = MinPLogitsWarper(float(min_p))(ids, s)
    return torch.softmax(s, dim=-1)[0].numpy()


PARAM_SETS = [
    dict(temperature=0.7, top_k=20, top_p=0.8, min_p=0.0),
    dict(temperature=1.2, top_k=0, top_p=0.95, min_p=0.05, repetition_penalty=1.3),
    dict(temperature=0.3, top_k=50, top_p=1.0, min_p=0.0, presence_penalty=0.5, frequency_penalty=0.25),
    dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition_penalty=0.8, frequency_penalty=0.5),
    dict(temperature=0.9, top_k=1, top_p=0.5, min_p=0.5),
    dict(temperature=2.0, top_k=0, top_p=0.6, min_p=0.01, repetition_penalty=1.5, presence_penalty=0.3,
         frequency_penalty=0.1),
]


@pytest.mark.parametrize("pset", range(len(PARAM_SETS)))
def test_sampler_distribution_matches_hf_warpers(orc, pset):
    kw = PARAM_SETS[pset]
    rng = np.random.default_rng(100 + pset)
    rows, v = 12, 4096
    x = (rng.standard_normal((rows, v)) * 2.0).astype(np.float32)
    hists = [rng.integers(0, v, rng.integers(0, 600)).astype(np.int32) for _ in range(rows)]
    hists[0] = np.argsort(-x[0])[:40].astype(np.int32)   # penalties on the head of the row
    offs = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    prm = make_params(rows, **kw)
    prm["lane"] = np.arange(rows)
    prm["seed"] = 99
    _, _, probs, st, margins = orc.sample_rows(x, F32, prm, np.concatenate(hists), offs, want_probs=True)
    for r in range(rows):
        y = penalized_closed_form(x[r], hists[r], kw.get("repetition_penalty", 1.0),
                                  kw.get("presence_penalty", 0.0), kw.get("frequency_penalty", 0.0), F32)
        want = hf_filtered_probs(y, kw["temperature"], kw["top_k"], kw["top_p"], kw["min_p"])
        same = np.array_equal(probs[r] > 0, want > 0)
        if not same:
            assert margins[r, 1] < 1e-6 or margins[r, 2] < 1e-6, (r, (probs[r] > 0).sum(), (want > 0).sum())
            continue
        np.testing.assert_allclose(probs[r], want, rtol=1e-5, atol=1e-12)
        assert st["support"][r] == (want > 0).sum()


@pytest.mark.parametrize("dtype", [BF16, F16])
def test_sampler_16bit_rows_round_penalized_logits(orc, dtype):
    """16-bit rows: penalized logits are stored back in the row's dtype (many
    ties), so compare the multiset of probabilities."""
    rng = np.random.default_rng(31 + dtype)
    rows, v = 6, 2000
    bits = random_bits(rng, (rows, v), dtype, 1.5)
    x = decode(bits, dtype)
    hists = [rng.integers(0, v, 300).astype(np.int32) for _ in range(rows)]
    offs = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    kw = dict(temperature=0.8, top_p=0.9, min_p=0.02, repetition_penalty=1.2, presence_penalty=0.2,
              frequency_penalty=0.1)
    prm = make_params(rows, **kw)
    _, _, probs, st, margins = orc.sample_rows(bits, dtype, prm, np.concatenate(hists), offs, want_probs=True)
    for r in range(rows):
        y = penalized_closed_form(x[r], hists[r], 1.2, 0.2, 0.1, dtype)
        want = hf_filtered_probs(y, 0.8, 0, 0.9, 0.02)
        if (probs[r] > 0).sum() != (want > 0).sum():
            assert margins[r, 1] < 1e-6 or margins[r, 2] < 1e-6
            continue
        np.testing.assert_allclose(np.sort(probs[r])[::-1], np.sort(want)[::-1], rtol=1e-5, atol=1e-12)


def test_sampler_temperature_zero_is_penalized_argmax(orc):
    rng = np.random.default_rng(5)
    rows, v = 8, 3000
    x = rng.standard_normal((rows, v)).astype(np.float32)
    hists = [np.argsort(-x[r])[: r + 1].astype(np.int32) for r in range(rows)]
    offs = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.int64)
    prm = make_params(rows, temperature=0.0, repetition_penalty=1.1, presence_penalty=0.4, frequency_penalty=0.3)
    toks, _, _, st, _ = orc.sample_rows(x, F32, prm, np.concatenate(hists), offs)
    for r in range(rows):
        y = penalized_closed_form(x[r], hists[r], 1.1, 0.4, 0.3, F32)
        assert toks[r] == int(np.argmax(y))
        assert st["support"][r] == 1


def test_sampler_draw_law_over_positions(orc):
    """Philox draws at successive positions follow the filtered distribution."""
    rng = np.random.default_rng(17)
    v, n = 96, 30000
    x = np.tile((rng.standard_normal(v) * 1.5).astype(np.float32), (n, 1))
    prm = make_params(n, temperature=0.9, top_k=40, top_p=0.92, min_p=0.01)
    prm["seed"] = 0xC0FFEE
    prm["lane"] = 3
    prm["position"] = np.arange(n)
    toks, u, probs, st, _ = orc.sample_rows(x, F32, prm, want_probs=True)
    p = probs[0].astype(np.float64)
    counts = np.bincount(toks, minlength=v)
    assert chi2_pvalue(counts, p / p.sum()) > 1e-4
    for i in (0, 1, 777):
        assert u[i] == orc.uniform(0xC0FFEE, 3, i, 0)


def test_sampler_rejects_nothing_finite(orc):
    x = np.full((2, 50), np.nan, dtype=np.float32)
    x[1, 10] = 1.0
    toks, _, _, st, _ = orc.sample_rows(x, F32, make_params(2, temperature=1.0))
    assert st["flags"][0] & 2 and toks[0] == 50         # VI_FLAG_EMPTY, index V
    assert toks[1] == 10 and st["flags"][1] & 1         # VI_FLAG_NONFINITE


# ---------------------------------------------------------------- acceptance (fp64)

def test_accept_reference_known_answers(orc):
    """The five cases of test_exl3_sampled_acceptance_reference.cpp:16-45."""
    st, o, res = orc.accept(np.array([0.6, 0.4]), np.array([0.5, 0.5]), 0, 0.999, 0.25)
    assert st == 0 and o["accepted"] and not o["correction_draw_used"] and o["token"] == 0
    assert o["acceptance_probability"] == 1.0
    st, o, res = orc.accept(np.array([0.2, 0.8]), np.array([0.5, 0.5]), 0, 0.5, 0.75)
    assert st == 0 and not o["accepted"] and o["correction_draw_used"] and o["token"] == 1
    assert abs(o["acceptance_probability"] - 0.4) < 1e-12 and res[0] == 0 and res[1] == 1
    st, o, res = orc.accept(np.array([0.25, 0.75]), np.array([0.0, 1.0]), 1, 0.9, 0.0)
    assert st == 0 and not o["accepted"] and o["token"] == 0 and res[0] == 1 and res[1] == 0
    st, _, _ = orc.accept(np.array([0.0, 0.5, 0.5]), np.array([0.0, 0.25, 0.75]), 0, 0.5, 0.5)
    assert st != 0                                      # zero-q proposal refused
    st, o, _ = orc.accept(np.array([0.5, 0.5]), np.array([0.5, 0.5]), 1, 0.999999, 0.5)
    assert st == 0 and o["accepted"] and not o["correction_draw_used"]
    assert orc.accept(np.array([np.inf, 0.4]), np.array([0.5, 0.5]), 0, 0.1, 0.1)[0] != 0
    assert orc.accept(np.array([0.4, 0.4]), np.array([0.5, 0.5]), 0, 0.1, 0.1)[0] != 0
    assert orc.accept(np.array([0.6, 0.4]), np.array([0.5, 0.5]), 0, 1.0, 0.1)[0] != 0


def test_accept_matches_reference_build(orc):
    """Differential against the reference's own header compiled into oracle/_ref."""
    import ctypes as C
    if not orc.REF_LIB_PATH.exists():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ref = C.CDLL(str(orc.REF_LIB_PATH))
    rng = np.random.default_rng(23)
    for case in range(400):
        v = int(rng.integers(2, 40))
        p = rng.dirichlet(np.full(v, 0.4))
        q = rng.dirichlet(np.full(v, 0.4))
        if case % 5 == 0:
            q[rng.integers(0, v)] = 0.0
            q /= q.sum()
        tok = int(rng.integers(0, v))
        ua, uc = float(rng.random()), float(rng.random())
        acc, cu, t = C.c_int32(), C.c_int32(), C.c_uint32()
        pr = C.c_double()
        rs = ref.ref_accept(p.ctypes.data_as(C.c_void_p), q.ctypes.data_as(C.c_void_p), C.c_size_t(v),
                            C.c_uint32(tok), C.c_double(ua), C.c_double(uc), C.byref(acc), C.byref(cu),
                            C.byref(t), C.byref(pr))
        st, o, _ = orc.accept(p, q, tok, ua, uc)
        assert (st == 0) == (rs == 0), case
        if st == 0:
            assert (o["accepted"], o["correction_draw_used"], o["token"]) == (bool(acc.value), bool(cu.value), t.value)
            assert o["acceptance_probability"] == pr.value


def test_accept_preserves_target_law(orc):
    """Speculative sampling: proposal ~ q, then accept / correct, yields p."""
    rng = np.random.default_rng(29)
    v, n = 10, 40000
    p = rng.dirichlet(np.ones(v))
    q = rng.dirichlet(np.ones(v))
    counts = np.zeros(v, dtype=np.int64)
    props = rng.choice(v, size=n, p=q)
    us = rng.random((n, 2))
    for i in range(n):
        st, o, _ = orc.accept(p, q, int(props[i]), float(us[i, 0]), float(us[i, 1]))
        assert st == 0
        counts[o["token"]] += 1
    assert chi2_pvalue(counts, p) > 1e-4


# ---------------------------------------------------------------- greedy prefix and verification

@pytest.mark.parametrize("target,tent,term,want", [
    ([5, 6, 7], [5, 6, 7], [], ([5, 6, 7], 3, False, False)),
    ([5, 6, 7], [5, 9, 7], [], ([5, 6], 1, True, False)),
    ([5, 6, 7], [4, 6, 7], [], ([5], 0, True, False)),
    ([5, 2, 7], [5, 2, 7], [2], ([5, 2], 2, False, True)),
    ([5, 2, 7], [5, 3, 7], [2], ([5, 2], 1, True, True)),
    ([9], [9], [9], ([9], 1, False, True)),
])
def test_outer_prefix_closed_form(orc, target, tent, term, want):
    assert orc.outer_prefix(target, tent, term) == want


def test_outer_prefix_extent_errors(orc):
    with pytest.raises(ValueError):
        orc.outer_prefix([], [])
    with pytest.raises(ValueError):
        orc.outer_prefix([1, 2], [1])


def test_verify_greedy_is_argmax_prefix_plus_bonus(orc):
    rng = np.random.default_rng(41)
    lanes, drafts, v = 5, 4, 700
    t = rng.standard_normal((lanes * (drafts + 1), v)).astype(np.float32)
    path = t.argmax(axis=1).reshape(lanes, drafts + 1)
    drafted = path[:, :drafts].copy()
    drafted[1, 2] = (drafted[1, 2] + 1) % v            # lane 1 rejects at depth 2
    drafted[2, 0] = (drafted[2, 0] + 1) % v            # lane 2 rejects at once
    acc, com, cnt, flg, _ = orc.verify_rows(0, t, F32, None, F32, lanes, drafts, drafted, None,
                                            terminal=[int(path[3, 1])])
    assert acc.tolist()[:3] == [4, 2, 0]
    assert com[0].tolist() == path[0].tolist() and cnt[0] == 5
    assert com[1, :3].tolist() == path[1, :3].tolist() and cnt[1] == 3
    assert com[2, 0] == path[2, 0] and cnt[2] == 1
    assert cnt[3] == 2 and acc[3] == 2                 # terminal token stops after depth 1


def test_verify_sampled_preserves_target_law(orc):
    """Lanes whose drafted token is drawn from q commit their first token with
    the target's filtered distribution p."""
    rng = np.random.default_rng(43)
    v, lanes = 24, 30000
    tgt = (rng.standard_normal(v) * 1.2).astype(np.float32)
    drf = (tgt + rng.standard_normal(v).astype(np.float32) * 0.8).astype(np.float32)
    prm = make_params(lanes, temperature=0.8, top_k=16, top_p=0.95)
    prm["seed"] = 77
    prm["lane"] = np.arange(lanes)
    p, _ = orc.row_distribution(tgt, F32, prm[0])
    q, _ = orc.row_distribution(drf, F32, prm[0])
    drafted = rng.choice(v, size=(lanes, 1), p=q / q.sum()).astype(np.int32)
    acc, com, cnt, flg, _ = orc.verify_rows(1, np.tile(tgt, (lanes, 1)), F32, np.tile(drf, (lanes, 1)), F32,
                                            lanes, 1, drafted, prm)
    assert np.all(flg & 4 == 0)
    counts = np.bincount(com[:, 0], minlength=v)
    assert chi2_pvalue(counts, p) > 1e-4


# ---------------------------------------------------------------- VeriCache row scores

def test_row_scores_closed_form(orc):
    """exact_row_score_kernel: argmax over values greater than -Inf (NaN and -Inf
    never win, +Inf can), lowest index; gap = max - logit(next)."""
    rng = np.random.default_rng(61)
    for dtype in (BF16, F16, F32):
        v = 777
        bits = random_bits(rng, (8, v), dtype, 2.0)
        inf_, ninf, nan = {F32: (np.float32(np.inf), np.float32(-np.inf), np.float32(np.nan)),
                           F16: (0x7C00, 0xFC00, 0x7E00), BF16: (0x7F80, 0xFF80, 0x7FC0)}[dtype]
        bits[1, [5, 300]] = inf_               # +Inf wins, first one
        bits[2, ::3] = nan                     # NaN never wins
        bits[3, :] = ninf                      # nothing beats -Inf: index V
        bits[4, :] = nan
        x = decode(bits, dtype)
        nxt = np.array([-1, 300, 7, 3, 4, v, 0, 0], dtype=np.int64)
        cand = x > -np.inf
        masked = np.where(cand, x, -np.inf)
        want_idx = np.where(cand.any(axis=1), masked.argmax(axis=1), v)
        nxt[6] = want_idx[6]                    # next == argmax: gap 0
        nxt[7] = (want_idx[7] + 1) % v
        greedy, gap = orc.row_scores(bits, dtype, nxt)
        assert np.array_equal(greedy, want_idx)
        with np.errstate(invalid="ignore"):
            for r in range(8):
                t = nxt[r]
                best = masked[r, want_idx[r]] if want_idx[r] < v else np.float32(-np.inf)
                exp = np.float32(best) - x[r, t] if (0 <= t < v and t != want_idx[r]) else np.float32(0)
                assert (np.isnan(exp) and np.isnan(gap[r])) or gap[r] == exp, (dtype, r, gap[r], exp)


def fma32(a, b, c):
    """fp32 fused multiply-add through fp64 (a*b is exact in fp64)."""
    return np.float32(np.float64(np.float32(a)) * np.float64(np.float32(b)) + np.float64(np.float32(c)))


def test_sampled_scores_trivial_and_greedy_cases(orc):
    rng = np.random.default_rng(67)
    rows, v = 6, 400
    bits = random_bits(rng, (rows, v), F16, 1.0)
    x = decode(bits, F16)
    # temperature 0 with presence: chosen = penalized argmax, gap = best - penalized logit
    fo = np.full(v, 2**31 - 1, dtype=np.int32)
    fo[np.argmax(x, axis=1)] = 2                       # seen before keys >= 3
    nxt = np.argsort(-x, axis=1)[:, 3].astype(np.int64)
    fo[nxt[::2]] = 0                                   # some next tokens carry the penalty too
    chosen, gap = orc.sampled_scores(bits, F16, 0.0, 0, 1.0, 0.0, 9, nxt, first_key=1, presence_penalty=0.7,
                                     first_occurrence=fo)
    for r in range(rows):
        key = 1 + r
        pen = np.where(fo < key, x[r] - np.float32(0.7), x[r]).astype(np.float32)
        assert chosen[r] == np.argmax(pen)
        assert gap[r] == max(np.float32(0), pen[chosen[r]] - pen[nxt[r]])
    # next == chosen or -1: gap 0; next >= V: infinite
    chosen, _ = orc.sampled_scores(bits, F16, 0.8, 0, 0.9, 0.0, 9, np.zeros(rows), first_key=5)
    _, gap = orc.sampled_scores(bits, F16, 0.8, 0, 0.9, 0.0, 9, chosen, first_key=5)
    assert np.all(gap == 0)
    _, gap = orc.sampled_scores(bits, F16, 0.8, 0, 0.9, 0.0, 9, np.full(rows, -1), first_key=5)
    assert np.all(gap == 0)
    _, gap = orc.sampled_scores(bits, F16, 0.8, 0, 0.9, 0.0, 9, np.full(rows, v), first_key=5)
    assert np.all(np.isinf(gap))


@pytest.mark.parametrize("tolerance", [0.0, 0.05, 0.5, 3.0])
def test_sampled_scores_against_the_packet_and_a_boosted_row(orc, tolerance):
    """In-support next: T times the perturbed-value gap of the coupled draw.
    Just outside the support: re-running the coupled sampler on the row with
    next's logit raised by `tolerance` decides admission, and the gap is
    measured against the best other support entry of that run."""
    rng = np.random.default_rng(71)
    v, temperature, top_p, min_p, seed = 300, 0.8, 0.85, 0.02, 1234
    checked_out, checked_in = 0, 0
    for trial in range(40):
        x = (rng.standard_normal((1, v)) * 1.5).astype(np.float32)
        key = 10 + trial
        out, det = orc.sampled_packet(x, F32, temperature, 0, top_p, min_p, seed=seed, first_key=key)
        d = det[0]
        sup, cap = int(d["support"]), int(d["cap"])
        sel = int(d["selected"])
        for rank in range(cap):
            want = int(d["cand_idx"][rank])
            chosen, gap = orc.sampled_scores(x, F32, temperature, 0, top_p, min_p, seed, [want], first_key=key,
                                             tolerance=tolerance)
            assert chosen[0] == out["token"][0]
            if rank == sel:
                assert gap[0] == 0
            elif rank < sup:
                exp = (np.float32(d["value"][sel]) - np.float32(d["value"][rank])) * np.float32(temperature)
                assert gap[0] == np.float32(exp) and gap[0] >= 0
                checked_in += 1
            elif tolerance == 0.0:
                assert np.isinf(gap[0])
            else:
                xb = x.copy()
                xb[0, want] = np.float32(x[0, want] + np.float32(tolerance))
                _, db = orc.sampled_packet(xb, F32, temperature, 0, top_p, min_p, seed=seed, first_key=key)
                db = db[0]
                ids = list(db["cand_idx"][: int(db["support"])])
                if want not in ids:
                    assert np.isinf(gap[0])
                    continue
                others = [db["value"][j] for j in range(int(db["support"])) if db["cand_idx"][j] != want]
                best = max(others) if others else np.float32(-np.inf)
                inv = np.float32(1.0) / np.float32(temperature)
                own = fma32(x[0, want], inv, orc.gumbel(seed, key, want))
                exp = max(np.float32(0), (np.float32(best) - own) * np.float32(temperature))
                assert gap[0] == np.float32(exp), (trial, rank, gap[0], exp)
                checked_out += 1
    assert checked_in > 20
    if tolerance > 0:
        assert checked_out > 10


# ---------------------------------------------------------------- DFlash2 draft coupled proposal

def draft_sampling(n, **kw):
    import oracle
    s = np.zeros(n, dtype=oracle.DRAFT_SAMPLING)
    s["top_p"] = 1.0
    for k, v in kw.items():
        s[k] = v
    return s


def test_draft_choice_greedy_is_first_maximum(orc):
    rng = np.random.default_rng(81)
    lanes, pos = 5, 4
    sc = rng.standard_normal((lanes, pos, 16)).astype(np.float32)
    sc[0, 0, [3, 9]] = 9.0                                   # tie: the first wins
    cd = rng.integers(0, 1000, (lanes, pos, 16))
    out = orc.draft_choice(sc, cd, draft_sampling(lanes, inv_temperature=0.0), vocabulary=1000)
    want = np.take_along_axis(cd, sc.argmax(axis=2)[..., None], axis=2)[..., 0]
    assert np.array_equal(out, want) and out[0, 0] == cd[0, 0, 3]


def test_draft_choice_presence_covers_seed_history_and_chain(orc):
    """The top candidate is penalized when it is the seed token, was generated
    before the key, or was proposed at an earlier position of the chain."""
    lanes, pos, v = 4, 3, 100
    sc = np.tile(np.linspace(3.0, 0.0, 16, dtype=np.float32), (lanes, pos, 1))
    cd = np.tile(np.arange(16, dtype=np.int64), (lanes, pos, 1))
    fo = np.full(v, 2**31 - 1, dtype=np.int32)
    fo[0] = 5                                                 # token 0 generated at index 5
    smp = draft_sampling(lanes, inv_temperature=1.0, top_k=1, presence_penalty=100.0, seed=3)
    smp["key_base"] = [0, 0, 10, 0]
    smp["first_occurrence"][2] = fo.ctypes.data
    out = orc.draft_choice(sc, cd, smp, seed_tokens=[50, 0, 50, 50], vocabulary=v)
    # lane 0: nothing seen -> 0, then 0 is in the chain -> 1, then 2
    assert out[0].tolist() == [0, 1, 2]
    # lane 1: the seed token is 0 -> 1, 2, 3
    assert out[1].tolist() == [1, 2, 3]
    # lane 2: key 10 > first occurrence 5 of token 0 -> 1, 2, 3
    assert out[2].tolist() == [1, 2, 3]
    # lane 3: keys 0..2 < 5 would not see token 0 even with the table
    smp["first_occurrence"][3] = fo.ctypes.data
    assert orc.draft_choice(sc, cd, smp, seed_tokens=[50, 0, 50, 50], vocabulary=v)[3].tolist() == [0, 1, 2]


@pytest.mark.parametrize("params", [(1.25, 0, 0.9, 0.02), (0.8, 6, 1.0, 0.0), (2.0, 0, 0.7, 0.1)])
def test_draft_choice_gumbel_max_law(orc, params):
    """Over seeds, the proposal follows softmax(score/T) over the truncated support."""
    inv_t, top_k, top_p, min_p = params
    rng = np.random.default_rng(83)
    x = rng.standard_normal(16).astype(np.float32)
    cand = rng.choice(5000, 16, replace=False).astype(np.int64)
    order = np.lexsort((np.arange(16), -x.astype(np.float64)))
    cap = top_k if 0 < top_k < 16 else 16
    w = np.exp((x[order[:cap]].astype(np.float64) - x[order[0]]) * inv_t)
    keep = np.ones(cap, bool)
    if min_p > 0:
        keep &= np.cumprod(w >= min_p).astype(bool)
    if top_p < 1:
        keep &= np.concatenate([[0.0], np.cumsum(w)[:-1]]) < top_p * w.sum()
    n = max(1, int(keep.sum()))
    probs = w[:n] / w[:n].sum()
    seeds = np.arange(1, 6001, dtype=np.uint64)
    smp = draft_sampling(len(seeds), inv_temperature=inv_t, top_k=top_k, top_p=top_p, min_p=min_p)
    smp["seed"] = seeds
    smp["key_base"] = np.arange(len(seeds)) % 97
    out = orc.draft_choice(np.tile(x, (len(seeds), 1, 1)), np.tile(cand, (len(seeds), 1, 1)), smp, vocabulary=5000)
    pos = {int(cand[order[j]]): j for j in range(n)}
    counts = np.zeros(n, dtype=np.int64)
    for t in out[:, 0]:
        counts[pos[int(t)]] += 1
    assert chi2_pvalue(counts, probs) > 1e-4


def test_draft_choice_couples_with_the_target_packet(orc):
    """Same candidates, scores and key as the target's coupled sampler: the draft
    proposes exactly the token the target packet draws (the coupling the
    reference relies on: key = absolute index of the proposed token)."""
    rng = np.random.default_rng(89)
    agree = 0
    for trial in range(200):
        bits = random_bits(rng, (1, 16), F16, 1.0)
        x = decode(bits, F16)[0]
        key = int(rng.integers(0, 10_000))
        seed = int(rng.integers(1, 2**62))
        temperature, top_k, top_p, min_p = 0.8, int(rng.choice([0, 5, 12])), 0.9, 0.02
        out, _ = orc.sampled_packet(bits, F16, temperature, top_k, top_p, min_p, seed=seed, first_key=key)
        smp = draft_sampling(1, inv_temperature=np.float32(1.0) / np.float32(temperature), top_k=top_k,
                             top_p=top_p, min_p=min_p, seed=seed, key_base=key)
        prop = orc.draft_choice(x.reshape(1, 1, 16), np.arange(16).reshape(1, 1, 16), smp, vocabulary=16)
        agree += int(prop[0, 0] == out["token"][0])
    assert agree == 200

"""GPU exact top-k (DFlash2 draft extraction) vs the oracle, bit-exact.

The qualification set of the reference (test_exl3_dflash2_topk.h:183-219): eight
xorshift32 patterns (random, all-equal, +-0, +-Inf, three-value ties, NaN at the
ends, NaN/Inf-rich, winners at the tail) over V in {16, 17, 31, 255, 257, 248319,
248320, 248321}; ids and value bits must equal the oracle's (partial_sort order,
serial-insertion order for NaN rows).  Log-probs within 1e-5 relative of the
oracle's fp64 logsumexp.  Plus config 3 (128 fp16 rows, top-8 + log-probs).
"""
import numpy as np
import pytest
import torch

from helpers import to_dev, xorshift_topk_case, xorshift_topk_case_fast

pytestmark = pytest.mark.gpu


def run(orc, dev, bits, dtype, k, logprobs=True):
    import voidinfer_amd as vi
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    ids, vals, lp = vi.topk_rows(to_dev(bits, dtype, dev), k, logprobs=logprobs, nonfinite_flag=flag)
    w_ids, w_vals, w_lp, w_nf = orc.topk_rows(bits, dtype, k)
    g_ids = ids.cpu().numpy()
    g_vals = vals.cpu().numpy()
    assert np.array_equal(g_ids, w_ids)
    nan = np.isnan(w_vals)
    assert np.array_equal(np.isnan(g_vals), nan)
    assert np.array_equal(g_vals[~nan].view(np.uint32), w_vals[~nan].view(np.uint32))
    assert int(flag.item()) == w_nf
    if logprobs:
        g_lp = lp.cpu().numpy()
        fin = np.isfinite(w_lp)
        assert np.array_equal(np.isfinite(g_lp), fin)
        np.testing.assert_allclose(g_lp[fin], w_lp[fin], rtol=1e-5, atol=1e-5)
    return g_ids, g_vals


@pytest.mark.parametrize("vocab", [16, 17, 31, 255, 257])
@pytest.mark.parametrize("pattern", range(8))
def test_qualification_small(orc, dev, vocab, pattern):
    for rows in range(1, 8):
        bits = xorshift_topk_case(rows, vocab, pattern)
        run(orc, dev, bits, 1, 16)


@pytest.mark.parametrize("vocab", [248319, 248320, 248321])
@pytest.mark.parametrize("pattern", range(8))
def test_qualification_full_vocab(orc, dev, vocab, pattern):
    rows = 7 if vocab == 248320 else 1
    bits = xorshift_topk_case_fast(rows, vocab, pattern)
    run(orc, dev, bits, 1, 16)


@pytest.mark.parametrize("k", [1, 8, 20, 50, 64])
@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_k_and_dtypes(orc, dev, rng, k, dtype):
    rows, vocab = 19, 70_001
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    x[:, rng.integers(0, vocab, 40)] = 3.0
    bits = x if dtype == 2 else (x.astype(np.float16).view(np.uint16) if dtype == 1 else
                                 (x.view(np.uint32) >> 16).astype(np.uint16))
    run(orc, dev, bits, dtype, k)


def test_config3_draft_top8_logprobs(orc, dev):
    from voidinfer_amd import workloads as W
    bits = W.config3(rows=128)
    ids, vals = run(orc, dev, bits, 1, 8)
    # every value above the 8th is in the list (closed form of "top-8")
    v = bits.view(np.float16).astype(np.float32)
    for r in range(0, 128, 17):
        assert set(ids[r]) >= set(np.flatnonzero(v[r] > vals[r, 7]))


def test_repeat_and_padding_guard(orc, dev, rng):
    import voidinfer_amd as vi
    bits = rng.integers(0, 0x7C00, (5, 3001)).astype(np.uint16)
    t = to_dev(bits, 1, dev)
    a = vi.topk_rows(t, 16)
    b = vi.topk_rows(t, 16)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert np.array_equal(t.view(torch.int16).cpu().numpy().view(np.uint16), bits)


def test_rejects_invalid(dev):
    import voidinfer_amd as vi
    t = torch.zeros(2, 15, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError):
        vi.topk_rows(t, 16)
    with pytest.raises(ValueError):
        vi.topk_rows(torch.zeros(2, 100, dtype=torch.float16, device=dev), 65)


@pytest.mark.parametrize("k", [8, 50])
def test_two_batch_slices(orc, dev, rng, k):
    """300 rows of 200,000 fp16 logits: 4 slices of 50,000 per row, so each
    lane of the held scan takes two batches of vectors (the second gated by the
    first batch's threshold)."""
    rows, vocab = 300, 200_000
    x = rng.standard_normal((rows, vocab)).astype(np.float32) * 1.5
    x[np.arange(rows)[:, None], rng.integers(0, vocab, (rows, 6))] = rng.uniform(6, 10, (rows, 6))
    run(orc, dev, x.astype(np.float16).view(np.uint16), 1, k)

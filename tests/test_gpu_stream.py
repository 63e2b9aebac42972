"""GPU full-vocabulary rows in one launch (csrc/sample_stream.hip) vs the CPU oracle.

The stream route serves the 16-bit full-route rows (temperature > 0, top_k 0 or
> 64) of vi_sample_rows / vi_sample_rows_state when no probabilities are
wanted and the rows are 16-byte aligned with a vocabulary that is a multiple of
8; these tests call the sampler that way.  Bar (north star): token ids equal
to the oracle's except where a cumulative-mass boundary lies within 1e-6 of
the drawn uniform or of a cut; support sizes, finite counts and flags equal
outside exempt rows; Philox uniforms bit-exact; support mass within 1e-6.
Cases: vocabularies from 64 to 248,320 and part boundaries (65,528 tokens),
one to 128 rows (one to sixteen parts per row), caps above 64, min-p, top-p,
ties, non-finite and empty rows, signed zeros, logits outside the fast
division's range, temperatures whose z overflows, repetition / presence /
frequency penalties from histories (the history view) and from penalty states
over recorded decode steps, tokens seen hundreds of times, bad history tokens,
and repeated calls on one workspace (the self-resetting counters).
"""
import numpy as np
import pytest
import torch

from helpers import exempt_draw, to_dev
from test_gpu_sample import compare, make_rows, params, run_both

pytestmark = pytest.mark.gpu


def stream(orc, dev, bits, dtype, p, hist=None, offs=None, label=""):
    print(f"[stream] {label} rows={len(p)} vocab={bits.shape[1]}", flush=True)
    return compare(*run_both(orc, dev, bits, dtype, p, hist, offs, want_probs=False), p, label)


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("vocab", [64, 1024, 65_528, 65_536, 131_072, 248_320])
def test_stream_filters(orc, dev, rng, dtype, vocab):
    rows = 16
    bits = make_rows(rng, rows, vocab, std=1.0, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.2, rows), top_k=rng.choice([0, 0, 100, 1000], rows),
               top_p=rng.choice([0.5, 0.9, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.0, 0.01, 0.1], rows))
    stream(orc, dev, bits, dtype, p, label=f"filters-{dtype}-{vocab}")


@pytest.mark.parametrize("rows", [1, 2, 3, 8, 9])
def test_stream_small_batches(orc, dev, rng, rows):
    """Few rows: up to sixteen parts per row, parts spread over every XCD."""
    vocab = 248_320
    bits = make_rows(rng, rows, vocab, std=2.0)
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.0, rows), top_k=0, top_p=rng.choice([0.8, 0.95], rows))
    stream(orc, dev, bits, 0, p, label=f"small-{rows}")


@pytest.mark.parametrize("dtype", [0, 1])
def test_stream_penalties_and_saturation(orc, dev, rng, dtype):
    rows, vocab = 8, 100_000
    bits = make_rows(rng, rows, vocab, std=0.5, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=0, top_p=rng.choice([0.9, 0.95], rows),
               repetition_penalty=rng.uniform(1.0, 1.2, rows), presence_penalty=rng.uniform(0, 0.5, rows),
               frequency_penalty=rng.uniform(0, 0.05, rows))
    L = 6000
    rows_h = []
    for r in range(rows):
        h = rng.integers(0, vocab, L).astype(np.int32)
        h[:600] = 77                     # one token seen 600 times
        h[600:900] = vocab - 1           # ... and one at the last id of the row
        h[900:1000] = rng.integers(0, 50, 100)
        rows_h.append(h)
    offs = np.arange(rows + 1, dtype=np.int64) * L
    stream(orc, dev, bits, dtype, p, np.concatenate(rows_h), offs, "penalties")


@pytest.mark.parametrize("dtype", [0, 1])
def test_stream_repeated_history_tokens(orc, dev, rng, dtype):
    """Tokens seen 2..7 times and at part boundaries: the count-1 penalty of the
    stream corrected from the repeat list at the end of each part."""
    rows, vocab = 8, 248_320
    bits = make_rows(rng, rows, vocab, std=0.5, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=0, top_p=rng.choice([0.9, 0.95], rows),
               repetition_penalty=rng.uniform(1.0, 1.3, rows), presence_penalty=rng.uniform(0, 0.5, rows),
               frequency_penalty=rng.uniform(0.05, 0.3, rows))
    rows_h = []
    for r in range(rows):
        pool = rng.choice(vocab, 400, replace=False)
        reps = np.concatenate([np.repeat(pool[:300], 2 + r % 3), np.repeat(pool[300:], 7)])
        edges = [15_519, 15_520, 62_079, 62_080, 124_159, 124_160, vocab - 1]
        h = np.concatenate([rng.integers(0, vocab, 3000), reps, np.repeat(edges, 3)])
        rows_h.append(rng.permutation(h).astype(np.int32))
    offs = np.concatenate([[0], np.cumsum([len(h) for h in rows_h])]).astype(np.int64)
    stream(orc, dev, bits, dtype, p, np.concatenate(rows_h), offs, "repeats")


def test_stream_nonfinite_and_ties(orc, dev, rng):
    rows, vocab = 6, 9_000
    bits = make_rows(rng, rows, vocab, std=1.0)
    bits[0, ::7] = 0x7FC0          # NaN
    bits[1, 5] = 0x7F80            # +inf
    bits[2, :] = 0x3F80            # all equal (1.0): pure tie-break by id
    bits[3, :4000] = 0x3F80
    bits[4, :] = 0x7FC0            # nothing finite
    p = params(rows, rng, temperature=0.9, top_k=0, top_p=rng.choice([0.3, 0.9], rows))
    g, w = run_both(orc, dev, bits, 0, p, want_probs=False)
    compare(g, w, p, "nonfinite")
    assert w["stats"]["flags"][4] & 2 and g["tokens"][4] == vocab


def test_stream_signed_zeros_extremes_and_temperatures(orc, dev, rng):
    """+0 / -0 (one key), logits beyond the fast division's range (|x| > 2^100,
    subnormal), temperatures whose z overflows, and T > 65,536 (refused)."""
    rows, vocab = 8, 4_096
    bits = make_rows(rng, rows, vocab, std=1.0)
    bits[0, ::2] = 0x0000
    bits[0, 1::2] = 0x8000
    bits[1, :64] = 0x7F00                          # 1.7e38
    bits[1, 64:128] = 0x0001                       # subnormal
    bits[2, :200] = 0x7F00
    bits[3, ::3] = 0x8000
    hist = np.concatenate([np.arange(0, 256, dtype=np.int32)] * rows)
    offs = np.arange(rows + 1, dtype=np.int64) * 256
    p = params(rows, rng, temperature=np.array([0.7, 0.9, 1e-30, 0.5, 1.0, 70_000.0, 0.3, 1.1], np.float32), top_k=0,
               top_p=rng.choice([0.6, 0.99], rows), repetition_penalty=np.array([1.3] * rows, np.float32),
               presence_penalty=0.2, frequency_penalty=0.1)
    g, w = run_both(orc, dev, bits, 0, p, hist, offs, want_probs=False)
    for r in range(rows):
        if r == 5:   # T above 65,536: the 16-bit routes refuse the row
            assert g["tokens"][r] == -1 and g["stats"]["flags"][r] & 0x80000000
            continue
        assert g["tokens"][r] == w["tokens"][r] or exempt_draw(w["margins"][r]), (r, g["tokens"][r], w["tokens"][r])
        assert g["stats"]["flags"][r] == w["stats"]["flags"][r], (r, g["stats"][r], w["stats"][r])


def test_stream_bad_history_tokens_flagged(orc, dev, rng):
    rows, vocab = 4, 5_000
    bits = make_rows(rng, rows, vocab)
    p = params(rows, rng, temperature=1.0, top_k=0, presence_penalty=0.5)
    hist = rng.integers(0, vocab, rows * 100).astype(np.int32)
    hist[5] = -3
    hist[250] = vocab + 10
    offs = np.arange(rows + 1, dtype=np.int64) * 100
    g, w = run_both(orc, dev, bits, 0, p, hist, offs, want_probs=False)
    compare(g, w, p, "badhist")
    assert (g["stats"]["flags"][0] & 16) and (g["stats"]["flags"][2] & 16)


def test_stream_repeat_calls_same_workspace(orc, dev, rng):
    """The part and arrival counters reset themselves: three calls in a row
    on one workspace give the same outputs."""
    import voidinfer_amd as vi
    rows, vocab = 24, 248_320
    bits = make_rows(rng, rows, vocab, std=1.0)
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=0, top_p=0.9)
    t = to_dev(bits, 0, dev)
    outs = []
    for i in range(3):
        print(f"[stream] repeat call {i}", flush=True)
        o = vi.sample_rows(t, p, want_probs=False)
        torch.cuda.synchronize()
        outs.append((o.tokens.cpu().numpy(), vi.stats_numpy(o.stats)))
    for tok, st in outs[1:]:
        assert np.array_equal(tok, outs[0][0])
        assert np.array_equal(st, outs[0][1])
    w_tok, _, _, _, margins = orc.sample_rows(bits, 0, p, None, None, want_probs=False)
    for r in range(rows):
        assert outs[0][0][r] == w_tok[r] or exempt_draw(margins[r]), r


@pytest.mark.parametrize("dtype", [0, 1])
def test_stream_state_route_steps(orc, dev, rng, dtype):
    """Penalties from penalty states over decode steps; odd steps record the
    sampled tokens in the same launch.  Every step against the oracle over the
    equivalent history."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    rows, vocab, L = 12, 248_320, 6000
    x = W.gaussian_zipf(rows, vocab, 1.0, int(rng.integers(1 << 30)))
    bits = W.encode(x, {0: "bf16", 1: "f16"}[dtype])
    p = vi.params_array(rows, seed=rng.integers(1, 2**62, rows), position=rng.integers(0, 10**5, rows),
                        temperature=rng.uniform(0.5, 1.2, rows), top_k=np.array([0, 0, 100, 0, 1000, 0] * 2),
                        top_p=rng.choice([0.9, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.02], rows),
                        repetition_penalty=rng.uniform(1.0, 1.3, rows), presence_penalty=rng.uniform(0, 0.5, rows),
                        frequency_penalty=rng.uniform(0.0, 0.3, rows))
    hist = []
    for r in range(rows):
        top = np.argsort(-x[r])[:300]                # penalties that reorder the top candidates
        h = np.concatenate([rng.integers(0, vocab, L), rng.choice(top, 800), np.repeat(top[:5], 40)])
        hist.append(rng.permutation(h).astype(np.int32))
    st = vi.PenaltyState(rows, vocab, 1 << 14, device=dev)
    toks, offs = np.concatenate(hist), np.concatenate([[0], np.cumsum([len(h) for h in hist])]).astype(np.int64)
    st.update(torch.from_numpy(toks).to(dev), torch.from_numpy(offs).to(dev))
    logits = to_dev(bits, dtype, dev)
    for step in range(4):
        print(f"[stream] state dtype={dtype} step={step}", flush=True)
        fused = step % 2 == 1
        b = vi.sample_rows_state(logits, p, st, record=fused, want_probs=False)
        torch.cuda.synchronize()
        toks = np.concatenate(hist)
        offs = np.concatenate([[0], np.cumsum([len(h) for h in hist])]).astype(np.int64)
        w_tok, w_u, _, w_stats, margins = orc.sample_rows(bits, dtype, p, toks, offs, want_probs=False)
        g_tok = b.tokens.cpu().numpy()
        g_st = vi.stats_numpy(b.stats)
        for r in range(rows):
            if g_tok[r] != w_tok[r] or g_st["support"][r] != w_stats["support"][r]:
                assert exempt_draw(margins[r]), (step, r, g_tok[r], w_tok[r], g_st[r], w_stats[r], margins[r])
        if not fused:
            st.update(b.tokens)
        hist = [np.append(h, t).astype(np.int32) for h, t in zip(hist, g_tok)]
        p["position"] += 1


def test_stream_config5_all_rows(orc, dev):
    """Configuration 5 at full size (128 rows, 32,768-token histories): the
    state route (as the benchmark runs it) and the history route."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    bits, hist, offs, p = W.config5()
    st = vi.PenaltyState(128, W.V_QWEN, 1 << 16, device=dev)
    st.update(torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev))
    logits = to_dev(bits, 0, dev)
    print("[stream] config5 state route", flush=True)
    b = vi.sample_rows_state(logits, p, st, want_probs=False)
    print("[stream] config5 history route", flush=True)
    a = vi.sample_rows(logits, p, torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev),
                       max_history=32768, want_probs=False)
    torch.cuda.synchronize()
    w_tok, w_u, _, w_stats, margins = orc.sample_rows(bits, 0, p, hist, offs, want_probs=False)
    for name, o in (("state", b), ("history", a)):
        g_tok = o.tokens.cpu().numpy()
        g_st = vi.stats_numpy(o.stats)
        exempt = 0
        for r in range(128):
            if g_tok[r] != w_tok[r] or g_st["support"][r] != w_stats["support"][r]:
                assert exempt_draw(margins[r]), (name, r, g_tok[r], w_tok[r], g_st[r], w_stats[r], margins[r])
                exempt += 1
                continue
            assert g_st["flags"][r] == w_stats["flags"][r] and g_st["finite"][r] == w_stats["finite"][r], (name, r)
            np.testing.assert_allclose(g_st["support_mass"][r], w_stats["support_mass"][r], rtol=1e-6)
        assert exempt <= 2, (name, exempt)

"""GPU batched sampler and coupled packet vs the CPU oracle.

Bar (north star): sampled token ids identical except where a cumulative-mass
boundary lies within 1e-6 (relative) of the drawn uniform or of a top-p / min-p
cut; filtered probabilities within 1e-5 relative; Philox uniforms bit-exact;
support sizes and flags equal outside exempt rows.  Both routes are covered:
the top-k route (1 <= top_k <= 64, temperature 0) and the full-vocabulary pair
kernel (top_k = 0 or > 64), with and without penalties over int32 histories.
"""
import numpy as np
import pytest
import torch

from helpers import exempt_draw, to_dev

pytestmark = pytest.mark.gpu

RTOL_PROBS = 1e-5
RTOL_MASS = 1e-6


def run_both(orc, dev, bits, dtype, params, hist=None, offs=None, want_probs=True):
    import voidinfer_amd as vi
    t = to_dev(bits, dtype, dev)
    h_dev = torch.from_numpy(hist).to(dev) if hist is not None else None
    o_dev = torch.from_numpy(offs).to(dev) if offs is not None else None
    max_h = int(np.max(np.diff(offs))) if offs is not None else 0
    out = vi.sample_rows(t, params, h_dev, o_dev, max_history=max(max_h, 1) if hist is not None else 0,
                         want_probs=want_probs)
    torch.cuda.synchronize()
    g = dict(tokens=out.tokens.cpu().numpy(), u=out.uniforms.cpu().numpy(),
             probs=out.probs.cpu().numpy() if want_probs else None, stats=vi.stats_numpy(out.stats))
    w_tok, w_u, w_probs, w_stats, margins = orc.sample_rows(bits, dtype, params, hist, offs, want_probs=want_probs)
    return g, dict(tokens=w_tok, u=w_u, probs=w_probs, stats=w_stats, margins=margins)


def compare(g, w, params, label=""):
    rows = len(params)
    exempt = 0
    for r in range(rows):
        ex = exempt_draw(w["margins"][r])
        if g["tokens"][r] != w["tokens"][r] or g["stats"]["support"][r] != w["stats"]["support"][r]:
            assert ex, (label, r, g["tokens"][r], w["tokens"][r], g["stats"][r], w["stats"][r], w["margins"][r],
                        params[r])
            exempt += 1
            continue
        assert g["stats"]["flags"][r] == w["stats"]["flags"][r], (label, r, g["stats"][r], w["stats"][r])
        assert g["stats"]["finite"][r] == w["stats"]["finite"][r], (label, r)
        if params["temperature"][r] > 0 and not (w["stats"]["flags"][r] & 2):
            assert g["u"][r] == w["u"][r], (label, r)
            # (the full route's coarse bin masses use single-precision weights:
            # within the north-star's 1e-6 relative mass tolerance)
            np.testing.assert_allclose(g["stats"]["support_mass"][r], w["stats"]["support_mass"][r], rtol=RTOL_MASS)
        if g["probs"] is not None:
            gp, wp = g["probs"][r], w["probs"][r]
            assert np.array_equal(gp > 0, wp > 0), (label, r, np.flatnonzero((gp > 0) != (wp > 0))[:10])
            nz = wp > 0
            np.testing.assert_allclose(gp[nz], wp[nz], rtol=RTOL_PROBS, err_msg=f"{label} row {r}")
    return exempt


def decode_rows(bits, dtype):
    if dtype == 2:
        return bits
    if dtype == 1:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def make_rows(rng, rows, vocab, std=2.0, dtype=0, zipf=True):
    from voidinfer_amd import workloads as W
    x = W.gaussian_zipf(rows, vocab, std, int(rng.integers(1 << 30)), zipf=zipf)
    return W.encode(x, {0: "bf16", 1: "f16", 2: "f32"}[dtype])


def params(rows, rng, **kw):
    import voidinfer_amd as vi
    p = vi.params_array(rows, seed=rng.integers(1, 2**62, rows), position=rng.integers(0, 100000, rows))
    for k, v in kw.items():
        p[k] = v
    return p


@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("top_k", [1, 5, 20, 50, 64])
def test_topk_route_no_penalty(orc, dev, rng, dtype, top_k):
    rows, vocab = 24, 50_000
    bits = make_rows(rng, rows, vocab, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.5, rows), top_k=top_k,
               top_p=rng.choice([0.5, 0.8, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.05, 0.2], rows))
    compare(*run_both(orc, dev, bits, dtype, p), p, f"topk{top_k}")


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_temperature_zero_penalized_argmax(orc, dev, rng, dtype):
    rows, vocab = 16, 30_000
    bits = make_rows(rng, rows, vocab, dtype=dtype)
    p = params(rows, rng, temperature=0.0, presence_penalty=rng.uniform(0, 2, rows),
               repetition_penalty=rng.uniform(1.0, 1.3, rows), frequency_penalty=rng.uniform(0, 0.5, rows))
    hist = rng.integers(0, vocab, rows * 300).astype(np.int32)
    # make each row's argmax a history token so the penalty moves it
    offs = np.arange(rows + 1, dtype=np.int64) * 300
    w = orc.greedy_rows(bits, dtype)
    for r in range(rows):
        hist[r * 300] = w["token"][r]
    g, wo = run_both(orc, dev, bits, dtype, p, hist, offs)
    assert np.array_equal(g["tokens"], wo["tokens"])
    assert not np.array_equal(wo["tokens"], w["token"])  # penalties changed some argmax


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_topk_route_penalties(orc, dev, rng, dtype):
    rows, vocab = 12, 40_000
    bits = make_rows(rng, rows, vocab, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.2, rows), top_k=rng.choice([10, 20, 50], rows),
               top_p=rng.choice([0.8, 0.95, 1.0], rows), repetition_penalty=rng.uniform(1.0, 1.5, rows),
               presence_penalty=rng.uniform(0, 1.0, rows), frequency_penalty=rng.uniform(0, 0.5, rows))
    L = 2000
    vals = decode_rows(bits, dtype)
    # histories drawn from each row's 200 largest logits, so penalties reorder candidates
    hist = np.concatenate([rng.choice(np.argsort(-vals[r])[:200], L) for r in range(rows)]).astype(np.int32)
    offs = np.arange(rows + 1, dtype=np.int64) * L
    compare(*run_both(orc, dev, bits, dtype, p, hist, offs), p, "topk-pen")


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_topk_route_ties_and_staging(orc, dev, rng, dtype):
    """Top-k route rows built to stress the batch scan's staging: values drawn
    from 12 levels (many exact ties, ordered by id), top_k 64 (a batch stages
    more than a wave's 64 slots and flushes mid-batch), penalties on tokens of
    the top level, one row with no history; and one row whose frequency
    penalty is too large for the batch scan's range check (element path)."""
    rows, vocab = 10, 30_000
    levels = rng.uniform(-4, 4, 12).astype(np.float32)
    x = levels[rng.integers(0, 12, (rows, vocab))]
    from voidinfer_amd import workloads as W
    bits = W.encode(x, {0: "bf16", 1: "f16", 2: "f32"}[dtype])
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=64, top_p=1.0,
               repetition_penalty=1.1, presence_penalty=0.25, frequency_penalty=0.05)
    p["frequency_penalty"][3] = 1.0e35 if dtype != 1 else 1.0e4
    vals = decode_rows(bits, dtype)
    L = 300
    hist = np.concatenate([rng.choice(np.flatnonzero(vals[r] == vals[r].max()), L) for r in range(rows)])
    hist = hist.astype(np.int32)
    offs = np.arange(rows + 1, dtype=np.int64) * L
    offs[5:] -= L   # row 4: empty history
    hist = np.concatenate([hist[: 4 * L], hist[5 * L:]])
    compare(*run_both(orc, dev, bits, dtype, p, hist, offs), p, "topk-ties")


def test_topk_route_increasing_penalties(orc, dev, rng):
    rows, vocab = 8, 20_000
    bits = make_rows(rng, rows, vocab)
    p = params(rows, rng, temperature=0.8, top_k=20, repetition_penalty=0.8, presence_penalty=-0.5,
               frequency_penalty=-0.1)
    hist = rng.integers(0, vocab, rows * 500).astype(np.int32)
    offs = np.arange(rows + 1, dtype=np.int64) * 500
    compare(*run_both(orc, dev, bits, 0, p, hist, offs), p, "topk-inc")


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("vocab", [64, 1000, 65_537, 248_320])
def test_full_route_filters(orc, dev, rng, dtype, vocab):
    rows = 16
    bits = make_rows(rng, rows, vocab, std=1.0, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.2, rows), top_k=rng.choice([0, 0, 100, 1000], rows),
               top_p=rng.choice([0.5, 0.9, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.0, 0.01, 0.1], rows))
    compare(*run_both(orc, dev, bits, dtype, p), p, f"full-{vocab}")


@pytest.mark.parametrize("dtype", [0, 1])
def test_full_route_penalties_and_saturation(orc, dev, rng, dtype):
    rows, vocab = 8, 100_000
    bits = make_rows(rng, rows, vocab, std=0.5, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=0, top_p=rng.choice([0.9, 0.95], rows),
               repetition_penalty=rng.uniform(1.0, 1.2, rows), presence_penalty=rng.uniform(0, 0.5, rows),
               frequency_penalty=rng.uniform(0, 0.05, rows))
    L = 6000
    rows_h = []
    for r in range(rows):
        h = rng.integers(0, vocab, L).astype(np.int32)
        h[:600] = 77                     # one token seen 600 times (> 255: exact side table)
        h[600:900] = vocab - 1           # ... and one at the last id of the row
        h[900:1000] = rng.integers(0, 50, 100)
        rows_h.append(h)
    hist = np.concatenate(rows_h)
    offs = np.arange(rows + 1, dtype=np.int64) * L
    compare(*run_both(orc, dev, bits, dtype, p, hist, offs), p, "full-pen")


@pytest.mark.parametrize("dtype", [0, 1])
def test_full_route_repeated_history_tokens(orc, dev, rng, dtype):
    """Tokens seen 2..7 times per history: the counts come from the first- and
    second-occurrence bitmaps plus the short list of further occurrences (a
    few hundred entries per half), without a second history pass."""
    rows, vocab = 8, 248_320
    bits = make_rows(rng, rows, vocab, std=0.5, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=0, top_p=rng.choice([0.9, 0.95], rows),
               repetition_penalty=rng.uniform(1.0, 1.3, rows), presence_penalty=rng.uniform(0, 0.5, rows),
               frequency_penalty=rng.uniform(0.05, 0.3, rows))
    rows_h = []
    for r in range(rows):
        pool = rng.choice(vocab, 400, replace=False)
        reps = np.concatenate([np.repeat(pool[:300], 2 + r % 3), np.repeat(pool[300:], 7)])
        h = np.concatenate([rng.integers(0, vocab, 3000), reps, [vocab // 2 - 1] * 4, [vocab // 2] * 5])
        rows_h.append(rng.permutation(h).astype(np.int32))
    offs = np.concatenate([[0], np.cumsum([len(h) for h in rows_h])]).astype(np.int64)
    compare(*run_both(orc, dev, bits, dtype, p, np.concatenate(rows_h), offs), p, "full-rep")


def test_full_route_nonfinite_and_ties(orc, dev, rng):
    rows, vocab = 6, 9_000
    bits = make_rows(rng, rows, vocab, std=1.0)
    bits[0, ::7] = 0x7FC0          # NaN
    bits[1, 5] = 0x7F80            # +inf
    bits[2, :] = 0x3F80            # all equal (1.0): pure tie-break by id
    bits[3, :4000] = 0x3F80
    bits[4, :] = 0x7FC0            # nothing finite
    p = params(rows, rng, temperature=0.9, top_k=0, top_p=rng.choice([0.3, 0.9], rows))
    compare(*run_both(orc, dev, bits, 0, p), p, "full-nonfinite")


def test_bad_history_tokens_flagged(orc, dev, rng):
    rows, vocab = 4, 5_000
    bits = make_rows(rng, rows, vocab)
    p = params(rows, rng, temperature=1.0, top_k=np.array([0, 20, 0, 20]), presence_penalty=0.5)
    hist = rng.integers(0, vocab, rows * 100).astype(np.int32)
    hist[5] = -3
    hist[250] = vocab + 10
    offs = np.arange(rows + 1, dtype=np.int64) * 100
    g, w = run_both(orc, dev, bits, 0, p, hist, offs)
    compare(g, w, p, "badhist")
    assert (w["stats"]["flags"][0] & 16) and (w["stats"]["flags"][2] & 16)


@pytest.mark.parametrize("dtype,vocab", [(0, 5_000), (1, 5_000), (2, 5_000), (0, 300_000)])
def test_topk_route_bad_history_tokens_flagged(orc, dev, rng, dtype, vocab):
    # top-k route rows whose histories hold tokens outside [0, V): flagged and
    # ignored (slices of up to 8,192 tokens count the histories in LDS, larger
    # ones look the counts up in the history hash)
    rows = 4
    bits = make_rows(rng, rows, vocab, dtype=dtype)
    p = params(rows, rng, temperature=1.0, top_k=20, presence_penalty=0.5, repetition_penalty=1.3)
    hist = rng.integers(0, vocab, rows * 100).astype(np.int32)
    hist[105] = -3
    hist[250] = vocab + 10
    offs = np.arange(rows + 1, dtype=np.int64) * 100
    g, w = run_both(orc, dev, bits, dtype, p, hist, offs, want_probs=False)
    compare(g, w, p, "badhist-topk")
    assert (w["stats"]["flags"][1] & 16) and (w["stats"]["flags"][2] & 16)
    assert not (w["stats"]["flags"][0] & 16) and not (w["stats"]["flags"][3] & 16)


def test_topk_route_history_past_max_is_an_error(dev, rng):
    # a history longer than max_history: token -1 and VI_FLAG_ERROR; the other rows are served
    import voidinfer_amd as vi
    rows, vocab = 3, 5_000
    bits = make_rows(rng, rows, vocab)
    p = params(rows, rng, temperature=1.0, top_k=20, presence_penalty=0.5)
    lens = np.array([40, 80, 40])
    hist = rng.integers(0, vocab, int(lens.sum())).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    out = vi.sample_rows(to_dev(bits, 0, dev), p, torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev),
                         max_history=50)
    torch.cuda.synchronize()
    tok, st = out.tokens.cpu().numpy(), vi.stats_numpy(out.stats)
    assert tok[1] == -1 and (int(st["flags"][1]) & 0x80000000)
    assert tok[0] >= 0 and tok[2] >= 0
    assert not (int(st["flags"][0]) & 0x80000000) and not (int(st["flags"][2]) & 0x80000000)


def test_config2_mixed_lanes(orc, dev):
    from voidinfer_amd import workloads as W
    bits, hist, offs, p = W.config2()
    compare(*run_both(orc, dev, bits, 0, p, hist, offs), p, "config2")


def test_config5_subset(orc, dev):
    from voidinfer_amd import workloads as W
    bits, hist, offs, p = W.config5(rows=16)
    compare(*run_both(orc, dev, bits, 0, p, hist, offs), p, "config5")


def test_config1_fp32(orc, dev):
    from voidinfer_amd import workloads as W
    import voidinfer_amd as vi
    x, hist, offs, p = W.config1()
    g = vi.greedy_packet(to_dev(x, 2, dev))
    assert g["token"][0] == orc.cpu_greedy(x[0])
    compare(*run_both(orc, dev, x, 2, p, hist, offs), p, "config1")


@pytest.mark.parametrize("vocab", [1000, 16_385, 151_936, 248_320])
def test_full_route_fp32_filters(orc, dev, rng, vocab):
    """fp32 logits on the full-vocabulary route (sample_wide.hip): top_k 0 or
    above 64 with top-p / min-p, single-slice and many-slice rows."""
    rows = 16
    bits = make_rows(rng, rows, vocab, std=1.0, dtype=2)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.2, rows), top_k=rng.choice([0, 0, 100, 1000], rows),
               top_p=rng.choice([0.5, 0.8, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.0, 0.01, 0.1], rows))
    compare(*run_both(orc, dev, bits, 2, p), p, f"full32-{vocab}")


def test_full_route_fp32_config1_shape(orc, dev, rng):
    """Config 1's row (1 x 151,936 fp32, its 256-token history) with top_k 0,
    top_p 0.8 / 0.95 and penalties; then 16 x 248,320 the same way."""
    from voidinfer_amd import workloads as W
    x, hist, offs, p = W.config1()
    for top_p in (0.8, 0.95):
        q = p.copy()
        q["top_k"], q["top_p"], q["presence_penalty"], q["frequency_penalty"] = 0, top_p, 0.3, 0.1
        compare(*run_both(orc, dev, x, 2, q, hist, offs), q, f"config1 top_p {top_p}")
    rows, vocab, L = 16, 248_320, 4096
    bits = make_rows(rng, rows, vocab, std=2.0, dtype=2)
    q = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=0, top_p=rng.choice([0.8, 0.95], rows),
               repetition_penalty=rng.uniform(1.0, 1.3, rows), presence_penalty=rng.uniform(0, 0.5, rows),
               frequency_penalty=rng.uniform(0.0, 0.2, rows))
    h = []
    for r in range(rows):
        top = np.argsort(-bits[r])[:200]             # penalties that reorder the top candidates
        h.append(rng.permutation(np.concatenate([rng.integers(0, vocab, L), rng.choice(top, 300)])).astype(np.int32))
    offs16 = np.concatenate([[0], np.cumsum([len(v) for v in h])]).astype(np.int64)
    compare(*run_both(orc, dev, bits, 2, q, np.concatenate(h), offs16), q, "fp32 16 x 248,320")


def test_full_route_fp32_edges(orc, dev, rng):
    """NaN / Inf, an all-equal row (one key over every slice), signed zeros,
    nothing finite, spreads far past the 64 binned below the top (cap and min-p
    cut in the deep bin), values around zero across many exponents, huge values,
    an overflow to Inf by the temperature, an unaligned row stride."""
    rows, vocab = 12, 40_000
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    x[0, ::7] = np.nan
    x[1, 5] = np.inf
    x[2, :] = 1.0
    x[3, :20_000] = 0.5
    x[3, 20_000:] = -0.0
    x[4, :] = np.nan
    x[5] *= 100.0
    x[6] *= np.float32(1e-30)
    x[7, :] = -10.0
    x[7, [123, 30_456]] = 60.0
    x[8] *= np.float32(1e30)
    x[9, 10] = np.float32(3e38)
    x[10] *= 100.0
    x[11] *= 0.01
    p = params(rows, rng, temperature=1.0, top_k=0, top_p=0.9)
    p["temperature"][[6, 9]] = [0.7, 0.5]
    p["top_k"][[2, 3, 5, 10]] = [30_000, 25_000, 30_000, 39_990]
    p["top_p"][[2, 5, 10, 11]] = [1.0, 1.0, 1.0, 0.3]
    p["min_p"][[7, 10, 11]] = [1e-30, 1e-30, 0.5]
    compare(*run_both(orc, dev, x, 2, p), p, "fp32 edges")
    # the same rows at a row stride of V + 3 (rows past the first start unaligned)
    import voidinfer_amd as vi
    wide = torch.zeros(rows, vocab + 3, dtype=torch.float32)
    wide[:, :vocab] = torch.from_numpy(x)
    view = wide.to(dev)[:, :vocab]
    out = vi.sample_rows(view, p, want_probs=True)
    torch.cuda.synchronize()
    g, w = run_both(orc, dev, x, 2, p)
    assert np.array_equal(out.tokens.cpu().numpy(), g["tokens"])
    assert torch.equal(out.probs.cpu(), torch.from_numpy(g["probs"]))


def test_draw_distribution_chi_square(orc, dev, rng):
    """Philox inverse-CDF draws follow the filtered distribution (full route)."""
    import scipy.stats
    import voidinfer_amd as vi
    vocab, rows = 512, 4096
    x = (rng.standard_normal(vocab) * 1.5).astype(np.float32)
    bits = np.tile((x.view(np.uint32) >> 16).astype(np.uint16), (rows, 1))
    p = params(rows, rng, temperature=0.8, top_k=0, top_p=0.9)
    p["lane"] = np.arange(rows)
    out = vi.sample_rows(to_dev(bits, 0, dev), p, want_probs=False)
    toks = out.tokens.cpu().numpy()
    prob, sup = orc.row_distribution(bits[0], 0, p[0])
    counts = np.bincount(toks, minlength=vocab)
    m = prob > 0
    assert counts[~m].sum() == 0
    exp = prob[m] * rows
    big = exp >= 5
    chi = ((counts[m][big] - exp[big]) ** 2 / exp[big]).sum()
    assert scipy.stats.chi2.sf(chi, big.sum() - 1) > 1e-4


# ------------------------------------------------------------- coupled packet
def packet_both(orc, dev, bits, dtype, cfg, fo=None, first_key=0, depths=None, inputs=None):
    import voidinfer_amd as vi
    fo_dev = torch.from_numpy(fo).to(dev) if fo is not None else None
    g = vi.sampled_packet(to_dev(bits, dtype, dev), cfg["temperature"], cfg["top_k"], cfg["top_p"], cfg["min_p"],
                          cfg["seed"], cfg.get("presence_penalty", 0.0), fo_dev, first_key, depths, inputs, serial=5)
    w, detail = orc.sampled_packet(bits, dtype, cfg["temperature"], cfg["top_k"], cfg["top_p"], cfg["min_p"],
                                   cfg["seed"], cfg.get("presence_penalty", 0.0), fo, first_key, depths, inputs,
                                   serial=5)
    return g, w, detail


def packet_compare(g, w, detail, cfg):
    """Tokens equal unless the oracle's decision sat within float rounding of a
    boundary: two perturbed values within 1e-5, or a truncation cut
    (cum vs top_p * sum, prob vs min_p * prob[0]) within 1e-5 relative."""
    assert np.array_equal(g["serial"], w["serial"]) and np.array_equal(g["nonfinite"], w["nonfinite"])
    for r in range(len(g)):
        if g["token"][r] != w["token"][r]:
            d = detail[r]
            vals = np.sort(d["value"][: d["support"]])[::-1]
            near = len(vals) > 1 and abs(vals[0] - vals[1]) <= 1e-5 * (1 + abs(vals[0]))
            prob = d["prob"][: d["cap"]].astype(np.float64)
            cum = np.cumsum(prob)
            if cfg["top_p"] < 1:
                near = near or bool(np.any(np.abs(cum - cfg["top_p"] * d["sum"]) <= 1e-5 * d["sum"]))
            if cfg["min_p"] > 0:
                near = near or bool(np.any(np.abs(prob - cfg["min_p"] * prob[0]) <= 1e-5 * prob[0]))
            assert near, (r, g["token"][r], w["token"][r], d)


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_packet_reference_semantics(orc, dev, rng, dtype):
    rows, vocab = 16, 248_320 if dtype == 1 else 60_000
    bits = make_rows(rng, rows, vocab, dtype=dtype)
    for cfg in [dict(temperature=0.7, top_k=20, top_p=0.8, min_p=0.0, seed=123),
                dict(temperature=1.0, top_k=0, top_p=0.95, min_p=0.05, seed=2**63 + 5),
                dict(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, seed=9, presence_penalty=1.5),
                dict(temperature=0.6, top_k=7, top_p=1.0, min_p=0.0, seed=77, presence_penalty=-0.7)]:
        fo = np.full(vocab, 0x7F7F7F7F, dtype=np.int32)
        seen = rng.integers(0, vocab, 300)
        fo[seen] = rng.integers(0, 40, 300)
        top = orc.greedy_rows(bits, dtype)["token"]
        fo[top[:8]] = 5
        g, w, d = packet_both(orc, dev, bits, dtype, cfg, fo, first_key=20,
                              depths=list(range(rows)), inputs=list(rng.integers(0, vocab, rows)))
        packet_compare(g, w, d, cfg)


def test_packet_tree_depths_and_paths(orc, dev, rng):
    rows, vocab = 12, 30_000
    bits = make_rows(rng, rows, vocab)
    top = orc.greedy_rows(bits, 0)["token"]
    cfg = dict(temperature=0.9, top_k=20, top_p=0.9, min_p=0.0, seed=31337, presence_penalty=2.0)
    depths = [0, 1, 2, 3, 4, 5, 1, 2, 3, 2, 1, 4]
    inputs = [int(t) for t in top]
    g, w, d = packet_both(orc, dev, bits, 0, cfg, None, first_key=100, depths=depths, inputs=inputs)
    packet_compare(g, w, d, cfg)


def test_presence_table_kernels(orc, dev, rng):
    import voidinfer_amd as vi
    vocab = 10_000
    table = torch.empty(vocab, dtype=torch.int32, device=dev)
    vi.presence_reset(table)
    assert (table.cpu().numpy() == 0x7F7F7F7F).all()
    toks = torch.tensor([5, 7, 5, 9999, 3, 7], dtype=torch.int64, device=dev)
    vi.presence_record(table, 10, toks)
    t = table.cpu().numpy()
    assert t[5] == 10 and t[7] == 11 and t[9999] == 13 and t[3] == 14 and t[0] == 0x7F7F7F7F
    vi.presence_truncate(table, 12)
    t = table.cpu().numpy()
    assert t[5] == 10 and t[7] == 11 and t[9999] == 0x7F7F7F7F and t[3] == 0x7F7F7F7F

"""GPU DFlash2 verification vs the oracle.

Greedy mode: decide_exl3_outer_prefix over the target rows' argmax, bit-exact
(accepted lengths, committed ids, stop tokens, bonus row).  Sampled mode: the FP64
rejection rule of sampled_acceptance_reference.h on the filtered target / draft
distributions (T .7, top_p .8, top_k 20), Philox u_a / u_c; accepted lengths and
committed ids must be bit-exact except where |u_a - min(1, p/q)| < 1e-9 at a
decided position (reported by the oracle).
"""
import numpy as np
import pytest
import torch

from helpers import to_dev

pytestmark = pytest.mark.gpu


def sampler_from_draft(orc, params):
    rng = np.random.default_rng(99)

    def draw(row_f32, lane, j):
        bits = row_f32.astype(np.float16).view(np.uint16)
        prob, _ = orc.row_distribution(bits, 1, params[lane])
        return int(rng.choice(prob.size, p=prob / prob.sum()))
    return draw


def run(orc, dev, mode, tbits, dbits, drafted, p, lanes, drafts, terminal=()):
    import voidinfer_amd as vi
    t = to_dev(tbits, 0, dev)
    d = to_dev(dbits, 1, dev) if dbits is not None else None
    dr = torch.from_numpy(np.ascontiguousarray(drafted, dtype=np.int32)).to(dev)
    g = vi.verify_rows(mode, t, dr, lanes, drafts, draft=d, params=p, terminal=terminal)
    w = orc.verify_rows(mode, tbits, 0, dbits, 1, lanes, drafts, drafted, p, terminal)
    return g, w


def assert_same(g, w, exempt_lanes=()):
    """Every lane equal to the oracle but the exempt ones; returns the lanes that
    differ (all exempt)."""
    ga, gc, gn, gf = g
    wa, wc, wn, wf, _ = w
    differ = []
    for l in range(len(wa)):
        same = ga[l] == wa[l] and gn[l] == wn[l] and np.array_equal(gc[l], wc[l]) and gf[l] == wf[l]
        if same:
            continue
        assert l in exempt_lanes, (l, ga[l], wa[l], gc[l], wc[l], gf[l], wf[l])
        differ.append(l)
    return differ


@pytest.mark.parametrize("bonus", [False, True])
def test_greedy_prefix(orc, dev, bonus):
    from voidinfer_amd import workloads as W
    lanes, drafts = 8, 16
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, bonus=bonus)
    # make lanes accept 0..drafts tokens: copy the target's argmax into the drafts
    trows = drafts + 1 if bonus else drafts
    targ = orc.greedy_rows(tb, 0)["token"].reshape(lanes, trows)
    for l in range(lanes):
        k = (2 * l + 1) % (drafts + 1) if l < lanes - 1 else drafts
        drafted[l, :k] = targ[l, :k]
    g, w = run(orc, dev, 0, tb, None, drafted, p, lanes, drafts)
    assert_same(g, w)
    assert w[0].max() == drafts


def test_greedy_bonus_then_no_bonus(orc, dev):
    """Both row counts share one workspace per (lanes, drafts, vocabulary): a
    call with the bonus row, then one without, must find the greedy arrival
    counters at zero (they are carved ahead of the shape-dependent partials)."""
    from voidinfer_amd import workloads as W
    lanes, drafts = 8, 16
    for bonus in (True, False, True, False):
        tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, bonus=bonus)
        trows = drafts + 1 if bonus else drafts
        targ = orc.greedy_rows(tb, 0)["token"].reshape(lanes, trows)
        for l in range(lanes):
            k = (3 * l + 2) % (drafts + 1)
            drafted[l, :k] = targ[l, :k]
        print(f"[verify] greedy bonus={bonus}", flush=True)
        g, w = run(orc, dev, 0, tb, None, drafted, p, lanes, drafts)
        assert_same(g, w)


def test_greedy_terminal_stop(orc, dev):
    from voidinfer_amd import workloads as W
    lanes, drafts = 4, 8
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, vocab=20_000)
    targ = orc.greedy_rows(tb, 0)["token"].reshape(lanes, drafts)
    drafted[:] = targ
    term = [int(targ[1, 3]), int(targ[2, 0])]
    g, w = run(orc, dev, 0, tb, None, drafted, p, lanes, drafts, terminal=term)
    assert_same(g, w)
    assert w[0][1] <= 4 and w[0][2] == 1


@pytest.mark.parametrize("bonus", [False, True])
def test_sampled_rejection(orc, dev, bonus):
    from voidinfer_amd import workloads as W
    lanes, drafts = 8, 16
    p0 = W.config4(lanes=lanes, drafts=drafts, vocab=W.V_QWEN, bonus=bonus)[3]
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, bonus=bonus, sample_fn=sampler_from_draft(orc, p0))
    g, w = run(orc, dev, 1, tb, db, drafted, p, lanes, drafts)
    margins = w[4]
    exempt = {l for l in range(lanes) if np.min(margins[l]) < 1e-9}
    assert_same(g, w, exempt)
    assert len(exempt) <= 1


def test_sampled_many_lanes_small_vocab(orc, dev, rng):
    from voidinfer_amd import workloads as W
    lanes, drafts, vocab = 64, 6, 3000
    p0 = W.config4(lanes=lanes, drafts=drafts, vocab=vocab)[3]
    p0["top_k"] = rng.choice([1, 5, 20, 64], lanes)
    p0["top_p"] = rng.choice([0.5, 0.9, 1.0], lanes)
    p0["min_p"] = rng.choice([0.0, 0.1], lanes)
    p0["temperature"] = rng.choice([0.0, 0.5, 1.0], lanes)
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, vocab=vocab, sample_fn=sampler_from_draft(orc, p0))
    p[:] = p0
    drafted[::5, 2] = 0        # some zero-q proposals
    g, w = run(orc, dev, 1, tb, db, drafted, p, lanes, drafts)
    exempt = {l for l in range(lanes) if np.min(w[4][l]) < 1e-9}
    assert_same(g, w, exempt)


def test_sampled_nonfinite_and_overflowing_targets(orc, dev, rng):
    """Target rows holding +-Inf / NaN, and finite bf16 logits that overflow once
    divided by the temperature (the exact per-element path of the slice scan),
    beside clean rows (its all-finite fast path)."""
    from voidinfer_amd import workloads as W
    lanes, drafts, vocab = 16, 4, 5000
    p0 = W.config4(lanes=lanes, drafts=drafts, vocab=vocab)[3]
    p0["temperature"] = rng.choice([0.0, 0.25, 0.5, 1.0], lanes)
    p0["top_k"] = rng.choice([1, 8, 20], lanes)
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, vocab=vocab, sample_fn=sampler_from_draft(orc, p0))
    p[:] = p0
    big = int(np.float32(3.0e38).view(np.uint32) >> 16)
    for r in range(0, tb.shape[0], 3):
        cols = rng.integers(0, vocab, 3)
        tb[r, cols[0]] = big                                        # overflows at T < 1
        tb[r, cols[1]] = [0x7F80, 0xFF80, 0x7FC0][r % 3]           # +Inf, -Inf, NaN
        tb[r, cols[2]] = big | 0x8000                               # huge negative
    g, w = run(orc, dev, 1, tb, db, drafted, p, lanes, drafts)
    exempt = {l for l in range(lanes) if np.min(w[4][l]) < 1e-9}
    assert_same(g, w, exempt)
    assert any(f != 0 for f in w[3])


def test_sampled_full_vocabulary_lanes(orc, dev):
    """Lanes with temperature > 0 and top_k in {0, 65, 200} take p and q from the
    full-vocabulary sampler's distributions; every lane matches the oracle
    (accepted lengths, committed ids, flags) outside decisions that lie within
    1e-6 of turning (1e-9 on the list lanes, whose fp64 sums are the oracle's)."""
    from voidinfer_amd import workloads as W
    lanes, drafts = 8, 16
    p0 = W.config4(lanes=lanes, drafts=drafts)[3]
    full = {1: 0, 4: 65, 6: 200}
    for l, k in full.items():
        p0["top_k"][l] = k
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, sample_fn=sampler_from_draft(orc, p0))
    p[:] = p0
    g, w = run(orc, dev, 1, tb, db, drafted, p, lanes, drafts)
    exempt = {l for l in range(lanes) if np.min(w[4][l]) < (1e-6 if l in full else 1e-9)}
    assert len(assert_same(g, w, exempt)) <= 1
    assert not any(g[3][l] & 0x80000000 for l in range(lanes))


@pytest.mark.parametrize("bonus", [False, True])
def test_sampled_config4_top_k_disabled(orc, dev, bonus):
    """Config 4 with top_k 0 and top_p 0.8 (T 0.7) on every lane: the whole
    verification runs on the full-vocabulary path, drafts sampled from the
    draft's full filtered distribution."""
    from voidinfer_amd import workloads as W
    lanes, drafts = 8, 16
    p0 = W.config4(lanes=lanes, drafts=drafts, bonus=bonus)[3]
    p0["top_k"] = 0
    p0["top_p"] = 0.8
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, bonus=bonus, sample_fn=sampler_from_draft(orc, p0))
    p[:] = p0
    g, w = run(orc, dev, 1, tb, db, drafted, p, lanes, drafts)
    exempt = {l for l in range(lanes) if np.min(w[4][l]) < 1e-6}
    assert len(assert_same(g, w, exempt)) <= 1
    assert w[0].sum() > 0 and (w[0] < drafts).any()   # both accepts and rejections were exercised


def test_sampled_full_vocabulary_mixed_dtypes_and_edges(orc, dev, rng):
    """fp32 targets with bf16 drafts (and the reverse) on small vocabularies, min-p
    and top-p cuts, zero-q proposals, temperature 0 lanes beside full lanes, a
    bonus row."""
    import voidinfer_amd as vi
    lanes, drafts, vocab = 12, 5, 40_000
    for tdt, ddt in ((2, 0), (0, 2), (1, 1)):
        x = rng.standard_normal((lanes * (drafts + 1), vocab)).astype(np.float32) * 2.0
        y = x[np.arange(lanes * (drafts + 1)).reshape(lanes, drafts + 1)[:, :drafts].reshape(-1)]
        y = y + rng.standard_normal(y.shape).astype(np.float32) * 0.5
        enc = {0: W_bf16, 1: W_f16, 2: lambda a: a}
        tb, db = enc[tdt](x), enc[ddt](y)
        p = vi.params_array(lanes, seed=rng.integers(1, 2**62, lanes), position=rng.integers(0, 10**5, lanes),
                            lane=np.arange(lanes), temperature=rng.choice([0.0, 0.7, 1.0], lanes),
                            top_k=rng.choice([0, 0, 100, 20], lanes), top_p=rng.choice([0.5, 0.9, 1.0], lanes),
                            min_p=rng.choice([0.0, 0.05], lanes))
        drafted = np.zeros((lanes, drafts), dtype=np.int32)
        for l in range(lanes):
            for j in range(drafts):
                prob, _ = orc.row_distribution(db[l * drafts + j], ddt, p[l])
                drafted[l, j] = rng.choice(vocab, p=prob / prob.sum()) if j != 2 or l % 4 else 7
        t = to_dev(tb, tdt, dev)
        d = to_dev(db, ddt, dev)
        dr = torch.from_numpy(drafted).to(dev)
        g = vi.verify_rows(1, t, dr, lanes, drafts, draft=d, params=p)
        w = orc.verify_rows(1, tb, tdt, db, ddt, lanes, drafts, drafted, p)
        exempt = {l for l in range(lanes) if np.min(w[4][l]) < 1e-6}
        assert len(assert_same(g, w, exempt)) <= 1, (tdt, ddt, exempt)


def W_bf16(a):
    from voidinfer_amd import workloads as W
    return W.encode(a, "bf16")


def W_f16(a):
    from voidinfer_amd import workloads as W
    return W.encode(a, "f16")


def test_sampled_topk_mode_refuses_full_vocabulary_lanes(orc, dev):
    """VI_VERIFY_SAMPLED_TOPK (the caller vouches for top-k lists on every
    sampled lane): lanes with top_k in {0, 65, 200} are refused with
    VI_FLAG_ERROR, accept and commit nothing, and leave the other config-4 lanes
    bit-exact with the oracle."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    from voidinfer_amd._abi import FLAG_ERROR, VERIFY_SAMPLED_TOPK
    lanes, drafts = 8, 16
    p0 = W.config4(lanes=lanes, drafts=drafts)[3]
    tb, db, drafted, p = W.config4(lanes=lanes, drafts=drafts, sample_fn=sampler_from_draft(orc, p0))
    refused = {1: 0, 4: 65, 6: 200}
    for l, k in refused.items():
        p["top_k"][l] = k
    t, d = to_dev(tb, 0, dev), to_dev(db, 1, dev)
    dr = torch.from_numpy(np.ascontiguousarray(drafted, dtype=np.int32)).to(dev)
    g = vi.verify_rows(VERIFY_SAMPLED_TOPK, t, dr, lanes, drafts, draft=d, params=p)
    w = orc.verify_rows(1, tb, 0, db, 1, lanes, drafts, drafted, p)
    ga, gc, gn, gf = g
    for l in refused:
        assert gf[l] == FLAG_ERROR and ga[l] == 0 and gn[l] == 0 and np.all(gc[l] == -1), (l, ga[l], gn[l], gf[l])
    keep = [l for l in range(lanes) if l not in refused]
    exempt = {l for l in keep if np.min(w[4][l]) < 1e-9} | set(refused)
    assert_same(g, w, exempt)
    assert len(exempt) <= len(refused) + 1

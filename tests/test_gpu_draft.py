"""GPU DFlash2 draft coupled proposals (vi_draft_choice) and the fused selector
chain (vi_selector_chain) vs the CPU oracle (dflash_sampled_choice,
dflash2_draft.cu:2554-2610; dflash_selector_fused_chain_kernel, :2615-2678).

Proposals equal position by position; a lane may differ only where the
oracle's decision sat within float rounding of a boundary (the two best
perturbed values within 1e-5, or a top-p / min-p cut within 1e-5 relative),
and is not compared past such a position (later positions depend on it
through the presence penalty).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def near_boundary(orc, scores, cands, s, key):
    x = scores.astype(np.float64)
    inv = float(s["inv_temperature"])
    order = np.argsort(-x, kind="stable")
    cap = int(s["top_k"]) if 0 < int(s["top_k"]) < 16 else 16
    w = np.exp((x[order[:cap]] - x[order[0]]) * inv)
    near = False
    if float(s["top_p"]) < 1:
        near |= bool(np.any(np.abs(np.cumsum(w) - float(s["top_p"]) * w.sum()) <= 1e-5 * w.sum()))
    if float(s["min_p"]) > 0:
        near |= bool(np.any(np.abs(w - float(s["min_p"])) <= 1e-5))
    g = np.array([orc.gumbel(int(s["seed"]), key, int(c)) for c in cands[order[:cap]]])
    v = np.sort(x[order[:cap]] * inv + g)[::-1]
    near |= bool(len(v) > 1 and abs(v[0] - v[1]) <= 1e-5 * (1 + abs(v[0])))
    return near


@pytest.mark.parametrize("case", range(4))
def test_draft_choice_vs_oracle(orc, dev, case):
    import voidinfer_amd as vi
    rng = np.random.default_rng(500 + case)
    lanes, pos, vocab = 96, 8, 50_000
    scores = (rng.standard_normal((lanes, pos, 16)) * 1.5).astype(np.float32)
    cands = np.stack([np.stack([rng.choice(vocab, 16, replace=False) for _ in range(pos)]) for _ in range(lanes)])
    cands[:, 1:, 0] = cands[:, :1, 0]                      # a repeated top candidate exercises the chain penalty
    scores[:, :, 0] += 2.0
    smp = np.zeros(lanes, dtype=vi.DRAFT_SAMPLING)
    smp["inv_temperature"] = [0.0, 1.4, 0.9, 2.5][case] if case else 0.0
    smp["top_k"] = rng.choice([0, 4, 12], lanes)
    smp["top_p"] = rng.choice([1.0, 0.9, 0.7], lanes)
    smp["min_p"] = rng.choice([0.0, 0.05], lanes)
    smp["seed"] = rng.integers(1, 2**62, lanes)
    smp["key_base"] = rng.integers(0, 100_000, lanes)
    smp["presence_penalty"] = [0.0, 0.0, 1.5, -0.5][case]
    fo = np.full(vocab, 0x7F7F7F7F, dtype=np.int32)
    fo[cands[:, 0, 1]] = 3
    seeds = cands[:, 0, 2].copy()
    fo_dev = torch.from_numpy(fo).to(dev)
    smp_dev = smp.copy()
    smp_host = smp.copy()
    if case >= 2:
        smp_dev["first_occurrence"] = fo_dev.data_ptr()
        smp_host["first_occurrence"] = fo.ctypes.data
    got = vi.draft_choice(torch.from_numpy(scores).to(dev), torch.from_numpy(cands).to(dev), smp_dev,
                          torch.from_numpy(seeds).to(dev), vocabulary=vocab)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    want = orc.draft_choice(scores, cands, smp_host, seed_tokens=seeds, vocabulary=vocab)
    for l in range(lanes):
        for p in range(pos):
            if got[l, p] != want[l, p]:
                assert near_boundary(orc, scores[l, p], cands[l, p], smp[l], int(smp["key_base"][l]) + p), (l, p)
                break


def test_draft_choice_rejects_invalid(dev):
    import ctypes as C
    from voidinfer_amd import _abi
    lib = _abi.load()
    assert lib.vi_draft_choice(0, 4, 100, None, None, None, None, None, None) == 0      # nothing to do
    assert lib.vi_draft_choice(2, 4, 100, None, None, None, None, None, None) == 1      # null arrays
    assert lib.vi_draft_choice(-1, 4, 100, None, None, None, None, None, None) == 1


def _chain_case(rng, lanes, positions, vocab):
    anchors = rng.integers(0, vocab, lanes).astype(np.int64)
    cands = np.stack([np.stack([rng.choice(vocab, 16, replace=False) for _ in range(positions)])
                      for _ in range(lanes)]).astype(np.int64)
    unary = (rng.standard_normal((lanes, positions, 16)) * 2).astype(np.float32)
    f16 = lambda shape: rng.standard_normal(shape).astype(np.float16)   # noqa: E731
    return anchors, cands, unary, f16((lanes, positions, 256)), f16((vocab, 256)), f16((vocab, 256))


def _run_chain(dev, anchors, cands, unary, hidden, pred, succ, smp=None):
    import voidinfer_amd as vi
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)   # noqa: E731
    got = vi.selector_chain(t(anchors), t(cands), t(unary), t(hidden), t(pred), t(succ), smp)
    torch.cuda.synchronize()
    return got.cpu().numpy()


def check_chain_fp64(got, anchors, cands, unary, hidden, pred, succ):
    """Greedy chains against a float64 replay: at each position, with the chain's
    own previous proposal as anchor, the proposal's score (products rounded in
    fp32 as (pred * hidden) * succ, summed exactly) is within the fp32 sums'
    rounding bound of the best score; a choice that differs from the float64
    first maximum is allowed only there (a near tie)."""
    bound_units = 10 * 2.0 ** -24          # 2 in-lane + 6 cross-lane additions, the unary add, slack
    near = 0
    for l in range(got.shape[0]):
        anchor = int(anchors[l])
        for p in range(got.shape[1]):
            if got[l, p] == -1:
                assert (got[l, p:] == -1).all()
                break
            ah = pred[anchor].astype(np.float32) * hidden[l, p].astype(np.float32)
            prods = ah[None, :] * succ[cands[l, p]].astype(np.float32)          # fp32 products
            exact = prods.astype(np.float64).sum(axis=1) + unary[l, p].astype(np.float64)
            bound = bound_units * (np.abs(prods).astype(np.float64).sum(axis=1) + np.abs(unary[l, p]))
            best = int(np.argmax(exact))
            chosen = int(np.flatnonzero(cands[l, p] == got[l, p])[0])
            if chosen != best:
                assert exact[chosen] >= exact[best] - (bound[chosen] + bound[best]), (l, p, exact[best] - exact[chosen])
                near += 1
            anchor = int(got[l, p])
    return near


def test_selector_chain_vs_oracle(orc, dev):
    """Greedy lanes against the float64 replay (this kernel sums in its own
    order: near ties may turn within the fp32 rounding bound); sampled lanes
    equal to the oracle up to a position within rounding of a boundary; invalid
    ids end a lane's chain."""
    import voidinfer_amd as vi
    rng = np.random.default_rng(77)
    lanes, positions, vocab = 24, 16, 30_000
    anchors, cands, unary, hidden, pred, succ = _chain_case(rng, lanes, positions, vocab)
    anchors[5] = -1
    cands[3, 9, 4] = vocab
    cands[:, 1:, 2] = anchors[:, None]          # the seed token keeps coming back (presence penalty)
    smp = np.zeros(lanes, dtype=vi.DRAFT_SAMPLING)
    sampled = np.arange(lanes) % 3 == 0
    smp["inv_temperature"] = np.where(sampled, 1 / 0.8, 0.0)
    smp["top_k"], smp["top_p"], smp["min_p"] = 10, 0.9, 0.0
    smp["seed"] = rng.integers(1, 2**62, lanes)
    smp["key_base"] = rng.integers(0, 100_000, lanes)
    smp["presence_penalty"] = 0.5
    hb, pb, sb = hidden.view(np.uint16), pred.view(np.uint16), succ.view(np.uint16)
    got = _run_chain(dev, anchors, cands, unary, hidden, pred, succ, smp)
    want = orc.selector_chain(anchors, cands, unary, hb, pb, sb, smp)
    assert (want[5] == -1).all() and (want[3, 9:] == -1).all()
    assert (got[5] == -1).all() and (got[3, 9:] == -1).all() and (got[3, :9] != -1).all()
    greedy = [l for l in range(lanes) if not sampled[l]]
    assert check_chain_fp64(got[greedy], anchors[greedy], cands[greedy], unary[greedy], hidden[greedy], pred,
                            succ) <= 2
    for l in range(lanes):
        if not sampled[l]:
            continue
        for p in range(positions):
            if got[l, p] != want[l, p]:
                assert near_boundary(orc, unary[l, p], cands[l, p], smp[l], int(smp["key_base"][l]) + p), (l, p)
                break


def test_selector_chain_full_vocabulary_greedy(orc, dev):
    rng = np.random.default_rng(78)
    anchors, cands, unary, hidden, pred, succ = _chain_case(rng, 4, 16, 248_320)
    got = _run_chain(dev, anchors, cands, unary, hidden, pred, succ)
    assert check_chain_fp64(got, anchors, cands, unary, hidden, pred, succ) <= 1
    assert (got >= 0).all()


def test_selector_chain_near_ties(orc, dev):
    """Candidates whose float64 scores differ by less than the fp32 sums' rounding
    (duplicated succ rows with the unary split by one ulp) and exact ties (the
    first candidate wins)."""
    rng = np.random.default_rng(79)
    lanes, positions, vocab = 8, 6, 4096
    anchors, cands, unary, hidden, pred, succ = _chain_case(rng, lanes, positions, vocab)
    reserved = vocab - 2 * lanes * positions                 # ids no other candidate or anchor uses
    anchors %= reserved
    cands %= reserved
    for l in range(lanes):
        for p in range(positions):
            i = l * positions + p
            cands[l, p, 3], cands[l, p, 7] = reserved + 2 * i, reserved + 2 * i + 1
            succ[cands[l, p, 7]] = succ[cands[l, p, 3]]          # same rank-256 term
            unary[l, p, 7] = unary[l, p, 3]                      # exact tie: candidate 3 first
    got = _run_chain(dev, anchors, cands, unary, hidden, pred, succ)
    check_chain_fp64(got, anchors, cands, unary, hidden, pred, succ)
    assert not (got == cands[:, :, 7]).any()

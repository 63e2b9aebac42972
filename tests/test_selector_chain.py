"""DFlash2 fused selector chain (dflash_selector_fused_chain_kernel,
src/exl3/dflash2_draft.cu:2615-2678): the oracle restatement pinned on the CPU.

* closed form: one-hot predecessor rows and a constant hidden state make every
  selector value one exact fp16 entry of the successor codebook, so the whole
  greedy chain (each pick becomes the next anchor) is known exactly;
* float64: random codebooks, the chain recomputed in float64 agrees up to the
  first position whose two best scores lie within 1e-3 (the fp32 reduction is
  the reference's order, which float64 cannot see below that);
* sampled lanes propose what the coupled draft choice proposes over the unary
  scores with the initial anchor as seed token (that oracle is pinned in
  test_oracle_pins.py);
* an anchor or a candidate outside the codebooks ends the lane's chain with -1.
"""
import numpy as np

import oracle

R, K = 256, 16


def fp16_bits(x):
    return np.asarray(x, dtype=np.float16).view(np.uint16)


def case(rng, lanes, positions, vocab, scale=1.0):
    anchors = rng.integers(0, vocab, lanes).astype(np.int64)
    cands = np.stack([np.stack([rng.choice(vocab, K, replace=False) for _ in range(positions)]) for _ in range(lanes)])
    unary = (rng.standard_normal((lanes, positions, K)) * 2).astype(np.float32)
    hidden = fp16_bits(rng.standard_normal((lanes, positions, R)) * scale)
    pred = fp16_bits(rng.standard_normal((vocab, R)) * scale)
    succ = fp16_bits(rng.standard_normal((vocab, R)) * scale)
    return anchors, cands.astype(np.int64), unary, hidden, pred, succ


def test_closed_form_one_hot_chain():
    rng = np.random.default_rng(1)
    lanes, positions, vocab = 4, 12, 600
    anchors, cands, unary, _, _, _ = case(rng, lanes, positions, vocab)
    pred = np.zeros((vocab, R), dtype=np.float16)
    pred[np.arange(vocab), np.arange(vocab) % R] = 1.0          # anchor v selects rank v mod 256
    hidden = np.ones((lanes, positions, R), dtype=np.float16)
    succ = (rng.integers(-64, 64, (vocab, R)) * 0.25).astype(np.float16)
    unary = (rng.integers(-8, 8, (lanes, positions, K)) * 0.125).astype(np.float32)
    want = np.zeros((lanes, positions), dtype=np.int64)
    for l in range(lanes):
        a = anchors[l]
        for p in range(positions):
            score = unary[l, p] + succ[cands[l, p], a % R].astype(np.float32)   # exact in fp32
            a = cands[l, p, int(np.argmax(score))]                            # first maximum
            want[l, p] = a
    got = oracle.selector_chain(anchors, cands, unary, hidden.view(np.uint16), pred.view(np.uint16),
                                succ.view(np.uint16))
    assert np.array_equal(got, want)


def test_float64_chain_until_near_tie():
    rng = np.random.default_rng(2)
    lanes, positions, vocab = 6, 16, 2000
    anchors, cands, unary, hidden, pred, succ = case(rng, lanes, positions, vocab)
    got = oracle.selector_chain(anchors, cands, unary, hidden, pred, succ)
    P, S = pred.view(np.float16).astype(np.float64), succ.view(np.float16).astype(np.float64)
    H = hidden.view(np.float16).astype(np.float64)
    checked = 0
    for l in range(lanes):
        a = anchors[l]
        for p in range(positions):
            score = unary[l, p].astype(np.float64) + (P[a] * H[l, p] * S[cands[l, p]]).sum(axis=1)
            top2 = np.sort(score)[-2:]
            if top2[1] - top2[0] < 1e-3:
                break
            a = cands[l, p, int(np.argmax(score))]
            assert got[l, p] == a, (l, p)
            checked += 1
    assert checked > lanes * positions // 2


def test_sampled_lanes_are_the_coupled_choice_over_unary():
    rng = np.random.default_rng(3)
    lanes, positions, vocab = 8, 10, 1500
    anchors, cands, unary, hidden, pred, succ = case(rng, lanes, positions, vocab)
    cands[:, :, 5] = anchors[:, None]                     # the seed token among the candidates (presence)
    smp = np.zeros(lanes, dtype=oracle.DRAFT_SAMPLING)
    smp["inv_temperature"] = np.where(np.arange(lanes) % 2 == 0, 1 / 0.7, 0.0)   # odd lanes greedy
    smp["top_k"], smp["top_p"], smp["min_p"] = 8, 0.9, 0.02
    smp["seed"] = rng.integers(1, 2**62, lanes)
    smp["key_base"] = rng.integers(0, 10000, lanes)
    smp["presence_penalty"] = 0.8
    got = oracle.selector_chain(anchors, cands, unary, hidden, pred, succ, smp)
    coupled = oracle.draft_choice(unary, cands, smp, seed_tokens=anchors, vocabulary=vocab)
    greedy = oracle.selector_chain(anchors, cands, unary, hidden, pred, succ)
    for l in range(lanes):
        assert np.array_equal(got[l], coupled[l] if l % 2 == 0 else greedy[l]), l


def test_invalid_ids_end_the_chain():
    rng = np.random.default_rng(4)
    lanes, positions, vocab = 3, 6, 500
    anchors, cands, unary, hidden, pred, succ = case(rng, lanes, positions, vocab)
    anchors[0] = vocab            # bad anchor: nothing proposed
    cands[1, 3, 7] = -2           # bad candidate at position 3
    got = oracle.selector_chain(anchors, cands, unary, hidden, pred, succ)
    ok = oracle.selector_chain(anchors[2:], cands[2:], unary[2:], hidden[2:], pred, succ)
    assert (got[0] == -1).all()
    assert (got[1, :3] >= 0).all() and (got[1, 3:] == -1).all()
    assert np.array_equal(got[2], ok[0])

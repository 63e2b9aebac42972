"""DFlash2 verification tree (exl3_build_verification_tree,
src/exl3/verification_tree.h:44-112) on the CPU: the oracle against the
reference's own header (oracle/_ref), the library's C ABI against the oracle,
and the search pinned by brute force over every admissible tree."""
import itertools

import numpy as np
import pytest

import oracle

CHAIN_HIT = np.array([0.32, 0.38, 0.35, 0.44, 0.42, 0.49, 0.57, 0.67, 0.78, 0.97], dtype=np.float32)
SIB_HIT = np.array([[0.04, 0.13, 0.18, 0.23, 0.26, 0.27, 0.13, 0.09, 0.06, 0.07],
                    [0.03, 0.10, 0.15, 0.09, 0.12, 0.12, 0.12, 0.12, 0.12, 0.12],
                    [0.03, 0.10, 0.15, 0.15, 0.15, 0.15, 0.15, 0.15, 0.15, 0.15]], dtype=np.float32)


def random_case(rng, depth, ties=True):
    ids = rng.integers(1000, 1040, (depth, 16)).astype(np.int64)
    un = (rng.random((depth, 16)) * 6 * rng.integers(1, 5, (depth, 1))).astype(np.float32)
    if ties:
        mask = rng.random((depth, 16)) < 0.3
        un[mask] = rng.integers(0, 3, int(mask.sum())).astype(np.float32)
    drafts = np.array([ids[d, rng.integers(0, 16)] if rng.random() < 0.8 else 5 for d in range(depth)],
                      dtype=np.int64)
    return drafts, ids, un


def cases(seed, n):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        depth = int(rng.integers(0, 9))
        drafts, ids, un = random_case(rng, depth)
        budget, max_sib = int(rng.integers(0, 13)), int(rng.integers(-1, 6))
        cost = [0.0, oracle.ROW_COST, float(rng.random() * 0.2)][int(rng.integers(0, 3))]
        yield drafts, ids, un, budget, max_sib, cost


def test_oracle_matches_reference_build():
    """The oracle restatement against the reference's header itself, ties included."""
    if oracle.ref_build_verification_tree([], np.zeros((0, 16)), np.zeros((0, 16)), 1, 1) is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    for k, (d, ids, un, b, ms, c) in enumerate(cases(41, 3000)):
        assert oracle.build_verification_tree(d, ids, un, b, ms, c) == \
            oracle.ref_build_verification_tree(d, ids, un, b, ms, c), k


def test_library_matches_oracle():
    """vi_build_verification_tree (the C++20 host layer behind the C ABI)."""
    import voidinfer_amd as vi
    for k, (d, ids, un, b, ms, c) in enumerate(cases(43, 3000)):
        assert vi.verification_tree(d, ids, un, b, ms, c) == oracle.build_verification_tree(d, ids, un, b, ms, c), k


def _nodes(drafts, ids, un):
    """Per depth: the chain token's hit rate and the (rate, token) of up to three
    siblings, from the top-16 softmax (float32, stable unary order)."""
    hits, leaves = [], []
    for d in range(len(drafts)):
        u = un[d].astype(np.float32)
        p = np.exp(u - u.max()).astype(np.float32)
        s = np.float32(0)
        for x in p:
            s = np.float32(s + x)
        chain = [c for c in range(16) if ids[d, c] == drafts[d]]
        cp = np.float32(p[chain[-1]] / s) if chain else np.float32(0)
        hits.append(CHAIN_HIT[min(max(int(cp * np.float32(10)), 0), 9)])
        order = sorted(range(16), key=lambda c: -float(u[c]))
        sib = [c for c in order if ids[d, c] != drafts[d]][:3]
        leaves.append([(SIB_HIT[r][min(max(int(np.float32(p[c] / s) * np.float32(10)), 0), 9)], int(ids[d, c]))
                       for r, c in enumerate(sib)])
    return hits, leaves


def _rate(hits, leaves, chain, chosen, cost):
    """(1 + E[accepted]) / (1 + cost * rows) of a chain prefix plus chosen (depth, rank) leaves."""
    surv, value = [], 0.0
    s = 1.0
    for d in range(chain):
        surv.append(s)
        s *= float(hits[d])
        value += s
    value += sum(surv[d] * float(leaves[d][r][0]) for d, r in chosen)
    return (1.0 + value) / (1.0 + cost * (chain + len(chosen)))


@pytest.mark.parametrize("seed", range(6))
def test_search_is_optimal_by_brute_force(seed):
    """Every chain length and every sibling subset within the budget and the
    sibling cap: the chosen tree attains the best rate (float rounding aside)."""
    rng = np.random.default_rng(100 + seed)
    for _ in range(25):
        depth = int(rng.integers(1, 4))
        drafts, ids, un = random_case(rng, depth, ties=False)
        budget, max_sib = int(rng.integers(1, 6)), int(rng.integers(0, 4))
        cost = float(rng.choice([0.0, oracle.ROW_COST, 0.1]))
        hits, leaves = _nodes(drafts, ids, un)
        best = -1.0
        for chain in range(1, min(depth, budget) + 1):
            slots = [(d, r) for d in range(chain) for r in range(len(leaves[d]))]
            for k in range(0, min(max_sib, budget - chain) + 1):
                for chosen in itertools.combinations(slots, k):
                    best = max(best, _rate(hits, leaves, chain, chosen, cost))
        chain, toks, offs = oracle.build_verification_tree(drafts, ids, un, budget, max_sib, cost)
        assert 1 <= chain <= min(depth, budget) and len(toks) <= max_sib and chain + len(toks) <= budget
        chosen = []
        for t, o in zip(toks, offs):
            r = [x[1] for x in leaves[o - 1]].index(t)
            chosen.append((o - 1, r))
        assert _rate(hits, leaves, chain, chosen, cost) == pytest.approx(best, rel=1e-5)


def test_closed_forms():
    rng = np.random.default_rng(7)
    drafts, ids, un = random_case(rng, 4, ties=False)
    assert oracle.build_verification_tree(drafts, ids, un, 0, 3) == (0, [], [])        # no rows
    assert oracle.build_verification_tree(drafts, ids, un, 1, 3)[1:] == ([], [])       # one row: the chain
    c, t, o = oracle.build_verification_tree(drafts, ids, un, 12, 0)                   # no siblings allowed
    assert t == [] and o == [] and 1 <= c <= 4
    # a prohibitive row cost keeps the smallest tree, a free one the largest
    assert oracle.build_verification_tree(drafts, ids, un, 8, 3, 1e6) == (1, [], [])
    c, t, _ = oracle.build_verification_tree(drafts, ids, un, 7, 3, 0.0)
    assert c + len(t) == 7
    # one depth, chain token certain (p > 0.9): hit 0.97; siblings are the next
    # three candidates in unary order, at offset 1
    ids1 = np.arange(100, 116, dtype=np.int64)[None]
    un1 = np.full((1, 16), -30.0, dtype=np.float32)
    un1[0, 3], un1[0, 7], un1[0, 1], un1[0, 9] = 10.0, 2.0, 1.5, 1.0
    chain, toks, offs = oracle.build_verification_tree([103], ids1, un1, 4, 3, 0.0)
    assert (chain, toks, offs) == (1, [107, 101, 109], [1, 1, 1])
    # chain token absent from the candidates: decile 0 and every sibling is a candidate
    chain, toks, _ = oracle.build_verification_tree([5], ids1, un1, 4, 3, 0.0)
    assert toks == [103, 107, 101]

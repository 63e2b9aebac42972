"""Per-lane penalty state (vi_penalty_state_*, vi_sample_rows_state) on the GPU.

The state's contents are checked against numpy occurrence counts of the same
token multiset (presence bitmap = count >= 1, repeat bitmap = count >= 2, hash
lookups = counts, header keys / total), after records, duplicate records inside
one call, removals (roll-back) and re-records.  The sampler reading the state
is checked bit for bit against the sampler reading an equivalent history (same
tokens, uniforms, flags, support and probabilities) and against the CPU oracle,
on both kernel routes, over several decode steps that record each step's
sampled tokens in the state (by the update entry point, or by the sampler
itself in the same launch).
"""
import numpy as np
import pytest
import torch

from helpers import exempt_draw, to_dev

pytestmark = pytest.mark.gpu

FLAG_BAD_HISTORY, FLAG_ERROR = 16, 0x80000000   # VI_FLAG_BAD_HISTORY, VI_FLAG_ERROR


def layout(vocab, slots):
    """Offsets of one lane's state: 64-byte header, presence bitmap of ceil(V / 32)
    words (rounded up to 4 words), then at a 64-byte boundary the hash
    (8 bytes per slot), the slots' repeat-list indices (4 bytes) and the repeat
    list (8 bytes per entry)."""
    words = -(-(-(-vocab // 32)) // 4) * 4
    off_hash = -(-(64 + 4 * words) // 64) * 64
    return words, 64, off_hash, off_hash + 8 * slots, off_hash + 12 * slots


def decode_state(st, lane):
    """(presence bits, hash counts per token, repeat list [(token, count)], header) of one lane."""
    raw = st.buf.view(st.lanes, st.lane_bytes)[lane].cpu().numpy()
    words, o1, oh, orx, ol = layout(st.vocabulary, st.slots)
    b1 = np.unpackbits(raw[o1:o1 + 4 * words].view(np.uint32).view(np.uint8), bitorder="little")[:st.vocabulary]
    tab = raw[oh:oh + 8 * st.slots].view(np.uint32).reshape(st.slots, 2)
    counts = np.zeros(st.vocabulary, dtype=np.int64)
    used = tab[:, 0] != 0
    keys = tab[used, 0].astype(np.int64) - 1
    assert len(np.unique(keys)) == len(keys), "a token holds two slots"
    counts[keys] = tab[used, 1]
    hdr = raw[:24]
    flags, nkeys, total, nrep = (int(hdr[:4].view(np.uint32)[0]), int(hdr[4:8].view(np.uint32)[0]),
                                 int(hdr[8:16].view(np.uint64)[0]), int(hdr[16:20].view(np.uint32)[0]))
    lst = raw[ol:ol + 8 * st.slots].view(np.uint32).reshape(st.slots, 2)
    assert not lst[nrep:].any(), "entries past the repeat list's end"
    ridx = raw[orx:orx + 4 * st.slots].view(np.uint32)
    assert (ridx[~used] == 0).all() and np.array_equal(np.sort(ridx[ridx > 0]), np.arange(1, nrep + 1))
    assert (lst[ridx[ridx > 0] - 1, 0] == tab[ridx > 0, 0] - 1).all(), "slot and entry name another token"
    return b1, counts, lst[:nrep], (flags, nkeys, total)


def check_lane(st, lane, tokens_multiset, flags=0):
    want = np.bincount(np.asarray(tokens_multiset, dtype=np.int64), minlength=st.vocabulary)
    b1, counts, lst, (f, keys, total) = decode_state(st, lane)
    assert np.array_equal(counts, want), (lane, np.flatnonzero(counts != want)[:8])
    assert np.array_equal(b1, (want >= 1).astype(np.uint8)), lane
    # one entry per token that reached 2, holding its current count; every token at >= 2 listed
    assert len(np.unique(lst[:, 0])) == len(lst), lane
    assert np.array_equal(lst[:, 1].astype(np.int64), want[lst[:, 0]]), lane
    assert set(np.flatnonzero(want >= 2)) <= set(lst[:, 0].tolist()), lane
    assert total == int(want.sum()) and f == flags, (lane, total, f)
    return keys


def csr(lists):
    offs = np.concatenate([[0], np.cumsum([len(x) for x in lists])]).astype(np.int64)
    toks = np.concatenate([np.asarray(x, dtype=np.int32) for x in lists]) if offs[-1] else np.zeros(1, np.int32)
    return toks, offs


def update(st, dev, lists, sign=1):
    toks, offs = csr(lists)
    st.update(torch.from_numpy(toks).to(dev), torch.from_numpy(offs).to(dev), sign)


def test_state_contents_record_remove(dev, rng):
    import voidinfer_amd as vi
    lanes, vocab, slots = 6, 248_320, 1 << 15
    st = vi.PenaltyState(lanes, vocab, slots, device=dev)
    hist = []
    for l in range(lanes):
        h = rng.integers(0, vocab, 5000 + 700 * l)
        h[:400] = rng.integers(0, 30, 400)          # heavy repeats (recorded concurrently in one call)
        h[400:450] = vocab - 1                     # the last id
        hist.append(h)
    update(st, dev, hist)
    for l in range(lanes):
        keys = check_lane(st, l, hist[l])
        assert keys == len(np.unique(hist[l]))
    # roll back a suffix of every lane (drafted tokens rejected), then record new ones
    cut = [len(h) - int(rng.integers(0, 1500)) for h in hist]
    update(st, dev, [h[c:] for h, c in zip(hist, cut)], sign=-1)
    for l in range(lanes):
        check_lane(st, l, hist[l][:cut[l]])
    extra = [rng.integers(0, vocab, int(rng.integers(0, 50))) for _ in range(lanes)]
    update(st, dev, extra)
    for l in range(lanes):
        check_lane(st, l, np.concatenate([hist[l][:cut[l]], extra[l]]))
    # one token per lane (the sampler's output), a failed row (-1) records nothing
    one = np.array([5, -1, 7, 7, vocab - 1, 0], dtype=np.int32)
    st.update(torch.from_numpy(one).to(dev))
    for l in range(lanes):
        base = np.concatenate([hist[l][:cut[l]], extra[l]])
        check_lane(st, l, np.concatenate([base, [one[l]]]) if one[l] >= 0 else base)
    st.reset()
    for l in range(lanes):
        assert check_lane(st, l, []) == 0


def test_state_error_flags(dev, rng):
    import voidinfer_amd as vi
    vocab = 5000
    st = vi.PenaltyState(3, vocab, 64, device=dev)
    update(st, dev, [[1, 2, -4, vocab + 3], list(range(100)), [9]])     # bad ids; 100 distinct in 64 slots
    update(st, dev, [[], [], [9, 10]], sign=-1)                         # 10 was never recorded
    h = st.header()
    assert h[0, 0] == FLAG_BAD_HISTORY and h[0, 2] == 2
    assert h[1, 0] & FLAG_ERROR and h[1, 1] == 64
    assert h[2, 0] == FLAG_ERROR and h[2, 2] == 0
    # every row sampled from an ERROR lane fails; a BAD_HISTORY lane reports it
    bits = np.stack([np.asarray(rng.standard_normal(vocab) * 2, np.float32).view(np.uint32) >> 16] * 3).astype(np.uint16)
    p = vi.params_array(3, seed=[1, 2, 3], temperature=1.0, top_k=np.array([0, 20, 0]), presence_penalty=0.5)
    out = vi.sample_rows_state(to_dev(bits, 0, dev), p, st)
    s = vi.stats_numpy(out.stats)
    tok = out.tokens.cpu().numpy()
    assert tok[0] >= 0 and s["flags"][0] & FLAG_BAD_HISTORY
    assert tok[1] == -1 and tok[2] == -1 and s["flags"][1] & FLAG_ERROR and s["flags"][2] & FLAG_ERROR


def same_outputs(a, b, label):
    import voidinfer_amd as vi
    assert torch.equal(a.tokens, b.tokens), label
    assert torch.equal(a.uniforms, b.uniforms), label
    sa, sb = vi.stats_numpy(a.stats), vi.stats_numpy(b.stats)
    assert sa.tobytes() == sb.tobytes(), label
    if a.probs is not None:
        assert torch.equal(a.probs, b.probs), label


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_state_route_equals_history_route_over_steps(orc, dev, rng, dtype):
    """Both routes (top_k 0 / 20 / 50 / 100), five decode steps: sample from the
    state and from the equivalent history, then record the sampled tokens."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    rows, vocab, L = 12, 248_320, 6000
    x = W.gaussian_zipf(rows, vocab, 1.0, int(rng.integers(1 << 30)))
    bits = W.encode(x, {0: "bf16", 1: "f16", 2: "f32"}[dtype])
    p = vi.params_array(rows, seed=rng.integers(1, 2**62, rows), position=rng.integers(0, 10**5, rows),
                        temperature=rng.uniform(0.5, 1.2, rows), top_k=np.array([0, 20, 0, 50, 100, 0] * 2),
                        top_p=rng.choice([0.9, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.02], rows),
                        repetition_penalty=rng.uniform(1.0, 1.3, rows), presence_penalty=rng.uniform(0, 0.5, rows),
                        frequency_penalty=rng.uniform(0.0, 0.3, rows))
    hist = []
    for r in range(rows):
        top = np.argsort(-x[r])[:300]                # penalties that reorder the top candidates
        h = np.concatenate([rng.integers(0, vocab, L), rng.choice(top, 800), np.repeat(top[:5], 40)])
        hist.append(rng.permutation(h).astype(np.int32))
    st = vi.PenaltyState(rows, vocab, 1 << 14, device=dev)
    update(st, dev, hist)
    logits = to_dev(bits, dtype, dev)
    for step in range(6):
        toks, offs = csr(hist)
        a = vi.sample_rows(logits, p, torch.from_numpy(toks).to(dev), torch.from_numpy(offs).to(dev),
                           max_history=int(np.diff(offs).max()), want_probs=True)
        fused = step % 2 == 1                         # odd steps: the sampler records its own tokens
        b = vi.sample_rows_state(logits, p, st, record=fused, want_probs=True)
        torch.cuda.synchronize()
        same_outputs(a, b, f"step {step}")
        if step == 0:   # and the oracle, once
            w_tok, w_u, _, w_stats, margins = orc.sample_rows(bits, dtype, p, toks, offs, want_probs=False)
            g_tok = b.tokens.cpu().numpy()
            for r in range(rows):
                assert g_tok[r] == w_tok[r] or exempt_draw(margins[r]), (r, g_tok[r], w_tok[r])
        new = b.tokens.cpu().numpy()
        if not fused:
            st.update(b.tokens)                       # one token per lane, straight from the sampler
        hist = [np.append(h, t).astype(np.int32) for h, t in zip(hist, new)]
        p["position"] += 1
    for r in range(rows):                             # the state holds exactly the grown histories
        check_lane(st, r, hist[r])


def test_state_route_config5_subset(orc, dev):
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    bits, hist, offs, p = W.config5(rows=16)
    st = vi.PenaltyState(16, W.V_QWEN, 1 << 16, device=dev)
    st.update(torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev))
    logits = to_dev(bits, 0, dev)
    a = vi.sample_rows(logits, p, torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev),
                       max_history=32768, want_probs=True)
    b = vi.sample_rows_state(logits, p, st, want_probs=True)
    torch.cuda.synchronize()
    same_outputs(a, b, "config5")


def test_state_route_without_distinct_token_limits(orc, dev, rng):
    """Lanes holding 40,000 distinct recorded tokens in the low vocabulary, or one
    token recorded 70,000 times (a count past the LDS repeat hash's 16 bits, so
    the slice counts in its dense table instead): every route samples them, the
    state route equals the history route bit for bit, and both match the oracle."""
    import voidinfer_amd as vi
    vocab = 248_320
    st = vi.PenaltyState(4, vocab, 1 << 18, device=dev)
    hist = [np.arange(40_000), np.full(70_000, 1234), np.arange(40_000), np.full(70_000, 1234)]
    update(st, dev, hist)
    bits = np.stack([np.asarray(rng.standard_normal(vocab), np.float32).view(np.uint32) >> 16] * 4).astype(np.uint16)
    bits[1, 1234] = 0x4200                                    # 32.0: the heavy token would win unpenalized
    p = vi.params_array(4, seed=[1, 2, 3, 4], position=[7, 8, 9, 10], temperature=1.0,
                        top_k=np.array([0, 0, 20, 20]), top_p=0.9, repetition_penalty=1.1,
                        frequency_penalty=0.001, presence_penalty=0.1)
    logits = to_dev(bits, 0, dev)
    toks, offs = csr(hist)
    a = vi.sample_rows(logits, p, torch.from_numpy(toks).to(dev), torch.from_numpy(offs).to(dev),
                       max_history=70_000, want_probs=True)
    b = vi.sample_rows_state(logits, p, st, want_probs=True)
    torch.cuda.synchronize()
    same_outputs(a, b, "limits")
    w_tok, w_u, w_probs, w_stats, margins = orc.sample_rows(bits, 0, p, toks, offs, want_probs=True)
    s = vi.stats_numpy(b.stats)
    assert not (s["flags"] & FLAG_ERROR).any()
    for r in range(4):
        if not exempt_draw(margins[r]):
            assert b.tokens[r].item() == w_tok[r] and s["support"][r] == w_stats["support"][r], r
            np.testing.assert_allclose(s["support_mass"][r], w_stats["support_mass"][r], rtol=1e-6)


@pytest.mark.parametrize("vocab", [64, 1000, 65_537])
def test_state_route_small_and_odd_vocabularies(orc, dev, rng, vocab):
    """Half boundaries that do not fall on a bitmap word, the last word masked,
    both routes, recording from the sampler: equal to the history route (whose
    histories of up to 3 V tokens take its general path at V = 65,537)."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    rows = 8
    bits = W.encode(W.gaussian_zipf(rows, vocab, 1.0, int(rng.integers(1 << 30))), "bf16")
    p = vi.params_array(rows, seed=rng.integers(1, 2**62, rows), position=rng.integers(0, 10**5, rows),
                        temperature=0.9, top_k=np.array([0, 20, 0, 0, 64, 0, 0, 10]), top_p=0.95,
                        repetition_penalty=1.2, presence_penalty=0.3, frequency_penalty=0.2)
    hist = [rng.integers(0, vocab, int(rng.integers(1, 3 * vocab))).astype(np.int32) for _ in range(rows)]
    hist[0] = np.full(50, vocab - 1, dtype=np.int32)          # only the last id, repeated
    st = vi.PenaltyState(rows, vocab, 1 << 18, device=dev)   # >= 2 x the distinct tokens (up to V)
    update(st, dev, hist)
    assert (st.header()[:, 0] == 0).all()
    logits = to_dev(bits, 0, dev)
    for step in range(3):
        toks, offs = csr(hist)
        a = vi.sample_rows(logits, p, torch.from_numpy(toks).to(dev), torch.from_numpy(offs).to(dev),
                           max_history=int(np.diff(offs).max()), want_probs=True)
        b = vi.sample_rows_state(logits, p, st, record=True, want_probs=True)
        torch.cuda.synchronize()
        same_outputs(a, b, f"V={vocab} step {step}")
        hist = [np.append(h, t).astype(np.int32) for h, t in zip(hist, b.tokens.cpu().numpy())]
        p["position"] += 1
    for r in range(rows):
        check_lane(st, r, hist[r])

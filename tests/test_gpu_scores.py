"""GPU VeriCache row scores vs the CPU oracle.

vi_row_scores (exact_row_score_kernel, text_model.cu:11393-11420): greedy ids
and gaps bit-exact, including rows with +Inf (which can win), NaN and -Inf
(which cannot), and next tokens that are -1, the argmax, or past the row.

vi_sampled_scores (exl3_sampled_score_kernel, sampled_select.cuh:300-360):
chosen ids equal and gaps within 1e-4 + 1e-5 relative, unless the oracle's
decision sits within float rounding of a boundary (two perturbed values within
1e-5, or a top-p / min-p cut within 1e-5 relative, of the row's support or of
the support re-ranked with next raised by the tolerance); infinite gaps agree
outside such rows.
"""
import numpy as np
import pytest
import torch

from helpers import to_dev

pytestmark = pytest.mark.gpu


def make_bits(rng, rows, vocab, dtype, scale=1.5):
    x = (rng.standard_normal((rows, vocab)) * scale).astype(np.float32)
    if dtype == 2:
        return x
    if dtype == 1:
        return x.astype(np.float16).view(np.uint16)
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def decode(bits, dtype):
    if dtype == 2:
        return bits.astype(np.float32)
    if dtype == 1:
        return bits.view(np.float16).astype(np.float32)
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("dtype", [0, 1, 2])
@pytest.mark.parametrize("rows,vocab", [(1, 1000), (32, 248320), (128, 4099)])
def test_row_scores_bit_exact(orc, dev, dtype, rows, vocab):
    import voidinfer_amd as vi
    rng = np.random.default_rng(rows * 7 + dtype)
    bits = make_bits(rng, rows, vocab, dtype)
    inf_, ninf, nan = {2: (np.float32(np.inf), np.float32(-np.inf), np.float32(np.nan)),
                       1: (0x7C00, 0xFC00, 0x7E00), 0: (0x7F80, 0xFF80, 0x7FC0)}[dtype]
    if rows >= 8:
        bits[1, [vocab // 3, vocab - 1]] = inf_
        bits[2, ::5] = nan
        bits[3, :] = ninf
        bits[4, :] = nan
        bits[5, 17] = bits[5, vocab - 2] = bits[5].max() if dtype == 2 else bits[5, 17]
    nxt = rng.integers(-1, vocab + 2, rows).astype(np.int64)
    want_g, want_gap = orc.row_scores(bits, dtype, nxt)
    nxt[::4] = want_g[::4]                          # next == argmax: gap 0
    want_g, want_gap = orc.row_scores(bits, dtype, nxt)
    g, gap = vi.row_scores(to_dev(bits, dtype, dev), torch.from_numpy(nxt))
    torch.cuda.synchronize()
    assert np.array_equal(g.cpu().numpy(), want_g)
    got = gap.cpu().numpy()
    both_nan = np.isnan(got) & np.isnan(want_gap)
    assert np.array_equal(got[~both_nan].view(np.uint32), want_gap[~both_nan].view(np.uint32))


def _near(detail, cfg):
    d = detail
    vals = np.sort(d["value"][: d["support"]])[::-1]
    near = len(vals) > 1 and abs(vals[0] - vals[1]) <= 1e-5 * (1 + abs(vals[0]))
    prob = d["prob"][: d["cap"]].astype(np.float64)
    cum = np.cumsum(prob)
    if cfg["top_p"] < 1:
        near = near or bool(np.any(np.abs(cum - cfg["top_p"] * d["sum"]) <= 1e-5 * d["sum"]))
    if cfg["min_p"] > 0:
        near = near or bool(np.any(np.abs(prob - cfg["min_p"] * prob[0]) <= 1e-5 * prob[0]))
    return near


CFGS = [
    dict(temperature=0.8, top_k=0, top_p=0.9, min_p=0.02, seed=123),
    dict(temperature=1.1, top_k=6, top_p=1.0, min_p=0.0, seed=2**63 + 1),
    dict(temperature=0.5, top_k=0, top_p=0.7, min_p=0.1, seed=99, presence_penalty=0.8),
    dict(temperature=0.0, top_k=0, top_p=1.0, min_p=0.0, seed=5, presence_penalty=1.25),
]


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cfg_i", range(len(CFGS)))
@pytest.mark.parametrize("tolerance", [0.0, 0.75])
def test_sampled_scores_vs_oracle(orc, dev, dtype, cfg_i, tolerance):
    import voidinfer_amd as vi
    cfg = CFGS[cfg_i]
    rng = np.random.default_rng(1000 + cfg_i * 10 + dtype)
    rows, vocab, first_key = 24, 248320 if cfg_i == 0 else 50_000, 40
    bits = make_bits(rng, rows, vocab, dtype)
    pres = cfg.get("presence_penalty", 0.0)
    fo = np.full(vocab, 0x7F7F7F7F, dtype=np.int32)
    top = np.argsort(-decode(bits, dtype), axis=1)[:, :30]
    fo[top[:, 0]] = 10
    fo[top[::3, 4]] = 60                      # generated after some keys
    # next tokens over every path: chosen, in support, just outside, far outside, -1, >= V
    chosen0, _ = orc.sampled_scores(bits, dtype, cfg["temperature"], cfg["top_k"], cfg["top_p"], cfg["min_p"],
                                    cfg["seed"], np.zeros(rows), first_key, tolerance, pres, fo)
    nxt = np.empty(rows, dtype=np.int64)
    for r in range(rows):
        kind = r % 6
        nxt[r] = [chosen0[r], top[r, 1], top[r, 8], top[r, 25], -1, vocab + 3][kind]
    want_c, want_gap = orc.sampled_scores(bits, dtype, cfg["temperature"], cfg["top_k"], cfg["top_p"],
                                          cfg["min_p"], cfg["seed"], nxt, first_key, tolerance, pres, fo)
    c, gap = vi.sampled_scores(to_dev(bits, dtype, dev), torch.from_numpy(nxt), cfg["temperature"], cfg["top_k"],
                               cfg["top_p"], cfg["min_p"], cfg["seed"], first_key, tolerance, pres,
                               torch.from_numpy(fo).to(dev))
    torch.cuda.synchronize()
    c, gap = c.cpu().numpy(), gap.cpu().numpy()
    x32 = decode(bits, dtype)
    for r in range(rows):
        key = first_key + r
        _, det = orc.sampled_packet(bits[r:r + 1], dtype, cfg["temperature"], cfg["top_k"], cfg["top_p"],
                                    cfg["min_p"], cfg["seed"], pres, fo, first_key=key)
        near = _near(det[0], cfg)
        if c[r] != want_c[r]:
            assert near, (r, c[r], want_c[r])
            continue
        if np.isinf(gap[r]) or np.isinf(want_gap[r]):
            if np.isinf(gap[r]) != np.isinf(want_gap[r]):
                boosted = x32[r:r + 1].copy()
                if 0 <= nxt[r] < vocab:
                    boosted[0, nxt[r]] = np.float32(boosted[0, nxt[r]] + np.float32(tolerance))
                _, bd = orc.sampled_packet(boosted, 2, cfg["temperature"], cfg["top_k"], cfg["top_p"],
                                           cfg["min_p"], cfg["seed"], pres, fo, first_key=key)
                assert near or _near(bd[0], cfg), (r, gap[r], want_gap[r])
            continue
        assert abs(gap[r] - want_gap[r]) <= 1e-4 + 1e-5 * abs(want_gap[r]), (r, gap[r], want_gap[r], near)


def test_scores_many_rows_and_rejects(orc, dev):
    """Row counts past the 16-row packet and invalid arguments."""
    import voidinfer_amd as vi
    from voidinfer_amd import _abi
    rng = np.random.default_rng(3)
    rows, vocab = 300, 2048
    bits = make_bits(rng, rows, vocab, 1)
    nxt = rng.integers(0, vocab, rows)
    want_c, want_gap = orc.sampled_scores(bits, 1, 0.9, 10, 0.95, 0.0, 77, nxt, 1000, 0.5)
    c, gap = vi.sampled_scores(to_dev(bits, 1, dev), torch.from_numpy(nxt), 0.9, 10, 0.95, 0.0, 77, 1000, 0.5)
    torch.cuda.synchronize()
    c = c.cpu().numpy()
    cfg = dict(temperature=0.9, top_k=10, top_p=0.95, min_p=0.0)
    for r in np.flatnonzero(c != want_c):
        _, det = orc.sampled_packet(bits[r:r + 1], 1, 0.9, 10, 0.95, 0.0, 77, first_key=1000 + int(r))
        assert _near(det[0], cfg), (r, c[r], want_c[r])
    lib = _abi.load()
    dcfg = _abi.DeviceSampling(0.9, 10, 0.95, 0.0, 77, 0.0, 0, None)
    import ctypes as C
    t = to_dev(bits, 1, dev)
    assert lib.vi_sampled_scores(t.data_ptr(), 1, rows, vocab, vocab, C.byref(dcfg), 0, -1.0, 0, 0, 0, None, 0,
                                 None) == 1
    assert lib.vi_row_scores(t.data_ptr(), 1, rows, vocab, vocab - 1, 0, 0, 0, None, 0, None) == 1

"""GPU full-vocabulary parts route (csrc/sample_parts.hip) vs the CPU oracle.

The parts route serves 16-bit full-route rows (temperature > 0, top_k 0 or
> 64) when no probabilities are wanted and the penalties come from penalty
states (or there are none), once VOIDINFER_AMD_FULL_ROUTE=parts selects it
(every test here sets it).  Bar (north star): sampled token ids identical
except where the oracle reports a cumulative-mass boundary within 1e-6
(relative) of the draw or of a top-p / min-p cut; Philox uniforms bit-exact;
support sizes, finite counts and flags equal outside exempt rows; support
masses within 1e-6 relative.  Covered: vocabularies that make one to four
parts (1,024 .. 248,320, and 65,504 / 65,512 on either side of one part),
bf16 and fp16, top-k caps above 64, min-p, top-p, non-finite logits, ties,
rows with nothing finite, penalty states with repeated tokens past the LDS
hash's capacity and counts past 16 bits, and recording sampled tokens.
"""
import numpy as np
import pytest
import torch

from helpers import exempt_draw, to_dev
from test_gpu_penalty_state import check_lane, csr, update

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def parts_route(monkeypatch):
    monkeypatch.setenv("VOIDINFER_AMD_FULL_ROUTE", "parts")

RTOL_MASS = 1e-6
FLAG_ERROR = 0x80000000


def make_rows(rng, rows, vocab, std=2.0, dtype=0, zipf=True):
    from voidinfer_amd import workloads as W
    x = W.gaussian_zipf(rows, vocab, std, int(rng.integers(1 << 30)), zipf=zipf)
    return W.encode(x, {0: "bf16", 1: "f16"}[dtype])


def params(rows, rng, **kw):
    import voidinfer_amd as vi
    p = vi.params_array(rows, seed=rng.integers(1, 2**62, rows), position=rng.integers(0, 100000, rows))
    for k, v in kw.items():
        p[k] = v
    return p


def check(out, w, p, label):
    """GPU outputs `out` (SampleOutputs) against the oracle's (tokens, u, _, stats, margins)."""
    import voidinfer_amd as vi
    w_tok, w_u, _, w_stats, margins = w
    g_tok = out.tokens.cpu().numpy()
    g_u = out.uniforms.cpu().numpy()
    g_st = vi.stats_numpy(out.stats)
    exempt = 0
    for r in range(len(p)):
        if g_tok[r] != w_tok[r] or g_st["support"][r] != w_stats["support"][r]:
            assert exempt_draw(margins[r]), (label, r, g_tok[r], w_tok[r], g_st[r], w_stats[r], margins[r], p[r])
            exempt += 1
            continue
        assert g_st["flags"][r] == w_stats["flags"][r], (label, r, g_st[r], w_stats[r])
        assert g_st["finite"][r] == w_stats["finite"][r], (label, r, g_st[r], w_stats[r])
        if p["temperature"][r] > 0 and not (w_stats["flags"][r] & 2):
            assert g_u[r] == w_u[r], (label, r)
            np.testing.assert_allclose(g_st["support_mass"][r], w_stats["support_mass"][r], rtol=RTOL_MASS,
                                       err_msg=f"{label} row {r}")
    return exempt


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("vocab", [1024, 65_504, 65_512, 151_936, 248_320])
def test_parts_filters(orc, dev, rng, dtype, vocab):
    import voidinfer_amd as vi
    rows = 16
    print(f"[parts] filters dtype={dtype} V={vocab}", flush=True)
    bits = make_rows(rng, rows, vocab, std=1.0, dtype=dtype)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.2, rows), top_k=rng.choice([0, 0, 100, 1000], rows),
               top_p=rng.choice([0.5, 0.9, 0.95, 1.0], rows), min_p=rng.choice([0.0, 0.0, 0.01, 0.1], rows))
    p["top_k"][3] = 20          # a top-k route row in the same call
    p["temperature"][5] = 0.0   # and an argmax row
    out = vi.sample_rows(to_dev(bits, dtype, dev), p, want_probs=False)
    torch.cuda.synchronize()
    w = orc.sample_rows(bits, dtype, p, None, None, want_probs=False)
    check(out, w, p, f"filters-{vocab}")


def test_parts_near_flat_rows(orc, dev, rng):
    """Config-5 style rows (N(0, 0.1), top_p 0.95): few distinct keys, the draw
    deep in the nucleus."""
    import voidinfer_amd as vi
    rows, vocab = 16, 248_320
    bits = make_rows(rng, rows, vocab, std=0.1, zipf=False)
    p = params(rows, rng, temperature=rng.uniform(0.3, 1.2, rows), top_k=0, top_p=0.95)
    out = vi.sample_rows(to_dev(bits, 0, dev), p, want_probs=False)
    torch.cuda.synchronize()
    check(out, orc.sample_rows(bits, 0, p, None, None, want_probs=False), p, "near-flat")


def test_parts_nonfinite_ties_and_limits(orc, dev, rng):
    import voidinfer_amd as vi
    rows, vocab = 10, 9_000
    bits = make_rows(rng, rows, vocab, std=1.0)
    bits[0, ::7] = 0x7FC0          # NaN
    bits[1, 5] = 0x7F80            # +inf
    bits[2, :] = 0x3F80            # all equal (1.0): pure tie-break by id
    bits[3, :4000] = 0x3F80
    bits[4, :] = 0x7FC0            # nothing finite
    bits[5, ::2] = 0x8000          # -0 and +0 share a key
    bits[5, 1::2] = 0x0000
    bits[6, :100] = 0x7F7F         # the largest finite bf16: z overflows at T < 1
    p = params(rows, rng, temperature=0.9, top_k=0, top_p=rng.choice([0.3, 0.9], rows))
    p["temperature"][6] = 0.5
    p["temperature"][7] = 70000.0  # above the 16-bit route's limit: the row fails
    p["top_k"][8] = 65             # a cap just above the top-k route
    p["min_p"][9] = 0.5
    out = vi.sample_rows(to_dev(bits, 0, dev), p, want_probs=False)
    torch.cuda.synchronize()
    st = vi.stats_numpy(out.stats)
    assert out.tokens[7].item() == -1 and (st["flags"][7] & FLAG_ERROR)
    keep = np.array([r for r in range(rows) if r != 7])
    kt = torch.from_numpy(keep).to(out.tokens.device)
    w = orc.sample_rows(bits[keep], 0, p[keep], None, None, want_probs=False)

    class Sub:
        tokens, uniforms, stats = out.tokens[kt], out.uniforms[kt], out.stats.view(rows, -1)[kt].reshape(-1)
    check(Sub, w, p[keep], "edges")


@pytest.mark.parametrize("dtype", [0, 1])
def test_parts_state_route_steps(orc, dev, rng, dtype):
    """Penalties from the lanes' states over three decode steps that record the
    sampled tokens in the same launch; the oracle reads the equivalent
    histories; the states hold exactly the grown histories afterwards."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    rows, vocab, L = 12, 248_320, 6000
    x = W.gaussian_zipf(rows, vocab, 1.0, int(rng.integers(1 << 30)))
    bits = W.encode(x, {0: "bf16", 1: "f16"}[dtype])
    p = params(rows, rng, temperature=rng.uniform(0.5, 1.2, rows), top_k=np.array([0, 20, 0, 500, 100, 0] * 2),
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
    for step in range(3):
        print(f"[parts] state dtype={dtype} step={step}", flush=True)
        toks, offs = csr(hist)
        out = vi.sample_rows_state(logits, p, st, record=True, want_probs=False)
        torch.cuda.synchronize()
        check(out, orc.sample_rows(bits, dtype, p, toks, offs, want_probs=False), p, f"state step {step}")
        hist = [np.append(h, t).astype(np.int32) for h, t in zip(hist, out.tokens.cpu().numpy())]
        p["position"] += 1
    for r in range(rows):
        check_lane(st, r, hist[r])


def test_parts_state_route_config5_subset(orc, dev):
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    bits, hist, offs, p = W.config5(rows=16)
    st = vi.PenaltyState(16, W.V_QWEN, 1 << 16, device=dev)
    st.update(torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev))
    out = vi.sample_rows_state(to_dev(bits, 0, dev), p, st, want_probs=False)
    torch.cuda.synchronize()
    check(out, orc.sample_rows(bits, 0, p, hist, offs, want_probs=False), p, "config5")


def test_parts_state_hash_overflow_and_large_counts(orc, dev, rng):
    """Lane 0: 5,000 tokens seen twice in one part (past the LDS repeat hash's
    3,072 entries: lookups read the lane's table); lane 1: one token recorded
    70,000 times (a count past 16 bits); lane 2: 40,000 distinct tokens once."""
    import voidinfer_amd as vi
    vocab = 248_320
    hist = [np.tile(np.arange(5000), 2), np.full(70_000, 1234), np.arange(40_000)]
    st = vi.PenaltyState(3, vocab, 1 << 18, device=dev)
    update(st, dev, hist)
    bits = make_rows(rng, 3, vocab, std=1.0)
    bits[1, 1234] = 0x4200                                    # 32.0: the heavy token would win unpenalized
    p = params(3, rng, temperature=1.0, top_k=0, top_p=0.9, repetition_penalty=1.1, frequency_penalty=0.01,
               presence_penalty=0.1)
    out = vi.sample_rows_state(to_dev(bits, 0, dev), p, st, want_probs=False)
    torch.cuda.synchronize()
    toks, offs = csr(hist)
    check(out, orc.sample_rows(bits, 0, p, toks, offs, want_probs=False), p, "overflow")

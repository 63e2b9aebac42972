"""GPU greedy argmax vs the oracle (greedy_packet.cuh semantics), bit-exact.

Inputs follow tests/test_exl3_greedy_device.cu:47-97 of the reference: authored
binary16 patterns, rows {1, 8, 16} x V {1, 255, 257, 1025, 248320}, stride V + 7
padded with NaN, ties across lanes, subnormals, signed zeros, +-Inf/NaN; plus
bf16 / fp32 random rows and the 128-row metric shape.  Expected values come from
the oracle and, independently, numpy's first-maximum argmax.
"""
import numpy as np
import pytest
import torch

from helpers import greedy_reference_patterns as reference_patterns, to_dev

pytestmark = pytest.mark.gpu


def check(orc, dev, bits: np.ndarray, dtype: int, vocab: int):
    import voidinfer_amd as vi
    rows, width = bits.shape
    got = vi.greedy_packet(to_dev(bits, dtype, dev)[:, :width], serial=91, vocabulary=vocab)
    want = orc.greedy_rows(bits, dtype, vocabulary=vocab, serial=91)
    assert np.array_equal(got["serial"], want["serial"])
    assert np.array_equal(got["nonfinite"], want["nonfinite"]), (got, want)
    assert np.array_equal(got["token"], want["token"]), (got, want)
    # independent: numpy first-maximum over finite values
    if dtype == 1:
        vals = bits[:, :vocab].view(np.float16).astype(np.float32)
    elif dtype == 0:
        vals = (bits[:, :vocab].astype(np.uint32) << 16).view(np.float32)
    else:
        vals = bits[:, :vocab]
    for r in range(rows):
        fin = np.isfinite(vals[r])
        assert bool(want["nonfinite"][r]) == (not fin.all())
        if fin.any():
            masked = np.where(fin, vals[r], -np.inf)
            assert want["token"][r] == int(np.argmax(masked)) or (masked[want["token"][r]] == masked.max())


@pytest.mark.parametrize("rows", [1, 8, 16])
@pytest.mark.parametrize("vocab", [1, 255, 257, 1025, 248320])
def test_reference_device_patterns(orc, dev, rows, vocab):
    for bits in reference_patterns(rows, vocab):
        check(orc, dev, bits, 1, vocab)


def test_private_winners_per_row(orc, dev):
    # test_exl3_greedy_device.cu:50-62: distinct rows, winners at 0 / 256 / V-1
    vocab, stride = 248320, 248327
    paired = np.full((16, stride), 0x7E00, dtype=np.uint16)
    for r in range(16):
        paired[r, :vocab] = 0xBC00
        paired[r, 0 if r < 8 else 256] = 0x3C00
        paired[r, vocab - 1] = 0x3C00
    check(orc, dev, paired, 1, vocab)
    paired[7, vocab - 1] = 0x7E01
    check(orc, dev, paired, 1, vocab)
    paired = np.concatenate([paired[8:], paired[:8]])
    check(orc, dev, paired, 1, vocab)


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_random_rows_all_dtypes(orc, dev, rng, dtype):
    rows, vocab = 37, 100_003
    x = rng.standard_normal((rows, vocab)).astype(np.float32)
    x[:, rng.integers(0, vocab, 5)] = 4.0          # ties across the row
    if dtype == 2:
        bits = x
    elif dtype == 1:
        bits = x.astype(np.float16).view(np.uint16)
    else:
        bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    check(orc, dev, bits, dtype, vocab)


def test_metric_shape_128_rows(orc, dev, rng):
    rows, vocab = 128, 248320
    bits = (rng.standard_normal((rows, vocab)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    check(orc, dev, bits, 0, vocab)


def test_repeat_and_unmutated(orc, dev, rng):
    import voidinfer_amd as vi
    bits = rng.integers(0, 0x7C00, (8, 5000)).astype(np.uint16)
    t = to_dev(bits, 1, dev)
    a = vi.greedy_packet(t)
    b = vi.greedy_packet(t)
    assert np.array_equal(a, b)
    assert np.array_equal(t.view(torch.int16).cpu().numpy().view(np.uint16), bits)


def test_ties_inside_vectors_and_signed_zeros(orc, dev, rng):
    """Maxima repeated inside one 16-byte vector (the first must win), and rows
    whose largest values are +0 / -0 mixed (the first zero wins, either sign)."""
    rows, vocab = 24, 40_960
    x = rng.standard_normal((rows, vocab)).astype(np.float16)
    for r in range(rows):
        v = int(rng.integers(0, vocab // 8)) * 8
        x[r, v + int(rng.integers(1, 8)):v + 8] = 6.0           # tie inside one vector
        x[r, int(rng.integers(0, vocab))] = 6.0 if r % 3 == 0 else x[r, 0]
    z = -np.abs(x[:8])
    z[:, rng.integers(0, vocab, 64)] = np.float16(0.0)
    z[:, rng.integers(0, vocab, 64)] = np.float16(-0.0)
    check(orc, dev, np.concatenate([x, z]).view(np.uint16), 1, vocab)

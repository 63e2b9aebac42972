"""Test helpers: move numpy logit patterns to the device, compare against the oracle."""
from __future__ import annotations

import functools

import numpy as np
import torch

DT_TORCH = {0: torch.bfloat16, 1: torch.float16, 2: torch.float32}


def to_dev(bits: np.ndarray, dtype: int, device) -> torch.Tensor:
    """uint16 patterns (bf16/fp16) or float32 -> device tensor of that dtype."""
    if dtype == 2:
        return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.float32)).to(device)
    t = torch.from_numpy(np.ascontiguousarray(bits).astype(np.uint16).view(np.int16)).to(device)
    return t.view(DT_TORCH[dtype])


def xorshift_topk_case(rows: int, vocab: int, pattern: int) -> np.ndarray:
    """The reference's 168-case top-k input generator (test_exl3_dflash2_topk.h:183-219):
    xorshift32 seeded 0x12345678 and the eight bit patterns of the qualification run."""
    state = 0x12345678
    out = np.empty(rows * vocab, dtype=np.uint16)
    k = 0
    for _ in range(rows):
        for c in range(vocab):
            state ^= (state << 13) & 0xFFFFFFFF
            state ^= state >> 17
            state ^= (state << 5) & 0xFFFFFFFF
            bits = (state & 0x8000) | (state % 0x7C00)
            if pattern == 1:
                bits = 0x3C00
            elif pattern == 2:
                bits = 0x8000 if (c & 1) else 0
            elif pattern == 3:
                bits = 0x7C00 if c % 17 == 0 else 0xFC00
            elif pattern == 4:
                bits = 0x3C00 + c % 3
            elif pattern == 5 and (c == 0 or c == 7 or c == vocab - 1):
                bits = 0xFC11 if c == 7 else 0x7E11
            elif pattern == 6:
                bits = 0x7C01 | (state & 0x83FF)
            elif pattern == 7:
                bits = 0x4000 if c >= vocab - 2 else 0xBC00
            out[k] = bits
            k += 1
    return out.reshape(rows, vocab)


@functools.lru_cache(maxsize=4)
def xorshift_states(n: int) -> np.ndarray:
    """The first n states of the reference generator's xorshift32 (seed 0x12345678)."""
    states = np.empty(n, dtype=np.uint32)
    st = 0x12345678
    for i in range(n):  # inherently serial
        st ^= (st << 13) & 0xFFFFFFFF
        st ^= st >> 17
        st ^= (st << 5) & 0xFFFFFFFF
        states[i] = st
    states.setflags(write=False)
    return states


def xorshift_topk_case_fast(rows: int, vocab: int, pattern: int) -> np.ndarray:
    """Vectorised version of xorshift_topk_case (same bits); used for large vocabularies."""
    states = xorshift_states(rows * vocab)
    c = np.tile(np.arange(vocab), rows)
    bits = (states & 0x8000) | (states % 0x7C00)
    if pattern == 1:
        bits[:] = 0x3C00
    elif pattern == 2:
        bits = np.where(c & 1, 0x8000, 0).astype(np.uint32)
    elif pattern == 3:
        bits = np.where(c % 17 == 0, 0x7C00, 0xFC00).astype(np.uint32)
    elif pattern == 4:
        bits = (0x3C00 + c % 3).astype(np.uint32)
    elif pattern == 5:
        m = (c == 0) | (c == 7) | (c == vocab - 1)
        bits = np.where(m, np.where(c == 7, 0xFC11, 0x7E11), bits).astype(np.uint32)
    elif pattern == 6:
        bits = (0x7C01 | (states & 0x83FF)).astype(np.uint32)
    elif pattern == 7:
        bits = np.where(c >= vocab - 2, 0x4000, 0xBC00).astype(np.uint32)
    return bits.astype(np.uint16).reshape(rows, vocab)


def exempt_draw(margins_row: np.ndarray, tol: float = 1e-6) -> bool:
    """Token mismatch allowed when the drawn uniform or a truncation cut lies
    within `tol` of a cumulative-mass boundary."""
    return bool(margins_row[0] < tol or margins_row[1] < tol or margins_row[2] < tol)


def greedy_reference_patterns(rows: int, vocab: int):
    """The authored binary16 greedy patterns of the reference's device test
    (test_exl3_greedy_device.cu:47-97): stride V + 7 padded with NaN, near-equal
    pairs at the row ends and lane boundary 256, signed zeros, +-Inf / NaN."""
    stride = vocab + 7
    base = np.full((rows, stride), 0x7E00, dtype=np.uint16)
    base[:, :vocab] = 0xBC00
    yield base.copy()
    for a, b in [(0x3C00, 0x3C01), (0x0001, 0x0002), (0x03FF, 0x0400), (0xFBFF, 0xFBFE), (0x7BFE, 0x7BFF)]:
        near = base.copy()
        near[:, :vocab] = a
        near[:, vocab - 1] = b
        if vocab > 256:
            near[:, 256] = b
        yield near
    x = base.copy()
    x[:, vocab - 1] = 0x0000
    x[:, 0] = 0x8000
    yield x.copy()
    x[:, vocab - 1] = 0x3C00
    if vocab > 256:
        x[:, 256] = 0x3C00
    yield x.copy()
    for bad in (0x7C00, 0xFC00, 0x7E01):
        inv = x.copy()
        inv[rows - 1, vocab - 1] = bad
        yield inv

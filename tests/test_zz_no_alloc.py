"""vi_greedy_rows_noalloc (the allocation-free greedy entry point) against
vi_greedy_rows with a caller workspace: bit-identical packet rows on two calls in
a row, the second smaller than the first (so it reads the library's scratch
array after a larger call left partials in it), then a shape that needs no
slices.  Runs through the C ABI."""
import numpy as np
import pytest
import torch

from helpers import to_dev

pytestmark = pytest.mark.gpu


def _noalloc(lib, t, dtype_code, rows, vocab, stride, serial):
    out = torch.empty(rows, 16, dtype=torch.uint8, device=t.device)
    st = lib.vi_greedy_rows_noalloc(t.data_ptr(), dtype_code, rows, vocab, stride, serial, out.data_ptr(), None)
    assert st == 0, st
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.dtype([("serial", "<u8"), ("token", "<i4"), ("nonfinite", "<u4")])).ravel()


def _with_workspace(lib, t, dtype_code, rows, vocab, stride, serial):
    out = torch.empty(rows, 16, dtype=torch.uint8, device=t.device)
    nb = lib.vi_greedy_workspace_bytes(rows, vocab)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=t.device)
    st = lib.vi_greedy_rows(t.data_ptr(), dtype_code, rows, vocab, stride, serial, out.data_ptr(), ws.data_ptr(),
                            ws.numel(), None)
    assert st == 0, st
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.dtype([("serial", "<u8"), ("token", "<i4"), ("nonfinite", "<u4")])).ravel()


@pytest.mark.parametrize("dtype_code", [0, 1, 2])
def test_noalloc_matches_workspace_entry(orc, dev, rng, dtype_code):
    import voidinfer_amd as vi
    lib = vi.load()
    shapes = [(96, 248_320), (7, 50_001), (1100, 4096)]   # large, then smaller, then one slice per row
    for serial, (rows, vocab) in enumerate(shapes, start=11):
        x = rng.standard_normal((rows, vocab)).astype(np.float32)
        x[:, rng.integers(0, vocab, 3)] = 7.5            # ties at the maximum: lowest id wins
        x[rows // 2, 5] = np.nan
        if dtype_code == 0:
            bits = (x.view(np.uint32) >> 16).astype(np.uint16)
        elif dtype_code == 1:
            bits = x.astype(np.float16).view(np.uint16)
        else:
            bits = x
        t = to_dev(bits, dtype_code, dev)
        print(f"noalloc dtype {dtype_code} rows {rows} vocab {vocab}", flush=True)
        a = _noalloc(lib, t, dtype_code, rows, vocab, vocab, serial)
        b = _with_workspace(lib, t, dtype_code, rows, vocab, vocab, serial)
        assert np.array_equal(a, b), (rows, vocab)
        want = orc.greedy_rows(bits, dtype_code)
        assert np.array_equal(a["token"], want["token"]) and np.array_equal(a["nonfinite"], want["nonfinite"])
        assert np.all(a["serial"] == serial)


def test_noalloc_rejects_bad_arguments(dev):
    import voidinfer_amd as vi
    lib = vi.load()
    t = torch.zeros(4, 100, dtype=torch.bfloat16, device=dev)
    out = torch.empty(4, 16, dtype=torch.uint8, device=dev)
    assert lib.vi_greedy_rows_noalloc(t.data_ptr(), 0, 4, 100, 99, 1, out.data_ptr(), None) == 1   # stride < V
    assert lib.vi_greedy_rows_noalloc(t.data_ptr(), 7, 4, 100, 100, 1, out.data_ptr(), None) == 1  # dtype
    assert lib.vi_greedy_rows_noalloc(t.data_ptr(), 0, 0, 100, 100, 1, out.data_ptr(), None) == 0  # no rows

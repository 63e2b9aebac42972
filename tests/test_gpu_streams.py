"""Calls that run part of their work on the library's second stream (a batch
with rows on both kernel routes: the top-k launch beside the full-vocabulary
route) issued from a non-default stream and from a captured HIP graph.  The
second stream is forked from the caller's stream and joined back into it, so
synchronizing the caller's stream alone must expose complete results, and a
graph captured from the call must replay them."""
import numpy as np
import pytest
import torch

from helpers import to_dev

pytestmark = pytest.mark.gpu

ROWS, VOCAB, HIST = 8, 65_536, 2048


def _batch(rng, dtype):
    """Eight lanes, top_k 0 on half of them (full-vocabulary route) and 20 / 50
    on the others (top-k route), with penalties over 2,048-token histories."""
    import voidinfer_amd as vi
    from voidinfer_amd import workloads as W
    x = W.gaussian_zipf(ROWS, VOCAB, 2.0, int(rng.integers(1 << 30)))
    bits = W.encode(x, {0: "bf16", 2: "f32"}[dtype])
    p = vi.params_array(ROWS, seed=rng.integers(1, 2**62, ROWS), position=rng.integers(0, 10**5, ROWS),
                        temperature=np.full(ROWS, 0.8), top_k=np.array([0, 20, 0, 50, 0, 0, 20, 0]),
                        top_p=np.full(ROWS, 0.9), repetition_penalty=np.full(ROWS, 1.1),
                        presence_penalty=np.full(ROWS, 0.2))
    hist = rng.integers(0, VOCAB, ROWS * HIST).astype(np.int32)
    offs = (np.arange(ROWS + 1) * HIST).astype(np.int64)
    return bits, p, hist, offs


@pytest.mark.parametrize("dtype", [0, 2])
def test_mixed_routes_from_a_non_default_stream(dev, rng, dtype):
    """The same call on the default stream is the reference (its parity with
    the oracle is the mixed-lane tests' subject)."""
    import voidinfer_amd as vi
    bits, p, hist, offs = _batch(rng, dtype)
    assert vi.route_mask(p) == vi.ROUTE_ALL
    logits = to_dev(bits, dtype, dev)
    h, o = torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev)
    ref = vi.sample_rows(logits, p, h, o, max_history=HIST)
    torch.cuda.synchronize()
    ref_tok = ref.tokens.cpu().numpy()
    assert (ref_tok >= 0).all() and (ref_tok < VOCAB).all(), ref_tok
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        outs = [vi.sample_rows(logits, p, h, o, max_history=HIST) for _ in range(4)]
    s.synchronize()   # (only the caller's stream: the second stream was joined into it)
    for i, out in enumerate(outs):
        assert (out.tokens.cpu().numpy() == ref_tok).all(), i


def test_mixed_routes_graph_replay(dev, rng):
    import voidinfer_amd as vi
    from voidinfer_amd.ops import SampleOutputs
    bits, p, hist, offs = _batch(rng, 0)
    logits = to_dev(bits, 0, dev)
    h, o = torch.from_numpy(hist).to(dev), torch.from_numpy(offs).to(dev)
    p_dev = vi.to_device_bytes(p, dev)
    out = SampleOutputs(torch.empty(ROWS, dtype=torch.int32, device=dev), None, None, None)

    def call():
        return vi.sample_rows(logits, p_dev, h, o, max_history=HIST, outputs=out, routes=vi.ROUTE_ALL)

    call()   # (creates the workspace and this thread's second stream before the capture)
    torch.cuda.synchronize()
    ref = out.tokens.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    for i in range(3):
        out.tokens.fill_(-7)   # eager work and a synchronization between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.tokens, ref), i

"""GPU greedy-packet transport (vi_packet_*): the rows one vi_greedy_rows launch
writes for several lanes come back through one pinned copy, equal to the
oracle's argmax rows; pool exhaustion, slot reuse, wrong row counts and
destroy with a copy in flight behave as documented."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_batched_readback_equals_oracle(orc, dev):
    import voidinfer_amd as vi
    from voidinfer_amd import ops, workloads as W
    lanes_rows = [1, 16, 4, 7]                      # four lanes' packets, end to end
    total = sum(lanes_rows)
    bits = W.encode(W.gaussian_zipf(total, 248_320, 2.0, 31), "bf16")
    logits = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    out = torch.zeros(total * vi.GREEDY_ROW.itemsize, dtype=torch.uint8, device=dev)
    t = vi.PacketTransport(slots=2, max_rows=64)
    for serial in (5, 6, 7):                        # three rounds reuse the two slots
        ops.greedy_rows_device(logits, out, serial=serial)
        slot = t.submit(out, total)
        rows = t.finish(slot, total)
        want = orc.greedy_rows(bits, orc.BF16)
        assert np.array_equal(rows["token"], want["token"])
        assert (rows["serial"] == serial).all() and (rows["nonfinite"] == 0).all()
    t.close()


def test_pool_limits_and_errors(dev):
    import voidinfer_amd as vi
    from voidinfer_amd._abi import VIError
    rows = torch.zeros(4 * vi.GREEDY_ROW.itemsize, dtype=torch.uint8, device=dev)
    t = vi.PacketTransport(slots=2, max_rows=4)
    a, b = t.submit(rows), t.submit(rows)
    with pytest.raises(VIError):                    # every slot in flight: VI_ERR_WORKSPACE
        t.submit(rows)
    with pytest.raises(ValueError):                 # wrong row count (VI_ERR_INVALID)
        t.finish(a, 3)
    torch.cuda.synchronize()
    assert t.query(a)
    t.finish(a, 4)
    c = t.submit(rows)                              # the freed slot is reused
    assert c == a
    with pytest.raises(ValueError):                 # more rows than a slot holds
        t.submit(torch.zeros(5 * vi.GREEDY_ROW.itemsize, dtype=torch.uint8, device=dev))
    t.close()                                       # b and c still in flight: destroy waits for them

"""The engine-facing C++ launchers on the GPU.

tests/cpp/test_launchers_gpu (built with the library by voidinfer_amd/build.py)
links libvoidinfer_sampling.so and calls exl3_launch_greedy_packet,
Exl3GreedyPacketTransport, exl3_presence_*, exl3_launch_sampled_packet,
dflash2_topk16_for_test and dflash_sampled_choices through
include/voidinfer_sampling.hpp, as the engine would.  This test writes its
inputs and the CPU oracle's outputs (oracle/liboracle.so) to a fixture
directory and runs it: greedy tokens, top-16 ids and values, presence tables
and draft proposals bit-exact; sampled-packet tokens bit-exact outside the
oracle's near-boundary rows (flagged in the fixture).
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "tests" / "cpp" / "test_launchers_gpu"


def f32_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def packet_near(detail, cfg) -> np.ndarray:
    """Rows whose oracle decision lay within float rounding of a boundary."""
    out = np.zeros(len(detail), dtype=np.uint8)
    for r, d in enumerate(detail):
        vals = np.sort(d["value"][: d["support"]])[::-1]
        near = len(vals) > 1 and abs(vals[0] - vals[1]) <= 1e-5 * (1 + abs(vals[0]))
        prob = d["prob"][: d["cap"]].astype(np.float64)
        cum = np.cumsum(prob)
        if cfg["top_p"] < 1:
            near = near or bool(np.any(np.abs(cum - cfg["top_p"] * d["sum"]) <= 1e-5 * d["sum"]))
        if cfg["min_p"] > 0:
            near = near or bool(np.any(np.abs(prob - cfg["min_p"] * prob[0]) <= 1e-5 * prob[0]))
        out[r] = near
    return out


def write_fixture(d: Path, orc) -> None:
    import voidinfer_amd as vi
    rng = np.random.default_rng(2024)
    meta = {}

    def put(name, arr):
        np.ascontiguousarray(arr).tofile(d / name)

    # greedy packet and its readback: 8 fp16 rows, the last with a NaN
    V = 50_000
    g_bits = (rng.standard_normal((8, V)) * 2).astype(np.float16).view(np.uint16)
    g_bits[2, [11, 40_000]] = 0x4B00          # a tie at the row maximum: the lower id wins
    g_bits[7, 123] = 0x7E00
    g = orc.greedy_rows(g_bits, orc.F16, serial=9)
    put("greedy_logits.bin", g_bits)
    put("greedy_tokens.bin", g["token"].astype(np.int32))
    put("greedy_nonfinite.bin", g["nonfinite"].astype(np.uint32))
    meta.update(greedy_rows=8, greedy_vocab=V, greedy_serial=9, greedy_clean_rows=7)

    # presence table (reset, record at position 40, truncate at 50), then the
    # sampled packet over it
    absent = vi.ABSENT_OCCURRENCE
    hist = rng.integers(-5, V + 5, 30).astype(np.int64)
    table = np.full(V, absent, dtype=np.int32)
    for i, t in enumerate(hist):
        if 0 <= t < V:
            table[t] = min(table[t], 40 + i)
    table[table >= 50] = absent
    put("presence_tokens.bin", hist)
    put("presence_table.bin", table)
    meta.update(presence_first=40, presence_truncate=50)
    p_bits = (rng.standard_normal((6, V)) * 2).astype(np.float16).view(np.uint16)
    top = orc.greedy_rows(p_bits, orc.F16)["token"]
    cfg = dict(temperature=0.8, top_k=20, top_p=0.9, min_p=0.02, seed=0x5EED, presence_penalty=1.25)
    depths = np.array([0, 1, 2, 1, 2, 3], dtype=np.int32)
    inputs = top.astype(np.int32)
    w, detail = orc.sampled_packet(p_bits, orc.F16, cfg["temperature"], cfg["top_k"], cfg["top_p"], cfg["min_p"],
                                   cfg["seed"], cfg["presence_penalty"], table, 60, depths, inputs, serial=5)
    put("packet_logits.bin", p_bits)
    put("packet_depths.bin", depths)
    put("packet_inputs.bin", inputs)
    put("packet_tokens.bin", w["token"].astype(np.int32))
    put("packet_near.bin", packet_near(detail, cfg))
    meta.update(packet_vocab=V, packet_rows=6, packet_first_key=60, packet_top_k=cfg["top_k"],
                packet_seed=cfg["seed"], packet_temperature=f32_bits(cfg["temperature"]),
                packet_top_p=f32_bits(cfg["top_p"]), packet_min_p=f32_bits(cfg["min_p"]),
                packet_presence=f32_bits(cfg["presence_penalty"]))

    # top-16 at the reference's qualification shape (rows 1..7, full vocabulary)
    TV = 248_320
    t_bits = (rng.standard_normal((7, TV)) * 1.5).astype(np.float16).view(np.uint16)
    t_bits[4, 1000] = 0x7C00                   # +Inf: the non-finite flag
    ids, vals, _, flag = orc.topk_rows(t_bits, orc.F16, 16)
    put("topk_logits.bin", t_bits)
    put("topk_ids.bin", ids.astype(np.int64))
    put("topk_values.bin", vals.astype(np.float32))
    meta.update(topk_rows=7, topk_vocab=TV, topk_nonfinite=int(flag))

    # draft proposals (coupled sampled choice on odd lanes, first maximum on even)
    lanes, positions, DV = 6, 8, 30_000
    scores = (rng.standard_normal((lanes, positions, 16)) * 2).astype(np.float32)
    cands = np.stack([np.stack([rng.choice(DV, 16, replace=False) for _ in range(positions)])
                      for _ in range(lanes)]).astype(np.int64)
    seeds = rng.integers(0, DV, lanes).astype(np.int64)
    cands[:, 1:, 3] = seeds[:, None]           # the seed token recurs (presence penalty)
    smp = np.zeros(lanes, dtype=vi.DRAFT_SAMPLING)
    smp["inv_temperature"] = np.where(np.arange(lanes) % 2 == 1, 1 / 0.8, 0.0)
    smp["top_k"], smp["top_p"], smp["min_p"] = 10, 0.9, 0.0
    smp["seed"] = 1000 + np.arange(lanes)
    smp["key_base"] = 77 * np.arange(lanes)
    smp["presence_penalty"] = 0.5
    want = orc.draft_choice(scores, cands, smp, seeds, vocabulary=DV)
    put("draft_scores.bin", scores)
    put("draft_candidates.bin", cands)
    put("draft_seed_tokens.bin", seeds)
    put("draft_sampling.bin", smp)
    put("draft_proposals.bin", want)
    meta.update(draft_lanes=lanes, draft_positions=positions, draft_vocab=DV)

    (d / "meta.txt").write_text("".join(f"{k}={int(v)}\n" for k, v in meta.items()))


def test_cpp_launchers_against_oracle_fixture(orc, dev, tmp_path):
    if not BIN.exists():
        pytest.fail("tests/cpp/test_launchers_gpu is not built (python voidinfer_amd/build.py)")
    write_fixture(tmp_path, orc)
    res = subprocess.run([str(BIN), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "launchers PASS" in res.stdout

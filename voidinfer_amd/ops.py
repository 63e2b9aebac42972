"""Torch-facing calls into libvoidinfer_sampling.so.

PyTorch supplies device memory and the current stream; every computation is a
HIP kernel of the library.  Function names follow the reference's launchers:

=========================  ==========================================================
``greedy_packet``           exl3_launch_greedy_packet (src/exl3/greedy_packet.cuh:256)
``topk_rows``               dflash2_topk16_for_test (src/exl3/dflash2_draft.cu:2390)
``sampled_packet``          exl3_launch_sampled_packet (src/exl3/sampled_select.cuh:362)
``presence_*``              exl3_presence_reset/truncate/record (sampled_select.h:33-35)
``sample_rows``             batched sampler (new entry; lanes x penalties x Philox)
``verify_rows``             decide_exl3_outer_prefix / IndependentAcceptanceReference,
                            on the device (exact_outer_reference.h:68,
                            sampled_acceptance_reference.h:48)
``verification_tree``       exl3_build_verification_tree (src/exl3/verification_tree.h:44),
                            a host function of the library
=========================  ==========================================================

Workspaces: each entry point and shape owns a zero-initialised workspace (its
arrival counters start at zero and the kernels leave them at zero), cached per
device here.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np
import torch

from . import _abi
from ._abi import (BF16, F16, F32, GREEDY_ROW, ROW_PARAMS, SAMPLE_STATS, DeviceSampling, check)

_DTYPES = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}
_workspaces: dict[tuple, torch.Tensor] = {}


def _lib():
    return _abi.load()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def workspace(key: tuple, nbytes: int, device: torch.device) -> torch.Tensor:
    """Zero-filled device workspace of at least `nbytes`, one per (key, device)."""
    k = (key, device.index if device.index is not None else torch.cuda.current_device())
    ws = _workspaces.get(k)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _workspaces[k] = ws
    return ws


def _logit_args(logits: torch.Tensor) -> tuple[int, int, int, int]:
    if logits.dim() != 2:
        raise ValueError("logits must be [rows, vocabulary]")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logit dtype {logits.dtype}")
    if logits.stride(1) != 1:
        raise ValueError("logit rows must be contiguous")
    if not logits.is_cuda:
        raise ValueError("logits must be on a HIP device")
    rows, vocab = logits.shape
    stride = logits.stride(0) if rows > 1 else max(vocab, logits.stride(0))
    return _DTYPES[logits.dtype], rows, vocab, stride


def _rows_view(logits: torch.Tensor, vocabulary: int | None) -> tuple[int, int, int, int]:
    dtype, rows, width, stride = _logit_args(logits)
    vocab = width if vocabulary is None else vocabulary
    if vocab > width:
        raise ValueError("vocabulary exceeds the row width")
    return dtype, rows, vocab, stride


def greedy_packet(logits: torch.Tensor, serial: int = 1, vocabulary: int | None = None) -> np.ndarray:
    """Argmax rows -> structured array of vi_greedy_row (serial, token, nonfinite)."""
    dtype, rows, vocab, stride = _rows_view(logits, vocabulary)
    out = torch.empty(rows * GREEDY_ROW.itemsize, dtype=torch.uint8, device=logits.device)
    nb = _lib().vi_greedy_workspace_bytes(rows, vocab)
    ws = workspace(("greedy", rows, vocab), nb, logits.device)
    check(_lib().vi_greedy_rows(logits.data_ptr(), dtype, rows, vocab, stride, serial, out.data_ptr(),
                                ws.data_ptr(), ws.numel(), _stream()), "vi_greedy_rows")
    return out.cpu().numpy().view(GREEDY_ROW)


def greedy_rows_device(logits: torch.Tensor, out: torch.Tensor, serial: int = 1) -> None:
    """Argmax into a caller-owned uint8 device buffer of rows * 16 bytes (no sync)."""
    dtype, rows, vocab, stride = _rows_view(logits, None)
    nb = _lib().vi_greedy_workspace_bytes(rows, vocab)
    ws = workspace(("greedy", rows, vocab), nb, logits.device)
    check(_lib().vi_greedy_rows(logits.data_ptr(), dtype, rows, vocab, stride, serial, out.data_ptr(),
                                ws.data_ptr(), ws.numel(), _stream()), "vi_greedy_rows")


def topk_rows(logits: torch.Tensor, k: int = 16, logprobs: bool = False, vocabulary: int | None = None,
              nonfinite_flag: torch.Tensor | None = None):
    """Exact top-k ids (int64), values (f32) and optional log-probs (f32)."""
    dtype, rows, vocab, stride = _rows_view(logits, vocabulary)
    dev = logits.device
    ids = torch.empty(rows, k, dtype=torch.int64, device=dev)
    vals = torch.empty(rows, k, dtype=torch.float32, device=dev)
    lp = torch.empty(rows, k, dtype=torch.float32, device=dev) if logprobs else None
    nb = _lib().vi_topk_workspace_bytes(rows, vocab, k)
    ws = workspace(("topk", rows, vocab), nb, dev)
    check(_lib().vi_topk_rows(logits.data_ptr(), dtype, rows, vocab, stride, k, ids.data_ptr(), vals.data_ptr(),
                              _ptr(lp), _ptr(nonfinite_flag), ws.data_ptr(), ws.numel(), _stream()),
          "vi_topk_rows")
    return ids, vals, lp


def sampled_packet(scores: torch.Tensor, temperature: float, top_k: int, top_p: float, min_p: float,
                   seed: int, presence_penalty: float = 0.0, first_occurrence: torch.Tensor | None = None,
                   first_key: int = 0, depths: Sequence[int] | None = None,
                   inputs: Sequence[int] | None = None, serial: int = 1) -> np.ndarray:
    """Coupled reference-semantics packet -> vi_greedy_row array."""
    dtype, rows, vocab, stride = _rows_view(scores, None)
    cfg = DeviceSampling(temperature, top_k, top_p, min_p, seed, presence_penalty, 0,
                         first_occurrence.data_ptr() if first_occurrence is not None else None)
    d = (C.c_int32 * rows)(*depths) if depths is not None else None
    i = (C.c_int32 * rows)(*inputs) if inputs is not None else None
    out = torch.empty(rows * GREEDY_ROW.itemsize, dtype=torch.uint8, device=scores.device)
    nb = _lib().vi_sampled_packet_workspace_bytes(rows, vocab)
    ws = workspace(("packet", rows, vocab), nb, scores.device)
    check(_lib().vi_sampled_packet(scores.data_ptr(), dtype, rows, vocab, stride, C.byref(cfg), first_key,
                                   C.cast(d, C.c_void_p) if d is not None else None,
                                   len(depths) if depths is not None else 0,
                                   C.cast(i, C.c_void_p) if i is not None else None,
                                   len(inputs) if inputs is not None else 0, serial, out.data_ptr(),
                                   ws.data_ptr(), ws.numel(), _stream()), "vi_sampled_packet")
    return out.cpu().numpy().view(GREEDY_ROW)


def row_scores(logits: torch.Tensor, next_tokens: torch.Tensor):
    """VeriCache exact row scores -> (greedy int64 [rows], gap f32 [rows]) on the device."""
    dtype, rows, vocab, stride = _rows_view(logits, None)
    nxt = next_tokens.to(device=logits.device, dtype=torch.int64).contiguous()
    greedy = torch.empty(rows, dtype=torch.int64, device=logits.device)
    gap = torch.empty(rows, dtype=torch.float32, device=logits.device)
    nb = _lib().vi_row_scores_workspace_bytes(rows, vocab)
    ws = workspace(("greedy", rows, vocab), nb, logits.device)
    check(_lib().vi_row_scores(logits.data_ptr(), dtype, rows, vocab, stride, nxt.data_ptr(), greedy.data_ptr(),
                               gap.data_ptr(), ws.data_ptr(), ws.numel(), _stream()), "vi_row_scores")
    return greedy, gap


def sampled_scores(scores: torch.Tensor, next_tokens: torch.Tensor, temperature: float, top_k: int, top_p: float,
                   min_p: float, seed: int, first_key: int = 0, tolerance: float = 0.0,
                   presence_penalty: float = 0.0, first_occurrence: torch.Tensor | None = None):
    """VeriCache sampled row scores -> (chosen int64 [rows], gap f32 [rows]) on the device."""
    dtype, rows, vocab, stride = _rows_view(scores, None)
    cfg = DeviceSampling(temperature, top_k, top_p, min_p, seed, presence_penalty, 0,
                         first_occurrence.data_ptr() if first_occurrence is not None else None)
    nxt = next_tokens.to(device=scores.device, dtype=torch.int64).contiguous()
    chosen = torch.empty(rows, dtype=torch.int64, device=scores.device)
    gap = torch.empty(rows, dtype=torch.float32, device=scores.device)
    nb = _lib().vi_sampled_scores_workspace_bytes(rows, vocab)
    ws = workspace(("packet", rows, vocab), nb, scores.device)
    check(_lib().vi_sampled_scores(scores.data_ptr(), dtype, rows, vocab, stride, C.byref(cfg), first_key, tolerance,
                                   nxt.data_ptr(), chosen.data_ptr(), gap.data_ptr(), ws.data_ptr(), ws.numel(),
                                   _stream()), "vi_sampled_scores")
    return chosen, gap


def draft_choice(scores: torch.Tensor, candidates: torch.Tensor, sampling: np.ndarray,
                 seed_tokens: torch.Tensor | None = None, vocabulary: int = 248320) -> torch.Tensor:
    """DFlash2 coupled proposals for every lane: scores f32 [lanes, positions, 16],
    candidates int64 [lanes, positions, 16], sampling DRAFT_SAMPLING [lanes] (its
    first_occurrence field a device address or 0) -> int64 [lanes, positions]."""
    if scores.dim() != 3 or scores.shape[2] != 16 or candidates.shape != scores.shape:
        raise ValueError("scores / candidates must be [lanes, positions, 16]")
    lanes, positions, _ = scores.shape
    dev = scores.device
    sc = scores.to(torch.float32).contiguous()
    cd = candidates.to(device=dev, dtype=torch.int64).contiguous()
    st = None if seed_tokens is None else seed_tokens.to(device=dev, dtype=torch.int64).contiguous()
    smp = to_device_bytes(np.ascontiguousarray(sampling, dtype=_abi.DRAFT_SAMPLING), dev)
    out = torch.empty(lanes, positions, dtype=torch.int64, device=dev)
    check(_lib().vi_draft_choice(lanes, positions, vocabulary, sc.data_ptr(), cd.data_ptr(), _ptr(st),
                                 smp.data_ptr(), out.data_ptr(), _stream()), "vi_draft_choice")
    return out


def selector_chain(anchors: torch.Tensor, candidates: torch.Tensor, unary: torch.Tensor, hidden: torch.Tensor,
                   pred_codebook: torch.Tensor, succ_codebook: torch.Tensor, sampling: np.ndarray | None = None,
                   vocabulary: int | None = None) -> torch.Tensor:
    """Fused selector chain (vi_selector_chain): anchors int64 [lanes], candidates
    int64 / unary f32 [lanes, positions, 16], hidden fp16 [lanes, positions, 256],
    codebooks fp16 [vocabulary, 256], sampling DRAFT_SAMPLING [lanes] or None ->
    proposals int64 [lanes, positions]."""
    if candidates.dim() != 3 or candidates.shape[2] != 16 or unary.shape != candidates.shape:
        raise ValueError("candidates / unary must be [lanes, positions, 16]")
    lanes, positions, _ = candidates.shape
    if hidden.shape != (lanes, positions, 256) or hidden.dtype != torch.float16:
        raise ValueError("hidden must be fp16 [lanes, positions, 256]")
    vocab = pred_codebook.shape[0] if vocabulary is None else vocabulary
    for cb in (pred_codebook, succ_codebook):
        if cb.dtype != torch.float16 or cb.dim() != 2 or cb.shape[1] != 256 or cb.shape[0] < vocab:
            raise ValueError("codebooks must be fp16 [vocabulary, 256]")
    dev = candidates.device
    an = anchors.to(device=dev, dtype=torch.int64).contiguous()
    cd = candidates.to(torch.int64).contiguous()
    un = unary.to(torch.float32).contiguous()
    hd, pc, sc = hidden.contiguous(), pred_codebook.contiguous(), succ_codebook.contiguous()
    smp = None if sampling is None else to_device_bytes(np.ascontiguousarray(sampling, dtype=_abi.DRAFT_SAMPLING), dev)
    out = torch.empty(lanes, positions, dtype=torch.int64, device=dev)
    check(_lib().vi_selector_chain(lanes, positions, vocab, an.data_ptr(), cd.data_ptr(), un.data_ptr(), hd.data_ptr(),
                                   pc.data_ptr(), sc.data_ptr(), _ptr(smp), out.data_ptr(), _stream()),
          "vi_selector_chain")
    return out


class PacketTransport:
    """Pinned readback slots for greedy-packet rows (vi_packet_*)."""

    def __init__(self, slots: int = 2, max_rows: int = 16):
        h = C.c_void_p()
        check(_lib().vi_packet_transport_create(slots, max_rows, C.byref(h)), "vi_packet_transport_create")
        self.handle = h

    def close(self) -> None:
        if self.handle:
            check(_lib().vi_packet_transport_destroy(self.handle), "vi_packet_transport_destroy")
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def submit(self, device_rows: torch.Tensor, rows: int | None = None) -> int:
        """Start the copy of `rows` GREEDY_ROW records (a uint8 device tensor); returns the slot."""
        n = device_rows.numel() // GREEDY_ROW.itemsize if rows is None else rows
        slot = C.c_int(-1)
        check(_lib().vi_packet_submit(self.handle, device_rows.data_ptr(), n, _stream(), C.byref(slot)),
              "vi_packet_submit")
        return slot.value

    def query(self, slot: int) -> bool:
        r = C.c_int(0)
        check(_lib().vi_packet_query(self.handle, slot, C.byref(r)), "vi_packet_query")
        return bool(r.value)

    def finish(self, slot: int, rows: int) -> np.ndarray:
        out = np.zeros(rows, dtype=GREEDY_ROW)
        check(_lib().vi_packet_finish(self.handle, slot, out.ctypes.data, rows), "vi_packet_finish")
        return out


def presence_reset(table: torch.Tensor) -> None:
    check(_lib().vi_presence_reset(table.data_ptr(), table.numel(), _stream()), "vi_presence_reset")


def presence_truncate(table: torch.Tensor, start: int) -> None:
    check(_lib().vi_presence_truncate(table.data_ptr(), table.numel(), start, _stream()), "vi_presence_truncate")


def presence_record(table: torch.Tensor, first: int, tokens: torch.Tensor) -> None:
    check(_lib().vi_presence_record(table.data_ptr(), table.numel(), first, tokens.data_ptr(), tokens.numel(),
                                    _stream()), "vi_presence_record")


def params_array(rows: int, **fields) -> np.ndarray:
    """vi_row_params[rows] with neutral defaults; fields are scalars or arrays."""
    p = np.zeros(rows, dtype=ROW_PARAMS)
    p["temperature"] = 1.0
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    p["lane"] = np.arange(rows)
    for k, v in fields.items():
        p[k] = v
    return p


def to_device_bytes(arr: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).reshape(-1).copy()).to(device)


class SampleOutputs:
    def __init__(self, tokens, uniforms, probs, stats):
        self.tokens, self.uniforms, self.probs, self.stats = tokens, uniforms, probs, stats


def route_mask(params: np.ndarray) -> int:
    """Kernels a batch needs: top-k route (T == 0 or 1 <= top_k <= 64) / full route."""
    topk = (params["temperature"] <= 0) | ((params["top_k"] >= 1) & (params["top_k"] <= 64))
    return (_abi.ROUTE_TOPK if topk.any() else 0) | (_abi.ROUTE_FULL if (~topk).any() else 0)


def sample_rows(logits: torch.Tensor, params: np.ndarray | torch.Tensor,
                histories: torch.Tensor | None = None, offsets: torch.Tensor | None = None,
                max_history: int = 0, want_probs: bool = False, want_stats: bool = True,
                want_uniforms: bool = True, outputs: SampleOutputs | None = None,
                routes: int | None = None) -> SampleOutputs:
    """Batched sampler.  params: vi_row_params array (host numpy or device uint8);
    with device params pass `routes` (default: run both kernel routes)."""
    dtype, rows, vocab, stride = _rows_view(logits, None)
    dev = logits.device
    if routes is None:
        routes = _abi.ROUTE_ALL if isinstance(params, torch.Tensor) else route_mask(params)
    p_dev = params if isinstance(params, torch.Tensor) else to_device_bytes(params, dev)
    if histories is not None:
        if histories.dtype != torch.int32 or offsets is None or offsets.dtype != torch.int64:
            raise ValueError("histories must be int32 with int64 offsets[rows + 1]")
        if max_history <= 0:
            raise ValueError("max_history must bound the longest history")
    o = outputs
    if o is None:
        o = SampleOutputs(
            torch.empty(rows, dtype=torch.int32, device=dev),
            torch.empty(rows, dtype=torch.float64, device=dev) if want_uniforms else None,
            torch.empty(rows, vocab, dtype=torch.float32, device=dev) if want_probs else None,
            torch.empty(rows * SAMPLE_STATS.itemsize, dtype=torch.uint8, device=dev) if want_stats else None)
    nb = _lib().vi_sample_workspace_bytes(rows, vocab, max_history)
    ws = workspace(("sample", rows, vocab, max_history), nb, dev)
    check(_lib().vi_sample_rows(logits.data_ptr(), dtype, rows, vocab, stride, p_dev.data_ptr(),
                                _ptr(histories), _ptr(offsets), max_history, o.tokens.data_ptr(),
                                _ptr(o.uniforms), _ptr(o.probs), vocab, _ptr(o.stats), routes, ws.data_ptr(),
                                ws.numel(), _stream()), "vi_sample_rows")
    return o


class PenaltyState:
    """Per-lane occurrence counts on the device (vi_penalty_state_*): lane l's
    state is bytes [l * lane_bytes, (l + 1) * lane_bytes) of one uint8 tensor."""

    def __init__(self, lanes: int, vocabulary: int, slots: int = 65536, device="cuda"):
        self.lanes, self.vocabulary, self.slots = lanes, vocabulary, slots
        self.lane_bytes = _lib().vi_penalty_state_bytes(vocabulary, slots)
        if self.lane_bytes == 0:
            raise ValueError("slots must be a power of two >= 64")
        self.buf = torch.empty(lanes * self.lane_bytes, dtype=torch.uint8, device=device)
        self.reset()

    def reset(self) -> None:
        check(_lib().vi_penalty_state_reset(self.buf.data_ptr(), self.lanes, self.vocabulary, self.slots,
                                            _stream()), "vi_penalty_state_reset")

    def update(self, tokens: torch.Tensor, offsets: torch.Tensor | None = None, sign: int = 1) -> None:
        """Record (sign +1) or remove (-1) tokens[offsets[l]:offsets[l+1]] per lane,
        or tokens[l] per lane without offsets (negative tokens skipped)."""
        if tokens.dtype != torch.int32 or (offsets is not None and offsets.dtype != torch.int64):
            raise ValueError("tokens must be int32 (offsets int64)")
        check(_lib().vi_penalty_state_update(self.buf.data_ptr(), self.lanes, self.vocabulary, self.slots,
                                             tokens.data_ptr(), _ptr(offsets), sign, _stream()),
              "vi_penalty_state_update")

    def header(self) -> np.ndarray:
        """(flags, keys, total) per lane."""
        h = self.buf.view(self.lanes, self.lane_bytes)[:, :16].cpu().numpy()
        return np.stack([h[:, 0:4].copy().view(np.uint32)[:, 0], h[:, 4:8].copy().view(np.uint32)[:, 0],
                         h[:, 8:16].copy().view(np.uint64)[:, 0].astype(np.int64)], axis=1)


def sample_rows_state(logits: torch.Tensor, params: np.ndarray | torch.Tensor, state: PenaltyState,
                      record: bool = False, want_probs: bool = False, want_stats: bool = True,
                      want_uniforms: bool = True, outputs: SampleOutputs | None = None,
                      routes: int | None = None) -> SampleOutputs:
    """The batched sampler with penalties from `state` (row r uses lane r); with
    `record`, each row's sampled token is also recorded in its lane's state."""
    dtype, rows, vocab, stride = _rows_view(logits, None)
    if rows > state.lanes or vocab != state.vocabulary:
        raise ValueError("penalty state has too few lanes or another vocabulary")
    dev = logits.device
    if routes is None:
        routes = _abi.ROUTE_ALL if isinstance(params, torch.Tensor) else route_mask(params)
    p_dev = params if isinstance(params, torch.Tensor) else to_device_bytes(params, dev)
    o = outputs
    if o is None:
        o = SampleOutputs(
            torch.empty(rows, dtype=torch.int32, device=dev),
            torch.empty(rows, dtype=torch.float64, device=dev) if want_uniforms else None,
            torch.empty(rows, vocab, dtype=torch.float32, device=dev) if want_probs else None,
            torch.empty(rows * SAMPLE_STATS.itemsize, dtype=torch.uint8, device=dev) if want_stats else None)
    nb = _lib().vi_sample_workspace_bytes(rows, vocab, 0)
    ws = workspace(("sample", rows, vocab, 0), nb, dev)
    check(_lib().vi_sample_rows_state(logits.data_ptr(), dtype, rows, vocab, stride, p_dev.data_ptr(),
                                      state.buf.data_ptr(), state.slots, int(record), o.tokens.data_ptr(),
                                      _ptr(o.uniforms),
                                      _ptr(o.probs), vocab, _ptr(o.stats), routes, ws.data_ptr(), ws.numel(),
                                      _stream()), "vi_sample_rows_state")
    return o


def stats_numpy(stats: torch.Tensor) -> np.ndarray:
    return stats.cpu().numpy().view(SAMPLE_STATS)


def verify_rows(mode: int, target: torch.Tensor, drafted: torch.Tensor, lanes: int, drafts: int,
                draft: torch.Tensor | None = None, params: np.ndarray | None = None,
                terminal: Sequence[int] | None = None):
    """Per-lane acceptance.  Returns (accepted[lanes], committed[lanes, drafts+1],
    committed_count[lanes], lane_flags[lanes]) as numpy arrays."""
    tdt, trows_total, vocab, tstride = _rows_view(target, None)
    if trows_total % lanes:
        raise ValueError("target rows must be lanes x target_rows")
    trows = trows_total // lanes
    dev = target.device
    ddt, dstride, dptr = 0, 0, None
    if draft is not None:
        ddt, drows_total, dvocab, dstride = _rows_view(draft, None)
        if dvocab != vocab or drows_total != lanes * drafts:
            raise ValueError("draft must be [lanes * drafts, vocabulary]")
        dptr = draft.data_ptr()
    p_dev = to_device_bytes(params, dev) if params is not None else None
    if mode == _abi.VERIFY_SAMPLED and params is not None:
        sampled = params["temperature"] > 0
        k = params["top_k"]
        if not np.any(sampled & ((k < 1) | (k > 64))):   # every sampled lane has a top-k list
            mode = _abi.VERIFY_SAMPLED_TOPK
    term = torch.tensor(list(terminal), dtype=torch.int64, device=dev) if terminal else None
    acc = torch.empty(lanes, dtype=torch.int32, device=dev)
    com = torch.empty(lanes, drafts + 1, dtype=torch.int32, device=dev)
    cnt = torch.empty(lanes, dtype=torch.int32, device=dev)
    flg = torch.empty(lanes, dtype=torch.int32, device=dev)
    nb = _lib().vi_verify_workspace_bytes(lanes, drafts, vocab)
    ws = workspace(("verify", lanes, drafts, vocab), nb, dev)
    check(_lib().vi_verify_rows(mode, target.data_ptr(), tdt, tstride, trows, dptr, ddt, dstride, lanes, drafts,
                                vocab, drafted.data_ptr(), _ptr(p_dev), _ptr(term), len(terminal or ()),
                                acc.data_ptr(), com.data_ptr(), cnt.data_ptr(), flg.data_ptr(), ws.data_ptr(),
                                ws.numel(), _stream()), "vi_verify_rows")
    return acc.cpu().numpy(), com.cpu().numpy(), cnt.cpu().numpy(), flg.cpu().numpy().view(np.uint32)


def probe_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    check(_lib().vi_probe_read(buf.data_ptr(), buf.numel() * buf.element_size(), sink.data_ptr(), _stream()),
          "vi_probe_read")


def probe_copy(dst: torch.Tensor, src: torch.Tensor) -> None:
    check(_lib().vi_probe_copy(dst.data_ptr(), src.data_ptr(), src.numel() * src.element_size(), _stream()),
          "vi_probe_copy")


def verification_tree(drafts: Sequence[int], candidate_ids, candidate_unary, budget: int, max_siblings: int,
                      row_cost: float = 0.0141):
    """DFlash2 verification tree from the draft's top-16 (host arrays): chain
    length, sibling tokens and their offsets (depths).  candidate_ids /
    candidate_unary: [depth, 16] in unary order (vi_topk_rows' output)."""
    d = np.ascontiguousarray(drafts, dtype=np.int64)
    ids = np.ascontiguousarray(candidate_ids, dtype=np.int64).reshape(-1)
    un = np.ascontiguousarray(candidate_unary, dtype=np.float32).reshape(-1)
    if ids.size < 16 * d.size or un.size < 16 * d.size:
        raise ValueError("candidate arrays must be [depth, 16]")
    cap = max(1, int(budget))
    toks = np.zeros(cap, dtype=np.int64)
    offs = np.zeros(cap, dtype=np.int32)
    chain, n = np.zeros(1, dtype=np.int32), np.zeros(1, dtype=np.int32)
    vp = lambda a: a.ctypes.data_as(C.c_void_p)  # noqa: E731
    check(_lib().vi_build_verification_tree(vp(d), d.size, vp(ids), vp(un), int(budget), int(max_siblings),
                                            C.c_float(row_cost), vp(chain), vp(toks), vp(offs), vp(n)),
          "vi_build_verification_tree")
    return int(chain[0]), [int(t) for t in toks[: n[0]]], [int(o) for o in offs[: n[0]]]


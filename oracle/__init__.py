"""Python view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py import this module as the checker.  The product
package (voidinfer_amd) never imports it.  All arrays are numpy; logits are
passed as raw 16-bit patterns (bf16 / fp16) or float32.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_LIB_PATH = HERE / "_ref" / "libvoidinfer_ref.so"
REF_DIFF_PATH = HERE / "_ref" / "ref_diff"

BF16, F16, F32 = 0, 1, 2

GREEDY_ROW = np.dtype([("serial", "<u8"), ("token", "<i4"), ("nonfinite", "<u4")])
ROW_PARAMS = np.dtype([
    ("temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"),
    ("repetition_penalty", "<f4"), ("presence_penalty", "<f4"), ("frequency_penalty", "<f4"),
    ("top_k", "<i4"), ("lane", "<u4"), ("seed", "<u8"), ("position", "<i4"), ("reserved", "<u4"),
])
SAMPLE_STATS = np.dtype([
    ("flags", "<u4"), ("support", "<u4"), ("finite", "<u4"), ("reserved", "<u4"),
    ("support_mass", "<f8"), ("uniform", "<f8"),
])
PACKET_DETAIL = np.dtype([
    ("cap", "<i4"), ("support", "<i4"), ("selected", "<i4"), ("key", "<i4"),
    ("cand_val", "<f4", 20), ("cand_idx", "<i4", 20), ("value", "<f4", 20), ("prob", "<f4", 20),
    ("sum", "<f4"),
])


class DeviceSampling(C.Structure):
    _fields_ = [
        ("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
        ("seed", C.c_uint64), ("presence_penalty", C.c_float), ("reserved", C.c_int32),
        ("first_occurrence", C.c_void_p),
    ]


class AcceptOutcome(C.Structure):
    _fields_ = [("accepted", C.c_int32), ("correction_draw_used", C.c_int32), ("token", C.c_uint32),
                ("reserved", C.c_uint32), ("acceptance_probability", C.c_double)]


_lib = None


def build() -> Path:
    """Compile the oracle (g++) from oracle/oracle.cpp."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    return LIB_PATH


def build_ref() -> Path | None:
    """Compile oracle/_ref from the reference's host headers when they are mounted."""
    ref = Path(os.environ.get("VOIDINFER_REFERENCE", "/root/reference"))
    if not (ref / "src" / "exl3" / "sampling_policy.h").exists():
        return None
    subprocess.run(["make", "-s", "-C", str(HERE), "ref", "diff", f"REF={ref}"], check=True)
    return REF_LIB_PATH


def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo), for baseline records."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


_native = None


def native_lib() -> tuple[C.CDLL, str]:
    """The oracle compiled for this host's CPU (g++ -O3 -march=native into a
    temporary directory) for CPU-baseline timing, with the flags used; falls back
    to the portable build (-march=x86-64-v2) when no compiler is available."""
    global _native
    if _native is None:
        import tempfile
        out = Path(tempfile.gettempdir()) / f"voidinfer_oracle_native_{os.getuid()}.so"
        flags = ["-std=c++20", "-O3", "-march=native", "-fPIC", "-ffp-contract=off", "-fno-fast-math"]
        try:
            subprocess.run(["g++", *flags, "-shared", "-o", str(out), str(HERE / "oracle.cpp"), "-lpthread"],
                           check=True, capture_output=True, timeout=300)
            _native = (_load(out), " ".join(["g++", *flags]))
        except (OSError, subprocess.SubprocessError):
            _native = (lib(), "prebuilt oracle/liboracle.so (-O3 -march=x86-64-v2)")
    return _native


def use_native() -> str:
    """Route every wrapper below through native_lib() (same IEEE semantics:
    -ffp-contract=off, no fast math); returns the build flags."""
    global _lib
    L, flags = native_lib()
    _lib = L
    return flags


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = _load(LIB_PATH)
    return _lib


def _load(path) -> C.CDLL:
    if True:
        L = C.CDLL(str(path))
        vp, i, i64, u32, u64, d = C.c_void_p, C.c_int, C.c_int64, C.c_uint32, C.c_uint64, C.c_double
        sig = {
            "or_decode": ([i, u32], C.c_float),
            "or_round_to_dtype": ([i, C.c_float], u32),
            "or_order_key": ([C.c_float], u32),
            "or_splitmix64": ([u64], u64),
            "or_gumbel": ([u64, C.c_int32, C.c_int32], C.c_float),
            "or_philox4x32_10": ([vp, vp, vp], None),
            "or_uniform": ([u64, u32, C.c_int32, u32], d),
            "or_greedy_rows": ([vp, i, i, i, i64, u64, vp], i),
            "or_cpu_greedy": ([vp, i64], i64),
            "or_topk_rows": ([vp, i, i, i, i64, i, vp, vp, vp, vp], i),
            "or_sampled_packet": ([vp, i, i, i, i64, C.POINTER(DeviceSampling), i, vp, i, vp, i, u64, vp, vp], i),
            "or_sampled_scores": ([vp, i, i, i, i64, C.POINTER(DeviceSampling), i, C.c_float, vp, vp, vp], i),
            "or_row_scores": ([vp, i, i, i, i64, vp, vp, vp], i),
            "or_draft_choice": ([i, i, i, vp, vp, vp, vp, vp], i),
            "or_selector_chain": ([i, i, i, vp, vp, vp, vp, vp, vp, vp, vp], i),
            "or_sample_rows": ([vp, i, i, i, i64, vp, vp, vp, vp, vp, vp, i64, vp, vp, i], i),
            "or_accept": ([vp, vp, i64, u32, d, d, C.POINTER(AcceptOutcome), vp], i),
            "or_outer_prefix": ([vp, vp, i, vp, i, vp, vp, vp, vp, vp], i),
            "or_verify_rows": ([i, vp, i, i64, i, vp, i, i64, i, i, i, vp, vp, vp, i, vp, vp, vp, vp, vp, i], i),
            "or_row_distribution": ([vp, i, i, vp, vp, vp], i),
            "or_build_verification_tree": ([vp, i, vp, vp, i, i, C.c_float, vp, vp, vp, vp], i),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
    return L


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _dtype_of(bits: np.ndarray) -> int:
    if bits.dtype == np.float32:
        return F32
    raise ValueError("pass dtype explicitly for 16-bit patterns")


def decode(dtype: int, bits: int) -> float:
    return lib().or_decode(dtype, bits)


def round_to_dtype(dtype: int, value: float) -> int:
    return lib().or_round_to_dtype(dtype, value)


def splitmix64(x: int) -> int:
    return lib().or_splitmix64(x)


def gumbel(seed: int, key: int, token: int) -> float:
    return lib().or_gumbel(seed, key, token)


def philox(counter, key) -> np.ndarray:
    c = np.asarray(counter, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().or_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def uniform(seed: int, lane: int, position: int, purpose: int) -> float:
    return lib().or_uniform(seed, lane, position, purpose)


def greedy_rows(logits: np.ndarray, dtype: int, vocabulary: int | None = None, serial: int = 1) -> np.ndarray:
    rows, width = logits.shape
    v = width if vocabulary is None else vocabulary
    out = np.zeros(rows, dtype=GREEDY_ROW)
    lib().or_greedy_rows(_p(np.ascontiguousarray(logits)), dtype, rows, v, width, serial, _p(out))
    return out


def cpu_greedy(logits_f32: np.ndarray) -> int:
    x = np.ascontiguousarray(logits_f32, dtype=np.float32)
    return int(lib().or_cpu_greedy(_p(x), x.size))


def topk_rows(logits: np.ndarray, dtype: int, k: int, vocabulary: int | None = None, threads: int = 1):
    """Rows split over `threads` host threads (ctypes releases the GIL)."""
    rows, width = logits.shape
    v = width if vocabulary is None else vocabulary
    x = np.ascontiguousarray(logits)
    ids = np.zeros((rows, k), dtype=np.int64)
    vals = np.zeros((rows, k), dtype=np.float32)
    lp = np.zeros((rows, k), dtype=np.float32)
    nf = np.zeros(max(1, rows), dtype=np.uint32)

    def part(lo: int, hi: int) -> int:
        return lib().or_topk_rows(_p(x[lo:hi]), dtype, hi - lo, v, width, k, _p(ids[lo:hi]), _p(vals[lo:hi]),
                                  _p(lp[lo:hi]), _p(nf[lo:]))
    t = max(1, min(threads, rows))
    if t == 1:
        sts = [part(0, rows)]
    else:
        from concurrent.futures import ThreadPoolExecutor
        cuts = [rows * i // t for i in range(t + 1)]
        with ThreadPoolExecutor(t) as ex:
            sts = list(ex.map(lambda i: part(cuts[i], cuts[i + 1]), range(t)))
    if any(sts):
        raise ValueError("oracle top-k: invalid arguments")
    return ids, vals, lp, int(nf.max())


def sampled_packet(scores: np.ndarray, dtype: int, temperature: float, top_k: int, top_p: float, min_p: float,
                   seed: int, presence_penalty: float = 0.0, first_occurrence: np.ndarray | None = None,
                   first_key: int = 0, depths=None, inputs=None, serial: int = 1):
    rows, width = scores.shape
    fo = None if first_occurrence is None else np.ascontiguousarray(first_occurrence, dtype=np.int32)
    cfg = DeviceSampling(temperature, top_k, top_p, min_p, seed, presence_penalty, 0,
                         fo.ctypes.data if fo is not None else None)
    d = None if depths is None else np.asarray(depths, dtype=np.int32)
    i = None if inputs is None else np.asarray(inputs, dtype=np.int32)
    out = np.zeros(rows, dtype=GREEDY_ROW)
    detail = np.zeros(rows, dtype=PACKET_DETAIL)
    st = lib().or_sampled_packet(_p(np.ascontiguousarray(scores)), dtype, rows, width, width, C.byref(cfg),
                                 first_key, _p(d), 0 if d is None else d.size, _p(i), 0 if i is None else i.size,
                                 serial, _p(out), _p(detail))
    if st:
        raise ValueError("oracle packet: invalid arguments")
    return out, detail


def sampled_scores(scores: np.ndarray, dtype: int, temperature: float, top_k: int, top_p: float, min_p: float,
                   seed: int, next_tokens, first_key: int = 0, tolerance: float = 0.0, presence_penalty: float = 0.0,
                   first_occurrence: np.ndarray | None = None):
    """VeriCache sampled row scores: (chosen int64[rows], gap float32[rows])."""
    rows, width = scores.shape
    fo = None if first_occurrence is None else np.ascontiguousarray(first_occurrence, dtype=np.int32)
    cfg = DeviceSampling(temperature, top_k, top_p, min_p, seed, presence_penalty, 0,
                         fo.ctypes.data if fo is not None else None)
    nxt = np.ascontiguousarray(next_tokens, dtype=np.int64)
    chosen = np.zeros(rows, dtype=np.int64)
    gap = np.zeros(rows, dtype=np.float32)
    st = lib().or_sampled_scores(_p(np.ascontiguousarray(scores)), dtype, rows, width, width, C.byref(cfg),
                                 first_key, tolerance, _p(nxt), _p(chosen), _p(gap))
    if st:
        raise ValueError("oracle sampled scores: invalid arguments")
    return chosen, gap


DRAFT_SAMPLING = np.dtype([
    ("inv_temperature", "<f4"), ("top_p", "<f4"), ("min_p", "<f4"), ("top_k", "<i4"), ("seed", "<u8"),
    ("key_base", "<i4"), ("reserved", "<i4"), ("presence_penalty", "<f4"), ("reserved2", "<i4"),
    ("first_occurrence", "<u8"),
])


def draft_choice(scores: np.ndarray, candidates: np.ndarray, sampling: np.ndarray, seed_tokens=None,
                 vocabulary: int = 248320) -> np.ndarray:
    """DFlash2 coupled proposals: scores f32 [lanes, positions, 16], candidates int64
    [lanes, positions, 16], sampling DRAFT_SAMPLING [lanes] (first_occurrence = host
    address or 0) -> proposals int64 [lanes, positions]."""
    lanes, positions, _ = scores.shape
    sc = np.ascontiguousarray(scores, dtype=np.float32)
    cd = np.ascontiguousarray(candidates, dtype=np.int64)
    st = None if seed_tokens is None else np.ascontiguousarray(seed_tokens, dtype=np.int64)
    smp = np.ascontiguousarray(sampling, dtype=DRAFT_SAMPLING)
    out = np.zeros((lanes, positions), dtype=np.int64)
    if lib().or_draft_choice(lanes, positions, vocabulary, _p(sc), _p(cd), _p(st), _p(smp), _p(out)):
        raise ValueError("oracle draft choice: invalid arguments")
    return out


def selector_chain(anchors, candidates, unary, hidden, pred_codebook, succ_codebook, sampling=None,
                   vocabulary: int | None = None) -> np.ndarray:
    """Fused selector chain: anchors int64 [lanes], candidates int64 / unary f32
    [lanes, positions, 16], hidden fp16 bits [lanes, positions, 256], codebooks fp16
    bits [vocabulary, 256], sampling DRAFT_SAMPLING [lanes] or None -> int64
    [lanes, positions]."""
    lanes, positions, _ = candidates.shape
    vocabulary = pred_codebook.shape[0] if vocabulary is None else vocabulary
    an = np.ascontiguousarray(anchors, dtype=np.int64)
    cd = np.ascontiguousarray(candidates, dtype=np.int64)
    un = np.ascontiguousarray(unary, dtype=np.float32)
    hd = np.ascontiguousarray(hidden, dtype=np.uint16)
    pc = np.ascontiguousarray(pred_codebook, dtype=np.uint16)
    sc = np.ascontiguousarray(succ_codebook, dtype=np.uint16)
    smp = None if sampling is None else np.ascontiguousarray(sampling, dtype=DRAFT_SAMPLING)
    out = np.zeros((lanes, positions), dtype=np.int64)
    if lib().or_selector_chain(lanes, positions, vocabulary, _p(an), _p(cd), _p(un), _p(hd), _p(pc), _p(sc),
                               _p(smp), _p(out)):
        raise ValueError("oracle selector chain: invalid arguments")
    return out


def row_scores(logits: np.ndarray, dtype: int, next_tokens):
    """VeriCache exact row scores: (greedy int64[rows], gap float32[rows])."""
    rows, width = logits.shape
    nxt = np.ascontiguousarray(next_tokens, dtype=np.int64)
    greedy = np.zeros(rows, dtype=np.int64)
    gap = np.zeros(rows, dtype=np.float32)
    st = lib().or_row_scores(_p(np.ascontiguousarray(logits)), dtype, rows, width, width, _p(nxt), _p(greedy),
                             _p(gap))
    if st:
        raise ValueError("oracle row scores: invalid arguments")
    return greedy, gap


def sample_rows(logits: np.ndarray, dtype: int, params: np.ndarray, histories: np.ndarray | None = None,
                offsets: np.ndarray | None = None, want_probs: bool = False, threads: int = 0):
    rows, width = logits.shape
    toks = np.zeros(rows, dtype=np.int32)
    u = np.zeros(rows, dtype=np.float64)
    probs = np.zeros((rows, width), dtype=np.float32) if want_probs else None
    stats = np.zeros(rows, dtype=SAMPLE_STATS)
    margins = np.zeros((rows, 4), dtype=np.float64)
    h = None if histories is None else np.ascontiguousarray(histories, dtype=np.int32)
    o = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64)
    st = lib().or_sample_rows(_p(np.ascontiguousarray(logits)), dtype, rows, width, width,
                              _p(np.ascontiguousarray(params)), _p(h), _p(o), _p(toks), _p(u), _p(probs), width,
                              _p(stats), _p(margins), threads)
    if st:
        raise ValueError("oracle sampler: invalid arguments")
    return toks, u, probs, stats, margins


def row_distribution(row: np.ndarray, dtype: int, params_row: np.ndarray) -> tuple[np.ndarray, int]:
    width = row.shape[-1]
    p = np.zeros(width, dtype=np.float64)
    sup = np.zeros(1, dtype=np.uint32)
    prm = np.ascontiguousarray(np.asarray(params_row, dtype=ROW_PARAMS).reshape(1))
    lib().or_row_distribution(_p(np.ascontiguousarray(row)), dtype, width, _p(prm), _p(p), _p(sup))
    return p, int(sup[0])


def accept(p: np.ndarray, q: np.ndarray, token: int, ua: float, uc: float):
    """Returns (status, outcome dict, residual)."""
    p = np.ascontiguousarray(p, dtype=np.float64)
    q = np.ascontiguousarray(q, dtype=np.float64)
    out = AcceptOutcome()
    res = np.zeros(p.size, dtype=np.float64)
    st = lib().or_accept(_p(p), _p(q), p.size, token, ua, uc, C.byref(out), _p(res))
    return st, {"accepted": bool(out.accepted), "correction_draw_used": bool(out.correction_draw_used),
                "token": int(out.token), "acceptance_probability": out.acceptance_probability}, res


def outer_prefix(target_path, tentative, terminal=()):
    t = np.asarray(target_path, dtype=np.int64)
    s = np.asarray(tentative, dtype=np.int64)
    term = np.asarray(terminal, dtype=np.int64) if len(terminal) else None
    com = np.zeros(max(1, t.size), dtype=np.int64)
    n, a, r, st = (np.zeros(1, dtype=np.int32) for _ in range(4))
    status = lib().or_outer_prefix(_p(t), _p(s), t.size if t.size == s.size else -1, _p(term),
                                   0 if term is None else term.size, _p(com), _p(n), _p(a), _p(r), _p(st))
    if status:
        raise ValueError("outer decision extent")
    return list(com[: n[0]]), int(a[0]), bool(r[0]), bool(st[0])


def verify_rows(mode: int, target: np.ndarray, tdtype: int, draft: np.ndarray | None, ddtype: int, lanes: int,
                drafts: int, drafted: np.ndarray, params: np.ndarray | None, terminal=(), threads: int = 0):
    trows_total, width = target.shape
    trows = trows_total // lanes
    acc = np.zeros(lanes, dtype=np.int32)
    com = np.zeros((lanes, drafts + 1), dtype=np.int32)
    cnt = np.zeros(lanes, dtype=np.int32)
    flg = np.zeros(lanes, dtype=np.uint32)
    margins = np.zeros((lanes, drafts), dtype=np.float64)
    term = np.asarray(terminal, dtype=np.int64) if len(terminal) else None
    dr = np.ascontiguousarray(drafted, dtype=np.int32)
    st = lib().or_verify_rows(mode, _p(np.ascontiguousarray(target)), tdtype, width, trows,
                              _p(None if draft is None else np.ascontiguousarray(draft)), ddtype,
                              width if draft is not None else 0, lanes, drafts, width, _p(dr),
                              _p(None if params is None else np.ascontiguousarray(params)), _p(term),
                              0 if term is None else term.size, _p(acc), _p(com), _p(cnt), _p(flg), _p(margins),
                              threads)
    if st:
        raise ValueError("oracle verify: invalid arguments")
    return acc, com, cnt, flg, margins


def _tree_call(fn, drafts, candidate_ids, candidate_unary, budget: int, max_siblings: int, row_cost: float):
    d = np.ascontiguousarray(drafts, dtype=np.int64)
    ids = np.ascontiguousarray(candidate_ids, dtype=np.int64).reshape(-1)
    un = np.ascontiguousarray(candidate_unary, dtype=np.float32).reshape(-1)
    if ids.size < 16 * d.size or un.size < 16 * d.size:
        raise ValueError("verification tree candidate extent")
    cap = max(1, budget)
    toks = np.zeros(cap, dtype=np.int64)
    offs = np.zeros(cap, dtype=np.int32)
    chain, n = np.zeros(1, dtype=np.int32), np.zeros(1, dtype=np.int32)
    st = fn(_p(d), d.size, _p(ids), _p(un), budget, max_siblings, C.c_float(row_cost), _p(chain), _p(toks),
            _p(offs), _p(n))
    if st:
        raise ValueError(f"verification tree status {st}")
    return int(chain[0]), [int(t) for t in toks[: n[0]]], [int(o) for o in offs[: n[0]]]


ROW_COST = 0.0141   # kExl3TreeRowCost (verification_tree.h:33)


def build_verification_tree(drafts, candidate_ids, candidate_unary, budget: int, max_siblings: int,
                            row_cost: float = ROW_COST):
    """(chain_drafts, sibling_tokens, sibling_offsets) of the DFlash2 verification
    tree (verification_tree.h:44-112)."""
    return _tree_call(lib().or_build_verification_tree, drafts, candidate_ids, candidate_unary, budget,
                      max_siblings, row_cost)


def ref_build_verification_tree(drafts, candidate_ids, candidate_unary, budget: int, max_siblings: int,
                                row_cost: float = ROW_COST):
    """The same through the reference's own header compiled into oracle/_ref
    (None when that library is not built)."""
    if not REF_LIB_PATH.exists():
        return None
    ref = C.CDLL(str(REF_LIB_PATH))
    fn = ref.ref_build_verification_tree
    vp, i = C.c_void_p, C.c_int
    fn.argtypes = [vp, i, vp, vp, i, i, C.c_float, vp, vp, vp, vp]
    fn.restype = i
    return _tree_call(fn, drafts, candidate_ids, candidate_unary, budget, max_siblings, row_cost)


"""CPU checks of the C-ABI boundary: the built library loads, exports every
entry point include/voidinfer_sampling.h declares, the Python binding table
covers them, and the host-only entry points (version, status strings,
workspace sizing) answer without a GPU."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "voidinfer_sampling.h"
LIB = ROOT / "voidinfer_amd" / "libvoidinfer_sampling.so"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(vi_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.skip("library not built (run python voidinfer_amd/build.py)")
    return C.CDLL(str(LIB))


def test_header_declares_the_entry_points():
    names = declared()
    for must in ("vi_init", "vi_greedy_rows", "vi_topk_rows", "vi_sampled_packet", "vi_sample_rows",
                 "vi_verify_rows", "vi_row_scores", "vi_sampled_scores", "vi_presence_record", "vi_probe_read"):
        assert must in names
    assert len(names) >= 22


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing
    for n in declared():
        getattr(lib, n)


def test_binding_table_covers_the_header():
    from voidinfer_amd import _abi
    assert sorted(_abi.SIGNATURES) == declared()


def test_host_only_entry_points(lib):
    lib.vi_abi_version.restype = C.c_uint32
    assert lib.vi_abi_version() == 1
    lib.vi_status_string.restype = C.c_char_p
    lib.vi_status_string.argtypes = [C.c_int]
    assert lib.vi_status_string(0) == b"ok" and b"invalid" in lib.vi_status_string(1)
    for name, args in [("vi_greedy_workspace_bytes", (128, 248320)), ("vi_topk_workspace_bytes", (128, 248320, 8)),
                       ("vi_sampled_packet_workspace_bytes", (16, 248320)),
                       ("vi_row_scores_workspace_bytes", (32, 248320)),
                       ("vi_sampled_scores_workspace_bytes", (32, 248320)),
                       ("vi_verify_workspace_bytes", (128, 16, 248320))]:
        fn = getattr(lib, name)
        fn.restype = C.c_size_t
        fn.argtypes = [C.c_int] * len(args)
        assert fn(*args) > 0, name
        assert fn(*((0,) + args[1:])) == 0, name
    fn = lib.vi_sample_workspace_bytes
    fn.restype = C.c_size_t
    fn.argtypes = [C.c_int, C.c_int, C.c_int64]
    # full route at the headline shape: barriers, summaries, lists, dense penalised logits
    assert fn(128, 248320, 32768) >= 128 * 2 * 65536 * 4 + 128 * 2 * 32768 * 2
    assert fn(128, 248320, -1) == 0

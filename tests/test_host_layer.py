"""CPU tests of the C++20 host layer (include/voidinfer_sampling.hpp).

* tests/cpp/test_host_contracts.cpp — the reference's own contract scenarios
  (tests/test_exl3_sampling_policy.cpp and its siblings) against this layer;
* tests/cpp/test_transport_host.cpp — the greedy-packet transport classes over
  a host stand-in of the vi_packet_* entry points;
* tests/cpp/test_markstein.cpp — the samplers' FMA-corrected division of a
  penalized logit by the repetition penalty, bit for bit against IEEE division;
* oracle/_ref/ref_diff — random scripts run side by side through this layer and
  the reference's host headers compiled from /root/reference (skipped where the
  reference tree is absent and the binary was not built).
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BUILD = ROOT / "_build"


def _compile(src: Path, out: Path) -> Path:
    gxx = shutil.which("g++") or "g++"
    BUILD.mkdir(exist_ok=True)
    cmd = [gxx, "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror", "-I", str(ROOT / "include"), str(src),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return out


def test_markstein_division_matches_ieee():
    gxx = shutil.which("g++") or "g++"
    BUILD.mkdir(exist_ok=True)
    exe = BUILD / "test_markstein"
    cmd = [gxx, "-std=c++20", "-O2", "-ffp-contract=off", "-Wall", "-Werror", str(ROOT / "tests/cpp/test_markstein.cpp"),
           "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 mismatches" in res.stdout


def test_host_contracts_program():
    exe = _compile(ROOT / "tests" / "cpp" / "test_host_contracts.cpp", BUILD / "test_host_contracts")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "host contracts PASS" in res.stdout


def test_transport_host_layer():
    """Exl3GreedyPacketTransport over a host stand-in of the vi_packet_* entry points."""
    exe = _compile(ROOT / "tests" / "cpp" / "test_transport_host.cpp", BUILD / "test_transport_host")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "transport host layer PASS" in res.stdout


def test_host_layer_matches_reference_headers():
    import oracle
    ref = Path(os.environ.get("VOIDINFER_REFERENCE", "/root/reference"))
    if (ref / "src" / "exl3" / "sampling_policy.h").exists():
        oracle.build_ref()
    if not oracle.REF_DIFF_PATH.exists():
        pytest.skip("oracle/_ref/ref_diff not built (reference tree absent)")
    res = subprocess.run([str(oracle.REF_DIFF_PATH), "20000"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches=0" in res.stdout

"""Source-level drop-in proof: compiled C and C++ callers of include/ix_gdn.h linked with
-lixgdn (tests/dropin/).

The C caller uses the header's C mode (no default stream argument); the C++ caller makes the
reference acceptance test's five launcher calls as tests/test_gdn.cu:28, :39, :46, :51, :55
make them, with the stream defaulted; the projection caller makes the GEMV calls of
tests/test_bf16_gemv.cu:27-38 and the namespaced ix_mmvq::ix_mmvq_q8_0 call of
tests/test_mmvq_wave.cu:46. Without a GPU the programs are built here and run their
validation checks, which the library answers before any launch; on a GPU the C++ callers
run the reference tests' shapes and tolerances against double references.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "tests", "dropin")
BIN = os.path.join(DROPIN, "_build")


def _run(args, timeout=120):
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    return r


def test_callers_build_and_validate():
    r = subprocess.run(["make", "-s", "-C", DROPIN], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    r = _run([os.path.join(BIN, "dropin_c")])
    assert r.returncode == 0 and "C caller: PASS" in r.stdout, r.stdout + r.stderr
    r = _run([os.path.join(BIN, "dropin_cxx"), "--validate"])
    assert r.returncode == 0 and "PASS" in r.stdout, r.stdout + r.stderr
    r = _run([os.path.join(BIN, "dropin_proj"), "--validate"])
    assert r.returncode == 0 and "PASS" in r.stdout and "ix_mmvq::ix_mmvq_q8_0" in r.stdout, r.stdout + r.stderr


@pytest.mark.gpu
def test_cxx_caller_reference_checks_on_gpu():
    exe = os.path.join(BIN, "dropin_cxx")
    assert os.path.exists(exe), f"{exe} is missing: build it with `make -C tests/dropin` (or __graft_entry__.build())"
    r = _run([exe])
    assert r.returncode == 0 and "C++ caller, libixgdn" in r.stdout and "PASS" in r.stdout, r.stdout + r.stderr
    for name in ("step.o     h_k=16", "step.state h_k=48", "conv.state", "l2 cols=1024", "out_norm S=65", "beta_gate"):
        assert name in r.stdout, name


@pytest.mark.gpu
def test_projection_caller_reference_checks_on_gpu():
    exe = os.path.join(BIN, "dropin_proj")
    assert os.path.exists(exe), f"{exe} is missing: build it with `make -C tests/dropin` (or __graft_entry__.build())"
    r = _run([exe], timeout=300)
    assert r.returncode == 0 and "drop-in projection caller, libixgdn" in r.stdout and "PASS" in r.stdout, \
        r.stdout + r.stderr
    assert "mmvq_q8_0 cases=" in r.stdout and "ref_fail=0 column_dependence=0" in r.stdout
    assert "pair.y1" in r.stdout and "bitwise mismatches vs split(64)=0" in r.stdout

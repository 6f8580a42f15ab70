"""Runs the C++ API self-check (tests/cpp/api_selfcheck.cpp, built by
`make -C dnn-flash_amd selfcheck`): every entry point of
include/onednn_flash/*.hpp on the GPU against standard_attention, the
counterpart of the reference's benchmarks/bench_attention.cpp self-check."""

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parents[1] / "dnn-flash_amd" / "build" / "api_selfcheck"


def test_cpp_api_selfcheck():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert BIN.exists(), f"{BIN} not built (make -C dnn-flash_amd selfcheck)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0 and "ALL OK" in r.stdout

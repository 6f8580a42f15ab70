"""The C++ API (include/onednn_flash/*.hpp) on the GPU.

test_cpp_api_selfcheck runs tests/cpp/api_selfcheck.cpp (built by
`make -C dnn-flash_amd selfcheck`): every entry point against this library's
standard_attention, the counterpart of the reference's
benchmarks/bench_attention.cpp self-check, plus the error contract.
test_cpp_api_against_compiled_reference runs tests/cpp/api_golden.cpp on every
golden case and compares each entry point with the outputs of the reference
compiled from its own sources."""

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


GOLDEN = Path(__file__).resolve().parent / "golden"
GOLDEN_BIN = BIN.parent / "api_golden"
GOLDEN_CASES = sorted(p.stem for p in GOLDEN.glob("*.npz") if p.stem != "qk_score")


def _write_case(path, z):
    import numpy as np

    M, N, D, Dv = (int(z[n]) for n in ("M", "N", "D", "Dv"))
    tiles = np.asarray(z["tiles"], np.int64).reshape(-1, 2)
    has_mask = "mask" in z.files
    mask = np.asarray(z["mask"], np.uint8) if has_mask else None
    hdr = np.array([M, N, D, Dv, int(z["causal"]), int(has_mask),
                    int(z["mask_qbs"]) if has_mask else 0, int(z["mask_kbs"]) if has_mask else 0,
                    mask.shape[0] if has_mask else 0, mask.shape[1] if has_mask else 0,
                    int("alibi_slope" in z.files), len(tiles)], np.int64)
    slope = float(z["alibi_slope"]) if "alibi_slope" in z.files else 0.0
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(tiles.tobytes())
        f.write(np.array([float(z["scale"]), slope], np.float32).tobytes())
        for name in ("q", "k", "v"):
            f.write(np.ascontiguousarray(z[name], np.float32).tobytes())
        if has_mask:
            f.write(np.ascontiguousarray(mask).tobytes())
    return M, Dv, len(tiles)


@pytest.mark.parametrize("case", GOLDEN_CASES)
def test_cpp_api_against_compiled_reference(case, tmp_path):
    """Every C++ entry point on the GPU against the outputs of the reference's
    own standard_attention / flash_attention_qk_pv_tile_ws (and, for the
    bench_attention.cpp self-check inputs, flash_attention_tiled / _q_tile /
    _qk_pv_tile) compiled from its sources: max-abs <= 1e-5, the bar of the
    reference's self-check (benchmarks/bench_attention.cpp:152-160)."""
    import numpy as np

    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert GOLDEN_BIN.exists(), f"{GOLDEN_BIN} not built (make -C dnn-flash_amd selfcheck)"
    z = np.load(GOLDEN / f"{case}.npz")
    M, Dv, nt = _write_case(tmp_path / "case.bin", z)
    r = subprocess.run([str(GOLDEN_BIN), str(tmp_path / "case.bin"), str(tmp_path / "out.bin")],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0
    outs = np.fromfile(tmp_path / "out.bin", np.float32).reshape(-1, M, Dv)
    std = z["standard"]
    names = ["standard_attention", "flash_attention_tiled", "flash_attention_q_tile",
             "flash_attention_qk_pv_tile"] + [f"flash_attention_qk_pv_tile_ws{tuple(t)}" for t in z["tiles"]] + \
            ["flash_attention_batched_qk_pv_tile", "run_attention(StandardReference)",
             "run_attention(FlashTiledReference)", "run_attention(FlashMfmaHip)"]
    expected = [std, z["tiled"] if "tiled" in z.files else std,
                z["q_tile"] if "q_tile" in z.files else std,
                z["qk_pv_tile"] if "qk_pv_tile" in z.files else std] + list(z["flash_ws"]) + [std, std, std, std]
    if "alibi_slope" in z.files:
        names.append("flash_attention_tiled(alibi_slopes)")
        expected.append(std)
    assert outs.shape[0] == len(names)
    for name, got, ref in zip(names, outs, expected):
        d = float(np.abs(got.astype(np.float64) - ref).max())
        print(f"{case} {name}: max-abs {d:.3e}")
        assert np.isfinite(got).all(), f"{case} {name}: non-finite"
        assert d <= 1e-5, f"{case} {name}: max-abs {d:.3e} > 1e-5"

"""Planner parity (CPU): this library's ScoreModPlan / RuntimePlan planner
(include/onednn_flash/{score_mod_plan,runtime_plan}.hpp) against the
reference's (src/onednn_flash/score_mod_plan.cpp:115-182,
runtime_plan.cpp:71-182).

tests/cpp/planner_dump.cpp prints every decision over a grid of inputs. The
reference's build of it wrote tests/golden/planner_ref.txt.xz
(tests/golden/make_planner_golden.py); this library's build
(dnn-flash_amd/build/planner_dump) must print the same lines, except two
fields where this library deliberately differs and which are checked against
their closed forms instead:
  can_skip_tiles (causal):   reference key_length > query_length,
                             here key_length > 1 (some key tile lies above the
                             diagonal as soon as there are two keys);
  all_masked_row_possible:   reference k_start > q_start + q_size - 1 (every
                             row masked), here k_start > q_start (some row).
With a GPU present (--hip) the planner lowers to the HIP kernels; those
decisions are checked against the rules the kernels implement.
"""

from __future__ import annotations

import lzma
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
OURS = ROOT / "dnn-flash_amd" / "build" / "planner_dump"
REF_BIN = ROOT / "oracle" / "_ref" / "planner_dump_ref"
GOLDEN = ROOT / "tests" / "golden" / "planner_ref.txt.xz"


def _run(binary: Path, *args: str) -> list[str]:
    if not binary.exists():
        pytest.fail(f"{binary} is missing: run __graft_entry__.build()")
    return subprocess.run([str(binary), *args], check=True, capture_output=True, text=True,
                          timeout=60).stdout.splitlines()


def _fields(part: str) -> dict[str, str]:
    return dict(kv.split("=", 1) for kv in part.strip().split(";") if kv)


def _golden() -> list[str]:
    return lzma.decompress(GOLDEN.read_bytes()).decode().splitlines()


_SKIP = re.compile(r"can_skip_tiles=([01])")
_ROW = re.compile(r"all_masked_row_possible=([01])")


def _expected_skip(kind: str, m: int, n: int, ours: bool) -> str:
    if kind != "causal":
        return "0"
    return "1" if (n > 1 if ours else n > m) else "0"


def _check_deliberate_fields(ref: str, got: str) -> tuple[str, str]:
    """Checks the two deliberately different fields of one line against their
    closed forms and returns both lines with those fields blanked."""
    tag = ref[0]
    inputs = _fields(ref[2:].split(" | ", 1)[0])
    if tag in "BR":
        if tag == "B":
            kind, m, n = inputs["kind"], int(inputs["m"]), int(inputs["n"])
        else:
            dims = [int(x) for x in inputs["shape"].split("x")]
            kind, m, n = inputs["mask"], dims[2], dims[3]
        # Unsupported masks never reach the causal branch.
        assert _SKIP.search(ref).group(1) == _expected_skip(kind, m, n, ours=False), ref
        assert _SKIP.search(got).group(1) == _expected_skip(kind, m, n, ours=True), got
        return _SKIP.sub("can_skip_tiles=?", ref), _SKIP.sub("can_skip_tiles=?", got)
    if tag == "T":
        qs, ks, qz = int(inputs["q_start"]), int(inputs["k_start"]), int(inputs["q_size"])
        assert _ROW.search(ref).group(1) == ("1" if ks > qs + qz - 1 else "0"), ref
        assert _ROW.search(got).group(1) == ("1" if ks > qs else "0"), got
        return _ROW.sub("all_masked_row_possible=?", ref), _ROW.sub("all_masked_row_possible=?", got)
    return ref, got


def test_golden_is_current_reference_build():
    """Where the reference planner is built here, its live output is the fixture."""
    if not REF_BIN.exists():
        pytest.skip("reference planner not built here (make -C oracle ref)")
    assert _run(REF_BIN) == _golden()


def test_planner_matches_reference():
    ref_lines, got_lines = _golden(), _run(OURS)
    assert len(ref_lines) == len(got_lines) == 11304
    counts = {}
    for ref, got in zip(ref_lines, got_lines):
        assert ref.split(" | ", 1)[0] == got.split(" | ", 1)[0], (ref, got)
        r, g = _check_deliberate_fields(ref, got)
        assert r == g, f"\nreference: {ref}\nthis lib:  {got}"
        counts[ref[0]] = counts.get(ref[0], 0) + 1
    assert counts == {"S": 360, "B": 18, "T": 126, "R": 10800}


def test_reference_planner_known_answers():
    """Decisions the reference's own sources fix, read from the fixture: fp32
    only (score_mod_plan.cpp:129-135), same-shape bias only for post-ops, and
    the fallback chain order of runtime_plan.cpp:136-152."""
    lines = {ln.split(" | ", 1)[0]: ln.split(" | ")[1:] for ln in _golden()}
    s = _fields(lines["S dtype=bf16;kind=scale;has_scale=1;bias=none;post_ops=1"][0])
    assert (s["fallback"], s["signature"]) == ("unsupported_dtype", "unsupported:unsupported_dtype")
    s = _fields(lines["S dtype=f32;kind=scale_additive_bias;has_scale=1;bias=broadcast_row;post_ops=1"][0])
    assert (s["lowering"], s["fallback"]) == ("onednn_flash_epilogue", "unsupported_broadcast")
    s = _fields(lines["S dtype=f32;kind=scale_additive_bias;has_scale=1;bias=same_shape_tile;post_ops=1"][0])
    assert (s["lowering"], s["signature"]) == ("lowered_to_onednn_post_ops",
                                               "scale_additive_bias:same_shape_tile:f32")
    key = ("R shape=1x1x0x64x32x32;dtypes=unsupported,f32,f32,f32;kind=none;has_scale=0;bias=none;"
           "mask=none;force_reference=1;enable_onednn=1;onednn=1;post_ops=1")
    assert _fields(lines[key][2])["fallback"] == "unsupported_shape"   # shape is checked first


HIP_DTYPES = {("f32",) * 4, ("bf16",) * 4, ("bf16", "bf16", "bf16", "f32"), ("f16",) * 4,
              ("f16", "f16", "f16", "f32")}


def test_hip_lowering_rules():
    lines = _run(OURS, "--hip")
    assert len(lines) == 11520
    lowered = 0
    for ln in lines:
        head, sm, _bm, rp = ln.split(" | ")
        inp, sm, rp = _fields(head[2:]), _fields(sm), _fields(rp)
        dtypes = tuple(inp["dtypes"].split(","))
        use_hip = (inp["enable_hip"] == "1" and inp["force_reference"] == "0" and int(inp["m"]) > 0
                   and dtypes in HIP_DTYPES)
        if not use_hip:
            assert rp["backend"] in ("reference", "onednn_matmul"), ln
            assert "hip" not in rp["lowering"], ln
            continue
        if inp["kind"] == "unsupported":
            want = "unsupported_score_mod"
        elif inp["bias"] == "broadcast_col":
            want = "unsupported_broadcast"
        elif inp["bias"] == "unsupported":
            want = "unsupported_bias_layout"
        elif inp["mask"] == "unsupported":
            want = "unsupported_block_mask"
        else:
            want = "none"
        assert rp["fallback"] == want, ln
        if want != "none":
            assert (rp["backend"], rp["lowering"]) == ("reference", "reference_fallback"), ln
            continue
        lowered += 1
        assert (rp["backend"], rp["lowering"]) == ("hip", "lowered_to_hip_kernel"), ln
        assert sm["lowering"] == "lowered_to_hip_kernel" and sm["dtype"] == dtypes[0], ln
        assert sm["signature"].endswith(":softcap=30") == (inp["softcap"] == "30"), ln
        assert rp["signature"].endswith("|hip|row_major_k_strided"), ln
    assert lowered == 5 * 4 * 4 * 2 * 2

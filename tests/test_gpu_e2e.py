"""The decoder-block benchmark (dnn-flash_amd/python/bench_decoder_e2e.py) on
small shapes: the library's attention matches materialised attention alone
and inside the block, eagerly and replayed from a captured HIP graph (every
replay of the timing loop runs between the capture and the final comparison
with an eager call)."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "dnn-flash_amd" / "python"))


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


@pytest.mark.parametrize("args,tol", [
    (["--dtype", "f32"], 1e-5),                                            # reference defaults: D=32, rowwise kernel
    (["--dtype", "bf16", "--seq", "512", "--heads", "4", "--head-dim", "128"], 3e-2),
    (["--dtype", "f16", "--seq", "300", "--heads", "2", "--head-dim", "64", "--no-causal"], 5e-3),
])
@pytest.mark.parametrize("graph", [False, True])
def test_decoder_block_matches_materialized(ofh, tmp_path, args, tol, graph):
    import bench_decoder_e2e as E

    argv = args + ["--warmup", "1", "--repeat", "3", "--output-json", str(tmp_path / "e2e.json")]
    if graph:
        argv.append("--graph")
    print("e2e", argv, flush=True)
    rec = E.main(argv)[0]
    assert rec["attention_max_abs_diff"] <= tol
    assert rec["decoder_max_abs_diff"] <= 20 * tol
    assert rec["graph_replay_max_abs_diff_onednn_flash"] == 0.0
    assert rec["graph_replay_max_abs_diff_materialized"] <= tol
    assert (tmp_path / "e2e.json").exists()

"""Writes tests/golden/planner_ref.txt.xz: the reference planner's decisions
(src/onednn_flash/{score_mod_plan,runtime_plan}.cpp, compiled with
tests/cpp/planner_dump.cpp by `make -C oracle ref`) over the dump's input grid.

    make -C oracle ref && python tests/golden/make_planner_golden.py
"""

import lzma
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
BIN = ROOT / "oracle" / "_ref" / "planner_dump_ref"
OUT = Path(__file__).resolve().parent / "planner_ref.txt.xz"


def main() -> None:
    text = subprocess.run([str(BIN)], check=True, capture_output=True, text=True).stdout
    OUT.write_bytes(lzma.compress(text.encode(), preset=9 | lzma.PRESET_EXTREME))
    print(f"{OUT}: {text.count(chr(10))} lines")


if __name__ == "__main__":
    main()

"""Host check of the cell-list encode rules (no GPU): grids set up from a box
as the box kernel sets them, coarse and fine lists built as the build kernels
build them, and for random and adversarial vectors (on codewords, near
bisectors, on and beside cell edges, duplicate and lattice codebooks,
subnormal and large scales) every vector lies in its cell's box and its
cell's list holds the reference's first-index argmin
(src/util/vec.zig:109-175,271-283), whose lexicographic minimum equals it
bit for bit; two planted mistakes (no rounding margin, cell intervals
without the (1 +- u)^2 widening) are caught."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_cell_rules(tmp_path):
    exe = tmp_path / "cell_rules_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "native" / "cell_rules_check.cpp")],
                   check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 box_miss, 0 wrong;" in r.stdout, r.stdout

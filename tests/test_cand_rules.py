"""Host check of the candidate-set rules the GPU assignment and encode kernels
use (no GPU): for random and adversarial codebooks (duplicates, few distinct
points, scales 1e-19 to 1e18) and any anchor, the selected candidate set
holds the reference's first-index argmin (src/util/vec.zig:109-175,271-283)
and its lexicographic minimum equals it bit for bit; two planted mistakes
(a radius of rho instead of 2 rho, ties by scan order) are caught."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_cand_rules(tmp_path):
    exe = tmp_path / "cand_rules_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "native" / "cand_rules_check.cpp")],
                   check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 wrong;" in r.stdout, r.stdout
    assert "row_overrun 0" in r.stdout, r.stdout
    assert " 0 search_mismatch" in r.stdout, r.stdout

"""Host check of the chunked fold evaluation the GPU kernels use (no GPU):
the serial fold of non-negative float terms with an fp32 accumulator (the
wcss of src/tac/kmeans.zig:179) or an f64 one (weightedSample,
src/util/rng.zig:60-81), taken a chunk at a time by quantizing the terms to
the accumulator's ulp, equals the term-by-term fold bit for bit on random and
adversarial sequences, and weightedSample's pick through the exact chunk
start values equals the plain loop's."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_fold_rules(tmp_path):
    exe = tmp_path / "fold_rules_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "native" / "fold_rules_check.cpp")],
                   check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout and "fold rules check passed" in r.stdout

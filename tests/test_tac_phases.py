"""Host check of the library's TAC budget phases (csrc/tac_phases.hpp)
against the oracle's literal restatement of src/tac/tac.zig:97-401, on
random inputs (no GPU)."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_tac_phases_match_oracle(tmp_path):
    exe = tmp_path / "tac_phases_check"
    objs = []
    for c in ("pq_oracle.c", "tac_oracle.c"):
        o = tmp_path / (c + ".o")
        subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-c", "-o", str(o),
                        str(ROOT / "oracle" / c)], check=True, timeout=120)
        objs.append(str(o))
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "native" / "tac_phases_check.cpp"), *objs,
                    "-lpthread", "-lm"], check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout

"""Host check of the k-means++ seeding rules the GPU kernels use (no GPU):
the restated Zig PRNG agrees with the oracle's independent restatement, and
the band test never accepts an index the reference's sequential
weightedSample (src/util/rng.zig:57-82) would not return."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_kpp_rules(tmp_path):
    exe = tmp_path / "kpp_rules_check"
    lib = ROOT / "oracle" / "_build" / "libpq_oracle.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-o", str(exe),
                    str(ROOT / "tests" / "native" / "kpp_rules_check.cpp"), str(lib),
                    f"-Wl,-rpath,{lib.parent}"], check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 wrong" in r.stdout

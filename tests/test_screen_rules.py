"""Host check of the matrix-core screen's rules (screen_rules.hpp, no GPU):
with the bf16 hi/lo pieces emulated bit for bit (round to nearest even, and
with subnormal pieces flushed) and the 33-term fp32 sum taken in seven
orders, the screen value stays within its bound for random and adversarial
pairs; and for random and adversarial codebooks at sub-dimensions 5-8 and
K 2-256 (duplicates, near-duplicates, bisectors, vectors far from the
codebook, aligned worst-case pieces), whenever the screen settles a vector
the reference's first-index argmin (src/util/vec.zig:109-175,271-283) lies in
the winning block of 8 and the block's (distance, index) minimum equals it
bit for bit.  Planted mistakes are caught: a bound of a sixteenth fails the
bound check, a threshold of a thirty-second and one without the reference
distance's rounding term settle vectors wrongly."""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_screen_rules(tmp_path):
    exe = tmp_path / "screen_rules_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    str(ROOT / "tests" / "native" / "screen_rules_check.cpp")],
                   check=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    out = r.stdout
    assert " 0 over the bound" in out, out
    assert " 0 wrong;" in out, out
    over16 = int(re.search(r"(\d+) over a sixteenth", out).group(1))
    small = int(re.search(r"thirty-second of the bound (\d+) wrong", out).group(1))
    gamma = int(re.search(r"no rounding term (\d+) wrong", out).group(1))
    assert over16 > 0 and small > 0 and gamma > 0, out

#!/usr/bin/env python3
"""PQ build benchmark on one MI355X: pq.train (20 Lloyd iterations) + pq.encode.

Headline workload: the full-corpus shape — 1,521,797 synthetic fp32
residuals of dim 64 (Zipf 1.1 over 32,768 unit-sphere centres, sigma 0.15),
m=16 subspaces of dsub 4, ksub=256, seeded-shuffle initial codebooks,
exactly 20 Lloyd iterations, then encode of every vector.  One step = one
full train + one full encode with residuals already resident in HBM.

Prints ONE JSON line.  value = pq.train seconds per 20 iterations (lower is
better).  Beside it: encode throughput, the dominant kernel's roofline (live
HIP-event time of every kernel over the timed steps, HBM traffic and VALU
counters from the committed rocprofv3 summaries), the CPU baseline (the
oracle on this host's cores), rows for the subspace-shape sweep, the 60M
resident train and the 200M encode stream, and the stages around the path.

Other modes:
  --counter-pass W      one run of workload W's GPU work for rocprofv3 counter passes
  --summarize-trace OUT DIR   kernel table of a rocprofv3 --kernel-trace --stats run
  --cpu-protocol OUT W...   the CPU baseline protocol of workloads W (profiles)
  --summarize-pmc OUT DIR...   per-kernel summary of rocprofv3 counter CSVs
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ir-multivector-retrieval_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "pq.train s/20 iters + pq.encode Mvec/s, 1.52M×64 fp32, m16×k256; % roofline"
WORKLOAD = "corpus-1.52m"
PEAK_FP32_TFLOPS = 157.3   # MI355X fp32 vector peak (packed)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
# VALU issue: 256 CUs x 4 SIMDs, one wave64 VALU instruction per SIMD every 4
# cycles (16 lanes), at 2.4 GHz.
PEAK_VALU_GINSTR = 256 * 4 * 2.4 / 4
NEVER = float("-inf")
TRAFFIC_FILE = ROOT / "profiles" / f"pq_build_{WORKLOAD}_hbm_traffic.json"
VALU_FILE = ROOT / "profiles" / f"pq_build_{WORKLOAD}_valu_counters.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def host_cpu() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def median_of(fn, runs: int = 3):
    """Median wall time of `runs` calls (the first call's result is returned)."""
    times, first = [], None
    for r in range(runs):
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
        if r == 0:
            first = out
    return statistics.median(times), first


# ---------------------------------------------------------------------------
# CPU baseline: the oracle with the reference's threading
# ---------------------------------------------------------------------------
def cpu_baseline(x: np.ndarray, init: np.ndarray, w, gpu_cb2: np.ndarray | None,
                 full: bool = False):
    """The oracle (the C restatement of the reference, its threading: work
    stealing over subspaces, static chunks inside a subspace and for encode)
    on this host's cores, at T = every available thread and T = 1.

    Protocol: one discarded warm-up (the 2-iteration run that also checks the
    GPU's codebooks at full size), then the median of 3 runs of each timing.
    Bounded mode (default) times 4 Lloyd iterations at T and extrapolates to
    20, and 1 iteration of 2 subspaces at T = 1, extrapolated to 20
    iterations of all subspaces; encode times the whole corpus at T and
    100,000 vectors at T = 1.  Full mode times all 20 iterations at T."""
    from oracle import binding as orc

    T = host_threads()
    t0 = time.perf_counter()
    ref2 = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=2, tol=NEVER, n_threads=T)
    warm_s = time.perf_counter() - t0
    assert ref2.status == 0
    parity = None
    if gpu_cb2 is not None:
        parity = bool(np.array_equal(gpu_cb2.view(np.uint32), ref2.codebooks.view(np.uint32)))
    iters = w.iters if full else 4
    t_train, _ = median_of(lambda: orc.pq_train(x, w.dim, w.m, w.ksub, init=init,
                                                 max_iters=iters, tol=NEVER, n_threads=T))
    t_enc, _ = median_of(lambda: orc.pq_encode(x, w.dim, w.m, w.ksub, ref2.codebooks,
                                               n_threads=T))
    # T = 1: the first two subspaces (dim 2 * dsub) stand for all of them
    dsub = w.dim // w.m
    x2 = np.ascontiguousarray(x[:, :2 * dsub])
    it1 = 2 if full else 1
    t1_train, _ = median_of(lambda: orc.pq_train(x2, 2 * dsub, 2, w.ksub, init=init[:2],
                                                  max_iters=it1, tol=NEVER, n_threads=1))
    ns = 100_000
    t1_enc, _ = median_of(lambda: orc.pq_encode(x[:ns], w.dim, w.m, w.ksub, ref2.codebooks,
                                                n_threads=1))
    return {
        "value": round(t_train / iters * w.iters, 3), "unit": "s/20 iters",
        "encode_mvec_per_s": round(w.n / t_enc / 1e6, 3),
        "threads": T, "cores": T, "kind": "port",
        "t1_train_s_per_20_iters": round(t1_train / it1 * w.iters * (w.m / 2), 2),
        "t1_encode_mvec_per_s": round(ns / t1_enc / 1e6, 4),
        "median_of": 3, "warmup_discarded": 1, "extrapolated": iters < w.iters,
        "host_cpu": host_cpu(),
        "sample": (f"T={T}: median of 3 runs of {iters} Lloyd iterations of all {w.m} "
                   f"subspaces over the full {w.n:,}-vector corpus"
                   + (f", scaled x{w.iters // iters} to {w.iters}" if iters < w.iters else "")
                   + f"; encode of all {w.n:,} vectors, median of 3. T=1: {it1} iteration(s) "
                     f"of 2 subspaces scaled to {w.iters} x {w.m}, encode of {ns:,} vectors. "
                     f"Warm-up {warm_s:.1f} s discarded."),
        "parity_full_size_2_iters": parity,
    }


# The CPU protocol of every workload: how much of it is timed (Lloyd
# iterations at T, at T = 1 on 2 subspaces, vectors encoded at T = 1) and
# for the encode stream the chunk that stands for the whole of it.
CPU_PLAN = {
    "chunk-117k": dict(iters_T=20, iters_T1=20, enc_T1=117_645),
    "corpus-1.52m": dict(iters_T=20, iters_T1=2, enc_T1=100_000),
    "corpus-1.52m-m32d2": dict(iters_T=20, iters_T1=2, enc_T1=100_000),
    "corpus-1.52m-m8d8": dict(iters_T=20, iters_T1=2, enc_T1=100_000),
    "corpus-1.52m-k1024": dict(iters_T=20, iters_T1=1, enc_T1=50_000),
    "paper-60m": dict(iters_T=1, iters_T1=1, enc_T1=100_000),
    "stream-200m": dict(chunk=10_000_000, enc_T1=100_000),
}


def cpu_protocol(name: str) -> dict:
    """The CPU baseline protocol for one workload: the oracle on this host at
    T = every available thread and T = 1, one discarded warm-up, median of 3.
    Training workloads time CPU_PLAN's iterations of all subspaces at T
    (all of them up to the 1.52M corpus; one for the 60M sample, scaled to
    its 25) and iterations of the first 2 subspaces at T = 1, scaled to all
    subspaces and iterations (subspaces train independently,
    src/index/pq.zig:200-205); encode runs the whole workload at T and a
    prefix at T = 1.  The 200M stream times the encode of its first 10M
    chunk, scaled x20.  Every scaled figure is labelled."""
    from oracle import binding as orc
    from tac_gpu import synth

    w = synth.WORKLOADS[name]
    plan = CPU_PLAN[name]
    T = host_threads()
    t0 = time.perf_counter()
    rec = {"workload": name, "n": w.n, "dim": w.dim, "m": w.m, "dsub": w.dsub, "ksub": w.ksub,
           "threads": T, "cores": T, "kind": "port", "host_cpu": host_cpu(), "median_of": 3,
           "warmup_discarded": 1}
    if name == "stream-200m":
        chunk = plan["chunk"]
        x = synth.residuals(w, chunk)
        rec["generate_s"] = round(time.perf_counter() - t0, 1)
        cb = synth.gauss_codebooks(w.seed, w.m, w.ksub, w.dsub, 0.05)
        orc.pq_encode(x, w.dim, w.m, w.ksub, cb, n_threads=T)  # warm-up
        t_enc, _ = median_of(lambda: orc.pq_encode(x, w.dim, w.m, w.ksub, cb, n_threads=T))
        ns = plan["enc_T1"]
        t1_enc, _ = median_of(lambda: orc.pq_encode(x[:ns], w.dim, w.m, w.ksub, cb,
                                                    n_threads=1))
        scale = w.n / chunk
        rec.update({
            "value": round(t_enc * scale, 2), "unit": "s per 200M-vector encode",
            "encode_mvec_per_s": round(chunk / t_enc / 1e6, 3),
            "t1_encode_mvec_per_s": round(ns / t1_enc / 1e6, 4),
            "t1_s_per_200m": round(t1_enc / ns * w.n, 1),
            "extrapolated": True,
            "sample": (f"T={T}: encode of the first {chunk:,}-vector chunk (median of 3), "
                       f"scaled x{scale:.0f} to {w.n:,}; T=1: {ns:,} vectors, scaled.")})
        return rec
    x = synth.residuals(w)
    init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
    rec["generate_s"] = round(time.perf_counter() - t0, 1)
    it_T, it_1 = plan["iters_T"], plan["iters_T1"]
    ref = orc.pq_train(x, w.dim, w.m, w.ksub, init=init, max_iters=min(2, w.iters), tol=NEVER,
                       n_threads=T)  # warm-up; its codebooks serve the encode timing
    assert ref.status == 0
    t_train, _ = median_of(lambda: orc.pq_train(x, w.dim, w.m, w.ksub, init=init,
                                                 max_iters=it_T, tol=NEVER, n_threads=T))
    t_enc, _ = median_of(lambda: orc.pq_encode(x, w.dim, w.m, w.ksub, ref.codebooks,
                                               n_threads=T))
    d2 = 2 * w.dsub
    x2 = np.ascontiguousarray(x[:, :d2])
    t1_train, _ = median_of(lambda: orc.pq_train(x2, d2, 2, w.ksub, init=init[:2],
                                                  max_iters=it_1, tol=NEVER, n_threads=1))
    del x2
    ns = min(plan["enc_T1"], w.n)
    t1_enc, _ = median_of(lambda: orc.pq_encode(x[:ns], w.dim, w.m, w.ksub, ref.codebooks,
                                                n_threads=1))
    rec.update({
        "lloyd_iters": w.iters,
        "value": round(t_train / it_T * w.iters, 3), "unit": f"s/{w.iters} iters",
        "encode_mvec_per_s": round(w.n / t_enc / 1e6, 3),
        "t1_train_s": round(t1_train / it_1 * w.iters * (w.m / 2), 2),
        "t1_encode_mvec_per_s": round(ns / t1_enc / 1e6, 4),
        "extrapolated": it_T < w.iters,
        "sample": (f"T={T}: median of 3 runs of {it_T} Lloyd iteration(s) of all {w.m} "
                   f"subspaces over all {w.n:,} vectors"
                   + (f", scaled x{w.iters / it_T:g} to {w.iters}" if it_T < w.iters else
                      " (not extrapolated)")
                   + f"; encode of all {w.n:,} vectors. T=1: {it_1} iteration(s) of the "
                     f"first 2 subspaces, scaled to {w.iters} iterations x {w.m} subspaces"
                     f"; encode of {ns:,} vectors.")})
    return rec


def cpu_profile_row(name: str, gpu_s: float | None = None, gpu_enc_mvec: float | None = None):
    """The committed CPU protocol record of a workload
    (profiles/cpu_baseline_<name>.json, written by --cpu-protocol on the GPU
    box's host), with the speed-ups of this run's GPU figures over it."""
    rec = _load_json(ROOT / "profiles" / f"cpu_baseline_{name}.json")
    if not rec:
        return None
    keys = ("value", "unit", "encode_mvec_per_s", "threads", "t1_train_s",
            "t1_encode_mvec_per_s", "t1_s_per_200m", "kind", "host_cpu", "extrapolated",
            "sample")
    row = {k: rec[k] for k in keys if k in rec}
    row["source"] = f"profiles/cpu_baseline_{name}.json"
    if gpu_s and "value" in rec:
        row["speedup_train_or_stream"] = round(rec["value"] / gpu_s, 1)
    if gpu_enc_mvec and rec.get("encode_mvec_per_s"):
        row["speedup_encode"] = round(gpu_enc_mvec / rec["encode_mvec_per_s"], 1)
    return row


def write_cpu_profile(out_dir: Path, rec: dict, command: str) -> None:
    """profiles-style JSON and Markdown summary of one cpu_protocol record."""
    out_dir.mkdir(parents=True, exist_ok=True)
    stem = f"cpu_baseline_{rec['workload']}"
    (out_dir / f"{stem}.json").write_text(json.dumps(rec, indent=1) + "\n")
    stream = rec["workload"] == "stream-200m"
    lines = [
        f"# CPU baseline, {rec['workload']} ({rec['n']:,} x {rec['dim']} fp32, "
        f"m{rec['m']} dsub {rec['dsub']} k{rec['ksub']})", "",
        "The oracle (`oracle/pq_oracle.c`, the C restatement of the reference's `pq.train` / "
        "`PQ.encode` with its threading: work stealing over subspaces, static chunks inside a "
        "subspace and for encode; built `-O3 -march=x86-64-v3 -ffp-contract=off`) on the GPU "
        "box's host cores. No Zig toolchain exists in this image, so the reference itself "
        "cannot be timed (`kind: port`).", "",
        f"Protocol: {rec['sample']} One discarded warm-up, median of 3 runs of each timing.", "",
        f"Command (on the GPU box): `{command}`", ""]
    if stream:
        lines += ["| host CPU | threads | s per 200M encode (scaled) | encode Mvec/s | "
                  "T=1 encode Mvec/s | T=1 s per 200M (scaled) |",
                  "|---|---:|---:|---:|---:|---:|",
                  f"| {rec['host_cpu']} | {rec['threads']} | {rec['value']} | "
                  f"{rec['encode_mvec_per_s']} | {rec['t1_encode_mvec_per_s']} | "
                  f"{rec['t1_s_per_200m']} |"]
    else:
        lines += [f"| host CPU | threads | pq.train {rec['unit']}"
                  f"{' (scaled)' if rec['extrapolated'] else ''} | pq.encode Mvec/s | "
                  f"T=1 pq.train s (scaled) | T=1 pq.encode Mvec/s |",
                  "|---|---:|---:|---:|---:|---:|",
                  f"| {rec['host_cpu']} | {rec['threads']} | {rec['value']} | "
                  f"{rec['encode_mvec_per_s']} | {rec['t1_train_s']} | "
                  f"{rec['t1_encode_mvec_per_s']} |"]
    (out_dir / f"{stem}.md").write_text("\n".join(lines) + "\n")


# ---------------------------------------------------------------------------
# Counter summaries (rocprofv3 CSV -> profiles/*.json)
# ---------------------------------------------------------------------------
def _counter_rows(paths):
    for p in paths:
        p = Path(p)
        files = [p] if p.is_file() else sorted(p.rglob("*counter_collection.csv"))
        for f in files:
            with open(f, newline="") as fh:
                yield from csv.DictReader(fh)


def _agent(paths):
    for p in paths:
        p = Path(p)
        for f in ([p] if p.is_file() else sorted(p.rglob("*agent_info.csv"))):
            if not f.name.endswith("agent_info.csv"):
                continue
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    if r.get("Agent_Type") == "GPU":
                        return {"cu": int(r["Cu_Count"]), "simd": int(r["Simd_Count"]),
                                "xcc": int(r["Num_Xcc"])}
    return {"cu": 256, "simd": 1024, "xcc": 8}


def short_name(kernel: str) -> str:
    """'void tacgpu::cand_kernel<4, false, ...>(float const*, ...)' ->
    'cand_kernel<4, false, ...>'."""
    k = kernel.replace("void ", "", 1) if kernel.startswith("void ") else kernel
    k = k.removeprefix("(anonymous namespace)::")
    depth, cut = 0, len(k)
    for i, ch in enumerate(k):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    k = k[:cut]
    return k.split("::")[-1] if "::" in k.split("<")[0] else k


def _md_table(kernels: dict, cols) -> str:
    lines = ["| kernel | " + " | ".join(c for c, _ in cols) + " |",
             "|---|" + "---:|" * len(cols)]
    for name, rec in kernels.items():
        vals = []
        for _, f in cols:
            v = f(rec)
            vals.append("-" if v is None else (f"{v:,.4g}" if isinstance(v, float) else f"{v:,}"))
        lines.append(f"| {name} | " + " | ".join(vals) + " |")
    return "\n".join(lines)


def summarize_pmc(out_base: str, dirs, commands=()) -> None:
    """Per-kernel averages of every counter over its launches, plus derived
    figures: HBM bytes from FETCH_SIZE / WRITE_SIZE scaled by the 1 GiB copy
    kernel (the largest __amd_rocclr_copyBuffer launch), and VALU issue use
    from the SQ counters."""
    agent = _agent(dirs)
    per = {}  # kernel -> counter -> [values]
    for r in _counter_rows(dirs):
        name = short_name(r["Kernel_Name"])
        per.setdefault(name, {}).setdefault(r["Counter_Name"], []).append(
            float(r["Counter_Value"]))
    copy = per.get("__amd_rocclr_copyBuffer", {})
    gib_kib = float(1 << 20)
    fscale = gib_kib / max(copy["FETCH_SIZE"]) if copy.get("FETCH_SIZE") else None
    wscale = gib_kib / max(copy["WRITE_SIZE"]) if copy.get("WRITE_SIZE") else None
    kernels = {}
    for name, cs in sorted(per.items()):
        avg = {c: sum(v) / len(v) for c, v in cs.items()}
        rec = {"samples": max(len(v) for v in cs.values()), "counters": avg}
        if "FETCH_SIZE" in avg and fscale:
            rec["read_bytes"] = int(avg["FETCH_SIZE"] * 1024 * fscale)
        if "WRITE_SIZE" in avg and wscale:
            rec["write_bytes"] = int(avg["WRITE_SIZE"] * 1024 * wscale)
        gui = avg.get("GRBM_GUI_ACTIVE")
        if gui:
            cyc = gui / agent["xcc"]  # summed over the XCDs
            rec["cycles_per_xcd"] = round(cyc)
            if "SQ_INSTS_VALU" in avg:
                rec["valu_issue_frac"] = round(avg["SQ_INSTS_VALU"] / (agent["simd"] * cyc / 4), 4)
            if "SQ_ACTIVE_INST_VALU" in avg:
                rec["valu_busy"] = round(avg["SQ_ACTIVE_INST_VALU"] / (agent["cu"] * cyc), 4)
            if "SQ_LDS_BANK_CONFLICT" in avg:
                rec["lds_bank_conflict_frac"] = round(avg["SQ_LDS_BANK_CONFLICT"]
                                                      / (agent["cu"] * cyc), 4)
        if "SQ_THREAD_CYCLES_VALU" in avg and avg.get("SQ_ACTIVE_INST_VALU"):
            rec["valu_lane_util"] = round(avg["SQ_THREAD_CYCLES_VALU"]
                                          / (avg["SQ_ACTIVE_INST_VALU"] * 64), 4)
        kernels[name] = rec
    doc = {"agent": agent, "fetch_scale": fscale, "write_scale": wscale, "kernels": kernels}
    Path(out_base + ".json").write_text(json.dumps(doc, indent=1, sort_keys=True) + "\n")
    counters = sorted({c for rec in kernels.values() for c in rec["counters"]})
    cols = [("samples", lambda r: r["samples"])]
    if fscale:
        cols.append(("HBM read MB", lambda r: r.get("read_bytes", 0) / 1e6 if "read_bytes" in r
                     else None))
    if wscale:
        cols.append(("HBM write MB", lambda r: r.get("write_bytes", 0) / 1e6 if "write_bytes" in r
                     else None))
    for key, label in (("valu_issue_frac", "VALU issue"), ("valu_busy", "VALU busy"),
                       ("valu_lane_util", "VALU lanes"),
                       ("lds_bank_conflict_frac", "LDS conflict")):
        if any(key in r for r in kernels.values()):
            cols.append((label, lambda r, k=key: r.get(k)))
    for c in counters:
        cols.append((c, lambda r, k=c: (round(r["counters"][k]) if k in r["counters"] else None)))
    md = [f"# rocprofv3 counters per kernel: {Path(out_base).name}", "",
          "Values are averages over the samples of each kernel (one per launch per pass).",
          f"Device: {agent['cu']} CUs, {agent['simd']} SIMDs, {agent['xcc']} XCDs.", ""]
    if fscale or wscale:
        md += [f"HBM bytes: FETCH_SIZE x {fscale and round(fscale, 4)}, WRITE_SIZE x "
               f"{wscale and round(wscale, 4)} (KiB), the factors that make the 1 GiB "
               "__amd_rocclr_copyBuffer launch read and write 1 GiB.", ""]
    if any("valu_issue_frac" in r for r in kernels.values()):
        md += ["VALU issue = SQ_INSTS_VALU / (SIMDs x GRBM_GUI_ACTIVE / XCDs / 4): the share of "
               "the wave64 VALU issue slots (one per SIMD every 4 cycles) the kernel used. "
               "VALU busy = SQ_ACTIVE_INST_VALU / (CUs x cycles); VALU lanes = "
               "SQ_THREAD_CYCLES_VALU / (64 x SQ_ACTIVE_INST_VALU); LDS conflict = "
               "SQ_LDS_BANK_CONFLICT / (CUs x cycles).", ""]
    md += ["Commands:", "```", "cd /tmp && export TMPDIR=/tmp"] + list(commands) + [
        "python3 bench.py --summarize-pmc " + " ".join([out_base] + [str(d) for d in dirs]),
        "```", "", _md_table(kernels, cols), ""]
    Path(out_base + ".md").write_text("\n".join(md))
    log(f"wrote {out_base}.json and .md ({len(kernels)} kernels)")


def _load_json(path: Path):
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------------------
# Roofline of the dominant kernel
# ---------------------------------------------------------------------------
def algorithmic_bytes(name: str, n: int, dim: int, m: int, parts: int = 1):
    """Bytes a kernel must move per launch: an assignment or encode reads
    every residual once and writes one code per vector and subspace (2 bytes
    during training, 1 in the encode output); scatter reads the records and
    codes and writes the records; the fold reads the records.  Training
    launches cover m / parts subspaces each (parts = the streams the Lloyd
    loop splits the subspaces over).  None for the small kernels."""
    dsub = dim // m
    dp = 1 if dsub <= 1 else 2 if dsub <= 2 else 4 if dsub <= 4 else 8
    if name.startswith("cand_kernel") and ", true, true," in name:
        return n * (4 * dim + m)
    if name.startswith("encode_kernel"):
        return n * (4 * dim + m)
    if name.startswith("transpose_kernel"):
        return n * (4 * dim + 4 * m * dp)
    if name.startswith(("cand_kernel", "assign_kernel")):
        return n * (4 * dim + 2 * m) // parts
    if name.startswith("scatter_kernel"):
        return n * m * (2 * 4 * dp + 2) // parts
    if name.startswith("fold_kernel"):
        return n * m * 4 * dp // parts
    return None


def kernel_table(kt: dict, steps: int, train_ms: float):
    rows = {}
    for name, (ms, launches) in kt.items():
        rows[name] = {"avg_ms": round(ms / max(launches, 1), 4),
                      "launches_per_step": round(launches / steps, 2),
                      "ms_per_step": round(ms / steps, 4),
                      "share_of_step": round(ms / steps / train_ms, 4) if train_ms else None}
    return dict(sorted(rows.items(), key=lambda kv: -kv[1]["ms_per_step"]))


def algorithmic_flops(name: str, n: int, dim: int, m: int, ksub: int, parts: int = 1):
    """FLOP a launch stands for in the reference's exhaustive scan: dsub
    multiply-adds per (vector, subspace, codeword) pair, 2 * dim * ksub per
    vector over all subspaces (the candidate kernels evaluate a pruned subset
    of the pairs; the figure counts the work they replace).  None for kernels
    that compute no distances."""
    if name.startswith("cand_kernel") and ", true, true," in name:
        return 2 * n * dim * ksub
    if name.startswith("encode_kernel"):
        return 2 * n * dim * ksub
    if name.startswith(("cand_kernel", "assign_kernel")):
        return 2 * n * dim * ksub // parts
    return None


def roofline(name: str, row: dict, n: int, dim: int, m: int, ksub: int, traffic: dict,
             valu: dict, parts: int = 1):
    """The dominant kernel against the roof its counters show it is bound by.
    'valu': the kernel's wave64 VALU instructions per launch (committed
    rocprofv3 counters, taken on the two-stream default, scaled to this run's
    launch size) over its live average launch time, against the issue peak
    of one wave64 VALU instruction per SIMD every 4 cycles (614.4 G/s); used
    when that share exceeds the HBM share.  'hbm': algorithmic bytes over the
    live launch time against 8 TB/s.  Both shares are reported under their
    own names, with the exhaustive-scan FLOP rate (which a pruned search can
    push past the FLOP peak, so it is no roof for this kernel)."""
    ab = algorithmic_bytes(name, n, dim, m, parts)
    af = algorithmic_flops(name, n, dim, m, ksub, parts)
    avg_s = row["avg_ms"] * 1e-3
    hbm_gbs = ab / avg_s / 1e9 if ab else None
    hbm_frac = None if hbm_gbs is None else hbm_gbs / PEAK_HBM_GBS
    v = valu.get(name) if valu else None
    instr = None
    if v and "SQ_INSTS_VALU" in v["counters"]:
        # training kernels were counted as half launches (two streams)
        training = name.startswith(("cand_kernel", "assign_kernel")) and ", true, true," not in name
        instr = v["counters"]["SQ_INSTS_VALU"] * (2 / max(parts, 1) if training else 1)
    ginstr = instr / avg_s / 1e9 if instr else None
    issue_frac = None if ginstr is None else ginstr / PEAK_VALU_GINSTR
    tr = traffic.get(name) if traffic else None
    counted = None if not tr or "read_bytes" not in tr else tr["read_bytes"] + tr.get(
        "write_bytes", 0)
    if issue_frac is not None and hbm_frac is not None and issue_frac > hbm_frac:
        out = {"kernel": name, "bound": "valu", "achieved": round(ginstr, 1),
               "peak": PEAK_VALU_GINSTR, "unit": "G wave64 VALU instr/s",
               "frac": round(issue_frac, 4)}
    else:
        out = {"kernel": name, "bound": "hbm",
               "achieved": None if hbm_gbs is None else round(hbm_gbs, 1),
               "peak": PEAK_HBM_GBS, "unit": "GB/s",
               "frac": None if hbm_frac is None else round(hbm_frac, 4)}
    out.update({
        "traffic": counted,
        "hbm_achieved_gbs": None if hbm_gbs is None else round(hbm_gbs, 1),
        "hbm_frac": None if hbm_frac is None else round(hbm_frac, 4),
        "valu_issue_frac_live": None if issue_frac is None else round(issue_frac, 4),
        "exhaustive_scan_tflops": None if not af else round(af / avg_s / 1e12, 2),
        "avg_launch_ms": row["avg_ms"], "algorithmic_bytes_per_launch": ab,
        "launches_per_step": row["launches_per_step"], "share_of_step": row["share_of_step"],
    })
    if counted:
        out["counted_hbm_gbs"] = round(counted / avg_s / 1e9, 1)
        out["counted_over_algorithmic"] = round(counted / ab, 3) if ab else None
    if v:
        c = v["counters"]
        out["valu"] = {
            "issue_frac_counters": v.get("valu_issue_frac"), "busy": v.get("valu_busy"),
            "lane_util": v.get("valu_lane_util"),
            "lds_bank_conflict_frac": v.get("lds_bank_conflict_frac"),
            "instr_per_launch": int(c["SQ_INSTS_VALU"]) if "SQ_INSTS_VALU" in c else None,
            "live_ginstr_per_s": (round(c["SQ_INSTS_VALU"] / avg_s / 1e9, 1)
                                  if "SQ_INSTS_VALU" in c else None),
            "peak_ginstr_per_s": PEAK_VALU_GINSTR,
            "source": str(VALU_FILE.relative_to(ROOT)),
        }
    return out


# ---------------------------------------------------------------------------
# Rows beside the headline
# ---------------------------------------------------------------------------
def residual_stage(device, x, ids, w, reps: int):
    """storage.build stage 2 on the corpus tokens (rebuilt as centre +
    residual): average kernel time per call over `reps` timed calls."""
    from tac_gpu import synth

    cents = synth.centers(w.seed, w.n_centers, w.dim)
    v = (x + cents[ids]).astype(np.float32)
    dv = device.DeviceArray.from_host(v)
    dc = device.DeviceArray.from_host(cents)
    da = device.DeviceArray.from_host(ids)
    dr = device.DeviceArray(v.shape, np.float32)
    dn = device.DeviceArray((w.n,), np.float32)
    device.residuals_device(dv, w.n, w.dim, dc, w.n_centers, da, dr, dn)  # warm
    device.profile_enable(True)
    device.profile_read(reset=True)
    for _ in range(reps):
        device.residuals_device(dv, w.n, w.dim, dc, w.n_centers, da, dr, dn)
    p = device.profile_read(reset=True)
    device.profile_enable(False)
    ms = p.residual_ms / max(p.residual_launches, 1)
    for a in (dv, dc, da, dr, dn):
        a.free()
    nbytes = w.n * (8 * w.dim + 8) + w.n_centers * w.dim * 4
    return {
        "kernel": "residual_kernel (r = v - c[a], in-order norm, scale by 1/norm)",
        "avg_call_ms": round(ms, 4), "algorithmic_bytes": nbytes,
        "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
    }


def storage_and_query(device, x, ids, w, cents, with_cpu: bool):
    """The .tac rows around the PQ build on the corpus workload: per-document
    layouts of all tokens (documents of 1-100 tokens), the footer CRC-32 over
    those layouts, one query's distance table and refine of 1,000 candidate
    documents.  GPU call times (data resident), averaged over 5 calls."""
    import ctypes
    from tac_gpu import errors, lib, retrieval
    from tac_gpu import pq as pqmod

    rng = np.random.default_rng(7)
    lens = rng.integers(1, 101, w.n // 40)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint64)
    off = off[off < w.n]
    off = np.append(off, np.uint64(w.n))
    n_docs = off.size - 1
    codes = rng.integers(0, 256, (w.n, w.m)).astype(np.uint8)
    total_c = ctypes.c_uint64(0)
    errors.check(lib.tac_doc_payload_bytes(off.ctypes.data_as(ctypes.c_void_p), n_docs, w.m, 1,
                                           ctypes.byref(total_c)))
    total = int(total_c.value)
    d_off = device.DeviceArray.from_host(off)
    d_ids = device.DeviceArray.from_host(ids)
    d_codes = device.DeviceArray.from_host(codes)
    d_idx = device.DeviceArray((n_docs + 1,), np.uint64)
    d_pay = device.DeviceArray((total,), np.uint8)

    def timed(fn, reps=5):
        fn()
        device.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        device.synchronize()
        return (time.perf_counter() - t0) / reps

    t_lay = timed(lambda: errors.check(lib.tac_write_doc_layouts_device(
        d_off.ptr, n_docs, w.n, d_ids.ptr, d_codes.ptr, w.m, 1, d_idx.ptr, d_pay.ptr, total,
        None)))
    crc = ctypes.c_uint32(0)
    device.profile_enable(True)
    device.profile_read(reset=True)
    t_crc = timed(lambda: errors.check(lib.tac_crc32_device(d_pay.ptr, total, ctypes.byref(crc),
                                                             None)))
    pc = device.profile_read(reset=True)
    k_crc = pc.crc_ms / max(pc.crc_launches, 1) * 1e-3
    n_q, dim = 32, w.dim
    q = rng.standard_normal((n_q, dim)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    cb = rng.standard_normal((w.m, w.ksub, w.dsub)).astype(np.float32) * 0.05
    d_q = device.DeviceArray.from_host(q)
    d_cb = device.DeviceArray.from_host(cb)
    d_tab = device.DeviceArray((w.m * w.ksub * n_q,), np.float32)
    t_tab = timed(lambda: errors.check(lib.tac_pq_distance_table_device(
        d_q.ptr, n_q, dim, w.m, w.ksub, d_cb.ptr, d_tab.ptr, w.m * w.ksub * n_q, None)))
    norms = (1.0 + rng.random(w.n)).astype(np.float32)
    d_cent = device.DeviceArray.from_host(cents)
    d_norms = device.DeviceArray.from_host(norms)
    view = retrieval._DocIndexC(dim, cents.shape[0], w.m, w.ksub, n_docs, w.n, total, d_cent.ptr,
                                d_idx.ptr, d_pay.ptr, d_off.ptr, d_norms.ptr)
    cand = rng.choice(n_docs, 1000, replace=False).astype(np.uint32)
    d_cand = device.DeviceArray.from_host(cand)
    d_scores = device.DeviceArray((1000,), np.float32)
    device.profile_read(reset=True)
    t_ref = timed(lambda: errors.check(lib.tac_refine_device(
        ctypes.byref(view), d_tab.ptr, w.m * w.ksub * n_q, d_q.ptr, n_q, d_cand.ptr, 1000,
        d_scores.ptr, None)))
    pr = device.profile_read(reset=True)
    k_ref = pr.refine_ms / max(pr.refine_launches, 1) * 1e-3
    device.profile_enable(False)
    cand_tokens = int(sum(int(off[c + 1] - off[c]) for c in cand))
    row = {
        "doc_layouts": {"tokens": w.n, "docs": n_docs, "payload_bytes": total,
                        "ms": round(t_lay * 1e3, 4),
                        "hbm_gbs": round((w.n * (4 + w.m) + 16 * n_docs + total) / t_lay / 1e9,
                                         1)},
        "crc32": {"bytes": total, "call_ms": round(t_crc * 1e3, 4),
                  "kernel_ms": round(k_crc * 1e3, 4),
                  "kernel_gbs": round(total / k_crc / 1e9, 1),
                  "hbm_frac": round(total / k_crc / 1e9 / PEAK_HBM_GBS, 4)},
        "distance_table": {"n_q": n_q, "m": w.m, "ksub": w.ksub, "us": round(t_tab * 1e6, 1)},
        "refine": {"n_q": n_q, "candidates": 1000, "candidate_tokens": cand_tokens,
                   "call_ms": round(t_ref * 1e3, 4), "kernel_ms": round(k_ref * 1e3, 4),
                   "candidates_per_s": round(1000 / k_ref)},
        "note": "call times include launch, status readback and host synchronisation",
    }
    if with_cpu:
        from oracle import binding as orc
        tab = d_tab.to_host()
        idx_h, pay_h = d_idx.to_host(), d_pay.to_host()
        t0 = time.perf_counter()
        for c in cand[:100]:
            orc.refine(q, n_q, dim, cents, tab, w.m, w.ksub, idx_h, pay_h, off, norms, int(c))
        row["refine"]["cpu_oracle_ms_1thread"] = round((time.perf_counter() - t0) * 10 * 1e3, 1)
    for a in (d_off, d_ids, d_codes, d_idx, d_pay, d_q, d_cb, d_tab, d_cent, d_norms, d_cand,
              d_scores):
        a.free()
    return row


def tac_clustering(device, with_cpu: bool):
    """Token-aware clustering (tac.clusterFlat) on the 1.52M-token synthetic
    dump (dim 64, 30,522-id vocabulary, Zipf 1.05, kappa_total 40,960): call
    time (host inputs, includes the upload and the host-side budget phases)
    and the device time of seeding and Lloyd; the oracle and the GPU on the
    first 200,000 rows (same generator) for a like-for-like CPU comparison."""
    from oracle import binding as orc
    from tac_gpu import synth, tac

    d, ids, v = synth.tac_workload("tac-1.52m")
    p = tac.ClusteringParams(kappa_total=d["kappa_total"], seed=0)
    tac.cluster_flat(ids, v, d["dim"], p)  # warm-up: workspace allocation
    device.profile_enable(True)
    device.profile_read(reset=True)
    reps = 2
    t0 = time.perf_counter()
    for _ in range(reps):
        r = tac.cluster_flat(ids, v, d["dim"], p)
    call_s = (time.perf_counter() - t0) / reps
    pr = device.profile_read(reset=True)
    device.profile_enable(False)
    f = np.bincount(ids)
    row = {
        "workload": "tac-1.52m", "n": int(ids.size), "dim": d["dim"],
        "distinct_tokens": int((f > 0).sum()), "kappa_total": d["kappa_total"],
        "max_kappa_per_token": int(r.kappa_per_token.max()),
        "pairs_per_iteration": int((f.astype(np.int64) * r.kappa_per_token[:f.size]).sum()),
        "call_s": round(call_s, 4),
        "device_kpp_ms": round(pr.cluster_kpp_ms / max(pr.cluster_calls, 1), 2),
        "device_lloyd_ms": round(pr.cluster_lloyd_ms / max(pr.cluster_calls, 1), 2),
        "host_prep_ms": round(pr.cluster_prep_ms / max(pr.cluster_calls, 1), 2),
        "library_call_ms": round(pr.cluster_call_ms / max(pr.cluster_calls, 1), 2),
        "kappa_sum_ok": bool(int(r.kappa_per_token.sum()) == d["kappa_total"]),
    }
    # The same call on token vectors already resident on the device
    # (tac_cluster_flat_device): no 390 MB upload inside the call.
    dv = device.DeviceArray.from_host(np.ascontiguousarray(v))
    rd = tac.cluster_flat(ids, dv, d["dim"], p)  # warm-up
    device.profile_enable(True)
    device.profile_read(reset=True)
    t0 = time.perf_counter()
    for _ in range(reps):
        rd = tac.cluster_flat(ids, dv, d["dim"], p)
    row["device_input_call_s"] = round((time.perf_counter() - t0) / reps, 4)
    prd = device.profile_read(reset=True)
    device.profile_enable(False)
    row["device_input_host_prep_ms"] = round(prd.cluster_prep_ms / max(prd.cluster_calls, 1), 2)
    row["device_input_same_bits"] = bool(rd.centroids.tobytes() == r.centroids.tobytes() and
                                         np.array_equal(rd.assignments, r.assignments))
    dv.free()
    if with_cpu:
        ns = 200_000
        fs = np.bincount(ids[:ns])
        kap = int(((fs > 0) & (fs < 128)).sum() + 2 * ((fs >= 128) & (fs < 256)).sum()
                  + 0.6 * (fs[fs >= 256] // 39).sum())
        t0 = time.perf_counter()
        ref = orc.tac_cluster_flat(ids[:ns], v[:ns], d["dim"], orc.tac_params(kap, 0))
        cpu_s = time.perf_counter() - t0
        t0 = time.perf_counter()
        got = tac.cluster_flat(ids[:ns], v[:ns], d["dim"], tac.ClusteringParams(kap, 0))
        gpu_s = time.perf_counter() - t0
        row["cpu_sample"] = {
            "rows": ns, "kappa_total": kap, "oracle_s_1thread": round(cpu_s, 3),
            "gpu_call_s": round(gpu_s, 4), "speedup": round(cpu_s / gpu_s, 1),
            "bit_exact": bool(ref.status == 0 and got.centroids.tobytes() == ref.centroids.tobytes()
                              and np.array_equal(got.assignments, ref.assignments)),
        }
    return row


def train_encode_timing(device, dx, n, dim, m, ksub, dinit, steps, warmup):
    """Median train and encode seconds over `steps` (after `warmup`) on
    resident data, with the encode stage's device time."""
    from tac_gpu import pq as pqmod
    dcb = device.DeviceArray(dinit.shape, np.float32)
    dcodes = device.DeviceArray((n, m), pqmod.code_dtype(ksub))
    for _ in range(warmup):
        device.train_device(dx, n, dim, m, ksub, dinit, dcb, 20, NEVER)
        device.encode_device(dx, n, dim, m, ksub, dcb, dcodes)
    device.synchronize()
    tr, en = [], []
    device.profile_enable(True)
    device.profile_read(reset=True)
    for _ in range(steps):
        t0 = time.perf_counter()
        device.train_device(dx, n, dim, m, ksub, dinit, dcb, 20, NEVER)
        device.synchronize()
        t1 = time.perf_counter()
        device.encode_device(dx, n, dim, m, ksub, dcb, dcodes)
        device.synchronize()
        tr.append(t1 - t0)
        en.append(time.perf_counter() - t1)
    p = device.profile_read(reset=True)
    # one more encode alone: the share of vectors its first pass (candidate
    # sets or the matrix-core screen) deferred
    device.encode_device(dx, n, dim, m, ksub, dcb, dcodes)
    device.synchronize()
    pe = device.profile_read(reset=True)
    p.encode_deferred_frac = deferred_frac(pe)
    # the train-then-encode entry: its encode stage is one candidate pass
    # anchored at the last Lloyd codes (device time of that pass)
    te = []
    for _ in range(steps):
        device.profile_read(reset=True)
        device.train_encode_device(dx, n, dim, m, ksub, dinit, dcb, dcodes, 20, NEVER)
        device.synchronize()
        q = device.profile_read(reset=True)
        te.append(q.encode_ms / max(q.encode_launches, 1))
    p.train_encode_stage_ms = statistics.median(te)
    device.profile_kernels(reset=True)
    device.profile_enable(False)
    dcb.free()
    dcodes.free()
    return statistics.median(tr), statistics.median(en), p


def deferred_frac(p) -> float:
    """The share of (vector, subspace) searches the first pass (candidate
    sets or the matrix-core screen) left to the pruned exact search."""
    return (p.cand_deferred + p.screen_deferred) / max(p.cand_vectors + p.screen_vectors, 1)


def search_kind(dsub: int, ksub: int) -> str:
    """The first pass the library picks in the Lloyd loop and in encode
    (cand_wanted / screen_wanted in tac_gpu.hip): candidate sets up to dsub 4
    (and beyond K = 256), the matrix-core screen from dsub 5 on."""
    if ksub > 256 or dsub <= 4:
        return "candidate sets"
    return "matrix-core screen"


def shape_sweep(device, dx, x, steps: int):
    """(m32, dsub 2), (m8, dsub 8) and (m16, ksub 1024) on the resident
    corpus: 20 Lloyd iterations from seeded-shuffle codebooks, then encode."""
    from tac_gpu import synth
    rows = {}
    for name in ("corpus-1.52m-m32d2", "corpus-1.52m-m8d8", "corpus-1.52m-k1024"):
        w = synth.WORKLOADS[name]
        init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
        dinit = device.DeviceArray.from_host(init)
        t_tr, t_en, p = train_encode_timing(device, dx, w.n, w.dim, w.m, w.ksub, dinit, steps, 1)
        dinit.free()
        cb = 1 if w.ksub <= 256 else 2
        enc_ms = p.encode_ms / max(p.encode_launches, 1)
        ebytes = w.n * (4 * w.dim + w.m * cb)
        rows[name] = {
            "m": w.m, "dsub": w.dim // w.m, "ksub": w.ksub, "lloyd_iters": 20,
            "train_s": round(t_tr, 5),
            "assign": search_kind(w.dim // w.m, w.ksub),
            "encode_s": round(t_en, 6), "encode_mvec_per_s": round(w.n / t_en / 1e6, 1),
            "encode_stage_ms": round(enc_ms, 4),
            "encode_hbm_frac": round(ebytes / (enc_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "train_encode_entry_stage_ms": round(p.train_encode_stage_ms, 4),
            "train_encode_entry_hbm_frac": round(
                ebytes / (p.train_encode_stage_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "update_ms_per_iter": round(p.update_ms / max(p.update_iters, 1), 4),
            "assign_ms_per_iter": round(p.assign_ms / max(p.assign_launches, 1), 4),
            "train_streams": int(p.train_streams),
            "candidate_deferred_frac_train": round(deferred_frac(p), 5),
            "candidate_deferred_frac_encode": round(p.encode_deferred_frac, 5),
        }
        rows[name]["cpu_baseline"] = cpu_profile_row(name, t_tr, w.n / t_en / 1e6)
        log(f"{name}: {rows[name]}")
    return rows


def paper_60m(device, steps: int):
    """60,000,000 x 64 residuals generated on the device (Zipf 1.05 over
    262,144 centres, sigma 0.12), resident; m16 k256, 25 Lloyd iterations
    from seeded-shuffle codebooks."""
    from tac_gpu import synth
    w = synth.WORKLOADS["paper-60m"]
    gen = synth.DeviceCorpus(w)
    dx = device.DeviceArray((w.n, w.dim), np.float32)
    t0 = time.perf_counter()
    gen.fill(dx, w.n)
    gen_s = time.perf_counter() - t0
    init = gen.shuffle_init(dx, w.n, w.m, w.ksub, w.seed)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, w.iters, NEVER)  # warm-up
    device.synchronize()
    times = []
    device.profile_enable(True)
    device.profile_read(reset=True)
    for _ in range(steps):
        t0 = time.perf_counter()
        device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, w.iters, NEVER)
        device.synchronize()
        times.append(time.perf_counter() - t0)
    p = device.profile_read(reset=True)
    device.profile_kernels(reset=True)
    device.profile_enable(False)
    for a in (dx, dinit, dcb):
        a.free()
    gen.free()
    t = statistics.median(times)
    return {"workload": "paper-60m", "n": w.n, "dim": w.dim, "m": w.m, "ksub": w.ksub,
            "lloyd_iters": w.iters, "train_s": round(t, 4),
            "ms_per_iter": round(t / w.iters * 1e3, 3),
            "assign_ms_per_iter": round(p.assign_ms / max(p.assign_launches, 1), 3),
            "update_ms_per_iter": round(p.update_ms / max(p.update_iters, 1), 3),
            "train_streams": int(p.train_streams),
            "resident_input_gb": round(w.n * w.dim * 4 / 1e9, 2),
            "device_generation_s": round(gen_s, 2), "timed_runs": steps,
            "data": "synthetic, generated on the device",
            "cpu_baseline": cpu_profile_row("paper-60m", t)}


def stream_200m(device):
    """200,000,000 residuals in 10M-vector chunks (generated on the device as
    the 60M corpus is), encoded against fixed N(0, 0.05^2) codebooks, m16
    k256: device encode time per chunk and the whole stream's HBM rate."""
    from tac_gpu import synth
    w = synth.WORKLOADS["stream-200m"]
    chunk = 10_000_000
    gen = synth.DeviceCorpus(w)
    cb = synth.gauss_codebooks(w.seed, w.m, w.ksub, w.dsub, 0.05)
    dcb = device.DeviceArray.from_host(cb)
    dx = device.DeviceArray((chunk, w.dim), np.float32)
    dcodes = device.DeviceArray((chunk, w.m), np.uint8)
    gen.fill(dx, chunk, 0)
    device.encode_device(dx, chunk, w.dim, w.m, w.ksub, dcb, dcodes)  # warm-up
    device.synchronize()
    enc = []
    deferred = vectors = cell_subspaces = 0
    hist = np.zeros(w.ksub, np.int64)
    t_all = time.perf_counter()
    for k in range(w.n // chunk):
        gen.fill(dx, chunk, k * chunk)
        device.profile_enable(True)
        device.profile_read(reset=True)
        device.encode_device(dx, chunk, w.dim, w.m, w.ksub, dcb, dcodes)
        p = device.profile_read(reset=True)
        device.profile_enable(False)
        enc.append(p.encode_ms)
        deferred += p.cand_deferred
        vectors += p.cand_vectors
        cell_subspaces += p.cell_subspaces
        if k == 0:
            hist += np.bincount(dcodes.to_host().reshape(-1), minlength=w.ksub)
    wall = time.perf_counter() - t_all
    device.profile_kernels(reset=True)
    for a in (dcb, dx, dcodes):
        a.free()
    gen.free()
    tot_ms = float(sum(enc))
    nbytes = w.n * (4 * w.dim + w.m)
    return {"workload": "stream-200m", "n": w.n, "chunk": chunk, "chunks": len(enc),
            "encode_ms_per_chunk": round(statistics.median(enc), 4),
            "encode_s_total": round(tot_ms * 1e-3, 4),
            "encode_mvec_per_s": round(w.n / (tot_ms * 1e-3) / 1e6, 1),
            "hbm_gbs": round(nbytes / (tot_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (tot_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "stream_wall_s": round(wall, 2),
            "codes_in_range_chunk0": int(hist.sum()) == chunk * w.m,
            "candidate_deferred_frac": round(deferred / max(vectors, 1), 5),
            "cell_list_subspaces_per_chunk": round(cell_subspaces / max(len(enc), 1), 2),
            "data": "synthetic, generated on the device chunk by chunk",
            "cpu_baseline": cpu_profile_row("stream-200m", tot_ms * 1e-3,
                                            w.n / (tot_ms * 1e-3) / 1e6)}


# ---------------------------------------------------------------------------
# Counter passes and trace summaries
# ---------------------------------------------------------------------------
COUNTER_PASSES = {
    "corpus": "corpus-1.52m: the benchmarked train (20 Lloyd iterations from seeded-shuffle "
              "codebooks) and encode, one residual-stage call",
    "m8d8": "corpus-1.52m-m8d8: 20-iteration train and encode",
    "m32d2": "corpus-1.52m-m32d2: 20-iteration train and encode",
    "k1024": "corpus-1.52m-k1024: 20-iteration train and encode",
    "stream-chunk": "stream-200m: encode of its first 10M-vector chunk (device-generated rows, "
                    "fixed N(0, 0.05^2) codebooks)",
    "paper-60m": "paper-60m: one 25-iteration train of the 60M-vector corpus (device-generated, "
                 "resident; the generator's launches come first)",
}


def counter_pass(device, errors, lib, synth, which, x, ids, dx):
    """One run of a workload's benchmarked GPU work, for one rocprofv3 counter
    pass, then a 1 GiB device-to-device copy whose counters calibrate the
    byte counts."""
    from tac_gpu import pq as pqmod
    if which == "stream-chunk":
        ws = synth.WORKLOADS["stream-200m"]
        chunk = 10_000_000
        gen = synth.DeviceCorpus(ws)
        xs = device.DeviceArray((chunk, ws.dim), np.float32)
        gen.fill(xs, chunk, 0)
        dcb = device.DeviceArray.from_host(synth.gauss_codebooks(ws.seed, ws.m, ws.ksub,
                                                                 ws.dsub, 0.05))
        codes = device.DeviceArray((chunk, ws.m), np.uint8)
        device.encode_device(xs, chunk, ws.dim, ws.m, ws.ksub, dcb, codes)
        for a in (xs, dcb, codes):
            a.free()
        gen.free()
    elif which == "paper-60m":
        w = synth.WORKLOADS["paper-60m"]
        gen = synth.DeviceCorpus(w)
        xs = device.DeviceArray((w.n, w.dim), np.float32)
        gen.fill(xs, w.n)
        dinit = device.DeviceArray.from_host(gen.shuffle_init(xs, w.n, w.m, w.ksub, w.seed))
        dcb = device.DeviceArray((w.m, w.ksub, w.dsub), np.float32)
        device.train_device(xs, w.n, w.dim, w.m, w.ksub, dinit, dcb, w.iters, NEVER)
        device.synchronize()
        for a in (xs, dinit, dcb):
            a.free()
        gen.free()
    else:
        name = {"corpus": WORKLOAD, "m8d8": "corpus-1.52m-m8d8", "m32d2": "corpus-1.52m-m32d2",
                "k1024": "corpus-1.52m-k1024"}[which]
        w = synth.WORKLOADS[name]
        init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
        dinit = device.DeviceArray.from_host(init)
        dcb = device.DeviceArray(init.shape, np.float32)
        codes = device.DeviceArray((w.n, w.m), pqmod.code_dtype(w.ksub))
        device.train_device(dx, w.n, w.dim, w.m, w.ksub, dinit, dcb, w.iters, NEVER)
        device.encode_device(dx, w.n, w.dim, w.m, w.ksub, dcb, codes)
        for a in (dinit, dcb, codes):
            a.free()
        if which == "corpus":
            residual_stage(device, x, ids, synth.WORKLOADS[WORKLOAD], 1)
    a = device.DeviceArray((1 << 28,), np.float32)
    b = device.DeviceArray((1 << 28,), np.float32)
    errors.check(lib.tac_gpu_memcpy_dtod(b.ptr, a.ptr, a.nbytes))
    device.synchronize()
    print(json.dumps({"counter_pass": which, "work": COUNTER_PASSES[which],
                      "copy_bytes": a.nbytes}), flush=True)


def summarize_trace(out_base: str, trace_dir: str, title: str, commands=()) -> None:
    """OUT.md: every kernel of a rocprofv3 --kernel-trace --stats run (its
    *kernel_stats.csv), with calls, total and average duration."""
    paths = sorted(Path(trace_dir).rglob("*kernel_stats.csv"))
    if not paths:
        raise SystemExit(f"no kernel_stats.csv under {trace_dir}")
    rows = []
    with open(paths[0], newline="") as f:
        for r in csv.DictReader(f):
            name = (r["Name"].removeprefix("(anonymous namespace)::").split("(")[0]
                    .removeprefix("void ").removeprefix("tacgpu::"))
            rows.append((name, int(r["Calls"]), float(r["TotalDurationNs"]),
                         float(r["AverageNs"])))
    rows.sort(key=lambda t: -t[2])
    total = sum(t[2] for t in rows)
    md = [f"# Kernel trace: {title}", "", "Command:", "```"] + list(commands) + ["```", "",
          "| kernel | calls | total ms | share | average us |", "|---|---:|---:|---:|---:|"]
    for name, calls, tot, avg in rows:
        md.append(f"| {name} | {calls} | {tot / 1e6:.3f} | {tot / total:.4f} | {avg / 1e3:.2f} |")
    Path(out_base + ".md").write_text("\n".join(md) + "\n")
    log(f"wrote {out_base}.md ({len(rows)} kernels)")


# ---------------------------------------------------------------------------
def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="skip the shape sweep, 60M, 200M and the rows around the path")
    ap.add_argument("--counter-pass", choices=sorted(COUNTER_PASSES),
                    help="one run of a workload's benchmarked work for rocprofv3 counter "
                         "passes, then a 1 GiB device-to-device copy (the calibration kernel)")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("OUT", "DIR"),
                    help="write OUT.md: the per-kernel table of a rocprofv3 --kernel-trace "
                         "--stats run in DIR")
    ap.add_argument("--trace-title", default="", help="title line for --summarize-trace")
    ap.add_argument("--cpu-protocol", nargs="+", metavar=("OUT_DIR", "WORKLOAD"),
                    help="the CPU baseline protocol of each named workload; writes "
                         "OUT_DIR/cpu_baseline_<workload>.json and .md")
    ap.add_argument("--summarize-pmc", nargs="+", metavar=("OUT", "DIR"),
                    help="write OUT.json and OUT.md: per-kernel averages of rocprofv3 counter "
                         "CSVs in DIRs")
    ap.add_argument("--pmc-command", action="append", default=[],
                    help="a command line that produced the counters or the trace, quoted in OUT.md")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace[0], args.summarize_trace[1], args.trace_title,
                        args.pmc_command)
        return 0
    if args.summarize_pmc:
        if len(args.summarize_pmc) < 2:
            ap.error("--summarize-pmc OUT DIR [DIR ...]")
        summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1:], args.pmc_command)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build runs the PQ path on a single MI355X).", file=sys.stderr)
        return 2

    from tac_gpu import device, errors, lib, synth

    if args.cpu_protocol:
        if len(args.cpu_protocol) < 2:
            ap.error("--cpu-protocol OUT_DIR WORKLOAD [WORKLOAD ...]")
        out_dir = Path(args.cpu_protocol[0])
        for name in args.cpu_protocol[1:]:
            t0 = time.perf_counter()
            rec = cpu_protocol(name)
            write_cpu_profile(out_dir, rec, f"python3 bench.py --cpu-protocol profiles {name}")
            log(f"cpu protocol {name}: {json.dumps(rec)} ({time.perf_counter() - t0:.0f} s)")
        return 0

    w = synth.WORKLOADS[WORKLOAD]
    errors.check(lib.tac_gpu_set_device(0))
    info = device.device_info(0)
    info["name"] = info["name"] or info["arch"]
    t0 = time.perf_counter()
    x, ids = synth.residuals(w, with_ids=True)
    init = synth.shuffle_init(x, w.m, w.ksub, w.seed)
    log(f"generated {w.n:,} x {w.dim} residuals in {time.perf_counter() - t0:.1f} s on {info['name']}")

    n, dim, m, ksub, iters = w.n, w.dim, w.m, w.ksub, w.iters
    dx = device.DeviceArray.from_host(x)
    dinit = device.DeviceArray.from_host(init)
    dcb = device.DeviceArray(init.shape, np.float32)
    dcodes = device.DeviceArray((n, m), np.uint8)

    if args.counter_pass:
        counter_pass(device, errors, lib, synth, args.counter_pass, x, ids, dx)
        return 0

    for i in range(args.warmup):
        device.train_device(dx, n, dim, m, ksub, dinit, dcb, iters, NEVER)
        device.encode_device(dx, n, dim, m, ksub, dcb, dcodes)
        device.synchronize()
        log(f"warmup step {i + 1}/{args.warmup} done")

    # Timed region: host clock around each synchronised train and encode.
    train_s, encode_s = [], []
    device.synchronize()
    t_all = time.perf_counter()
    for i in range(args.steps):
        ts = time.perf_counter()
        device.train_device(dx, n, dim, m, ksub, dinit, dcb, iters, NEVER)
        device.synchronize()
        tm = time.perf_counter()
        device.encode_device(dx, n, dim, m, ksub, dcb, dcodes)
        device.synchronize()
        te = time.perf_counter()
        train_s.append(tm - ts)
        encode_s.append(te - tm)
        log(f"step {i + 1}/{args.steps}: train {1e3 * (tm - ts):.2f} ms, encode {1e3 * (te - tm):.3f} ms")
    total = time.perf_counter() - t_all
    # The same steps again with every kernel bracketed by HIP events on the
    # library's stream (the events themselves lengthen a step, so the value
    # above is timed without them).
    device.profile_enable(True)
    device.profile_read(reset=True)
    device.profile_kernels(reset=True)
    for i in range(args.steps):
        device.train_device(dx, n, dim, m, ksub, dinit, dcb, iters, NEVER)
        device.encode_device(dx, n, dim, m, ksub, dcb, dcodes)
    device.synchronize()
    prof = device.profile_read(reset=True)
    kt = device.profile_kernels(reset=True)
    # The train-then-encode entry (storage.build's chain): whole-call wall
    # time and the device time of its encode pass, which is anchored at the
    # last Lloyd codes instead of grid cells.
    te_wall, te_stage = [], []
    for i in range(args.steps):
        device.train_encode_device(dx, n, dim, m, ksub, dinit, dcb, dcodes, iters, NEVER)
        device.synchronize()
        q = device.profile_read(reset=True)
        te_stage.append(q.encode_ms / max(q.encode_launches, 1))
    device.profile_kernels(reset=True)
    device.profile_enable(False)
    for i in range(args.steps):  # wall time without the per-kernel events
        t0 = time.perf_counter()
        device.train_encode_device(dx, n, dim, m, ksub, dinit, dcb, dcodes, iters, NEVER)
        device.synchronize()
        te_wall.append(time.perf_counter() - t0)
    mean_train = float(np.mean(train_s))
    mean_encode = float(np.mean(encode_s))
    step_ms = 1e3 * (mean_train + mean_encode)
    kernels = kernel_table(kt, args.steps, step_ms)
    traffic = (_load_json(TRAFFIC_FILE) or {}).get("kernels", {})
    valu = (_load_json(VALU_FILE) or {}).get("kernels", {})
    dominant = next(iter(kernels)) if kernels else None
    parts = max(1, int(prof.train_streams))
    roof = (roofline(dominant, kernels[dominant], n, dim, m, ksub, traffic, valu, parts)
            if dominant else None)
    enc_names = [k for k in kernels if ", true, true," in k or k.startswith(
        ("encode_kernel", "encode_list_kernel"))]
    enc_ms = prof.encode_ms / max(prof.encode_launches, 1)
    ebytes = n * (4 * dim + m)
    # With two training streams the stage timers cover the first half of the
    # subspaces (the second runs beside it), and so do the stage bytes.
    update_ms = prof.update_ms / max(prof.update_iters, 1)
    ubytes = n * (4 * dim + 2 * m) // parts
    assign_ms = prof.assign_ms / max(prof.assign_launches, 1)
    out = {
        "metric": METRIC,
        "value": round(mean_train, 5),
        "unit": "s/20 iters",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * total / args.steps, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": WORKLOAD, "n": n, "dim": dim, "m": m, "dsub": dim // m,
                   "ksub": ksub, "lloyd_iters": iters, "init": "seeded-shuffle prefix",
                   "tol": "never (fixed iterations)", "codes": "u8 token-major"},
        "train_s": round(mean_train, 5),
        "encode_s": round(mean_encode, 6),
        "encode_mvec_per_s": round(n / mean_encode / 1e6, 2),
        "roofline": roof,
        "train_encode_entry": {
            "call_s": round(statistics.median(te_wall), 5),
            "encode_stage_ms": round(statistics.median(te_stage), 4),
            "encode_hbm_frac": round(n * (4 * dim + m) / (statistics.median(te_stage) * 1e-3)
                                     / 1e9 / PEAK_HBM_GBS, 4),
            "anchors": "last Lloyd codes (tac_pq_train_encode_device)"},
        "encode_roofline": {
            "stage": " + ".join(enc_names) if enc_names else None,
            "avg_stage_ms": round(enc_ms, 4), "algorithmic_bytes": ebytes,
            "hbm_gbs": round(ebytes / (enc_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(ebytes / (enc_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "traffic": sum(traffic[k]["read_bytes"] + traffic[k].get("write_bytes", 0)
                           for k in enc_names if k in traffic and "read_bytes" in traffic[k])
                       or None,
        },
        "assign_stage_ms_per_iter": round(assign_ms, 4),
        "train_streams": parts,
        "update_roofline": {
            "avg_iter_ms": round(update_ms, 4), "algorithmic_bytes": ubytes,
            "hbm_gbs": round(ubytes / (update_ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(ubytes / (update_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "traffic": sum(traffic[k]["read_bytes"] + traffic[k].get("write_bytes", 0)
                           for k in traffic if "read_bytes" in traffic[k] and k.startswith(
                               ("hist_kernel", "scan_partial", "scan_apply", "scatter_kernel",
                                "fold_kernel", "reseed_kernel")))
                       or None,
        },
        "kernels": {k: v for k, v in list(kernels.items())[:12]},
        "kernel_timing": (f"HIP events around every kernel on the stream it runs on over "
                          f"{args.steps} further steps of the same workload; training "
                          f"launches cover {m // parts} of the {m} subspaces each, "
                          f"{parts} streams side by side"),
        "candidate_deferred_frac": round(prof.cand_deferred / max(prof.cand_vectors, 1), 4),
        "device": info["name"],
    }
    log(f"train {mean_train * 1e3:.3f} ms, encode {mean_encode * 1e3:.3f} ms; dominant {dominant}")

    # The reference's drop-in defaults (src/index/pq.zig:319-325): k-means++,
    # tol 1e-4, at most 25 iterations.
    device.synchronize()
    t0 = time.perf_counter()
    it_run, _, _ = device.train_device(dx, n, dim, m, ksub, None, dcb, 25, 1e-4, stats=True,
                                       seed=0xa1b2c3d4)
    device.synchronize()
    out["drop_in_defaults"] = {"init": "k-means++ (GPU)", "tol": 1e-4, "max_iters": 25,
                               "iters_run_min": int(it_run.min()),
                               "iters_run_max": int(it_run.max()),
                               "train_s": round(time.perf_counter() - t0, 5)}

    # Full-size parity: 2 GPU iterations, checked inside the CPU baseline.
    device.train_device(dx, n, dim, m, ksub, dinit, dcb, 2, NEVER)
    gpu_cb2 = dcb.to_host().reshape(-1)
    if not args.headline_only:
        out["shape_sweep"] = shape_sweep(device, dx, x, 3)
    for a in (dinit, dcb, dcodes):
        a.free()
    dx.free()
    device.synchronize()
    errors.check(lib.tac_gpu_release_workspace())
    if not args.headline_only:
        out["paper_60m"] = paper_60m(device, 2)
        log(f"paper-60m: {out['paper_60m']}")
        errors.check(lib.tac_gpu_release_workspace())
        out["stream_200m"] = stream_200m(device)
        log(f"stream-200m: {out['stream_200m']}")
        errors.check(lib.tac_gpu_release_workspace())
        out["residual_stage"] = residual_stage(device, x, ids, w, 5)
        out["storage_query"] = storage_and_query(device, x, ids, w,
                                                 synth.centers(w.seed, w.n_centers, w.dim),
                                                 not args.no_cpu_baseline)
        out["tac_clustering"] = tac_clustering(device, not args.no_cpu_baseline)
        log("rows around the path done")

    if not args.no_cpu_baseline:
        log(f"CPU baseline (oracle) on {host_threads()} threads")
        cpu = cpu_baseline(x, init, w, gpu_cb2)
        out["parity_full_size_2_iters_bit_exact"] = cpu.pop("parity_full_size_2_iters")
        full = cpu_profile_row(WORKLOAD)
        if full:
            cpu["full_protocol"] = full
        out["cpu_baseline"] = cpu
        out["speedup_vs_cpu_train"] = round(cpu["value"] / mean_train, 1)
        out["speedup_vs_cpu_encode"] = round(out["encode_mvec_per_s"] / cpu["encode_mvec_per_s"],
                                             1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Summaries of rocprofv3 CSV output for this library's kernels.

Three reports, each printed as a short text table (the files under ``profiles/`` are these
reports with the commands that produced them):

* ``stats DIR``   -- per-kernel launch statistics from ``--kernel-trace --stats`` output
  (``*_kernel_stats.csv``): calls, average / min / max duration, share of GPU time.
* ``pmc DIR``     -- per-kernel per-dispatch averages of every counter in a ``--pmc`` run
  (``*_counter_collection.csv``).
* ``traffic``     -- HBM bytes per call of a stage (the per-dispatch means of the kernels
  matching a pattern, summed) from a ``FETCH_SIZE`` run and a ``WRITE_SIZE`` run, each scaled
  by the factor that makes the same counter read exactly the known bytes of a plain copy kernel
  (``bench.py --copy-calibration``), written as JSON.
* ``util DIR...`` -- per-kernel compute utilisation from one or more ``--pmc`` runs of the same
  command (counters merged by kernel): MFMA busy, MFMA/VALU co-execution, VALU activity, the
  shader clock, and the MFMA operation count, each with the formula it is computed by.
* ``gemm-loop``    -- runs one projection shape back to back for a fixed time, first on this
  build's GEMM (``ops.linear``), then, after an idle gap, on torch's ``F.linear`` (hipBLASLt),
  and prints each one's rate and end time: a steady load for reading the package power and
  clock with ``amd-smi`` / ``rocm-smi`` beside it (GPU box only).

Usage::

    python -m tiktok_techjam_2026_track3_amd.profiling stats gpurun_out/prof_C2
    python -m tiktok_techjam_2026_track3_amd.profiling pmc gpurun_out/fetch_C2
    python -m tiktok_techjam_2026_track3_amd.profiling util gpurun_out/pmc1_C2 gpurun_out/pmc2_C2
    python -m tiktok_techjam_2026_track3_amd.profiling traffic --config C2 --kernel 'attn_fwd_mfma|attn_key_bound' \\
        --fetch gpurun_out/fetch_C2 --write gpurun_out/write_C2 \\
        --copy-fetch gpurun_out/fetch_copy --copy-write gpurun_out/write_copy --copy-bytes N
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys
from collections import defaultdict
from typing import Dict, List

_OURS = re.compile(r"(gemm_kernel|gemm_splitk|gemm_f32_splitk|attn_fwd_mfma|attn_fwd_valu|attn_fwd_f32|attn_key_bound|quant_rows_kernel|layernorm_rows|layernorm_stats)(<[^(]*>|I\w*?EEv)?")
_MANGLED_ARG = re.compile(r"DF16b|DF16_|Li(-?\d+)E|Lb([01])E|[afhsi]")
_TYPE = {"DF16b": "bf16", "DF16_": "f16", "a": "i8", "f": "f32", "h": "u8", "s": "i16", "i": "i32"}
COPY_KERNEL = "neg_kernel"  # the calibration kernel: y = -x, reads and writes every byte once


def _template_args(raw: str) -> str:
    """'<_Float16, 64, true>' or the Itanium-mangled 'IDF16_Li64ELb1EEEv' as 'f16,64,1'."""
    if raw.startswith("<"):
        args = [a.strip() for a in raw[1:-1].split(",")]
        conv = {"float": "f32", "_Float16": "f16", "__bf16": "bf16", "signed char": "i8",
                "true": "1", "false": "0"}
        return ",".join(conv.get(a, a) for a in args)
    out = []
    for m in _MANGLED_ARG.finditer(raw[1:-3]):
        tok = m.group(0)
        out.append(m.group(1) if m.group(1) is not None else
                   m.group(2) if m.group(2) is not None else _TYPE[tok])
    return ",".join(out)


def short_name(name: str) -> str:
    m = _OURS.search(name)
    if m:
        return f"{m.group(1)}<{_template_args(m.group(2)) if m.group(2) else ''}>"[:80]
    m = re.search(r"at::native::[^<(]*?(\w+_kernel\w*)", name)
    if m:
        return ("torch " + m.group(1))[:80]
    return name[:80]


def _find(d: str, suffix: str) -> List[str]:
    files = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return files


def kernel_stats(d: str) -> List[dict]:
    rows = []
    for path in _find(d, "_kernel_stats.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append({"name": r["Name"], "calls": int(r["Calls"]),
                             "total_ns": float(r["TotalDurationNs"]), "avg_ns": float(r["AverageNs"]),
                             "min_ns": float(r["MinNs"]), "max_ns": float(r["MaxNs"]),
                             "pct": float(r["Percentage"])})
    rows.sort(key=lambda r: -r["total_ns"])
    return rows


DURATION = "duration_ns"  # pseudo-counter: the dispatch's duration, when the CSV carries it


def counters(d: str) -> Dict[str, Dict[str, List[float]]]:
    """kernel name -> counter -> per-dispatch values (summed over dimensions of one dispatch);
    ``DURATION`` holds each dispatch's duration when the rows carry start / end timestamps."""
    per = defaultdict(lambda: defaultdict(float))
    names, span = {}, {}
    for path in _find(d, "_counter_collection.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                key = (path, r["Dispatch_Id"])
                names[key] = r["Kernel_Name"]
                per[key][r["Counter_Name"]] += float(r["Counter_Value"])
                if r.get("Start_Timestamp") and r.get("End_Timestamp"):
                    span[key] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    out: Dict[str, Dict[str, List[float]]] = defaultdict(lambda: defaultdict(list))
    for key, vals in per.items():
        for c, v in vals.items():
            out[names[key]][c].append(v)
        if key in span:
            out[names[key]][DURATION].append(span[key])
    return out


def _select(table: Dict[str, Dict[str, List[float]]], pattern: str, counter: str) -> List[float]:
    vals = [v for name, cs in table.items() if re.search(pattern, name) for v in cs.get(counter, [])]
    if not vals:
        raise ValueError(f"no dispatch of a kernel matching {pattern!r} carries {counter}")
    return vals


def _mean(v: List[float]) -> float:
    return sum(v) / len(v)


def stage_sum(rows: List[dict], pattern: str) -> dict:
    """Per-call time of a stage made of several launches (e.g. the attention's key-norm bound
    pass, sweep and redo launch): the average durations of the kernels matching ``pattern``,
    summed (each is launched once per call of the stage)."""
    hit = [r for r in rows if re.search(pattern, r["name"])]
    return {"kernels": [short_name(r["name"]) for r in hit],
            "calls": min((r["calls"] for r in hit), default=0),
            "avg_us": sum(r["avg_ns"] for r in hit) / 1e3}


def print_stats(d: str, groups: List[str] = ()) -> None:
    rows = kernel_stats(d)
    print(f"{'kernel':82s} {'calls':>6s} {'avg_us':>11s} {'min_us':>11s} {'max_us':>11s} {'pct':>6s}")
    for r in rows[:14]:
        print(f"{short_name(r['name']):82s} {r['calls']:6d} {r['avg_ns'] / 1e3:11.2f} "
              f"{r['min_ns'] / 1e3:11.2f} {r['max_ns'] / 1e3:11.2f} {r['pct']:6.1f}")
    for gspec in groups:
        name, _, pattern = gspec.partition("=")
        s = stage_sum(rows, pattern)
        print(f"stage {name}: {s['avg_us']:.2f} us per call (sum of the averages of "
              f"{', '.join(s['kernels'])})")


def print_pmc(d: str) -> None:
    table = counters(d)
    for name in sorted(table, key=lambda n: short_name(n)):
        cs = table[name]
        n = max(len(v) for v in cs.values())
        vals = ", ".join(f"{c}={_mean(v):.6g}" for c, v in sorted(cs.items()))
        print(f"{short_name(name)} [{n} dispatches]: {vals}")


# MI355X: 8 XCDs of 32 CUs, 4 SIMDs per CU; GRBM_GUI_ACTIVE is counted once per XCD
N_XCD, N_CU, SIMD_PER_CU = 8, 256, 4
UTIL_FORMULAS = """\
  cycles      = GRBM_GUI_ACTIVE / 8                      (kernel cycles; the counter is per XCD)
  clock GHz   = cycles / duration
  MFMA busy   = SQ_VALU_MFMA_BUSY_CYCLES / (cycles * 1024 SIMDs)
  co-exec     = SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES
                (share of MFMA-busy cycles in which a VALU instruction also issued)
  VALU active = 4 * SQ_ACTIVE_INST_VALU / (cycles * 1024)  (wave-cycles on VALU instructions,
                MFMA issue included, per SIMD-cycle; two resident waves can each count)
  MFMA ops    = 512 * SQ_INSTS_VALU_MFMA_MOPS_{F16,BF16,I8}  (multiply-adds counted as 2)
  MFMA rate   = MFMA ops / duration
  wait        = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES        (wave time waiting to issue)"""


def utilisation(dirs: List[str]) -> List[dict]:
    """Derived compute utilisation per kernel from one or more ``--pmc`` runs of one command."""
    merged: Dict[str, Dict[str, List[float]]] = defaultdict(dict)
    for d in dirs:
        for name, cs in counters(d).items():
            for c, v in cs.items():
                if c == DURATION and c in merged[name]:
                    merged[name][c] = merged[name][c] + v
                else:
                    merged[name][c] = v
    rows = []
    for name, cs in merged.items():
        m = {c: _mean(v) for c, v in cs.items()}
        cyc = m.get("GRBM_GUI_ACTIVE", 0.0) / N_XCD
        simd_cycles = cyc * N_CU * SIMD_PER_CU
        r = {"kernel": short_name(name),
             "dispatches": max(len(v) for c, v in cs.items() if c != DURATION),
             "cycles": cyc}
        dur = m.get(DURATION)
        if dur:
            r["duration_us"] = dur / 1e3
            r["clock_ghz"] = cyc / dur if cyc else None
        if simd_cycles and "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            r["mfma_busy"] = m["SQ_VALU_MFMA_BUSY_CYCLES"] / simd_cycles
            if "SQ_VALU_MFMA_COEXEC_CYCLES" in m and m["SQ_VALU_MFMA_BUSY_CYCLES"]:
                r["coexec"] = m["SQ_VALU_MFMA_COEXEC_CYCLES"] / m["SQ_VALU_MFMA_BUSY_CYCLES"]
        if simd_cycles and "SQ_ACTIVE_INST_VALU" in m:
            r["valu_active"] = 4.0 * m["SQ_ACTIVE_INST_VALU"] / simd_cycles
        ops = sum(m.get(f"SQ_INSTS_VALU_MFMA_MOPS_{t}", 0.0) for t in ("F16", "BF16", "I8")) * 512
        if ops:
            r["mfma_ops"] = ops
            if dur:
                r["mfma_tops"] = ops / dur / 1e3
        if m.get("SQ_WAVE_CYCLES") and "SQ_WAIT_INST_ANY" in m:
            r["wait"] = m["SQ_WAIT_INST_ANY"] / m["SQ_WAVE_CYCLES"]
        for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT"):
            if c in m:
                r[c] = m[c]
        rows.append(r)
    rows.sort(key=lambda r: -r["cycles"])
    return rows


def print_util(dirs: List[str]) -> None:
    print(UTIL_FORMULAS)
    print()
    hdr = (f"{'kernel':44s} {'n':>3s} {'dur_us':>10s} {'GHz':>5s} {'MFMA':>6s} {'coex':>6s} "
           f"{'VALU':>6s} {'wait':>6s} {'MFMA TOP/s':>10s} {'VALU inst':>11s} {'MFMA inst':>10s}")
    print(hdr)
    pct = lambda r, k: f"{100 * r[k]:5.1f}%" if r.get(k) is not None else "     -"
    for r in utilisation(dirs)[:12]:
        print(f"{r['kernel'][:44]:44s} {r['dispatches']:3d} {r.get('duration_us', 0):10.1f} "
              f"{r.get('clock_ghz') or 0:5.2f} {pct(r, 'mfma_busy')} {pct(r, 'coexec')} "
              f"{pct(r, 'valu_active')} {pct(r, 'wait')} {r.get('mfma_tops', 0):10.1f} "
              f"{r.get('SQ_INSTS_VALU', 0):11.4g} {r.get('SQ_INSTS_MFMA', 0):10.4g}")


def _per_kernel_mean(table: Dict[str, Dict[str, List[float]]], pattern: str, counter: str) -> Dict[str, float]:
    """Mean per dispatch of ``counter`` for every kernel (short name) matching ``pattern``."""
    out: Dict[str, List[float]] = defaultdict(list)
    for name, cs in table.items():
        if re.search(pattern, name) and cs.get(counter):
            out[short_name(name)].extend(cs[counter])
    if not out:
        raise ValueError(f"no dispatch of a kernel matching {pattern!r} carries {counter}")
    return {k: _mean(v) for k, v in out.items()}


def traffic(config: str, kernel: str, fetch: str, write: str, copy_fetch: str, copy_write: str,
            copy_bytes: float, stage: str = "attn") -> dict:
    """HBM bytes per call of a stage whose launches are the kernels matching ``kernel`` (a
    regular expression: e.g. the attention kernel's sweep and redo instances and its key-norm
    bound pass): the per-dispatch means of each matching kernel, summed. FETCH_SIZE /
    WRITE_SIZE are in KiB per dispatch."""
    cf = _mean(_select(counters(copy_fetch), COPY_KERNEL, "FETCH_SIZE")) * 1024.0
    cw = _mean(_select(counters(copy_write), COPY_KERNEL, "WRITE_SIZE")) * 1024.0
    f_fetch, f_write = copy_bytes / cf, copy_bytes / cw
    kf = _per_kernel_mean(counters(fetch), kernel, "FETCH_SIZE")
    kw = _per_kernel_mean(counters(write), kernel, "WRITE_SIZE")
    names = sorted(set(kf) | set(kw))
    per = {n: {"fetch_bytes": kf.get(n, 0.0) * 1024.0 * f_fetch,
               "write_bytes": kw.get(n, 0.0) * 1024.0 * f_write} for n in names}
    fb = sum(v["fetch_bytes"] for v in per.values())
    wb = sum(v["write_bytes"] for v in per.values())
    return {"config": config, "stage": stage, "kernel": kernel, "kernels": per,
            "fetch_bytes": fb, "write_bytes": wb, "bytes_per_launch": fb + wb,
            "raw_fetch_kib": sum(kf.values()), "raw_write_kib": sum(kw.values()),
            "copy_bytes": copy_bytes, "copy_fetch_factor": f_fetch, "copy_write_factor": f_write}


def gemm_loop(shape: str, dtype: str, out_dtype: str, seconds: float, gap: float) -> None:
    """The ``gemm-loop`` report (see the module docstring)."""
    import time
    import torch
    from . import ops
    M, N, K = (int(v) for v in shape.split(","))
    dt, odt = getattr(torch, dtype), getattr(torch, out_dtype)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(M, K, device=dev, generator=g).to(dt)
    w = (torch.randn(N, K, device=dev, generator=g) * 0.02).to(dt)
    b = torch.randn(N, device=dev, generator=g) * 0.02
    out = torch.empty(M, N, device=dev, dtype=odt)
    runs = (("this build", lambda: ops.linear(a, w, b, out=out, out_dtype=odt)),
            ("hipBLASLt", lambda: torch.nn.functional.linear(a, w, b.to(dt))))
    for i, (name, f) in enumerate(runs):
        f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0, n = time.time(), 0
        e0.record()
        while time.time() - t0 < seconds:
            for _ in range(50):
                f()
            n += 50
            torch.cuda.synchronize()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        print(f"{name}: {ms:.4f} ms per GEMM, {2.0 * M * N * K / ms / 1e9:.1f} TFLOP/s over {n} calls; "
              f"ended at {time.time():.1f}", flush=True)
        if i == 0:
            time.sleep(gap)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--stage", action="append", default=[], metavar="NAME=REGEX",
                   help="also print the per-call time of a stage made of the matching kernels")
    p = sub.add_parser("pmc")
    p.add_argument("dir")
    t = sub.add_parser("traffic")
    for a in ("config", "kernel", "fetch", "write", "copy-fetch", "copy-write"):
        t.add_argument("--" + a, required=True)
    t.add_argument("--copy-bytes", type=float, required=True)
    t.add_argument("--stage", default="attn", help="the bench stage the kernels make up")
    t.add_argument("--json-out", help="merge the record into this JSON file (keyed by config)")
    u = sub.add_parser("util")
    u.add_argument("dirs", nargs="+")
    gl = sub.add_parser("gemm-loop")
    gl.add_argument("--shape", default="32768,6144,2048", help="M,N,K")
    gl.add_argument("--dtype", default="bfloat16")
    gl.add_argument("--out-dtype", default="float16")
    gl.add_argument("--seconds", type=float, default=12.0)
    gl.add_argument("--gap", type=float, default=3.0)
    a = ap.parse_args(argv)
    if a.cmd == "gemm-loop":
        gemm_loop(a.shape, a.dtype, a.out_dtype, a.seconds, a.gap)
    elif a.cmd == "stats":
        print_stats(a.dir, a.stage)
    elif a.cmd == "pmc":
        print_pmc(a.dir)
    elif a.cmd == "util":
        print_util(a.dirs)
    else:
        rec = traffic(a.config, a.kernel, a.fetch, a.write, a.copy_fetch, a.copy_write, a.copy_bytes,
                      a.stage)
        print(json.dumps(rec, indent=1))
        if a.json_out:
            data = {}
            if os.path.exists(a.json_out):
                with open(a.json_out) as f:
                    data = json.load(f)
            data[a.config] = rec
            with open(a.json_out, "w") as f:
                json.dump(data, f, indent=1, sort_keys=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

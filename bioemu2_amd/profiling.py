"""Summaries of rocprofv3 output for the kernels of this library.

    python -m bioemu2_amd.profiling stats  <kernel_stats.csv> --title T --cmd C [--out F]
    python -m bioemu2_amd.profiling traffic --fetch <counter_collection.csv> --write <counter_collection.csv>
                                            --workload block --calib-bytes B --cmd C [--out F] [--json J]
    python -m bioemu2_amd.profiling pmc <counter_collection.csv>... --title T --cmd C [--bench F] [--flops k=GF,...]

``stats`` turns a ``--kernel-trace --stats -f csv`` kernel table into a short
markdown table.  ``pmc`` averages any ``--pmc`` counters per kernel and adds
the MFMA-busy fraction (rocprofv3's MfmaUtil formula) and the executed bf16
MFMA flops.  ``traffic`` turns two ``--pmc FETCH_SIZE`` / ``--pmc
WRITE_SIZE`` runs of ``bench.py --calibrate-bytes B`` into HBM bytes per launch
for every kernel: each counter (KiB per dispatch) is scaled by what the same
counter reads for torch's elementwise negation of a B-byte bf16 tensor, which
moves exactly B bytes in and B bytes out.  The per-kernel figures are merged
into ``profiles/traffic.json`` under the workload name, together with a hash
of the kernel sources they were measured on; ``bench.py`` reports them as
``roofline.traffic`` only while that hash matches the current sources.
"""

from __future__ import annotations

import argparse
import csv
import hashlib
import json
import re
from collections import defaultdict
from pathlib import Path

TRAFFIC_JSON = Path(__file__).resolve().parents[1] / "profiles" / "traffic.json"
CSRC = Path(__file__).resolve().parent / "csrc"


def csrc_hash() -> str:
    """First 16 hex digits of the SHA-256 of every kernel source (csrc/*.hip, csrc/*.h), in name order."""
    h = hashlib.sha256()
    for f in sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.h"))):
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]

# Kernel-timer names whose kernel function is named differently.
TIMER_TO_KERNEL = {"apb_pair_bias": "pair_bias", "token_layernorm": "token_ln",
                   "transition_pair": "transition_rows", "transition_msa": "transition_rows"}


def short_name(mangled: str) -> str:
    """`_ZN6bioemu12_GLOBAL__N_1<len><name>...` -> name (with a bool/int template tag)."""
    m = re.match(r"_ZN6bioemu12_GLOBAL__N_1(\d+)", mangled)
    if m:
        k = int(m.group(1))
        name = mangled[m.end():m.end() + k]
        rest = mangled[m.end() + k:]
        if rest.startswith("ILb1"):
            return name + "<true>"
        if rest.startswith("ILb0"):
            return name + "<false>"
        mm = re.match(r"ILi(\d+)ELb(\d)", rest)
        if mm:
            return f"{name}<epi={mm.group(1)},trans={mm.group(2)}>"
        mm = re.match(r"ILi(\d+)E", rest)
        if mm:
            return f"{name}<{mm.group(1)}>"
        return name
    m = re.search(r"bioemu::\(anonymous namespace\)::(\w+)(<[^>(]*>)?", mangled)
    if m:
        return m.group(1) + (m.group(2) or "")
    return mangled[:60]


def is_library_kernel(name: str) -> bool:
    return name.startswith("_ZN6bioemu") or re.match(r"(void )?bioemu::", name) is not None


def base_name(short: str) -> str:
    """Kernel function name without template tag and `_kernel` suffix."""
    return re.sub(r"<.*>$", "", short).removesuffix("_kernel")


def stats_markdown(path: str, title: str, cmd: str) -> str:
    rows = list(csv.DictReader(open(path)))
    out = [f"# {title}", "", "Command (from the repo root on the MI355X box):", "", "```", cmd, "```", "",
           "| kernel | calls | avg µs | min µs | max µs | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in rows:
        out.append(f"| `{short_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
    return "\n".join(out) + "\n"


def _per_dispatch(path: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, counter value in KiB) per dispatch, summed over dimensions."""
    acc: dict[int, list] = {}
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        e = acc.setdefault(d, [r["Kernel_Name"], 0.0])
        e[1] += float(r["Counter_Value"])
    return [tuple(acc[d]) for d in sorted(acc)]


def _calibration(dispatches: list[tuple[str, float]]) -> float:
    cal = [v for n, v in dispatches if "neg_kernel" in n]
    if not cal:
        raise SystemExit("no calibration dispatch (torch neg kernel) in the counter file")
    return max(cal)


def traffic(fetch_csv: str, write_csv: str, calib_bytes: int) -> tuple[dict, float, float]:
    """Per kernel base name: average HBM read/write bytes per launch after calibration."""
    fetch = _per_dispatch(fetch_csv, "FETCH_SIZE")
    write = _per_dispatch(write_csv, "WRITE_SIZE")
    f_scale = calib_bytes / _calibration(fetch)
    w_scale = calib_bytes / _calibration(write)
    table: dict[str, dict] = {}
    for counter, disp, scale in (("read", fetch, f_scale), ("write", write, w_scale)):
        sums: dict[str, list] = defaultdict(lambda: [0.0, 0])
        for name, v in disp:
            if not is_library_kernel(name):
                continue
            s = sums[base_name(short_name(name))]
            s[0] += v * scale
            s[1] += 1
        for k, (tot, n) in sums.items():
            table.setdefault(k, {})[counter] = tot / n
    for k, v in table.items():
        v["total"] = v.get("read", 0.0) + v.get("write", 0.0)
    # KiB of counter per real KiB moved: 1 / scale
    return table, 1024.0 / f_scale, 1024.0 / w_scale


def gpu_agent(counter_csv: str) -> tuple[int, int]:
    """(SIMD count, XCD count) of the GPU from the ``*_agent_info.csv`` rocprofv3 writes next to the counters
    (MI355X: 1024 SIMDs, 8 XCDs when the file is absent)."""
    for f in sorted(Path(counter_csv).parent.glob("*agent_info.csv")):
        for r in csv.DictReader(open(f)):
            if r.get("Agent_Type") == "GPU":
                return int(r["Simd_Count"]), int(r["Num_Xcc"])
    return 1024, 8


def pmc(csv_paths: list[str]) -> tuple[dict[str, dict[str, float]], int]:
    """Per library kernel (base name): every counter averaged over its dispatches.

    rocprofv3 writes one value per dispatch and counter, summed over the counter's instances (SEs,
    SIMDs, XCDs); GRBM_GUI_ACTIVE, one per XCD over the same busy window, is therefore divided by the
    XCD count to give the kernel's busy cycles, and MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES /
    (busy cycles x SIMDs), rocprofv3's MfmaUtil."""
    per: dict[str, dict[str, list]] = defaultdict(lambda: defaultdict(lambda: [0.0, set()]))
    simds = 1024
    for path in csv_paths:
        simds, xcc = gpu_agent(path)
        acc: dict[tuple, float] = defaultdict(float)
        names: dict[int, str] = {}
        for r in csv.DictReader(open(path)):
            if not is_library_kernel(r["Kernel_Name"]):
                continue
            d = int(r["Dispatch_Id"])
            names[d] = base_name(short_name(r["Kernel_Name"]))
            v = float(r["Counter_Value"])
            acc[(d, r["Counter_Name"])] += v / xcc if r["Counter_Name"].startswith("GRBM_") else v
        for (d, c), v in acc.items():
            e = per[names[d]][c]
            e[0] += v
            e[1].add((path, d))
    out: dict[str, dict[str, float]] = {}
    for k, counters in per.items():
        row = {c: tot / len(ds) for c, (tot, ds) in counters.items()}
        busy, active = row.get("SQ_VALU_MFMA_BUSY_CYCLES"), row.get("GRBM_GUI_ACTIVE")
        if busy is not None and active:
            row["mfma_busy_pct"] = 100.0 * busy / (active * simds)
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in row:
            row["mfma_bf16_flops"] = 512.0 * row["SQ_INSTS_VALU_MFMA_MOPS_BF16"]
        out[k] = row
    return out, simds


def pmc_markdown(table: dict, title: str, cmd: str, simds: int, flops: dict[str, float]) -> str:
    counters = sorted({c for row in table.values() for c in row if c.isupper() or c.startswith(("SQ_", "GRBM_"))})
    out = [f"# {title}", "", "Commands (from the repo root on the MI355X box):", "", "```", cmd, "```", "",
           f"Per-dispatch averages over every dispatch of each kernel (GRBM_GUI_ACTIVE per XCD).  MFMA busy = "
           f"SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x {simds} SIMDs) (rocprofv3's MfmaUtil); executed bf16 MFMA flops = "
           "SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 (includes non-algorithmic MFMAs); algorithmic = the kernel's "
           "counted work per launch.", "",
           "| kernel | MFMA busy % | executed bf16 MFMA GFLOP | algorithmic GFLOP | " + " | ".join(counters) + " |",
           "|---|---|---|---|" + "---|" * len(counters)]
    for k, row in sorted(table.items(), key=lambda kv: -kv[1].get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)):
        busy = row.get("mfma_busy_pct")
        fl = row.get("mfma_bf16_flops")
        alg = flops.get(k)
        cells = [f"`{k}`", "" if busy is None else f"{busy:.1f}", "" if fl is None else f"{fl / 1e9:.1f}",
                 "" if alg is None else f"{alg / 1e9:.1f}"]
        cells += [f"{row[c]:.4g}" if c in row else "" for c in counters]
        out.append("| " + " | ".join(cells) + " |")
    return "\n".join(out) + "\n"


def bench_flops(path: str) -> dict[str, float]:
    """Algorithmic flops per launch of every MFMA-bound kernel in a ``bench.py`` output line (the last JSON
    line of ``path``), keyed by kernel base name.  Timers that share a kernel (two transition shapes) are
    averaged weighted by launches, as the counters average over every dispatch."""
    line = [ln for ln in open(path) if ln.startswith("{")][-1]
    acc: dict[str, list[float]] = defaultdict(lambda: [0.0, 0.0])
    for timer, v in json.loads(line)["kernels"].items():
        if v.get("bound") != "mfma":
            continue
        work = v["work"] if "work" in v else v["rate"] * v["avg_ms"] * 1e9
        e = acc[TIMER_TO_KERNEL.get(timer, timer)]
        e[0] += work * v["launches_per_step"]
        e[1] += v["launches_per_step"]
    return {k: tot / n for k, (tot, n) in acc.items()}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd_name", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--title", required=True)
    s.add_argument("--cmd", required=True)
    s.add_argument("--out")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--workload", required=True)
    t.add_argument("--calib-bytes", type=int, required=True)
    t.add_argument("--cmd", required=True, help="the two rocprofv3 commands, as run")
    t.add_argument("--out")
    t.add_argument("--json", default=str(TRAFFIC_JSON))
    m = sub.add_parser("pmc")
    m.add_argument("csv", nargs="+")
    m.add_argument("--title", required=True)
    m.add_argument("--cmd", required=True)
    m.add_argument("--flops", default="", help="kernel=GFLOP,... algorithmic work per launch, for the table")
    m.add_argument("--bench", help="a bench.py output file: algorithmic flops per launch of its MFMA kernels")
    m.add_argument("--out")
    a = ap.parse_args(argv)
    if a.cmd_name == "pmc":
        flops = bench_flops(a.bench) if a.bench else {}
        flops.update({kv.split("=")[0]: float(kv.split("=")[1]) * 1e9 for kv in a.flops.split(",") if kv})
        table, simds = pmc(a.csv)
        text = pmc_markdown(table, a.title, a.cmd, simds, flops)
    elif a.cmd_name == "stats":
        text = stats_markdown(a.csv, a.title, a.cmd)
    else:
        table, f_per_kib, w_per_kib = traffic(a.fetch, a.write, a.calib_bytes)
        lines = [f"# HBM traffic per launch — workload `{a.workload}`", "",
                 "Commands (from the repo root on the MI355X box):", "", "```", a.cmd, "```", "",
                 f"Calibration: torch's negation of a {a.calib_bytes} B bf16 tensor (reads and writes exactly that many "
                 f"bytes) read FETCH_SIZE {f_per_kib:.4f} KiB and WRITE_SIZE {w_per_kib:.4f} KiB per real KiB; "
                 "kernel counters below are divided by those factors.", "",
                 f"Kernel sources: `csrc` SHA-256 prefix `{csrc_hash()}`.", "",
                 "| kernel | read MB | write MB | total MB |", "|---|---|---|---|"]
        for k, v in sorted(table.items(), key=lambda kv: -kv[1]["total"]):
            lines.append(f"| `{k}` | {v.get('read', 0) / 1e6:.1f} | {v.get('write', 0) / 1e6:.1f} | "
                         f"{v['total'] / 1e6:.1f} |")
        text = "\n".join(lines) + "\n"
        path = Path(a.json)
        try:
            data = json.loads(path.read_text())
        except (OSError, ValueError):
            data = {}
        data[a.workload] = {"csrc_sha16": csrc_hash(), "kernels": {k: round(v["total"]) for k, v in table.items()}}
        data.setdefault("_calibration", {})[a.workload] = {"fetch_kib_per_kib": round(f_per_kib, 5),
                                                           "write_kib_per_kib": round(w_per_kib, 5)}
        path.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    if a.out:
        Path(a.out).write_text(text)
    else:
        print(text, end="")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

"""Summaries of rocprofv3 output for the MXFP4 MoE expert path.

Command line (run from the repository root on the MI355X box)::

    python -m agent_factory_3_amd.profiling ktrace  <run>_kernel_trace.csv [<run>_marker_api_trace.csv RANGE]
    python -m agent_factory_3_amd.profiling traffic <fetch>_counter_collection.csv \\
                                                     <write>_counter_collection.csv
    python -m agent_factory_3_amd.profiling mfma <run>_counter_collection.csv <run>_agent_info.csv

``ktrace`` turns a ``rocprofv3 --kernel-trace --output-format csv`` trace into
a markdown table (one row per kernel name and grid size: calls, average /
minimum / total duration), optionally restricted to the dispatches that start
inside the roctx range RANGE of a ``--marker-trace`` (``bench.py`` wraps its
timed steps in the range ``bench_timed``).

``traffic`` takes two ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE``
counter collections of ``bench.py --probe traffic`` (which runs one plain
elementwise device copy of a known size, then the layer) and reports, per kernel, the
HBM-side bytes per dispatch: each counter (KiB per dispatch) is scaled by
the factor that makes the copy kernel's reading equal its known size.  The
last line is a machine-readable JSON comment that ``bench.py`` reads for the
``roofline.traffic`` field.

``mfma`` takes one ``rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES
GRBM_GUI_ACTIVE`` collection and the run's agent info and reports, per kernel
and grid, the share of the SIMDs' active cycles with the MFMA pipe busy:
SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x CUs x SIMDs per CU)
(GRBM_GUI_ACTIVE comes summed over the XCDs), and the CUs' busy share
SQ_BUSY_CU_CYCLES / (GRBM_GUI_ACTIVE / XCDs x CUs).
"""
from __future__ import annotations

import collections
import csv
import json
import re
import sys

# the calibration copy of ``bench.py --probe traffic`` (an elementwise
# dst = src * 1 kernel, so it runs as a kernel and not on a copy engine):
# bytes read == bytes written
COPY_BYTES = 512 * 1024 * 1024
COPY_KERNEL = "MulFunctor"

# grouped-GEMM entry points timed by bench.py -> the kernel their default tile
# configuration launches (forward: tile_cfg 26, input gradient: tile_cfg 28)
GEMM_KERNELS = {"moe_gemm_fwd": "gemm7_fwd_kernel", "moe_gemm_dgrad": "gemm8_dgrad_kernel"}


def short_name(name: str) -> str:
    s = name.replace("(anonymous namespace)::", "")
    s = re.sub(r"^void ", "", s)
    depth, out = 0, []
    for ch in s:  # cut the argument list, keep template arguments
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            break
        out.append(ch)
    return "".join(out).strip()


def marker_window(path: str, name: str) -> tuple[int, int]:
    """(start, end) timestamps of the roctx range ``name`` in a ``rocprofv3
    --marker-trace`` CSV (the earliest start and latest end of the rows that
    carry the name in any column)."""
    spans = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in csv.DictReader(open(path))
             if name in r.values()]
    if not spans:
        raise SystemExit(f"no marker named {name!r} in {path}")
    return min(s for s, _ in spans), max(e for _, e in spans)


def ktrace(path: str, window: tuple[int, int] | None = None) -> str:
    """Markdown table of a kernel trace, one row per (kernel, grid); with
    ``window`` only the dispatches that start inside it.  A second table gives
    the average duration over all grids of each grouped-GEMM entry point's
    kernel, the per-launch figure bench.py reports as ``roofline.avg_launch_us``."""
    rows = list(csv.DictReader(open(path)))
    agg = collections.defaultdict(list)
    for r in rows:
        if window and not window[0] <= int(r["Start_Timestamp"]) <= window[1]:
            continue
        grid = r.get("Grid_Size_X") or r.get("Grid_Size") or ""
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        agg[(short_name(r["Kernel_Name"]), grid)].append(dur)
    tot = sum(sum(v) for v in agg.values()) or 1.0
    lines = ["| kernel | grid | calls | avg us | min us | total us | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for (k, g), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        k = k if len(k) <= 100 else k[:96] + " ..."  # library kernels (hipBLASLt's Cijk_*) carry very long names
        lines.append(f"| `{k}` | {g} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {sum(v):.1f} | "
                     f"{100 * sum(v) / tot:.2f} |")
    lines += ["", "| entry point | kernel | launches | avg us per launch (all grids) |", "|---|---|---:|---:|"]
    for tag, kname in GEMM_KERNELS.items():
        v = [d for (k, _), ds in agg.items() if k.startswith(kname) for d in ds]
        if v:
            lines.append(f"| {tag} | `{kname}` | {len(v)} | {sum(v) / len(v):.2f} |")
    return "\n".join(lines)


def _counter_means(path: str, counter: str) -> dict:
    """(kernel, grid) -> mean counter value per dispatch (counter rows summed per dispatch)."""
    per_dispatch = collections.defaultdict(float)
    key_of = {}
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        d = r["Dispatch_Id"]
        per_dispatch[d] += float(r["Counter_Value"])
        key_of[d] = (short_name(r["Kernel_Name"]), r.get("Grid_Size") or r.get("Grid_Size_X") or "")
    agg = collections.defaultdict(list)
    for d, v in per_dispatch.items():
        agg[key_of[d]].append(v)
    return {k: sum(v) / len(v) for k, v in agg.items()}


def _copy_key(means: dict):
    """The calibration copy kernel (largest reading among the matching names)."""
    cands = [k for k in means if COPY_KERNEL in k[0]]
    if not cands:
        raise SystemExit(f"no {COPY_KERNEL} copy kernel found in the counter collection")
    return max(cands, key=lambda k: means[k])


def traffic(fetch_csv: str, write_csv: str) -> str:
    fetch = _counter_means(fetch_csv, "FETCH_SIZE")
    write = _counter_means(write_csv, "WRITE_SIZE")
    cf, cw = _copy_key(fetch), _copy_key(write)
    f_scale = COPY_BYTES / (fetch[cf] * 1024.0)
    w_scale = COPY_BYTES / (write[cw] * 1024.0)
    lines = [f"Calibration copy `{cf[0]}` (grid {cf[1]}): {COPY_BYTES} B read and written; FETCH_SIZE reads "
             f"{fetch[cf]:.0f} KiB (scale {f_scale:.4f}), WRITE_SIZE reads {write[cw]:.0f} KiB "
             f"(scale {w_scale:.4f}).", "",
             "| kernel | grid | FETCH_SIZE KiB/dispatch | WRITE_SIZE KiB/dispatch | HBM bytes/dispatch (scaled) |",
             "|---|---:|---:|---:|---:|"]
    out = {}
    for k in sorted(set(fetch) & set(write), key=lambda k: -(fetch[k] + write[k])):
        b = fetch[k] * 1024.0 * f_scale + write[k] * 1024.0 * w_scale
        out[f"{k[0]}|{k[1]}"] = {"fetch_kib": fetch[k], "write_kib": write[k], "bytes": b}
        lines.append(f"| `{k[0]}` | {k[1]} | {fetch[k]:.0f} | {write[k]:.0f} | {b:.4g} |")
    lines += ["", "<!-- traffic-json: " + json.dumps({"fetch_scale": f_scale, "write_scale": w_scale,
                                                       "kernels": out}) + " -->"]
    return "\n".join(lines)


def read_traffic(md_path: str) -> dict | None:
    """The JSON block written by ``traffic`` (None when absent)."""
    try:
        text = open(md_path).read()
    except OSError:
        return None
    m = re.search(r"<!-- traffic-json: (.*) -->", text)
    return json.loads(m.group(1)) if m else None


def _gpu_agent(agent_csv: str) -> tuple[int, int, int]:
    """(XCDs, CUs, SIMDs per CU) of the first GPU agent of a rocprofv3 agent-info CSV."""
    for r in csv.DictReader(open(agent_csv)):
        if r.get("Agent_Type", "").strip('"').upper() == "GPU":
            return int(r["Num_Xcc"]), int(r["Cu_Count"]), int(r["Simd_Per_Cu"])
    raise SystemExit("no GPU agent in the agent info")


def mfma(counters_csv: str, agent_csv: str, kernels: tuple[str, ...] = ("gemm", "lug_", "lwg_", "lrows_")) -> str:
    xcd, cus, simds = _gpu_agent(agent_csv)
    busy = _counter_means(counters_csv, "SQ_VALU_MFMA_BUSY_CYCLES")
    cu = _counter_means(counters_csv, "SQ_BUSY_CU_CYCLES")
    gui = _counter_means(counters_csv, "GRBM_GUI_ACTIVE")
    lines = [f"GPU: {xcd} XCDs, {cus} CUs, {simds} SIMDs per CU.", "",
             "| kernel | grid | GUI-active cycles per XCD | MFMA busy share | CU busy share |",
             "|---|---:|---:|---:|---:|"]
    for k in sorted(set(busy) & set(gui), key=lambda k: -gui[k]):
        if not any(n in k[0] for n in kernels) or gui[k] <= 0:
            continue
        g = gui[k] / xcd
        cu_s = f"{cu[k] / (g * cus):.3f}" if k in cu else "-"
        lines.append(f"| `{k[0]}` | {k[1]} | {g:.4g} | {busy[k] / (g * cus * simds):.3f} | {cu_s} |")
    return "\n".join(lines)


def main(argv: list[str]) -> int:
    if len(argv) in (2, 4) and argv[0] == "ktrace":
        print(ktrace(argv[1], marker_window(argv[2], argv[3]) if len(argv) == 4 else None))
        return 0
    if len(argv) >= 3 and argv[0] == "traffic":
        print(traffic(argv[1], argv[2]))
        return 0
    if len(argv) == 3 and argv[0] == "mfma":
        print(mfma(argv[1], argv[2]))
        return 0
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))

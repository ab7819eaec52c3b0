"""Summaries of rocprofv3 CSV output for the k-quant kernels.

    python -m engine_amd.profiling trace <dir-or-kernel_trace.csv>
    python -m engine_amd.profiling pmc <dir-or-counter_collection.csv> [--copy-bytes N]
    python -m engine_amd.profiling source-hash
    python -m engine_amd.profiling decode-steps <dir-or-kernel_trace.csv> [--steps N]
    python -m engine_amd.profiling prompt <dir-or-kernel_trace.csv> [--prompts N]

`trace` groups dispatches by (kernel, grid size), since one kernel instance can
serve launches of different shapes (the q/k/v and gate/up groups share one),
and prints count / mean / median / min duration in microseconds.

`pmc` groups counter values the same way and prints the mean per dispatch.
FETCH_SIZE and WRITE_SIZE are reported by rocprofv3 in KiB; with
`--copy-bytes N` the summary also reads the counter on the largest copy kernel
in the run (a device-to-device copy of N bytes reads N and writes N bytes) and
prints the scale factor that maps the counter onto true bytes.

`decode-steps` summarises the last N generation steps of each batch size in
a trace of the decoder: a step ends with its greedy-selection dispatch
(`argmax_final_kernel`, one 64-thread workgroup per member; `argmax_kernel`
in traces of the one-launch form), whose grid tells the batch sizes apart. Per kernel and
grid it prints launches per step, mean duration and time per step, and per
batch size the span and busy time of the window.

`prompt` summarises the prompt-prefill dispatches of a trace (the prefill
matmul, its activation stages, the chunk K/V append and the chunk attention:
kernels no decode step launches) per kernel and grid: launches, mean duration
and time per prompt (`--prompts N`: the trace holds N prompt prefills).

`source-hash` prints the hash of the decode GEMV's sources, recorded in
profile summaries so a stale measurement is recognisable.
"""
from __future__ import annotations

import csv
import glob
import hashlib
import os
import re
import statistics
import sys
from collections import defaultdict

HERE = os.path.dirname(os.path.abspath(__file__))
# The decode GEMV's sources (the kernel the roofline and traffic figures are
# about), including the dispatcher that routes member counts to launch groups.
KERNEL_SOURCES = ("csrc/gemv_f32.hip", "csrc/wave_rows.hpp", "csrc/kquant_device.hpp", "csrc/kquant_launch.hpp",
                  "csrc/gemv_mfma.hip")


def source_hash() -> str:
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(HERE, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def _find(path: str, suffix: str) -> list[str]:
    if os.path.isfile(path):
        return [path]
    return sorted(glob.glob(os.path.join(path, "**", f"*{suffix}"), recursive=True))


def _demangle(name: str) -> str:
    """`_ZN<len>ns<len>name I <literal args> E ...` -> `ns::name<args>` (the kernels' own
    mangling: a namespace, a function and integer/bool template arguments); other
    names come back unchanged."""
    m = re.match(r"_ZN((?:\d+[A-Za-z_][A-Za-z0-9_]*)+)I((?:L[a-z]\d+E)+)E", name)
    if not m:
        return name
    parts, rest = [], m.group(1)
    while rest:
        n = re.match(r"\d+", rest).group(0)
        parts.append(rest[len(n):len(n) + int(n)])
        rest = rest[len(n) + int(n):]
    args = []
    for kind, val in re.findall(r"L([a-z])(\d+)E", m.group(2)):
        args.append(("true" if val == "1" else "false") if kind == "b" else val)
    return "::".join(parts) + "<" + ", ".join(args) + ">"


def short_name(name: str) -> str:
    name = _demangle(name)
    name = name.replace("void ", "", 1).replace("ribn_amd::", "").replace("(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in name:  # drop the argument list, keep template arguments
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out)[:90]


def _grid(row) -> int:
    """Work-items of a dispatch (X * Y * Z of the grid)."""
    if row.get("Grid_Size_X"):
        return int(row["Grid_Size_X"]) * int(row.get("Grid_Size_Y") or 1) * int(row.get("Grid_Size_Z") or 1)
    return int(row.get("Grid_Size") or 0)


def trace_summary(path: str, match: str = "") -> list[tuple]:
    """[(kernel, grid, count, mean_us, median_us, min_us)] sorted by total time."""
    groups: dict[tuple, list[int]] = defaultdict(list)
    for f in _find(path, "kernel_trace.csv"):
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                name = short_name(row["Kernel_Name"])
                if match and match not in name:
                    continue
                grid = _grid(row)
                groups[(name, grid)].append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    out = [(k[0], k[1], len(v), statistics.mean(v) / 1e3, statistics.median(v) / 1e3, min(v) / 1e3)
           for k, v in groups.items()]
    out.sort(key=lambda r: -r[2] * r[3])
    return out


def _dispatches(path: str) -> list[tuple[str, int, int, int]]:
    """[(kernel, grid, start_ns, end_ns)] of a kernel trace in start order."""
    rows = []
    for f in _find(path, "kernel_trace.csv"):
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                rows.append((short_name(row["Kernel_Name"]), _grid(row), int(row["Start_Timestamp"]),
                             int(row["End_Timestamp"])))
    rows.sort(key=lambda r: r[2])
    return rows


def decode_steps_summary(path: str, steps: int = 32) -> list[dict]:
    """Per batch size (argmax grid): the last `steps` steps' kernels, see the module doc."""
    rows = _dispatches(path)
    ends: dict[int, list[int]] = defaultdict(list)
    for i, (name, grid, _, _) in enumerate(rows):
        if name.startswith(("argmax_final_kernel", "argmax_kernel")):
            ends[grid].append(i)
    out = []
    for grid in sorted(ends):
        idx = ends[grid]
        if len(idx) < steps + 1:
            continue
        window = rows[idx[-steps - 1] + 1:idx[-1] + 1]
        groups: dict[tuple, list[int]] = defaultdict(list)
        for name, g, t0, t1 in window:
            groups[(name, g)].append(t1 - t0)
        kernels = sorted(((k[0], k[1], len(v) / steps, statistics.mean(v) / 1e3, sum(v) / steps / 1e3)
                          for k, v in groups.items()), key=lambda r: -r[4])
        span = (window[-1][3] - window[0][2]) / 1e3
        busy = sum(t1 - t0 for _, _, t0, t1 in window) / 1e3
        out.append({"argmax_grid": grid, "steps": steps, "dispatches": len(window), "span_us": span,
                    "busy_us": busy, "kernels": kernels})
    return out


# Kernels only the prompt prefill launches (ribn_amd_qwen3_prefill_prompt).
PROMPT_KERNELS = ("act_f16_kernel", "qgemm", "attn_prefill_kernel", "kv_append_seq_kernel")


def prompt_summary(path: str, prompts: int = 1) -> dict:
    """Prompt-prefill kernels per (kernel, grid): launches per prompt, mean
    duration and time per prompt, plus their busy time per prompt."""
    groups: dict[tuple, list[int]] = defaultdict(list)
    for name, grid, t0, t1 in _dispatches(path):
        if name.startswith(PROMPT_KERNELS):
            groups[(name, grid)].append(t1 - t0)
    kernels = sorted(((k[0], k[1], len(v) / prompts, statistics.mean(v) / 1e3, sum(v) / prompts / 1e3)
                      for k, v in groups.items()), key=lambda r: -r[4])
    busy = sum(r[4] for r in kernels)
    return {"prompts": prompts, "busy_us": busy, "kernels": kernels}


def pmc_summary(path: str) -> dict[tuple, dict[str, float]]:
    """{(kernel, grid): {counter: mean value per dispatch}}."""
    acc: dict[tuple, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    for f in _find(path, "counter_collection.csv"):
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                name = short_name(row["Kernel_Name"])
                grid = int(row.get("Grid_Size") or row.get("Grid_Size_X") or 0)
                acc[(name, grid)][row["Counter_Name"]].append(float(row["Counter_Value"]))
    return {k: {c: statistics.mean(v) for c, v in cs.items()} for k, cs in acc.items()}


def copy_scale(summary: dict, counter: str, copy_bytes: int) -> float | None:
    """True bytes per counter unit, from the copy kernel with the largest counter value."""
    best = None
    for (name, _grid), cs in summary.items():
        if "copy" in name.lower() and counter in cs and cs[counter] > 0:
            if best is None or cs[counter] > best:
                best = cs[counter]
    return None if best is None else copy_bytes / best


def _main(argv: list[str]) -> int:
    if not argv or argv[0] not in ("trace", "pmc", "source-hash", "decode-steps", "prompt"):
        print(__doc__)
        return 2
    if argv[0] == "source-hash":
        print(source_hash())
        return 0
    if argv[0] == "decode-steps":
        steps = int(argv[argv.index("--steps") + 1]) if "--steps" in argv else 32
        for w in decode_steps_summary(argv[1], steps):
            print(f"== argmax grid {w['argmax_grid']}: {w['steps']} steps, {w['dispatches']} dispatches, "
                  f"span {w['span_us'] / w['steps']:.1f} us/step, busy {w['busy_us'] / w['steps']:.1f} us/step")
            print(f"{'kernel':60s} {'grid':>9s} {'per_step':>8s} {'mean_us':>9s} {'us/step':>9s}")
            for name, grid, n, mean, per in w["kernels"]:
                print(f"{name:60s} {grid:9d} {n:8.1f} {mean:9.3f} {per:9.1f}")
        return 0
    if argv[0] == "prompt":
        prompts = int(argv[argv.index("--prompts") + 1]) if "--prompts" in argv else 1
        w = prompt_summary(argv[1], prompts)
        print(f"== {w['prompts']} prompt(s): prompt-prefill kernels busy {w['busy_us']:.1f} us per prompt")
        print(f"{'kernel':66s} {'grid':>9s} {'n/prompt':>8s} {'mean_us':>9s} {'us/prompt':>10s} {'share':>6s}")
        for name, grid, n, mean, per in w["kernels"]:
            print(f"{name:66s} {grid:9d} {n:8.1f} {mean:9.3f} {per:10.1f} {per / w['busy_us']:6.1%}")
        return 0
    if argv[0] == "trace":
        match = argv[2] if len(argv) > 2 else ""
        print(f"{'kernel':90s} {'grid':>9s} {'n':>6s} {'mean_us':>9s} {'median_us':>9s} {'min_us':>9s}")
        for name, grid, n, mean, med, mn in trace_summary(argv[1], match):
            print(f"{name:90s} {grid:9d} {n:6d} {mean:9.3f} {med:9.3f} {mn:9.3f}")
        return 0
    copy_bytes = None
    if "--copy-bytes" in argv:
        copy_bytes = int(argv[argv.index("--copy-bytes") + 1])
    summary = pmc_summary(argv[1])
    counters = sorted({c for cs in summary.values() for c in cs})
    print(f"{'kernel':90s} {'grid':>9s} " + " ".join(f"{c:>14s}" for c in counters))
    for (name, grid), cs in sorted(summary.items()):
        print(f"{name:90s} {grid:9d} " + " ".join(f"{cs.get(c, float('nan')):14.1f}" for c in counters))
    if copy_bytes:
        for c in counters:
            scale = copy_scale(summary, c, copy_bytes)
            if scale is not None:
                print(f"scale {c}: {scale:.3f} bytes per unit (copy of {copy_bytes} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(_main(sys.argv[1:]))

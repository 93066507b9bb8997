"""Measurement helpers: HIP-event timing of library launches and summaries of
rocprofv3 output.

EventTimer is a profile-context factory (see _native.set_profile_ctx_factory):
for the labels it is asked to watch it records a torch.cuda.Event pair on the
current stream around the launch, so the averages are device time of exactly
those kernels, measured inside a larger timed region.

Command line (summaries of rocprofv3 CSV output, written as markdown/JSON):

  python -m repo_amd.profiling stats DIR --title T --cmd "rocprofv3 ..." [--top 20]
      kernel table from DIR/**/*kernel_stats.csv
  python -m repo_amd.profiling traffic --fetch DIR1 --write DIR2 --kernel NAME
      --copy-kernel copyBuffer --copy-bytes B --cmd-fetch "..." --cmd-write "..."
      [--json OUT.json] [--md OUT.md]
      per-dispatch HBM bytes of kernel NAME from FETCH_SIZE / WRITE_SIZE runs,
      scaled by what the same counters read for a plain copy of B bytes.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
from contextlib import contextmanager, nullcontext


class EventTimer:
    """Profile-context factory that times the watched labels with HIP events."""

    def __init__(self, labels):
        self.labels = set(labels)
        self.pairs = {k: [] for k in self.labels}
        self.enabled = True

    def __call__(self, label):
        if not self.enabled or label not in self.labels:
            return nullcontext()
        return self._bracket(label)

    @contextmanager
    def _bracket(self, label):
        import torch
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        yield
        b.record()
        self.pairs[label].append((a, b))

    def mean_ms(self, label):
        """Mean device time (ms) of the label's launches; call after a sync."""
        p = self.pairs.get(label) or []
        if not p:
            return None
        return sum(a.elapsed_time(b) for a, b in p) / len(p)

    def count(self, label):
        return len(self.pairs.get(label) or [])


def _csvs(directory, suffix):
    return sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))


def _short(name):
    name = name.split("(")[0].replace("void ", "")
    return name[:80]


def kernel_stats_md(directory, title, cmd, top=20):
    paths = _csvs(directory, "kernel_stats.csv")
    if not paths:
        raise FileNotFoundError(f"no *kernel_stats.csv under {directory}")
    rows = []
    for p in paths:
        with open(p) as f:
            rows += list(csv.DictReader(f))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    out = [f"# {title}", "", "Command (from the repository root, one MI355X):", "", "```", cmd,
           "```", "", "| kernel | calls | avg us | min us | max us | % of GPU time |",
           "|---|---:|---:|---:|---:|---:|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"]))[:top]:
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} "
                   f"| {float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} "
                   f"| {100 * float(r['TotalDurationNs']) / tot:.1f} |")
    return "\n".join(out) + "\n"


def counter_values(directory, counter, kernel_substr, last=None):
    """Per-dispatch values of `counter` for dispatches whose kernel name
    contains kernel_substr (counter_collection.csv of a --pmc run).  With
    `last`, only the last `last` such dispatches of the run are kept (the
    calibration copies bench.py issues at its very end, not the runtime's
    staging copies)."""
    vals = {}
    for p in _csvs(directory, "counter_collection.csv"):
        with open(p) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != counter or kernel_substr not in r["Kernel_Name"]:
                    continue
                key = (p, int(r["Dispatch_Id"]))
                vals[key] = vals.get(key, 0.0) + float(r["Counter_Value"])
    keys = sorted(vals)
    if last is not None:
        keys = keys[-last:]
    return [vals[k] for k in keys]


def traffic(fetch_dir, write_dir, kernel, copy_kernel, copy_bytes, copy_dispatches=3):
    """HBM bytes per dispatch of `kernel`, each counter scaled by
    copy_bytes / (its mean reading on the copy kernel).  FETCH_SIZE and
    WRITE_SIZE are in KiB."""
    res = {"kernel": kernel, "copy_kernel": copy_kernel, "copy_bytes": copy_bytes}
    runs = (("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE"))
    for name, d, counter in runs:
        k = counter_values(d, counter, kernel)
        c = counter_values(d, counter, copy_kernel, last=copy_dispatches)
        if not k or not c:
            raise RuntimeError(f"{counter}: no dispatches of {kernel!r} or {copy_kernel!r} in {d}")
        raw = statistics.mean(k) * 1024.0
        copy_raw = statistics.mean(c) * 1024.0
        factor = copy_bytes / copy_raw
        res[name] = {"counter": counter, "dispatches": len(k), "copy_dispatches": len(c),
                     "raw_bytes": raw,
                     "copy_raw_bytes": copy_raw, "scale": factor, "bytes": raw * factor}
    res["bytes_per_launch"] = res["fetch"]["bytes"] + res["write"]["bytes"]
    return res


def traffic_md(t, cmd_fetch, cmd_write):
    lines = [f"# HBM traffic per launch of `{t['kernel']}`", "",
             "FETCH_SIZE and WRITE_SIZE (KiB per dispatch) from two rocprofv3 --pmc runs, each "
             f"scaled by what the same counter reads for a plain copy of {t['copy_bytes']} bytes "
             f"(kernel `{t['copy_kernel']}`, which reads and writes exactly that many bytes).",
             "", "Commands (from the repository root, one MI355X):", "", "```", cmd_fetch,
             cmd_write, "```", "", "| counter | dispatches | raw MB | copy reads MB | scale | "
             "bytes per launch (MB) |", "|---|---:|---:|---:|---:|---:|"]
    for k in ("fetch", "write"):
        r = t[k]
        lines.append(f"| {r['counter']} | {r['dispatches']} | {r['raw_bytes'] / 1e6:.3f} | "
                     f"{r['copy_raw_bytes'] / 1e6:.3f} | {r['scale']:.4f} | "
                     f"{r['bytes'] / 1e6:.3f} |")
    lines += ["", f"Total HBM traffic per launch: {t['bytes_per_launch'] / 1e6:.3f} MB", ""]
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m repo_amd.profiling")
    sub = ap.add_subparsers(dest="what", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--title", required=True)
    s.add_argument("--cmd", required=True)
    s.add_argument("--top", type=int, default=20)
    s.add_argument("--out")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-kernel", default="copyBuffer")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--cmd-fetch", required=True)
    t.add_argument("--cmd-write", required=True)
    t.add_argument("--json")
    t.add_argument("--md")
    a = ap.parse_args(argv)
    if a.what == "stats":
        md = kernel_stats_md(a.dir, a.title, a.cmd, a.top)
        if a.out:
            with open(a.out, "w") as f:
                f.write(md)
        print(md)
    else:
        res = traffic(a.fetch, a.write, a.kernel, a.copy_kernel, a.copy_bytes)
        res["commands"] = [a.cmd_fetch, a.cmd_write]
        if a.json:
            with open(a.json, "w") as f:
                json.dump(res, f, indent=1)
        md = traffic_md(res, a.cmd_fetch, a.cmd_write)
        if a.md:
            with open(a.md, "w") as f:
                f.write(md)
        print(md)


if __name__ == "__main__":
    main()

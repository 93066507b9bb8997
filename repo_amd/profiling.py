"""Measurement helpers: HIP-event timing of library launches and summaries of
rocprofv3 output.

EventTimer is a profile-context factory (see _native.set_profile_ctx_factory):
for the labels it is asked to watch it records a HIP event pair on the
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
  python -m repo_amd.profiling counters DIR... --title T --cmd "..." [--kernel K]
      VALU / SALU busy, lane utilisation, LDS bank conflicts per kernel from
      SQ counter runs.
  python -m repo_amd.profiling hbm --stats D --fetch D1 --write D2 --copy-bytes B
      --title T --cmd "..." [--kernel K] [--alg SUBSTRING=BYTES]
      HBM GB/s per kernel (scaled FETCH_SIZE + WRITE_SIZE over the mean
      duration of a kernel-trace run).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
from contextlib import nullcontext


class _Bracket:
    __slots__ = ("timer", "label", "a", "b")

    def __init__(self, timer, label, a, b):
        self.timer, self.label, self.a, self.b = timer, label, a, b

    def __enter__(self):
        t = self.timer
        rc = t._rec(self.a, t._stream(t._dev()))
        if rc:
            t._N.hip_check(rc, "hipEventRecord")

    def __exit__(self, *exc):
        t = self.timer
        rc = t._rec(self.b, t._stream(t._dev()))
        if rc:
            t._N.hip_check(rc, "hipEventRecord")
        t.pairs[self.label].append((self.a, self.b))
        return False


class EventTimer:
    """Profile-context factory that times the watched labels with HIP events
    recorded on the current stream around the launch.  Event pairs are created
    up front (`reserve` per label) and reused, so a timed launch costs two
    event records on the host and nothing else.  close() releases the events
    (after the averages have been read)."""

    _NULL = nullcontext()

    def __init__(self, labels, reserve=128):
        import torch
        from . import _native as N
        self.labels = set(labels)
        self.pairs = {k: [] for k in self.labels}
        self._N = N
        self._rec = N.hip().hipEventRecord
        self._stream = torch._C._cuda_getCurrentRawStream
        self._dev = torch.cuda.current_device
        self._all = []
        self._pool = [self._pair() for _ in range(reserve * len(self.labels))]
        self.enabled = True

    def _pair(self):
        a, b = self._N.event_create(timing=True), self._N.event_create(timing=True)
        self._all += [a, b]
        return a, b

    def __call__(self, label):
        if not self.enabled or label not in self.labels:
            return self._NULL
        a, b = self._pool.pop() if self._pool else self._pair()
        return _Bracket(self, label, a, b)

    def mean_ms(self, label):
        """Mean device time (ms) of the label's launches; call after a sync."""
        p = self.pairs.get(label) or []
        if not p:
            return None
        return sum(self._N.event_elapsed_ms(a, b) for a, b in p) / len(p)

    def count(self, label):
        return len(self.pairs.get(label) or [])

    def close(self):
        for h in self._all:
            self._N.event_destroy(h)
        self._all, self._pool = [], []
        self.pairs = {k: [] for k in self.labels}


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


# MI355X: 256 compute units in 8 XCDs; GRBM_GUI_ACTIVE is reported per XCD
# and summed over them in a dispatch's counter record.
CU_NUM = 256
XCD_NUM = 8
HBM_PEAK_GBS = 8000.0


def per_kernel_counters(directories):
    """{kernel: {counter: mean per dispatch}} over the counter_collection.csv
    files of several --pmc runs (one counter set each)."""
    acc = {}
    for d in directories:
        for p in _csvs(d, "counter_collection.csv"):
            per_dispatch = {}
            with open(p) as f:
                for r in csv.DictReader(f):
                    key = (_short(r["Kernel_Name"]), int(r["Dispatch_Id"]))
                    per_dispatch.setdefault(key, {}).setdefault(r["Counter_Name"], 0.0)
                    per_dispatch[key][r["Counter_Name"]] += float(r["Counter_Value"])
            for (name, _), vals in per_dispatch.items():
                for c, v in vals.items():
                    acc.setdefault(name, {}).setdefault(c, []).append(v)
    return {k: {c: statistics.mean(v) for c, v in cs.items()} for k, cs in acc.items()}


def derived_metrics(c):
    """rocprofv3's derived metrics from raw SQ counters of one dispatch
    (GRBM_GUI_ACTIVE summed over the XCDs, so its per-XCD value is / 8)."""
    out = {}
    grbm = c.get("GRBM_GUI_ACTIVE")
    if not grbm:
        return out
    active = grbm / XCD_NUM
    if "SQ_ACTIVE_INST_VALU" in c:
        out["VALUBusy %"] = 100.0 * c["SQ_ACTIVE_INST_VALU"] / CU_NUM / active
    if "SQ_THREAD_CYCLES_VALU" in c and c.get("SQ_ACTIVE_INST_VALU"):
        out["VALU lane util %"] = 100.0 * c["SQ_THREAD_CYCLES_VALU"] / (
            c["SQ_ACTIVE_INST_VALU"] * 64.0)
    if "SQ_INST_CYCLES_SALU" in c:
        out["SALUBusy %"] = 100.0 * c["SQ_INST_CYCLES_SALU"] / CU_NUM / active
    if "SQ_LDS_BANK_CONFLICT" in c:
        out["LDS bank conflict %"] = 100.0 * c["SQ_LDS_BANK_CONFLICT"] / active / CU_NUM
    if "SQ_WAVE_CYCLES" in c:  # counted per 4 cycles (rocprofv3's OccupancyPercent)
        out["waves per CU"] = 4.0 * c["SQ_WAVE_CYCLES"] / active / CU_NUM
    for k in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_SMEM", "SQ_INSTS_LDS"):
        if k in c and c.get("SQ_WAVES"):
            out[k.replace("SQ_INSTS_", "") + " / wave"] = c[k] / c["SQ_WAVES"]
    return out


def counters_md(directories, kernels, title, cmds):
    kc = per_kernel_counters(directories)
    rows = []
    cols = ["VALUBusy %", "VALU lane util %", "SALUBusy %", "LDS bank conflict %",
            "waves per CU", "VALU / wave", "SALU / wave", "SMEM / wave", "LDS / wave"]
    for name in sorted(kc):
        if kernels and not any(k in name for k in kernels):
            continue
        d = derived_metrics(kc[name])
        rows.append((name, d))
    out = [f"# {title}", "", "rocprofv3 --pmc passes (each a separate run of the same command, "
           "from the repository root, one MI355X):", "", "```", *cmds, "```", "",
           "Derived as rocprofv3 defines them (VALUBusy = SQ_ACTIVE_INST_VALU / CU_NUM / "
           "GRBM_GUI_ACTIVE; VALU lane util = SQ_THREAD_CYCLES_VALU / (SQ_ACTIVE_INST_VALU x 64); "
           "SALUBusy = SQ_INST_CYCLES_SALU / CU_NUM / GRBM_GUI_ACTIVE; LDS bank conflict = "
           "SQ_LDS_BANK_CONFLICT / GRBM_GUI_ACTIVE / CU_NUM; waves per CU = 4 SQ_WAVE_CYCLES "
           "/ GRBM_GUI_ACTIVE / CU_NUM, at most 32), GRBM_GUI_ACTIVE per XCD, "
           f"CU_NUM = {CU_NUM}; means over each kernel's dispatches.", "",
           "| kernel | " + " | ".join(cols) + " |", "|---|" + "---:|" * len(cols)]
    for name, d in rows:
        out.append(f"| `{name}` | " + " | ".join(
            (f"{d[c]:.1f}" if c in d else "-") for c in cols) + " |")
    return "\n".join(out) + "\n"


def kernel_avg_ns(directory):
    out = {}
    for p in _csvs(directory, "kernel_stats.csv"):
        with open(p) as f:
            for r in csv.DictReader(f):
                out[_short(r["Name"])] = (float(r["AverageNs"]), int(r["Calls"]))
    return out


def hbm_md(stats_dir, fetch_dir, write_dir, copy_kernel, copy_bytes, title, cmds, kernels,
           algorithmic=None):
    """Per kernel: HBM bytes per dispatch (FETCH_SIZE and WRITE_SIZE scaled by
    a copy of copy_bytes), mean duration from a kernel-trace run, GB/s and
    the fraction of the 8 TB/s peak; with `algorithmic` ({substring: bytes})
    also the algorithmic bytes' rate."""
    ns = kernel_avg_ns(stats_dir)
    fk = per_kernel_counters([fetch_dir])
    wk = per_kernel_counters([write_dir])
    cf = counter_values(fetch_dir, "FETCH_SIZE", copy_kernel, last=3)
    cw = counter_values(write_dir, "WRITE_SIZE", copy_kernel, last=3)
    sf = copy_bytes / (statistics.mean(cf) * 1024.0)
    sw = copy_bytes / (statistics.mean(cw) * 1024.0)
    out = [f"# {title}", "", "Commands (from the repository root, one MI355X):", "", "```", *cmds,
           "```", "", f"FETCH_SIZE scaled by x{sf:.3f} and WRITE_SIZE by x{sw:.3f}: the factors "
           f"that make each counter read {copy_bytes} bytes for the plain device copy "
           f"(`{copy_kernel}`) at the end of the same runs.  Durations: mean over the "
           "kernel-trace run's dispatches.  Peak: 8 TB/s.", "",
           "| kernel | us | fetched MB | written MB | HBM GB/s | % of peak | algorithmic MB "
           "| algorithmic GB/s |", "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for name in sorted(ns, key=lambda n: -ns[n][0] * ns[n][1]):
        if kernels and not any(k in name for k in kernels):
            continue
        if name not in fk or name not in wk:
            continue
        t = ns[name][0] * 1e-9
        fb = fk[name].get("FETCH_SIZE", 0.0) * 1024.0 * sf
        wb = wk[name].get("WRITE_SIZE", 0.0) * 1024.0 * sw
        gbs = (fb + wb) / t / 1e9
        alg = None
        for k, v in (algorithmic or {}).items():
            if k in name:
                alg = v
        out.append(f"| `{name}` | {t * 1e6:.1f} | {fb / 1e6:.2f} | {wb / 1e6:.2f} | {gbs:.0f} "
                   f"| {100 * gbs / HBM_PEAK_GBS:.1f} | "
                   + (f"{alg / 1e6:.2f} | {alg / t / 1e9:.0f} |" if alg else "- | - |"))
    return "\n".join(out) + "\n"


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
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--title", required=True)
    c.add_argument("--cmd", action="append", required=True)
    c.add_argument("--kernel", action="append")
    c.add_argument("--out")
    h = sub.add_parser("hbm")
    h.add_argument("--stats", required=True)
    h.add_argument("--fetch", required=True)
    h.add_argument("--write", required=True)
    h.add_argument("--copy-kernel", default="copyBuffer")
    h.add_argument("--copy-bytes", type=int, required=True)
    h.add_argument("--title", required=True)
    h.add_argument("--cmd", action="append", required=True)
    h.add_argument("--kernel", action="append")
    h.add_argument("--alg", action="append", default=[],
                   help="SUBSTRING=BYTES algorithmic bytes per dispatch")
    h.add_argument("--out")
    a = ap.parse_args(argv)
    if a.what in ("counters", "hbm"):
        if a.what == "counters":
            md = counters_md(a.dirs, a.kernel, a.title, a.cmd)
        else:
            alg = {k: float(v) for k, v in (x.split("=", 1) for x in a.alg)}
            md = hbm_md(a.stats, a.fetch, a.write, a.copy_kernel, a.copy_bytes, a.title, a.cmd,
                        a.kernel, alg)
        if a.out:
            with open(a.out, "w") as f:
                f.write(md)
        print(md)
        return
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

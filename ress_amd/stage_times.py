"""GPU time per stage from a rocprofv3 run with the stage ranges on (ress_amd.trace):

    RESS_ROCTX=1 rocprofv3 --marker-trace --hip-runtime-trace --kernel-trace -d DIR -o PREFIX \\
        --output-format csv -- python3 bench.py
    python -m ress_amd.stage_times DIR PREFIX

Each kernel in PREFIX_kernel_trace.csv is tied, by its correlation id, to the HIP call that launched it
(PREFIX_hip_api_trace.csv), and that call to the innermost roctx range open on the same thread when it
started (PREFIX_marker_api_trace.csv). A stage's GPU time is the sum of its kernels' execution times.
Kernels launched outside every range (the caller's own work) are reported as one line."""

import collections
import csv
import os
import sys

OUTSIDE = "(outside any range)"


def _rows(d, prefix, what):
    with open(os.path.join(d, f"{prefix}_{what}.csv"), newline="") as f:
        return list(csv.DictReader(f))


def short_name(kernel_name):
    """A kernel's name without return type, namespace, template arguments or parameters."""
    n = kernel_name.replace("(anonymous namespace)::", "")
    if n.startswith("void "):
        n = n[5:]
    return n.split("(")[0].split("<")[0]


def stage_times(d, prefix):
    """{stage: (ranges, kernels, GPU ns, {kernel: ns})} for one rocprofv3 output directory."""
    ranges = collections.defaultdict(list)
    opened = collections.Counter()
    for m in _rows(d, prefix, "marker_api_trace"):
        ranges[m["Thread_Id"]].append((int(m["Start_Timestamp"]), int(m["End_Timestamp"]), m["Function"]))
        opened[m["Function"]] += 1
    launch = {a["Correlation_Id"]: (a["Thread_Id"], int(a["Start_Timestamp"]))
              for a in _rows(d, prefix, "hip_api_trace")}
    out = {}
    for k in _rows(d, prefix, "kernel_trace"):
        stage, at = OUTSIDE, launch.get(k["Correlation_Id"])
        if at is not None:
            inner = None
            for s, e, name in ranges.get(at[0], ()):
                if s <= at[1] <= e and (inner is None or s > inner[0]):
                    inner = (s, name)
            if inner is not None:
                stage = inner[1]
        ns = int(k["End_Timestamp"]) - int(k["Start_Timestamp"])
        n_ranges, n_kernels, total, per_kernel = out.get(stage, (opened.get(stage, 0), 0, 0, collections.Counter()))
        per_kernel[short_name(k["Kernel_Name"])] += ns
        out[stage] = (n_ranges, n_kernels + 1, total + ns, per_kernel)
    return out


def report(times):
    grand = sum(t[2] for t in times.values()) or 1
    lines = [f"{'stage':26s} {'ranges':>6s} {'kernels':>7s} {'GPU ms':>10s} {'us/range':>9s} {'share':>6s}  top kernels"]
    for stage, (n, nk, ns, per) in sorted(times.items(), key=lambda kv: -kv[1][2]):
        top = ", ".join(f"{name} {t / 1e6:.2f} ms" for name, t in per.most_common(3))
        lines.append(f"{stage:26s} {n:6d} {nk:7d} {ns / 1e6:10.3f} {(ns / n / 1e3 if n else 0):9.1f} "
                     f"{100 * ns / grand:5.1f}%  {top}")
    lines.append(f"all kernels: {grand / 1e6:.3f} ms")
    return "\n".join(lines)


if __name__ == "__main__":
    if len(sys.argv) != 3:
        sys.exit("usage: python -m ress_amd.stage_times DIR PREFIX")
    print(report(stage_times(sys.argv[1], sys.argv[2])))

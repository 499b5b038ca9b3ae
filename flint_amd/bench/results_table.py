"""Renders flint_bench's "flint-bench/1" JSON logs as Markdown tables (the
counterpart of the reference's scripts/results_table.py:1-236).

Usage: python -m flint_amd.bench.results_table LOG.json [LOG.json ...]

Each log gets a heading line (device, commit, command, protocol) and one row per
case. Bandwidth cases (copy) show GB/s and the fraction of the 8 TB/s HBM peak;
compute cases (mma, gemm) show TFLOP/s and the fraction of the dense FP16 MFMA
peak at the rated clock; with monitor statistics, also the mean graphics clock
over Flint's samples, the fraction of the peak at that clock, and the share of
the time the firmware's power cap (PPT) held the clock down. Two-sided cases add the baseline and the median ratio
(baseline time / Flint time, above 1 when Flint is faster) with its range.
A log whose numbers should not be quoted (a --quick run, options below the
standard protocol, an unknown or dirty commit, a case that is not ok) says why.
"""

import argparse
import json
import sys


def problems(log):
    """Why a log's numbers should not be quoted, if they should not."""
    found = []
    if log["quick"]:
        found.append("a --quick run")
    elif not log["standard_protocol"]:
        found.append("options below the standard protocol")
    if log["git"]["sha"] == "unknown":
        found.append("built outside a git checkout")
    elif log["git"]["dirty"]:
        found.append("built from a tree with uncommitted changes")
    if not all(case["ok"] for case in log["cases"]):
        found.append("a case that is not ok")
    return found


def case_name(case):
    name = case["benchmark"]
    if case.get("layout"):
        name += " " + case["layout"]
        if case.get("epilogue") not in (None, "none"):
            name += "+" + case["epilogue"]
    return f"{name} {case['label']}"


def pct(fraction):
    return f"{100 * fraction:.1f}%"


def rate(case, side):
    if case["flops"] > 0:
        return f"{side['tflops']:.1f}", pct(side["rated_compute_fraction"])
    return f"{side['gbs']:.1f}", pct(side["rated_fraction"])


def algorithm(case):
    a = case.get("baseline_algorithm")
    if not a:
        return "-"
    used = a["candidates"][a["used"]]
    return f"{a['selection']}: #{used['index']} of {len(a['candidates'])} (solution {used['solution_index']})"


def table(log):
    lines = []
    d = log["device"]
    sha = log["git"]["sha"][:12]
    lines.append(f"{d['name']} ({d['arch']}, {d['cu_count']} CUs, {d['rated_sm_clock_mhz']:.0f} MHz), "
                 f"commit {sha}, `flint_bench {' '.join(log['args'])}`, {log['timestamp_utc']}")
    why = problems(log)
    if why:
        lines.append("")
        lines.append("Not for quoting: " + "; ".join(why) + ".")
    lines.append("")
    compute = any(c["flops"] > 0 for c in log["cases"])
    unit = "TFLOP/s" if compute else "GB/s"
    peak = "of FP16 peak" if compute else "of HBM peak"
    has_baseline = any(not c["one_sided"] for c in log["cases"])
    has_algo = any(c.get("baseline_algorithm") for c in log["cases"])
    monitored = any(c["flint"].get("stats") for c in log["cases"])
    head = ["Case", "Flint ms", f"Flint {unit}", peak]
    if monitored and compute:
        head += ["SCLK MHz", "of peak at SCLK", "power-capped"]
    elif monitored:
        head += ["MCLK MHz", "of HBM peak at MCLK"]
    if has_baseline:
        head += ["Baseline", f"Baseline {unit}", "Ratio (median)", "Ratio range"]
    if has_algo:
        head += ["Baseline algorithm"]
    head += ["Rounds", "Check"]
    lines.append("| " + " | ".join(head) + " |")
    lines.append("|" + "---|" * len(head))
    for c in log["cases"]:
        value, frac = rate(c, c["flint"])
        row = [case_name(c), f"{c['flint']['ms_per_launch']:.4f}", value, frac]
        if monitored and compute:
            st = c["flint"].get("stats")
            adj = c["flint"].get("clock_adjusted_compute_fraction")
            row += [f"{st['sm_mhz']:.0f}" if st else "-", pct(adj) if adj else "-",
                    pct(st["power_cap_share"]) if st else "-"]
        elif monitored:
            st = c["flint"].get("stats")
            adj = c["flint"].get("clock_adjusted_fraction")
            row += [f"{st['mem_mhz']:.0f}" if st else "-", pct(adj) if adj else "-"]
        if has_baseline:
            if c["one_sided"]:
                row += ["-", "-", "-", "-"]
            else:
                row += [c["baseline_name"], rate(c, c["baseline"])[0], f"{c['ratio']['median']:.3f}",
                        f"{c['ratio']['min']:.3f}-{c['ratio']['max']:.3f}"]
        if has_algo:
            row += [algorithm(c)]
        check = "ok" if c["ok"] else ("too few rounds" if c["outputs_match"] else "OUTPUT MISMATCH")
        if c.get("output_check"):
            check += f", rel L2 {c['output_check']['rel_l2']:.1e}"
        row += [f"{c['valid_rounds']}/{len(c['rounds'])}", check]
        lines.append("| " + " | ".join(row) + " |")
    return "\n".join(lines)


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("logs", nargs="+")
    args = parser.parse_args(argv)
    out = []
    for path in args.logs:
        with open(path, encoding="utf-8") as f:
            log = json.load(f)
        if log.get("schema") != "flint-bench/1":
            print(f"{path}: not a flint-bench/1 log", file=sys.stderr)
            return 2
        out.append(table(log))
    print("\n\n".join(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())

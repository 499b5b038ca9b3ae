"""flint_bench: its command-line contract (CPU: parsing needs no GPU), quick
end-to-end runs with their "flint-bench/1" JSON logs (GPU), and the results
table (CPU).

The command-line contract is written down as data: which options belong to
which benchmark, the accepted values of each enumerated option, and the shape
rules of each layout and epilogue. The rejection and acceptance cases are
generated from those tables, so each rule is stated once. Option names and the
message texts are the reference harness's interface (ref bench/cli.cpp:222-444),
with rocBLAS and hipBLASLt as the baselines and amd-smi as the monitor."""

import json
import statistics
import subprocess

import pytest

from flint_amd import flint_lib

EXE = flint_lib.library_path().parent / "flint_bench"
PREFIX = "flint_bench: "


@pytest.fixture(scope="module")
def exe():
    if not EXE.is_file():
        pytest.fail(f"{EXE} not found; build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    return str(EXE)


def run(exe, *args, timeout=300):
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)


def first_line(result):
    return result.stderr.splitlines()[0]


# ------------------------------------------------------------------ CPU: the contract as data

BENCHMARKS = ("copy", "mma", "gemm")
# option -> (the benchmark it belongs to, a value that benchmark accepts)
OWNED = {"--sizes": ("copy", "1M"), "--chains": ("mma", "4"), "--shapes": ("gemm", "8x8x8"),
         "--layout": ("gemm", "nt"), "--epilogue": ("gemm", "bias"), "--lt-algo": ("gemm", "first")}
LAYOUTS = ("nt", "nn", "tn")
EPILOGUE_LAYOUT = {"none": None, "bias": "nt", "bias-gelu": "nt", "bias-residual": "nt", "dgelu": "nn"}
PROTOCOL = ("--rounds", "--max-rounds", "--warmup", "--sample-ms", "--allow-busy", "--quick", "--out", "--help")


def both_orders(a, b):
    """The two orders of two option pairs: the parser checks combinations
    after reading every option, so the order must not matter."""
    return [a + b, b + a]


def rejections():
    """(argv, exact first stderr line or (prefix, substring))."""
    cases = [((), "no benchmark given"), (("nope",), ("unknown benchmark: nope", "")),
             (("copy", "--bogus"), ("unknown option: --bogus", ""))]
    for option, (owner, value) in OWNED.items():
        for other in BENCHMARKS:
            if other != owner:
                cases.append(((other, option, value), f"{option} applies to {owner} only"))
    for value in ("Fastest", "second", "all", "1", ""):
        cases.append((("gemm", "--lt-algo", value), f"--lt-algo: must be fastest or first: '{value}'"))
    for value in ("Bias", "relu", "gelu", "bias_gelu", ""):
        cases.append((("gemm", "--epilogue", value),
                      ("--epilogue:", "none, bias, bias-gelu, bias-residual or dgelu")))
    for value in ("TN", "NN", "nx", ""):
        cases.append((("gemm", "--layout", value), ("--layout:", "nt, nn or tn")))
    for epilogue, needs in EPILOGUE_LAYOUT.items():
        for layout in LAYOUTS:
            if needs is None or layout == needs:
                continue
            for argv in both_orders(("--layout", layout), ("--epilogue", epilogue)):
                cases.append((("gemm", *argv), f"--epilogue {epilogue} needs --layout {needs}"))
    cases.append((("gemm", "--epilogue", "dgelu"), "--epilogue dgelu needs --layout nn"))
    for argv in both_orders(("--layout", "nn"), ("--shapes", "8x12x8")):
        cases.append((("gemm", *argv), ("--shapes:", "N must be a multiple of 8")))
    for argv in both_orders(("--epilogue", "bias-gelu"), ("--shapes", "8x12x8")):
        cases.append((("gemm", *argv),
                      "--shapes: N must be a multiple of 8 with --epilogue bias-gelu: '8x12x8'"))
    for shapes in ("8x13x8", "8x12x8,8x7x8"):
        bad = [s for s in shapes.split(",") if int(s.split("x")[1]) % 2][0]
        for argv in both_orders(("--epilogue", "bias-residual"), ("--shapes", shapes)):
            cases.append((("gemm", *argv),
                          f"--shapes: N must be even with --epilogue bias-residual: '{bad}'"))
    for shape, dim in (("12x8x8", "M"), ("8x12x8", "N"), ("12x12x8", "M")):
        for argv in both_orders(("--layout", "tn"), ("--shapes", shape)):
            cases.append((("gemm", *argv), ("--shapes:", f"{dim} must be a multiple of 8 with --layout tn")))
    for layout in ("nt", "nn"):
        cases.append((("gemm", "--layout", layout, "--shapes", "8x8x1001"), ("--shapes:", "K must be a multiple of 8")))
    cases.append((("gemm", "--layout", "tn", "--shapes", "8x8x65537"), ("--shapes:", "limits")))
    for shapes, why in (("8x8", "not a shape"), ("8x8x8x8", "not a shape"), ("axbxc", "not a shape"),
                        ("8x-8x8", "not a shape"), ("8x 8x8", "not a shape"), ("8x8x8,", "not a shape"),
                        ("99999999999999999999x8x8", "not a shape"), ("0x8x8", "positive"),
                        ("8x0x8", "positive"), ("8x8x0", "positive"), ("8x8x12", "multiple of 8"),
                        ("8388481x8x8", "limits"), ("8x8388481x8", "limits"), ("8x8x65544", "limits")):
        cases.append((("gemm", "--shapes", shapes), ("--shapes:", why)))
    for sizes, why in (("1X", "not a size"), ("-1", "not a size"), ("1M,", "not a size"),
                       ("0", "positive"), ("65G", "too large")):
        cases.append((("copy", "--sizes", sizes), ("--sizes:", why)))
    cases.append((("mma", "--chains", "5"), ("--chains", "'5'")))
    for argv, message in ((("--rounds", "0"), "--rounds: must be between 1 and 1000000: '0'"),
                          (("--rounds", "x"), "--rounds: not an integer: 'x'"),
                          (("--rounds", "12", "--max-rounds", "11"), "--max-rounds: 11 is below --rounds 12"),
                          (("--warmup", "-1"), "--warmup: must not be negative: '-1'"),
                          (("--sample-ms", "0"), "--sample-ms: must be positive: '0'"),
                          (("--out=",), "--out: empty path"),
                          (("--quick=1",), "--quick takes no value"),
                          (("--rounds",), "--rounds needs a value")):
        cases.append((("copy", *argv), message))
    return cases


def acceptances():
    """argv lists the parser takes (checked with --help, so nothing runs)."""
    ok = [("gemm", "--lt-algo", "first"), ("gemm", "--lt-algo=fastest"),
          ("gemm", "--epilogue", "bias", "--lt-algo", "first"),
          ("gemm", "--layout", "nt", "--shapes", "8x12x8"),
          ("gemm", "--epilogue", "bias", "--shapes", "8x12x8"),
          ("gemm", "--epilogue", "bias-residual", "--shapes", "8x14x8,8x2x8"),
          ("gemm", "--epilogue", "bias", "--shapes", "8x13x8"),
          ("gemm", "--layout", "tn", "--shapes", "8x8x1001,16x8x1,8x8x65536"),
          ("gemm", "--shapes", "8388480x8388480x65536,1x8x8")]
    for epilogue, needs in EPILOGUE_LAYOUT.items():
        layouts = LAYOUTS if needs is None else (needs,)
        for layout in layouts:
            ok.extend(("gemm", *argv) for argv in both_orders(("--layout", layout), ("--epilogue", epilogue)))
    ok.append(("gemm", "--epilogue", "bias"))
    return ok


def _id(argv):
    return " ".join(argv) or "(none)"


@pytest.mark.parametrize("argv,expect", rejections(), ids=[_id(a) for a, _ in rejections()])
def test_the_parser_rejects(exe, argv, expect):
    result = run(exe, *argv)
    assert result.returncode == 2, result.stdout
    line = first_line(result)
    if isinstance(expect, str):
        assert line == PREFIX + expect
    else:
        head, part = expect
        assert line.startswith(PREFIX + head) and part in line, line


@pytest.mark.parametrize("argv", acceptances(), ids=[_id(a) for a in acceptances()])
def test_the_parser_accepts(exe, argv):
    result = run(exe, *argv, "--help")
    assert result.returncode == 0, result.stderr


def test_help_names_every_benchmark_option_and_value(exe):
    result = run(exe, "--help")
    assert result.returncode == 0 and result.stdout.startswith("usage: flint_bench")
    words = set(BENCHMARKS) | set(OWNED) | set(PROTOCOL) | set(LAYOUTS) | set(EPILOGUE_LAYOUT)
    words |= {"fastest", "first"}
    missing = sorted(w for w in words if w not in result.stdout)
    assert not missing, missing


def test_the_generated_tables_cover_each_rule():
    """Every owned option is tried with every benchmark that does not own
    it, and every epilogue with every layout it does not allow."""
    argvs = [a for a, _ in rejections()]
    for option, (owner, _) in OWNED.items():
        assert sum(1 for a in argvs if option in a and a[0] != owner) >= len(BENCHMARKS) - 1
    pairs = {(a[a.index("--layout") + 1], a[a.index("--epilogue") + 1]) for a in argvs
             if "--layout" in a and "--epilogue" in a}
    for epilogue, needs in EPILOGUE_LAYOUT.items():
        for layout in LAYOUTS:
            assert ((layout, epilogue) in pairs) == (needs is not None and layout != needs)
    assert len(set(map(tuple, argvs))) == len(argvs), "duplicate cases"


# ------------------------------------------------------------------ GPU: quick runs
#
# Each run below is one quick invocation and the labels its cases must carry.
# The log's invariants are checked by small functions, each stating one
# property of the "flint-bench/1" format (its field names are the harness's
# interface): the header, the timing rounds, the monitor windows, and what a
# GEMM case must record. The shapes are chosen to mix GPT-2 sizes with edge
# tiles and short k.

BASELINES = {"none": "rocBLAS", "bias": "hipBLASLt, FP32 bias",
             "bias-gelu": "hipBLASLt, FP32 bias", "bias-residual": "hipBLASLt, residual in C",
             "dgelu": "hipBLASLt DGELU"}
# (layout, epilogue, shapes)
GEMM_RUNS = {
    "nt": ("nt", "none", "2048x2304x768,96x136x56"),
    "nt-bias": ("nt", "bias", "512x768x3072,72x264x32"),
    "nt-bias-gelu": ("nt", "bias-gelu", "2048x3072x768,40x520x64"),
    "nt-bias-residual": ("nt", "bias-residual", "1024x768x768,8x130x16"),
    "nn": ("nn", "none", "2048x768x3072,200x264x24"),
    "nn-dgelu": ("nn", "dgelu", "2048x3072x768,64x136x40"),
    "tn": ("tn", "none", "3072x768x2048,264x200x1000,16x8x8"),
}


def run_quick(exe, tmp_path, argv):
    """Runs one quick invocation with --out; its log, after the header checks."""
    out = tmp_path / "log.json"
    res = run(exe, *argv, "--out", str(out), timeout=600)
    assert res.returncode == 0, f"{res.stdout}\n{res.stderr}"
    raw = out.read_text()
    for private in (str(tmp_path), str(flint_lib.ROOT)):
        assert private not in raw, "the log names a local path"
    log = json.loads(raw)
    check_header(log, argv)
    return res, log


def check_header(log, argv):
    assert (log["schema"], log["args"]) == ("flint-bench/1", list(argv))
    assert (log["quick"], log["standard_protocol"]) == (True, False)
    util = log["gpu_at_start"]["utilization_percent"]
    assert util is None or 0 <= util <= 100
    assert type(log["gpu_at_start"]["process_detection"]) is bool


def median_of(values):
    return statistics.median(values)


def check_side_timing(case, side, opts, valid):
    """A side's time is the median of its valid rounds' times, every sample
    ran at least (nearly) the sample window."""
    per_round = [r[side]["ms_per_launch"] for r in valid]
    assert case[side]["ms_per_launch"] == pytest.approx(median_of(per_round))
    assert min(r[side]["sample_ms"] for r in valid) >= 0.9 * opts["sample_ms"]
    assert case[side]["min_sample_ms"] >= 0.9 * opts["sample_ms"]


def check_rounds(case, opts, sides):
    valid = [r for r in case["rounds"] if r["valid"]]
    assert len(valid) == case["valid_rounds"] and len(valid) >= opts["rounds"]
    assert case["warmup_seconds"] >= opts["warmup_seconds"]
    for side in sides:
        check_side_timing(case, side, opts, valid)
        if case[side]["stats"] is not None:
            check_monitor(case[side]["stats"], [r[side]["stats"] for r in valid])
    if sides == ("flint", "baseline"):
        # Interleaved rounds: the two sides alternate in going first, and each
        # round's ratio is baseline time over Flint time.
        assert [r["flint_first"] for r in valid] == [k % 2 == 0 for k in range(len(valid))]
        ratios = [r["baseline"]["ms_per_launch"] / r["flint"]["ms_per_launch"] for r in valid]
        assert [r["ratio"] for r in valid] == pytest.approx(ratios)
        summary = case["ratio"]
        assert (summary["min"], summary["median"], summary["max"]) == pytest.approx(
            (min(ratios), median_of(ratios), max(ratios)))


def check_monitor(merged, windows):
    """The merged monitor statistics of a side are its windows' totals, their
    means weighted by the seconds of the windows that hold readings, and
    their extremes."""
    for total in ("samples", "failed_reads"):
        assert merged[total] == sum(w[total] for w in windows), total
    assert merged["seconds"] == pytest.approx(sum(w["seconds"] for w in windows))
    assert merged["new_process"] == any(w["new_process"] for w in windows)
    with_reading = [w for w in windows if w["samples"] > 0]
    weight = sum(w["seconds"] for w in with_reading)
    for field in ("sm_mhz", "mem_mhz", "power_w", "gfx_activity_percent", "power_cap_share",
                  "thermal_share"):
        if with_reading:
            mean = sum(w[field] * w["seconds"] for w in with_reading) / weight
            assert merged[field] == pytest.approx(mean), field
        else:
            assert merged[field] is None, field
    if with_reading:
        assert merged["temp_c_max"] == max(w["temp_c_max"] for w in with_reading)
        assert all(w["sm_mhz"] > 0 and w["power_w"] > 0 for w in with_reading)


def gemm_bytes(layout, epilogue, m, n, k):
    """Bytes one launch's buffers hold: the operands, the output (FP32 for TN
    and the residual form), pre, the residual, the bias."""
    operands = 2 * (m * k + n * k)
    out = m * n * (4 if layout == "tn" or epilogue == "bias-residual" else 2)
    extra = {"bias": 4 * n, "bias-gelu": 2 * m * n + 4 * n, "dgelu": 2 * m * n,
             "bias-residual": 4 * m * n + 4 * n}.get(epilogue, 0)
    return operands + out + extra


def check_gemm_case(case, layout, epilogue, shape, l2_bytes):
    m, n, k = shape
    assert (case["layout"], case["epilogue"]) == (layout, epilogue)
    assert case["baseline_name"] == BASELINES[epilogue]
    assert case["ok"] and case["outputs_match"], case["output_check"]
    assert case["flops"] == 2 * m * n * k
    assert case["size_bytes"] == gemm_bytes(layout, epilogue, m, n, k)
    assert case["rotation_sets"] * case["size_bytes"] > 4 * l2_bytes
    for side in ("flint", "baseline"):
        t = case[side]
        assert t["tflops"] == pytest.approx(case["flops"] / t["ms_per_launch"] / 1e9)
    checks = [case["output_check"]]
    if epilogue == "bias-gelu":
        checks.append(case["pre_check"])
    else:
        assert case["pre_check"] is None
    for c in checks:
        assert c["deterministic"] is True and c["nonfinite"] == 0
        assert 0 <= c["rel_l2"] <= 2.0**-10 and c["max_abs_baseline"] > 0
    algo = case["baseline_algorithm"]
    if epilogue == "none":
        assert algo is None
    else:
        timed = [c["ms_per_launch"] for c in algo["candidates"] if c["ms_per_launch"] is not None]
        assert timed and len(algo["candidates"]) <= 8
        assert algo["candidates"][algo["used"]]["ms_per_launch"] == min(timed)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(GEMM_RUNS))
def test_quick_gemm_run(exe, tmp_path, name):
    layout, epilogue, shapes = GEMM_RUNS[name]
    argv = ["gemm", "--quick", "--allow-busy", "--layout", layout, "--epilogue", epilogue,
            "--shapes", shapes]
    res, log = run_quick(exe, tmp_path, argv)
    labels = shapes.split(",")
    assert [c["label"] for c in log["cases"]] == labels
    assert log["options"]["lt_algo"] == "fastest"
    tag = layout if epilogue == "none" else f"{layout}+{epilogue}"
    assert f"gemm {tag} {labels[0]}" in res.stdout
    for case, label in zip(log["cases"], labels):
        shape = tuple(int(v) for v in label.split("x"))
        check_gemm_case(case, layout, epilogue, shape, log["device"]["l2_bytes"])
        check_rounds(case, log["options"], ("flint", "baseline"))


@pytest.mark.gpu
def test_quick_copy_run(exe, tmp_path):
    argv = ["copy", "--quick", "--allow-busy", "--sizes", "3M,12345"]
    _, log = run_quick(exe, tmp_path, argv)
    dev = log["device"]
    assert dev["arch"].startswith("gfx950") and dev["rated_bandwidth_gbs"] == 8000
    assert [c["label"] for c in log["cases"]] == ["3 MiB", "12345 B"]
    for case in log["cases"]:
        assert case["ok"] and case["outputs_match"]
        assert (case["layout"], case["epilogue"], case["output_check"],
                case["baseline_algorithm"]) == (None, None, None, None)
        check_rounds(case, log["options"], ("flint", "baseline"))
        for side in ("flint", "baseline"):
            t = case[side]
            assert t["gbs"] == pytest.approx(case["bytes_moved"] / t["ms_per_launch"] / 1e6)
            assert 0 < t["gbs"] <= 1.1 * dev["rated_bandwidth_gbs"]
            st = t["stats"]
            if st is not None and st["samples"] > 0 and st["mem_mhz"] > 0:
                # HBM3E: four transfers per reported memory clock.
                peak = 4 * st["mem_mhz"] * 1e6 * dev["bus_width_bits"] / 8 / 1e9
                assert t["clock_adjusted_fraction"] == pytest.approx(t["gbs"] / peak)
        padded = -(-case["size_bytes"] // 256) * 256
        assert case["rotation_sets"] * 2 * padded > 4 * dev["l2_bytes"]


@pytest.mark.gpu
def test_quick_mma_run(exe, tmp_path):
    argv = ["mma", "--quick", "--allow-busy", "--chains", "16,4"]
    _, log = run_quick(exe, tmp_path, argv)
    cus = log["device"]["cu_count"]
    assert [c["label"] for c in log["cases"]] == [
        f"mfma 32x32x16 f16->f32, {c} chains, 2 blocks/CU" for c in (16, 4)]
    for case in log["cases"]:
        assert case["one_sided"] and case["baseline"] is None and case["ratio"] is None
        assert case["ok"] and case["outputs_match"]
        assert case["peak_flop_per_cu_per_clock"] == 4096
        # Two 4-wave blocks per CU, each wave 32,768 MFMAs of 32 x 32 x 16 x 2 FLOP.
        assert case["flops"] == (2 * cus) * 4 * 32768 * (32 * 32 * 16 * 2)
        assert 0 < case["flint"]["rated_compute_fraction"] <= 1.05
        check_rounds(case, log["options"], ("flint",))


# Runs whose point is one option: the hipBLASLt candidate choice, and the
# GPT-2 shapes an epilogue runs when --shapes is left out.
OPTION_RUNS = [
    (["--layout", "nt", "--epilogue", "bias-residual", "--lt-algo", "first", "--shapes",
      "512x768x768"], ["512x768x768"], "first"),
    (["--layout", "nn", "--epilogue", "dgelu", "--lt-algo", "first", "--shapes", "256x3072x768"],
     ["256x3072x768"], "first"),
    (["--epilogue", "bias-gelu"], ["8192x3072x768"], "fastest"),
    (["--epilogue", "bias-residual"], ["8192x768x768", "8192x768x3072"], "fastest"),
    (["--layout", "nn", "--epilogue", "dgelu"], ["8192x3072x768"], "fastest"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("extra,labels,choice", OPTION_RUNS,
                         ids=[" ".join(a) for a, _, _ in OPTION_RUNS])
def test_quick_option_run(exe, tmp_path, extra, labels, choice):
    _, log = run_quick(exe, tmp_path, ["gemm", "--quick", "--allow-busy", *extra])
    assert [c["label"] for c in log["cases"]] == labels
    assert log["options"]["lt_algo"] == choice
    for case in log["cases"]:
        assert case["ok"]
        algo = case["baseline_algorithm"]
        assert algo["selection"] == choice
        if choice == "first":
            assert algo["used"] == 0


# ------------------------------------------------------------------ CPU: results_table

def synthetic_log(quick=False, sha="0123456789abcdef", dirty=False, ok=True, stats=True):
    window = {"seconds": 1.0, "samples": 100, "failed_reads": 0, "sm_mhz": 2000.0, "mem_mhz": 2000.0,
              "power_w": 1400.0, "gfx_activity_percent": 100.0, "temp_c_max": 60, "power_cap_share": 0.25,
              "thermal_share": 0.0, "new_process": False}
    side = {"ms_per_launch": 0.5, "tflops": 800.0, "rated_compute_fraction": 800 / 2516.6, "gbs": 0,
            "rated_fraction": 0, "clock_adjusted_compute_fraction": 800 / (4096 * 256 * 2000e6 / 1e12),
            "stats": window if stats else None}
    case = {"benchmark": "gemm", "label": "8192x768x768", "layout": "nt", "epilogue": "bias", "flops": 2 * 8192 * 768 * 768,
            "one_sided": False, "baseline_name": "hipBLASLt, FP32 bias", "flint": side,
            "baseline": dict(side, ms_per_launch=0.6, tflops=666.7), "ratio": {"median": 1.2, "min": 1.1, "max": 1.3},
            "baseline_algorithm": {"selection": "fastest", "used": 1, "candidates": [
                {"index": 0, "solution_index": 7}, {"index": 1, "solution_index": 9}]},
            "ok": ok, "outputs_match": ok, "output_check": {"rel_l2": 1e-6}, "valid_rounds": 10,
            "rounds": [{}] * 10}
    return {"schema": "flint-bench/1", "quick": quick, "standard_protocol": not quick, "args": ["gemm"],
            "git": {"sha": sha, "dirty": dirty}, "timestamp_utc": "2026-01-01T00:00:00Z",
            "device": {"name": "AMD gfx950", "arch": "gfx950", "cu_count": 256, "rated_sm_clock_mhz": 2400.0},
            "cases": [case]}


def test_results_table_rows():
    from flint_amd.bench.results_table import table

    text = table(synthetic_log())
    assert "Not for quoting" not in text
    (row,) = [line for line in text.splitlines() if line.startswith("| gemm nt+bias 8192x768x768")]
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[1:8] == ["0.5000", "800.0", "31.8%", "2000", "38.1%", "25.0%", "hipBLASLt, FP32 bias"]
    assert cells[8:11] == ["666.7", "1.200", "1.100-1.300"]
    assert cells[11] == "fastest: #1 of 2 (solution 9)"
    assert cells[12:] == ["10/10", "ok, rel L2 1.0e-06"]
    # Without monitor statistics the clock columns are left out.
    assert "SCLK" not in table(synthetic_log(stats=False))


def test_results_table_bandwidth_at_the_memory_clock():
    from flint_amd.bench.results_table import table

    log = synthetic_log()
    case = log["cases"][0]
    case.update(benchmark="copy", label="1 GiB", layout=None, epilogue=None, flops=0)
    for name in ("flint", "baseline"):
        case[name] = dict(case[name], gbs=6000.0, rated_fraction=0.75, tflops=0,
                          clock_adjusted_fraction=6000 / 8192, clock_adjusted_compute_fraction=None)
    text = table(log)
    head = [line for line in text.splitlines() if line.startswith("| Case")][0]
    assert "MCLK MHz" in head and "SCLK" not in head
    (row,) = [line for line in text.splitlines() if line.startswith("| copy 1 GiB")]
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[1:6] == ["0.5000", "6000.0", "75.0%", "2000", "73.2%"]


@pytest.mark.parametrize("kwargs, reason", [
    ({"quick": True}, "a --quick run"), ({"sha": "unknown"}, "built outside a git checkout"),
    ({"dirty": True}, "uncommitted changes"), ({"ok": False}, "a case that is not ok"),
])
def test_results_table_says_why_a_log_is_not_for_quoting(kwargs, reason):
    from flint_amd.bench.results_table import table

    text = table(synthetic_log(**kwargs))
    assert "Not for quoting:" in text and reason in text

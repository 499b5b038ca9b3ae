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

def quick(exe, tmp_path, *args):
    out = tmp_path / "bench.json"
    result = run(exe, *args, "--out", str(out), timeout=600)
    assert result.returncode == 0, f"stdout:\n{result.stdout}\nstderr:\n{result.stderr}"
    text = out.read_text()
    assert str(tmp_path) not in text and str(flint_lib.ROOT) not in text
    data = json.loads(text)
    assert data["schema"] == "flint-bench/1"
    assert data["args"] == list(args)
    assert data["quick"] is True and data["standard_protocol"] is False
    start = data["gpu_at_start"]
    assert isinstance(start["process_detection"], bool)
    if start["utilization_percent"] is not None:
        assert 0 <= start["utilization_percent"] <= 100
    return result, data


def assert_rounds(case, options, two_sided=True):
    valid = [r for r in case["rounds"] if r["valid"]]
    assert case["valid_rounds"] == len(valid) >= options["rounds"]
    assert case["warmup_seconds"] >= options["warmup_seconds"]
    if two_sided:
        for r in valid:
            assert r["ratio"] == pytest.approx(r["baseline"]["ms_per_launch"] / r["flint"]["ms_per_launch"])
        ratios = [r["ratio"] for r in valid]
        assert case["ratio"]["median"] == pytest.approx(statistics.median(ratios))
        assert case["ratio"]["min"] == pytest.approx(min(ratios))
        assert case["ratio"]["max"] == pytest.approx(max(ratios))
        assert [r["flint_first"] for r in valid] == [i % 2 == 0 for i in range(len(valid))]
    for name in ("flint", "baseline") if two_sided else ("flint",):
        side = case[name]
        assert side["min_sample_ms"] >= 0.9 * options["sample_ms"]
        assert side["ms_per_launch"] == pytest.approx(statistics.median(
            [r[name]["ms_per_launch"] for r in valid]))
        for r in valid:
            assert r[name]["sample_ms"] >= 0.9 * options["sample_ms"]
        if side["stats"] is not None:
            assert_stats_follow_from_rounds(side["stats"], [r[name]["stats"] for r in valid])
            if case["flops"] > 0 and side["stats"]["samples"] > 0:
                # The firmware's clock readings lag short bursts of launches,
                # so only the sign is pinned here.
                assert side["clock_adjusted_compute_fraction"] > 0


def assert_stats_follow_from_rounds(stats, windows):
    """A side's stats merge its valid rounds' windows: counts add up, means are
    weighted by each window's seconds, maxima and the new-process flag carry."""
    seconds = sum(w["seconds"] for w in windows)
    assert stats["seconds"] == pytest.approx(seconds)
    assert stats["samples"] == sum(w["samples"] for w in windows)
    assert stats["failed_reads"] == sum(w["failed_reads"] for w in windows)
    # Means weigh only the windows that hold a reading; without any they are null.
    read = [w for w in windows if w["samples"] > 0]
    read_seconds = sum(w["seconds"] for w in read)
    for name in ("sm_mhz", "mem_mhz", "power_w", "gfx_activity_percent", "power_cap_share", "thermal_share"):
        if not read:
            assert stats[name] is None, name
            continue
        expect = sum(w[name] * w["seconds"] for w in read) / read_seconds
        assert stats[name] == pytest.approx(expect), name
    if read:
        assert stats["temp_c_max"] == max(w["temp_c_max"] for w in read)
    assert stats["new_process"] == any(w["new_process"] for w in windows)
    # A window with no reading of its own holds the last one before it, so
    # once the monitor has read the device every window has a clock.
    for w in windows:
        assert w["samples"] >= 0
        if w["samples"] > 0:
            assert w["sm_mhz"] > 0 and w["power_w"] > 0


@pytest.mark.gpu
def test_quick_copy(exe, tmp_path):
    args = ["copy", "--quick", "--sizes", "1M,4097", "--allow-busy"]
    _, data = quick(exe, tmp_path, *args)
    device, options = data["device"], data["options"]
    assert device["arch"].startswith("gfx950")
    assert device["rated_bandwidth_gbs"] == 8000
    cases = data["cases"]
    assert [c["label"] for c in cases] == ["1 MiB", "4097 B"]
    for case in cases:
        assert case["layout"] is None and case["epilogue"] is None
        assert case["ok"] and case["outputs_match"]
        assert case["output_check"] is None and case["baseline_algorithm"] is None
        assert_rounds(case, options)
        for name in ("flint", "baseline"):
            side = case[name]
            assert 0 < side["gbs"] <= 1.1 * device["rated_bandwidth_gbs"]
            assert side["gbs"] == pytest.approx(case["bytes_moved"] / (side["ms_per_launch"] * 1e-3) / 1e9)
            # Against the bandwidth at the monitored memory clock: HBM3E moves
            # four transfers per reported clock over the bus.
            st = side["stats"]
            if st is not None and st["samples"] > 0 and st["mem_mhz"] > 0:
                at_clock = 4 * st["mem_mhz"] * 1e6 * device["bus_width_bits"] / 8 / 1e9
                assert side["clock_adjusted_fraction"] == pytest.approx(side["gbs"] / at_clock)
            else:
                assert side["clock_adjusted_fraction"] is None
        stride = (case["size_bytes"] + 255) // 256 * 256
        assert case["rotation_sets"] * 2 * stride > 4 * device["l2_bytes"]


@pytest.mark.gpu
def test_quick_mma(exe, tmp_path):
    args = ["mma", "--quick", "--chains", "4,8,16", "--allow-busy"]
    _, data = quick(exe, tmp_path, *args)
    device, options = data["device"], data["options"]
    cases = data["cases"]
    assert [c["label"] for c in cases] == [f"mfma 32x32x16 f16->f32, {n} chains, 2 blocks/CU" for n in (4, 8, 16)]
    for case in cases:
        assert case["one_sided"] is True and case["baseline"] is None and case["ratio"] is None
        assert case["ok"] and case["outputs_match"]
        # 2 blocks/CU x CUs blocks of 4 waves, each wave 32768 MFMAs of 32768 FLOP.
        assert case["flops"] == 2 * device["cu_count"] * 4 * 32768 * 32768
        assert case["peak_flop_per_cu_per_clock"] == 4096
        assert_rounds(case, options, two_sided=False)
        assert 0 < case["flint"]["rated_compute_fraction"] <= 1.05


GEMM_CASES = [
    ("nt", "none", "1000x2304x768,129x257x40"),
    ("nt", "bias", "1000x2304x768,129x257x40"),
    ("nt", "bias-gelu", "1000x3072x768,129x264x40"),
    ("nt", "bias-residual", "1000x768x3072,129x266x40"),
    ("nn", "none", "1000x768x2304,129x264x40"),
    ("nn", "dgelu", "1000x3072x768,129x264x40"),
    ("tn", "none", "768x768x8192,136x120x3000,1032x8x4096,72x40x1001"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("layout, epilogue, shape_list", GEMM_CASES)
def test_quick_gemm(exe, tmp_path, layout, epilogue, shape_list):
    args = ["gemm", "--quick", "--shapes", shape_list, "--allow-busy"]
    if layout != "nt":
        args[1:1] = ["--layout", layout]
    if epilogue != "none":
        args[1:1] = ["--epilogue", epilogue]
    result, data = quick(exe, tmp_path, *args)
    first = shape_list.split(",")[0]
    for name in ("none", "bias", "bias-gelu", "dgelu", "bias-residual"):
        label = f"gemm {layout}" + ("" if name == "none" else f"+{name}") + f" {first}"
        assert (label in result.stdout) == (epilogue == name), label
    device, options = data["device"], data["options"]
    assert options["lt_algo"] == "fastest"
    shapes = [tuple(int(d) for d in item.split("x")) for item in shape_list.split(",")]
    assert [c["label"] for c in data["cases"]] == shape_list.split(",")
    for case, (m, n, k) in zip(data["cases"], shapes):
        assert case["layout"] == layout and case["epilogue"] == epilogue
        assert case["baseline_name"] == {
            "none": "rocBLAS", "bias": "hipBLASLt, FP32 bias", "bias-gelu": "hipBLASLt, FP32 bias",
            "dgelu": "hipBLASLt DGELU", "bias-residual": "hipBLASLt, residual in C"}[epilogue]
        assert case["ok"] and case["outputs_match"], case["output_check"]
        if epilogue == "none":
            assert case["baseline_algorithm"] is None
        else:
            algorithm = case["baseline_algorithm"]
            timed = [c for c in algorithm["candidates"] if c["ms_per_launch"] is not None]
            assert 1 <= len(algorithm["candidates"]) <= 8 and timed
            assert algorithm["candidates"][algorithm["used"]]["ms_per_launch"] == min(
                c["ms_per_launch"] for c in timed)
        checks = [case["output_check"]] + ([case["pre_check"]] if epilogue == "bias-gelu" else [])
        if epilogue != "bias-gelu":
            assert case["pre_check"] is None
        for check in checks:
            assert check["deterministic"] is True and check["nonfinite"] == 0
            assert 0 <= check["rel_l2"] <= 2**-10
            assert check["max_abs_baseline"] > 0
        assert case["flops"] == 2 * m * n * k
        assert_rounds(case, options)
        for name in ("flint", "baseline"):
            assert case[name]["tflops"] == pytest.approx(case["flops"] / (case[name]["ms_per_launch"] * 1e-3) / 1e12)
        assert case["size_bytes"] == (
            2 * (m * k + n * k)
            + m * n * (4 if layout == "tn" or epilogue == "bias-residual" else 2)
            + (2 * m * n if epilogue in ("bias-gelu", "dgelu") else 0)
            + (4 * m * n if epilogue == "bias-residual" else 0)
            + (4 * n if epilogue in ("bias", "bias-gelu", "bias-residual") else 0))
        assert case["rotation_sets"] * case["size_bytes"] > 4 * device["l2_bytes"]


@pytest.mark.gpu
@pytest.mark.parametrize("layout, epilogue", [("nt", "bias"), ("nn", "dgelu")])
def test_quick_gemm_lt_algo_first(exe, tmp_path, layout, epilogue):
    args = ["gemm", "--quick", "--layout", layout, "--epilogue", epilogue, "--lt-algo", "first",
            "--shapes", "1000x768x768", "--allow-busy"]
    _, data = quick(exe, tmp_path, *args)
    assert data["options"]["lt_algo"] == "first"
    (case,) = data["cases"]
    assert case["ok"]
    assert case["baseline_algorithm"]["selection"] == "first" and case["baseline_algorithm"]["used"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("args, labels", [
    (["--epilogue", "bias-gelu"], ["8192x3072x768"]),
    (["--epilogue", "bias-residual"], ["8192x768x768", "8192x768x3072"]),
    (["--layout", "nn", "--epilogue", "dgelu"], ["8192x3072x768"]),
])
def test_epilogue_defaults_are_the_gpt2_layers(exe, tmp_path, args, labels):
    _, data = quick(exe, tmp_path, "gemm", *args, "--quick", "--allow-busy")
    assert [c["label"] for c in data["cases"]] == labels
    assert all(c["ok"] for c in data["cases"])


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

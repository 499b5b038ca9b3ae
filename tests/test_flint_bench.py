"""flint_bench: the command line (CPU: parsing needs no GPU), and quick end-to-end
runs with their "flint-bench/1" JSON logs (GPU). Mirrors the reference's
tests/test_bench.py:113-700: the same option errors, defaults and log checks,
with rocBLAS and hipBLASLt as the baselines and amd-smi as the monitor."""

import json
import statistics
import subprocess

import pytest

from flint_amd import flint_lib

EXE = flint_lib.library_path().parent / "flint_bench"


@pytest.fixture(scope="module")
def exe():
    if not EXE.is_file():
        pytest.fail(f"{EXE} not found; build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    return str(EXE)


def run(exe, *args, timeout=300):
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)


def first_line(result):
    return result.stderr.splitlines()[0]


# ------------------------------------------------------------------ CPU: parsing

def test_help(exe):
    result = run(exe, "--help")
    assert result.returncode == 0, result.stderr
    assert "usage: flint_bench" in result.stdout
    for text in ("copy", "mma", "gemm", "--sizes", "--chains", "--shapes", "--layout", "tn", "--epilogue",
                 "bias", "bias-gelu", "dgelu", "bias-residual", "--lt-algo", "fastest", "first"):
        assert text in result.stdout


def test_unknown_option(exe):
    result = run(exe, "copy", "--bogus")
    assert result.returncode == 2
    assert "unknown option: --bogus" in result.stderr


def test_unknown_benchmark(exe):
    result = run(exe, "nope")
    assert result.returncode == 2
    assert "unknown benchmark: nope" in result.stderr


def test_no_benchmark(exe):
    result = run(exe)
    assert result.returncode == 2
    assert first_line(result) == "flint_bench: no benchmark given"


@pytest.mark.parametrize("option, value, owner", [
    ("--sizes", "1M", "copy"), ("--chains", "4", "mma"), ("--shapes", "8x8x8", "gemm"),
    ("--layout", "nt", "gemm"), ("--epilogue", "bias", "gemm"), ("--lt-algo", "first", "gemm"),
])
def test_options_rejected_for_other_benchmarks(exe, option, value, owner):
    for benchmark in ("copy", "mma", "gemm"):
        if benchmark == owner:
            continue
        result = run(exe, benchmark, option, value)
        assert result.returncode == 2
        assert first_line(result) == f"flint_bench: {option} applies to {owner} only"


def test_bad_chains_rejected(exe):
    result = run(exe, "mma", "--chains", "5")
    assert result.returncode == 2
    assert "--chains" in result.stderr and "'5'" in result.stderr


@pytest.mark.parametrize("sizes, reason", [("1X", "not a size"), ("0", "positive"), ("-1", "not a size"),
                                           ("1M,", "not a size"), ("65G", "too large")])
def test_bad_sizes_rejected(exe, sizes, reason):
    result = run(exe, "copy", "--sizes", sizes)
    assert result.returncode == 2
    assert first_line(result).startswith("flint_bench: --sizes:") and reason in first_line(result)


@pytest.mark.parametrize("value", ["Fastest", "second", "all", "1", ""])
def test_bad_lt_algo_rejected(exe, value):
    result = run(exe, "gemm", "--lt-algo", value)
    assert result.returncode == 2, result.stdout
    assert first_line(result) == f"flint_bench: --lt-algo: must be fastest or first: '{value}'"


def test_lt_algo_accepted_for_gemm(exe):
    for args in (("--lt-algo", "first"), ("--lt-algo=fastest",), ("--epilogue", "bias", "--lt-algo", "first")):
        result = run(exe, "gemm", *args, "--help")
        assert result.returncode == 0, result.stderr


@pytest.mark.parametrize("epilogue", ["Bias", "relu", "gelu", "bias_gelu", ""])
def test_bad_epilogue_rejected(exe, epilogue):
    result = run(exe, "gemm", "--epilogue", epilogue)
    assert result.returncode == 2, result.stdout
    assert first_line(result).startswith("flint_bench: --epilogue:")
    assert "none, bias, bias-gelu, bias-residual or dgelu" in first_line(result)


@pytest.mark.parametrize("epilogue", ["bias", "bias-gelu", "bias-residual"])
@pytest.mark.parametrize("layout", ["nn", "tn"])
def test_bias_needs_layout_nt(exe, layout, epilogue):
    for args in (("--layout", layout, "--epilogue", epilogue), ("--epilogue", epilogue, "--layout", layout)):
        result = run(exe, "gemm", *args)
        assert result.returncode == 2, result.stdout
        assert first_line(result) == f"flint_bench: --epilogue {epilogue} needs --layout nt"
    for args in (("--layout", "nt", "--epilogue", epilogue), ("--epilogue", epilogue),
                 ("--layout", layout, "--epilogue", "none")):
        result = run(exe, "gemm", *args, "--help")
        assert result.returncode == 0, result.stderr


@pytest.mark.parametrize("layout", ["nt", "tn"])
def test_dgelu_needs_layout_nn(exe, layout):
    cases = [("--layout", layout, "--epilogue", "dgelu"), ("--epilogue", "dgelu", "--layout", layout)]
    if layout == "nt":
        cases.append(("--epilogue", "dgelu"))
    for args in cases:
        result = run(exe, "gemm", *args)
        assert result.returncode == 2, result.stdout
        assert first_line(result) == "flint_bench: --epilogue dgelu needs --layout nn"
    for args in (("--layout", "nn", "--epilogue", "dgelu"), ("--epilogue", "dgelu", "--layout", "nn")):
        assert run(exe, "gemm", *args, "--help").returncode == 0


@pytest.mark.parametrize("layout", ["TN", "NN", "nx", ""])
def test_bad_layout_rejected(exe, layout):
    result = run(exe, "gemm", "--layout", layout)
    assert result.returncode == 2, result.stdout
    assert first_line(result).startswith("flint_bench: --layout:") and "nt, nn or tn" in first_line(result)


def test_nn_needs_n_a_multiple_of_8(exe):
    for args in (("--layout", "nn", "--shapes", "8x12x8"), ("--shapes", "8x12x8", "--layout", "nn")):
        result = run(exe, "gemm", *args)
        assert result.returncode == 2, result.stdout
        assert first_line(result).startswith("flint_bench: --shapes:")
        assert "N must be a multiple of 8" in first_line(result)
    assert run(exe, "gemm", "--layout", "nt", "--shapes", "8x12x8", "--help").returncode == 0
    assert run(exe, "gemm", "--shapes", "8x12x8", "--layout", "nn", "--help").returncode == 2


def test_bias_gelu_needs_n_a_multiple_of_8(exe):
    for args in (("--epilogue", "bias-gelu", "--shapes", "8x12x8"), ("--shapes", "8x12x8", "--epilogue", "bias-gelu")):
        result = run(exe, "gemm", *args)
        assert result.returncode == 2, result.stdout
        assert first_line(result) == (
            "flint_bench: --shapes: N must be a multiple of 8 with --epilogue bias-gelu: '8x12x8'")
    assert run(exe, "gemm", "--epilogue", "bias", "--shapes", "8x12x8", "--help").returncode == 0


def test_bias_residual_needs_n_even(exe):
    for args in (("--epilogue", "bias-residual", "--shapes", "8x13x8"),
                 ("--shapes", "8x13x8", "--epilogue", "bias-residual"),
                 ("--epilogue", "bias-residual", "--shapes", "8x12x8,8x7x8")):
        result = run(exe, "gemm", *args)
        assert result.returncode == 2, result.stdout
        line = first_line(result)
        assert line.startswith("flint_bench: --shapes: N must be even with --epilogue bias-residual: '8x")
        assert line.endswith("x8'")
    assert run(exe, "gemm", "--epilogue", "bias-residual", "--shapes", "8x14x8,8x2x8", "--help").returncode == 0
    assert run(exe, "gemm", "--epilogue", "bias", "--shapes", "8x13x8", "--help").returncode == 0


@pytest.mark.parametrize("shape, dimension", [("12x8x8", "M"), ("8x12x8", "N"), ("12x12x8", "M")])
def test_tn_needs_m_and_n_multiples_of_8(exe, shape, dimension):
    for args in (("--layout", "tn", "--shapes", shape), ("--shapes", shape, "--layout", "tn")):
        result = run(exe, "gemm", *args)
        assert result.returncode == 2, result.stdout
        assert first_line(result).startswith("flint_bench: --shapes:")
        assert f"{dimension} must be a multiple of 8 with --layout tn" in first_line(result)


def test_tn_takes_any_k(exe):
    result = run(exe, "gemm", "--layout", "tn", "--shapes", "8x8x1001,16x8x1,8x8x65536", "--help")
    assert result.returncode == 0, result.stderr
    for layout in ("nt", "nn"):
        result = run(exe, "gemm", "--layout", layout, "--shapes", "8x8x1001", "--help")
        assert result.returncode == 2
        assert "K must be a multiple of 8" in first_line(result)
    result = run(exe, "gemm", "--layout", "tn", "--shapes", "8x8x65537", "--help")
    assert result.returncode == 2
    assert "limits" in first_line(result)


@pytest.mark.parametrize("shapes, reason", [
    ("8x8", "not a shape"), ("8x8x8x8", "not a shape"), ("axbxc", "not a shape"), ("8x-8x8", "not a shape"),
    ("8x 8x8", "not a shape"), ("8x8x8,", "not a shape"), ("0x8x8", "positive"), ("8x0x8", "positive"),
    ("8x8x0", "positive"), ("8x8x12", "multiple of 8"), ("8388481x8x8", "limits"), ("8x8388481x8", "limits"),
    ("8x8x65544", "limits"), ("99999999999999999999x8x8", "not a shape"),
])
def test_bad_shapes_rejected(exe, shapes, reason):
    result = run(exe, "gemm", "--shapes", shapes)
    assert result.returncode == 2, result.stdout
    assert first_line(result).startswith("flint_bench: --shapes:") and reason in first_line(result)


def test_shapes_at_the_limits_are_accepted_by_the_parser(exe):
    assert run(exe, "gemm", "--shapes", "8388480x8388480x65536,1x8x8", "--help").returncode == 0


@pytest.mark.parametrize("args, message", [
    (("--rounds", "0"), "--rounds: must be between 1 and 1000000: '0'"),
    (("--rounds", "x"), "--rounds: not an integer: 'x'"),
    (("--rounds", "12", "--max-rounds", "11"), "--max-rounds: 11 is below --rounds 12"),
    (("--warmup", "-1"), "--warmup: must not be negative: '-1'"),
    (("--sample-ms", "0"), "--sample-ms: must be positive: '0'"),
    (("--out=",), "--out: empty path"),
    (("--quick=1",), "--quick takes no value"),
    (("--rounds",), "--rounds needs a value"),
])
def test_protocol_options_checked(exe, args, message):
    result = run(exe, "copy", *args)
    assert result.returncode == 2
    assert first_line(result) == f"flint_bench: {message}"


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
    for name in ("sm_mhz", "mem_mhz", "power_w", "gfx_activity_percent", "power_cap_share", "thermal_share"):
        assert stats[name] == pytest.approx(sum(w[name] * w["seconds"] for w in windows) / seconds), name
    assert stats["temp_c_max"] == max(w["temp_c_max"] for w in windows)
    assert stats["new_process"] == any(w["new_process"] for w in windows)
    # A short (--quick) sample can fall between two of the monitor's ~10 ms
    # readings; a window that holds readings has a clock and a power.
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


@pytest.mark.parametrize("kwargs, reason", [
    ({"quick": True}, "a --quick run"), ({"sha": "unknown"}, "built outside a git checkout"),
    ({"dirty": True}, "uncommitted changes"), ({"ok": False}, "a case that is not ok"),
])
def test_results_table_says_why_a_log_is_not_for_quoting(kwargs, reason):
    from flint_amd.bench.results_table import table

    text = table(synthetic_log(**kwargs))
    assert "Not for quoting:" in text and reason in text

"""The C ABI boundary, checked on the CPU: the header, the ctypes table and
the library's exports agree (ref tests/test_api.py:10-15), status strings
(ref src/api/status.cpp), and argument validation that fails before any HIP
call, with the reference's message text (ref src/api/*.cpp)."""

import ctypes
import subprocess

import pytest

from flint_amd import flint_lib


def test_header_matches_signatures():
    # flint.h: the reference's 40 functions; flint_train.h: the 4 of the
    # training-step extension, which has no counterpart in the reference.
    assert len(flint_lib.declared_functions(flint_lib.HEADER)) == 40
    assert len(flint_lib.declared_functions(flint_lib.TRAIN_HEADER)) == 4
    # flint_noalloc.h: one entry point for callers that cannot allocate.
    assert flint_lib.declared_functions(flint_lib.NOALLOC_HEADER) == ["flint_bias_gradient_noalloc"]
    # flint_attention.h: the fused causal attention and the model built on it,
    # additive.
    assert flint_lib.declared_functions(flint_lib.ATTENTION_HEADER) == [
        "flint_attention_forward", "flint_attention_backward_workspace",
        "flint_attention_backward", "flint_gpt2_bytes_fused", "flint_gpt2_create_fused"]
    # flint_tuning.h: the plan overrides for tests and sweeps.
    assert flint_lib.declared_functions(flint_lib.TUNING_HEADER) == ["flint_set_tuning"]
    declared = flint_lib.declared_functions()
    assert sorted(declared) == sorted(flint_lib.SIGNATURES)


def test_library_exports_exactly_the_header(flint):
    # Every defined dynamic symbol, of any kind (functions, data, weak
    # template instantiations): the set must be the headers' functions.
    out = subprocess.run(["nm", "-D", "--defined-only", str(flint.path)], capture_output=True,
                         text=True, check=True).stdout
    exported = [line.split()[-1] for line in out.splitlines() if line.strip()]
    assert sorted(exported) == sorted(flint_lib.declared_functions())


def test_tuning_names_are_checked_and_read_no_environment(flint):
    # Unknown names fail with a message; known ones set and clear. The
    # library's source reads no environment variable.
    from pathlib import Path

    assert flint.lib.flint_set_tuning(b"no_such_plan", b"1") == flint_lib.ERROR_INVALID_ARGUMENT
    assert "no_such_plan" in flint.last_error()
    assert flint.lib.flint_set_tuning(None, None) == flint_lib.ERROR_INVALID_ARGUMENT
    with flint.tuned(gemm_pipe="0", ln_defer="0"):
        pass
    src = Path(flint_lib.ROOT) / "flint_amd" / "csrc"
    for f in list(src.rglob("*.cpp")) + list(src.rglob("*.hip")) + list(src.rglob("*.h")):
        assert "getenv" not in f.read_text(), f


def test_links_only_the_hip_runtime(flint):
    out = subprocess.run(["readelf", "-d", str(flint.path)], capture_output=True, text=True,
                         check=True).stdout
    needed = [l for l in out.splitlines() if "NEEDED" in l]
    assert any("libamdhip64" in l for l in needed)
    for bad in ("cublas", "cudnn", "nvml", "cudart", "torch", "python"):
        assert not any(bad in l for l in needed)


def test_status_strings(flint):
    assert flint.version() == "0.1.0"
    assert flint.status_string(0) == "ok"
    assert flint.status_string(1) == "invalid argument"
    assert flint.status_string(2) == "CUDA error"
    assert flint.status_string(99) == "unknown status"


def _fails(flint, fn, *args, message):
    status = getattr(flint.lib, fn)(*args)
    assert status == flint_lib.ERROR_INVALID_ARGUMENT
    assert message in flint.last_error(), flint.last_error()


A = 0x10000  # a 16-byte-aligned fake device address: validation never dereferences


def test_gemm_validation(flint):
    _fails(flint, "flint_gemm_nt", A, A * 2, A * 3, 8, 8, 12, None,
           message="flint_gemm_nt: k (12) must be a positive multiple of 8")
    _fails(flint, "flint_gemm_nt", None, A, A, 8, 8, 8, None, message="flint_gemm_nt: y is null")
    _fails(flint, "flint_gemm_nt", A + 8, A * 2, A * 3, 8, 8, 8, None,
           message="flint_gemm_nt: y is not 16-byte aligned")
    _fails(flint, "flint_gemm_nt", A, A, A * 3, 8, 8, 8, None, message="flint_gemm_nt: y and x overlap")
    _fails(flint, "flint_gemm_nn", A, A * 2, A * 3, 8, 12, 8, None,
           message="flint_gemm_nn: n (12) must be a multiple of 8")
    _fails(flint, "flint_gemm_nt", A, A * 2, A * 3, 8, 8, 1 << 17, None, message="is too large")
    _fails(flint, "flint_gemm_nt_bias_residual", A, A * 2, A * 3, A * 4, A * 5, 8, 3, 8, None,
           message="flint_gemm_nt_bias_residual: n (3) must be even")
    _fails(flint, "flint_gemm_tn", A, A * 2, A * 3, 12, 8, 8, 0, None, 0, None,
           message="flint_gemm_tn: m (12) must be a multiple of 8")
    _fails(flint, "flint_gemm_nt_batched", A, A * 2, A * 3, 2, 8, 8, 8, ctypes.c_float(float("inf")),
           None, message="flint_gemm_nt_batched: scale (inf) must be finite")
    _fails(flint, "flint_gemm_nt_batched", A, A * 2, A * 3, 2, 1025, 8, 8, ctypes.c_float(1.0),
           None, message="flint_gemm_nt_batched: m (1025) can be up to 1024")


def test_zero_sizes_check_nothing(flint):
    """m or n of 0 returns OK before any check, even with null pointers
    (ref tests/test_gemm.py:640-650)."""
    assert flint.lib.flint_gemm_nt(None, None, None, 0, 8, 12, None) == 0
    assert flint.lib.flint_gemm_nn(None, None, None, 8, 0, 3, None) == 0
    assert flint.lib.flint_gemm_tn(None, None, None, 0, 0, 0, 0, None, 0, None) == 0
    assert flint.lib.flint_layernorm_forward(None, None, None, None, None, None, 0, 8,
                                             ctypes.c_float(1e-5), None) == 0


def test_reduction_validation(flint):
    _fails(flint, "flint_layernorm_forward", A, A * 2, A * 3, A * 4, A * 5, A * 6, 4, 0,
           ctypes.c_float(1e-5), None, message="flint_layernorm_forward: cols (0) must be from 1 to")
    _fails(flint, "flint_layernorm_forward", A, A * 2, A * 3, A * 4, A * 5, A * 6, 4, 8,
           ctypes.c_float(-1.0), None, message="eps (-1) must be finite and non-negative")
    _fails(flint, "flint_causal_softmax_forward", A, A * 2, 1, 12, None,
           message="flint_causal_softmax_forward: length (12) must be a multiple of 8 up to 1024")
    _fails(flint, "flint_softmax_cross_entropy", A, A * 2, A * 3, A * 4, ctypes.c_float(1.0), 4,
           20, 16, None, message="vocab (20) must be from 1 to cols (16)")
    _fails(flint, "flint_bias_gradient", A, A * 2, 256, 16, 0, A * 3, 8, None,
           message="flint_bias_gradient: needs 128 bytes of workspace, given 8")
    size = ctypes.c_size_t(0)
    assert flint.lib.flint_bias_gradient_workspace(257, 16, ctypes.byref(size)) == 0
    assert size.value == 2 * 16 * 8
    assert flint.lib.flint_layernorm_backward_workspace(8192, 768, ctypes.byref(size)) == 0
    assert size.value == 2 * 32 * 768 * 8   # the dbeta and dgamma chunk partials


def test_support_validation(flint):
    _fails(flint, "flint_copy", A, A + 4, 16, None, message="flint_copy: dst and src overlap")
    _fails(flint, "flint_heads_split", A, A * 2, 1, 8, 3, 64, 128, 0, None,
           message="3 heads of 64 columns from column 0 run past row_width (128)")
    _fails(flint, "flint_embedding_forward", A, A * 2, A * 3, A * 4, 1, 8, 0, 64, None,
           message="vocab (0) must be from 1 to 65536")


def test_gpt2_config_validation(flint):
    cfg = flint_lib.Gpt2Config(layers=12, heads=12, width=768, block_size=1024, vocab=50257,
                               padded_vocab=50304, sequences=8, length=1024, separate_buffers=0,
                               backward=0)
    size = ctypes.c_size_t(0)
    assert flint.lib.flint_gpt2_bytes(ctypes.byref(cfg), ctypes.byref(size)) == 0
    assert size.value > 124_000_000 * 4
    bad = flint_lib.Gpt2Config(**{f: getattr(cfg, f) for f, _ in cfg._fields_})
    bad.heads = 7
    assert flint.lib.flint_gpt2_bytes(ctypes.byref(bad), ctypes.byref(size)) == 1
    assert "heads (7) must split width (768) into multiples of 8" in flint.last_error()
    assert flint.lib.flint_gpt2_parameter_count(None) == 0


def test_attention_checks_fail_before_any_device_work(flint):
    from flint_amd.flint_lib import FlintError

    with pytest.raises(FlintError, match="head_width \\(32\\) must be 64"):
        flint.attention_forward(16, 32, 48, 64, 80, 2, 8, 32, 0.125, stream=0)
    with pytest.raises(FlintError, match="scale .* must be finite"):
        flint.attention_forward(16, 32, 48, 64, 80, 2, 8, 64, float("inf"), stream=0)
    with pytest.raises(FlintError, match="q is null"):
        flint.attention_forward(16, 1 << 20, None, 64, 80, 2, 8, 64, 0.125, stream=0)
    assert flint.attention_backward_workspace(96, 1024, 64) == 96 * 1024 * 4
    with pytest.raises(FlintError, match="needs 64 bytes of workspace, given 8"):
        flint.attention_backward(16, 32, 48, 64, 80, 96, 112, 128, 144, 2, 8, 64, 0.125,
                                 workspace=1 << 20, workspace_bytes=8, stream=0)
    # Empty calls succeed without touching anything.
    flint.attention_forward(None, None, None, None, None, 0, 8, 64, 0.125, stream=0)

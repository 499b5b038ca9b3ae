"""flint_gpt2_bytes / flint_gpt2_create: the model's device bytes against an
independent sum, its configuration limits, and validation messages (the
contracts of ref tests/test_gpt2.py:985-1056, :1582-1660 and
ref tests/test_gpt2_backward.py:998-1066, restated as this file's own cases).

The byte sum lists every buffer the model holds, each rounded up to 256 bytes.
flint_gpt2_create's model is the reference's: per-head q, k, v, the stored
scores and probabilities, and the heads' output. flint_gpt2_create_fused's
keeps each block's qkv projection and log-sum-exp instead. Without backward
the sums need no device (CPU tests); with backward the workspace sizes are
the device's answers to the *_workspace queries (GPU tests)."""

import ctypes

import pytest

from flint_amd import flint_lib
from flint_amd.flint_lib import Gpt2Config

ALIGN = 256


def _up(n):
    return (n + ALIGN - 1) // ALIGN * ALIGN


def _config(**f):
    return Gpt2Config(f["layers"], f["heads"], f["width"], f["block_size"], f["vocab"],
                      f["padded_vocab"], f["sequences"], f["length"], f.get("separate", 0),
                      f.get("backward", 0))


def _bytes(flint, fused=False, **f):
    out = ctypes.c_size_t(0)
    fn = flint.lib.flint_gpt2_bytes_fused if fused else flint.lib.flint_gpt2_bytes
    flint.check(fn(ctypes.byref(_config(**f)), ctypes.byref(out)))
    return out.value


def _masters(f):
    """The FP32 parameters, named_parameters order."""
    w, L = f["width"], f["layers"]
    per_layer = [w, w, 3 * w * w, 3 * w, w * w, w, w, w, 4 * w * w, 4 * w, 4 * w * w, w]
    return [f["padded_vocab"] * w, f["block_size"] * w] + per_layer * L + [w, w]


def expected_sum(f, fused=False, backward=False, workspaces=None):
    """Every buffer of the model in bytes (rounded up one by one, then added).
    workspaces: (shared, tn) byte counts, needed with backward."""
    w, L = f["width"], f["layers"]
    rows = f["sequences"] * f["length"]
    nb = f["sequences"] * f["heads"]
    hw = w // f["heads"]
    heads_rows = nb * f["length"] * hw * 2          # one [batches][length][head width] FP16
    square = nb * f["length"] * f["length"] * 2     # scores or probabilities, FP16
    lse = nb * f["length"] * 4
    resid, half_rows, row_f32 = rows * w * 4, rows * w * 2, rows * 4
    qkv, mlp = rows * 3 * w * 2, rows * 4 * w * 2
    parts = [4 * n for n in _masters(f)]
    if backward:
        parts += [4 * n for n in _masters(f)]       # a gradient per master
    parts += [f["padded_vocab"] * w * 2]            # wte's FP16 copy
    parts += [2 * n for _ in range(L) for n in (3 * w * w, w * w, 4 * w * w, 4 * w * w)]
    attention = [qkv, lse] if fused else [heads_rows] * 3 + [square]
    if backward:
        parts += [resid] * (2 * L + 1)               # x_in, x_mid per block; the last output
        for _ in range(L):
            parts += [half_rows, row_f32, row_f32] + attention + [half_rows]
            parts += [half_rows, row_f32, row_f32, mlp, mlp]
        parts += [half_rows, row_f32, row_f32, qkv]  # ln_f's output, mean, rstd; qkv scratch
        parts += [lse] if fused else [square, heads_rows] + [heads_rows] * 3   # D / S, O, dq, dk, dv
        parts += [resid, half_rows, half_rows, mlp]  # dres, its FP16 copy, dh, dpre
        parts += list(workspaces)
    else:
        parts += [resid, resid, half_rows, row_f32, row_f32, qkv]
        parts += [lse] if fused else [heads_rows] * 3 + [square, square, heads_rows]
        parts += [half_rows, mlp, mlp]
    parts += [rows * f["padded_vocab"] * 2] * 2 + [row_f32]   # logits, dlogits, row_loss
    return sum(_up(p) for p in parts)


def _workspaces(flint, f):
    rows, w = f["sequences"] * f["length"], f["width"]
    shared = [flint.bias_gradient_workspace(rows, c) for c in (w, 3 * w, 4 * w)]
    shared += [flint.layernorm_backward_workspace(rows, w),
               flint.embedding_backward_workspace(f["sequences"], f["length"],
                                                  f["padded_vocab"], w)]
    tn = [flint.gemm_tn_workspace(m, n, rows) for m, n in
          ((f["padded_vocab"], w), (3 * w, w), (w, w), (4 * w, w), (w, 4 * w))]
    return max(shared), max(tn)


GPT2 = dict(layers=12, heads=12, width=768, block_size=1024, vocab=50257, padded_vocab=50304)
# The reference's TINY model (ref scripts/gpt2_torch.py:34): heads of width 64.
REF_TINY = dict(layers=2, heads=2, width=128, block_size=64, vocab=50257, padded_vocab=50304)
ODDS = dict(layers=3, heads=4, width=96, block_size=40, vocab=100, padded_vocab=104)
# Legal configurations at the limits the validation allows: the most layers,
# the widest width, the most head batches (65,535), the most rows (8,388,480)
# and the smallest model, plus one past every size but the largest. Only sizes
# are asked of these; none is allocated.
LIMITS = {
    "layers-1024": dict(layers=1024, heads=4, width=256, block_size=1024, vocab=50000,
                        padded_vocab=50048, sequences=2, length=1024),
    "width-16384": dict(layers=3, heads=64, width=16384, block_size=1024, vocab=65536,
                        padded_vocab=65536, sequences=3, length=1024),
    "head-batches-65535": dict(layers=2, heads=15, width=960, block_size=512, vocab=30000,
                               padded_vocab=30000, sequences=4369, length=512),
    "rows-8388480": dict(layers=2, heads=1, width=32, block_size=256, vocab=40000,
                         padded_vocab=40000, sequences=65535, length=128),
    "smallest": dict(layers=1, heads=1, width=8, block_size=8, vocab=1, padded_vocab=8,
                     sequences=1, length=8),
    "largest": dict(layers=1024, heads=16, width=16384, block_size=1024, vocab=65536,
                    padded_vocab=65536, sequences=4095, length=1024),
}
CASES = {"gpt2-8x1024": {**GPT2, "sequences": 8, "length": 1024},
         "gpt2-16x1024": {**GPT2, "sequences": 16, "length": 1024},
         "ref-tiny-2x32": {**REF_TINY, "sequences": 2, "length": 32},
         "odd-3x24": {**ODDS, "sequences": 3, "length": 24},
         **LIMITS}


@pytest.mark.parametrize("name", list(CASES))
def test_forward_bytes_equal_the_independent_sum(flint, name):
    f = CASES[name]
    assert _bytes(flint, **f) == expected_sum(f)
    if f["width"] // f["heads"] == 64:
        assert _bytes(flint, fused=True, **f) == expected_sum(f, fused=True)


def test_the_largest_config_is_terabytes_without_wrapping(flint):
    total = _bytes(flint, **LIMITS["largest"])
    assert total > 2**40 and total == expected_sum(LIMITS["largest"])


def _backward_legal(f):
    return f["sequences"] * f["length"] <= 65536 and f["length"] * f["width"] <= 16776960


@pytest.mark.gpu
@pytest.mark.parametrize("name", [n for n, f in CASES.items() if _backward_legal(f)])
def test_backward_bytes_equal_the_independent_sum(flint, cuda, name):
    f = dict(CASES[name], backward=1)
    ws = _workspaces(flint, f)
    assert _bytes(flint, **f) == expected_sum(f, backward=True, workspaces=ws)
    if f["width"] // f["heads"] == 64:
        assert _bytes(flint, fused=True, **f) == expected_sum(f, fused=True, backward=True,
                                                              workspaces=ws)


def test_fused_needs_heads_of_width_64(flint):
    f = dict(ODDS, sequences=1, length=8)
    out = ctypes.c_size_t(0xDEAD)
    st = flint.lib.flint_gpt2_bytes_fused(ctypes.byref(_config(**f)), ctypes.byref(out))
    assert st == flint_lib.ERROR_INVALID_ARGUMENT and out.value == 0xDEAD
    assert "flint_gpt2_bytes_fused" in flint.last_error() and "64" in flint.last_error()


# Each case: the fields changed from a legal GPT-2 batch, and the argument
# whose value the message must name ("name (value)").
GOOD = dict(GPT2, sequences=2, length=64)
REJECTED = {
    "layers-0": ("layers", dict(layers=0)),
    "layers-1025": ("layers", dict(layers=1025)),
    "width-12": ("width", dict(width=12, heads=1)),
    "width-16392": ("width", dict(width=16392, heads=1)),
    "heads-0": ("heads", dict(heads=0)),
    "heads-of-4": ("heads", dict(heads=192)),
    "length-0": ("length", dict(length=0)),
    "length-1032": ("length", dict(length=1032, block_size=1024)),
    "block_size-below-length": ("block_size", dict(block_size=32)),
    "block_size-2048": ("block_size", dict(block_size=2048)),
    "padded_vocab-65544": ("padded_vocab", dict(padded_vocab=65544, vocab=100)),
    "padded_vocab-odd": ("padded_vocab", dict(padded_vocab=50305)),
    "vocab-0": ("vocab", dict(vocab=0)),
    "vocab-past-padded": ("vocab", dict(vocab=50305)),
    "sequences-0": ("sequences", dict(sequences=0)),
    "head-batches-65536": ("sequences", dict(sequences=65536, heads=1, width=8, length=8,
                                             block_size=8)),
    "sequences-2^63": ("sequences", dict(sequences=2**63)),
    "rows-8388608": ("sequences", dict(sequences=8192, heads=1, width=8, length=1024,
                                       block_size=1024)),
}


def _call(flint, fn, **fields):
    f = {**GOOD, **fields}
    if fn == "bytes":
        out = ctypes.c_size_t(0xDEAD)
        st = flint.lib.flint_gpt2_bytes(ctypes.byref(_config(**f)), ctypes.byref(out))
        return st, out.value, f
    handle = ctypes.c_void_p(0x1234)
    st = flint.lib.flint_gpt2_create(ctypes.byref(_config(**f)), ctypes.byref(handle))
    return st, handle.value, f


@pytest.mark.parametrize("case", list(REJECTED))
def test_a_rejected_config_names_its_argument(flint, case):
    arg, fields = REJECTED[case]
    st, value, f = _call(flint, "bytes", **fields)
    assert st == flint_lib.ERROR_INVALID_ARGUMENT and value == 0xDEAD
    msg = flint.last_error()
    assert msg.startswith("flint_gpt2_bytes: ") and f"{arg} ({f[arg]})" in msg, msg
    st, handle, _ = _call(flint, "create", **fields)
    assert st == flint_lib.ERROR_INVALID_ARGUMENT and handle is None
    assert flint.last_error().startswith("flint_gpt2_create: ")


def test_the_first_wrong_argument_is_the_one_named(flint):
    order = ["layers", "width", "heads", "length", "block_size", "padded_vocab", "vocab",
             "sequences"]
    broken = dict(layers=0, width=12, heads=0, length=12, block_size=0, padded_vocab=12,
                  vocab=0, sequences=0)
    for i, name in enumerate(order):
        st, _, _ = _call(flint, "bytes", **{k: broken[k] for k in order[i:]})
        assert st == flint_lib.ERROR_INVALID_ARGUMENT
        assert flint.last_error().startswith(f"flint_gpt2_bytes: {name} ("), flint.last_error()


def test_backward_limits_are_checked(flint):
    rows = dict(GPT2, sequences=65, length=1024, backward=1)
    st, _, _ = _call(flint, "bytes", **rows)
    assert st == flint_lib.ERROR_INVALID_ARGUMENT
    assert "with backward" in flint.last_error() and "sequences (65)" in flint.last_error()
    wide = dict(layers=1, heads=128, width=16384, block_size=1024, vocab=8, padded_vocab=8,
                sequences=1, length=1024, backward=1)
    st, _, _ = _call(flint, "bytes", **wide)
    assert st == flint_lib.ERROR_INVALID_ARGUMENT
    assert "length (1024) x width (16384)" in flint.last_error()


@pytest.mark.gpu
def test_a_model_too_large_for_the_gpu_fails_create_cleanly(flint, cuda):
    """A legal configuration of terabytes: create reports a HIP out-of-memory
    failure, leaves *model null, and keeps no device memory."""
    import torch

    f = {**GPT2, "sequences": 8000, "length": 1024, "heads": 6}
    assert _bytes(flint, **f) > torch.cuda.mem_get_info()[1]
    torch.cuda.synchronize()
    before = torch.cuda.mem_get_info()[0]
    for separate in (0, 1):
        handle = ctypes.c_void_p(0x1234)
        st = flint.lib.flint_gpt2_create(ctypes.byref(_config(**f, separate=separate)),
                                         ctypes.byref(handle))
        assert st == flint_lib.ERROR_CUDA and handle.value is None
        assert "out of memory" in flint.last_error().lower(), flint.last_error()
    assert before - torch.cuda.mem_get_info()[0] < 64 << 20

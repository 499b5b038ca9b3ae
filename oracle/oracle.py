"""CPU oracle for libflint's hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker: nothing in the product path calls it.

Two kinds of reference live here:
  * numpy float64 closed forms of every function on the path (GEMM layouts
    and epilogues, GELU and its derivative, LayerNorm, causal softmax,
    cross-entropy, their gradients), each citing the reference line whose
    semantics it restates;
  * `liboracle.so` (oracle/flint_oracle.c), a plain-C FP32 restatement of the
    reference's reduction kernels with their exact summation orders, used
    where the reference promises shape-only, bit-reproducible orders.

Inputs and outputs are numpy arrays. FP16 values are passed as float16 arrays
and widened here; results that the kernel rounds to FP16 are rounded with
numpy's float32 -> float16 cast, which is round-to-nearest-even.
"""

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_lib = None


def lib():
    """The C oracle, built from oracle/flint_oracle.c on first use if absent."""
    global _lib
    if _lib is None:
        if not LIB.is_file():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        _lib = ctypes.CDLL(str(LIB))
    return _lib


def _fp(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ GEMMs
# ref include/flint/flint.h:53-191, src/kernels/gemm.cu:198-412 (epilogue order)

SQRT_2_OVER_PI = np.sqrt(2.0 / np.pi)


def gelu64(s):
    """GPT-2's tanh GELU in float64 (ref flint.h:74-78)."""
    s = np.asarray(s, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        return 0.5 * s * (1.0 + np.tanh(SQRT_2_OVER_PI * (s + 0.044715 * s ** 3)))


def gelu_grad64(s):
    """d/ds of gelu64, with GELU's limits at +-inf and NaN kept (ref flint.h:104-111)."""
    s = np.asarray(s, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        u = SQRT_2_OVER_PI * (s + 0.044715 * s ** 3)
        t = np.tanh(u)
        du = SQRT_2_OVER_PI * (1.0 + 3 * 0.044715 * s ** 2)
        g = 0.5 * (1.0 + t) + 0.5 * s * (1.0 - t * t) * du
    g = np.where(np.isposinf(s), 1.0, g)
    g = np.where(np.isneginf(s), 0.0, g)
    # Far from 0 the product s (1 - t^2) du underflows to 0 * inf in float64.
    g = np.where(np.isfinite(s) & ~np.isfinite(g), np.where(s > 0, 1.0, 0.0), g)
    return g


def gemm64(x, w, layout):
    """y = x w^T (NT), x w (NN) or x^T w (TN) in float64."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    if layout == "nt":
        return x @ w.T
    if layout == "nn":
        return x @ w
    if layout == "tn":
        return x.T @ w
    raise ValueError(layout)


def gemm_epilogue64(s, epilogue, bias=None, residual=None, pre=None, scale=1.0):
    """The epilogue applied to float64 sums s (ref gemm.cu:247-412):
    'none' | 'bias' | 'bias_gelu' (returns (y, pre)) | 'bias_residual' | 'dgelu' | 'scale'."""
    if epilogue == "none":
        return s
    if epilogue == "scale":
        return s * scale
    if epilogue == "bias":
        return s + bias
    if epilogue == "bias_gelu":
        v = s + bias
        return gelu64(v), v
    if epilogue == "bias_residual":
        return residual + (s + bias)
    if epilogue == "dgelu":
        return s * gelu_grad64(pre)
    raise ValueError(epilogue)


# -------------------------------------------------------- row reductions, f64


def layernorm64(x, gamma, beta, eps):
    """Textbook LayerNorm in float64: returns (y, mean, rstd) (ref flint.h:193-213)."""
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    rstd = 1.0 / np.sqrt(var + eps)
    return (x - mu) * rstd * gamma + beta, mu[:, 0], rstd[:, 0]


def layernorm_backward64(dy, x, mean, rstd, gamma):
    """dx, dgamma, dbeta in float64 from the forward's statistics (ref flint.h:215-241)."""
    dy = np.asarray(dy, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    xhat = (x - mean[:, None]) * rstd[:, None]
    g = dy * gamma
    dx = rstd[:, None] * (g - g.mean(axis=1, keepdims=True)
                          - xhat * (g * xhat).mean(axis=1, keepdims=True))
    return dx, (dy * xhat).sum(axis=0), dy.sum(axis=0)


def causal_softmax64(s, length):
    """Row t of each batch over columns 0..t, +0 beyond (ref flint.h:350-369)."""
    s = np.asarray(s, dtype=np.float64).reshape(-1, length, length)
    mask = np.tril(np.ones((length, length), dtype=bool))
    z = np.where(mask, s, -np.inf)
    z = z - z.max(axis=2, keepdims=True)
    e = np.where(mask, np.exp(z), 0.0)
    return (e / e.sum(axis=2, keepdims=True)).reshape(-1, length)


def causal_softmax_backward64(p, dp, length, scale):
    """ds = scale p (dp - sum p dp) over visible columns (ref flint.h:371-392)."""
    p = np.asarray(p, dtype=np.float64).reshape(-1, length, length)
    dp = np.asarray(dp, dtype=np.float64).reshape(-1, length, length)
    mask = np.tril(np.ones((length, length), dtype=bool))
    p = np.where(mask, p, 0.0)
    dp = np.where(mask, dp, 0.0)
    d = (p * dp).sum(axis=2, keepdims=True)
    return np.where(mask, scale * p * (dp - d), 0.0).reshape(-1, length)


def cross_entropy64(logits, targets, vocab, scale):
    """(row_loss, dlogits) in float64 over the first vocab columns (ref flint.h:394-433)."""
    l = np.asarray(logits, dtype=np.float64)
    rows, cols = l.shape
    v = l[:, :vocab]
    mx = v.max(axis=1, keepdims=True)
    e = np.exp(v - mx)
    s = e.sum(axis=1, keepdims=True)
    t = np.asarray(targets, dtype=np.int64)
    loss = np.log(s[:, 0]) - (v[np.arange(rows), t] - mx[:, 0])
    d = np.zeros((rows, cols))
    d[:, :vocab] = e / s
    d[np.arange(rows), t] -= 1.0
    return loss, d * scale


# ---------------------------------------------------- FP32 order emulations (C)


def layernorm_forward(x, gamma, beta, eps):
    """FP32 emulation of the reference kernel; y rounded to FP16."""
    x = _f32(x)
    rows, cols = x.shape
    y = np.empty((rows, cols), np.float32)
    mean = np.empty(rows, np.float32)
    rstd = np.empty(rows, np.float32)
    lib().or_layernorm_forward(_fp(y), _fp(mean), _fp(rstd), _fp(x), _fp(_f32(gamma)),
                               _fp(_f32(beta)), ctypes.c_size_t(rows), ctypes.c_size_t(cols),
                               ctypes.c_float(eps))
    return y.astype(np.float16), mean, rstd


def bias_gradient(dy, old=None):
    """Column sums of FP16 dy in the reference's chunk order (FP32 out)."""
    dy = _f32(np.asarray(dy, dtype=np.float16))
    rows, cols = dy.shape
    out = np.zeros(cols, np.float32) if old is None else _f32(old).copy()
    lib().or_bias_gradient(_fp(out), _fp(dy), ctypes.c_size_t(rows), ctypes.c_size_t(cols),
                           ctypes.c_int(old is not None))
    return out


def layernorm_backward(dy, x, mean, rstd, gamma, dx_old=None, dgamma_old=None, dbeta_old=None):
    dy = _f32(np.asarray(dy, dtype=np.float16))
    x = _f32(x)
    rows, cols = x.shape
    acc_dx = dx_old is not None
    acc_p = dgamma_old is not None
    dx = _f32(dx_old).copy() if acc_dx else np.zeros((rows, cols), np.float32)
    dgamma = _f32(dgamma_old).copy() if acc_p else np.zeros(cols, np.float32)
    dbeta = _f32(dbeta_old).copy() if acc_p else np.zeros(cols, np.float32)
    lib().or_layernorm_backward(_fp(dx), _fp(dgamma), _fp(dbeta), _fp(dy), _fp(x),
                                _fp(_f32(mean)), _fp(_f32(rstd)), _fp(_f32(gamma)),
                                ctypes.c_size_t(rows), ctypes.c_size_t(cols), ctypes.c_int(acc_dx),
                                ctypes.c_int(acc_p))
    return dx, dgamma, dbeta


def softmax_forward(s, length):
    s = _f32(np.asarray(s, dtype=np.float16)).reshape(-1, length)
    p = np.empty_like(s)
    lib().or_softmax_forward(_fp(p), _fp(s), ctypes.c_size_t(s.shape[0]), ctypes.c_size_t(length))
    return p.astype(np.float16)


def softmax_backward(p, dp, length, scale):
    p = _f32(np.asarray(p, dtype=np.float16)).reshape(-1, length)
    dp = _f32(np.asarray(dp, dtype=np.float16)).reshape(-1, length)
    ds = np.empty_like(p)
    lib().or_softmax_backward(_fp(ds), _fp(p), _fp(dp), ctypes.c_size_t(p.shape[0]),
                              ctypes.c_size_t(length), ctypes.c_float(scale))
    return ds.astype(np.float16)


def cross_entropy(logits, targets, vocab, scale):
    """(row_loss FP32, dlogits FP16) as the reference kernel computes them."""
    l = _f32(np.asarray(logits, dtype=np.float16))
    rows, cols = l.shape
    t = np.ascontiguousarray(targets, dtype=np.uint16)
    d = np.empty_like(l)
    loss = np.full(rows, np.nan, np.float32)
    lib().or_cross_entropy(_fp(d), _fp(loss), _fp(l), _fp(t), ctypes.c_float(scale),
                           ctypes.c_size_t(rows), ctypes.c_size_t(vocab), ctypes.c_size_t(cols))
    return loss, d.astype(np.float16)


def embedding_backward(dx, tokens, sequences, length, vocab, width, dwte_old=None,
                       dwpe_old=None):
    dx = _f32(dx)
    t = np.ascontiguousarray(tokens, dtype=np.uint16)
    dwte = _f32(dwte_old).copy() if dwte_old is not None else np.zeros((vocab, width), np.float32)
    dwpe = _f32(dwpe_old).copy() if dwpe_old is not None else np.zeros((length, width), np.float32)
    lib().or_embedding_backward(_fp(dwte), _fp(dwpe), _fp(dx), _fp(t), ctypes.c_size_t(sequences),
                                ctypes.c_size_t(length), ctypes.c_size_t(vocab),
                                ctypes.c_size_t(width), ctypes.c_int(dwte_old is not None),
                                ctypes.c_int(dwpe_old is not None))
    return dwte, dwpe


def rel_max_err(got, ref):
    """max |got - ref| / max |ref| over finite reference values (the north-star metric)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref))
    if denom == 0:
        return float(np.max(np.abs(got - ref)))
    return float(np.max(np.abs(got - ref)) / denom)


# --------------------------------------------------------------------------
# AdamW step with clipping and a dynamic loss scale (the training-step
# extension, include/flint/flint_train.h). The reference's step is
# scripts/gpt2_torch.py:161-192 with the constants at :37-42, run by PyTorch
# (2.10 in this image): GradScaler.unscale_ (grad * float(1 / scale)),
# clip_grad_norm_ (norm over all tensors; coef = max_norm / (norm + 1e-6),
# clamped to 1), AdamW (param *= 1 - lr * wd; exp_avg.lerp_(g, 1 - beta1);
# exp_avg_sq = beta2 v + (1 - beta2) g^2; denom = sqrt(v) / sqrt(1 - beta2^t)
# + eps; param -= lr / (1 - beta1^t) * m / denom) and GradScaler.update
# (backoff on a non-finite gradient, growth after growth_interval finite
# steps). All elementwise arithmetic is FP32 as in PyTorch; the norm is FP64.
# Pinned in tests/test_train.py against torch.optim.AdamW, clip_grad_norm_ and
# torch.amp.GradScaler on the CPU.
# --------------------------------------------------------------------------

def adamw_step(tensors, state, lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, max_grad_norm=1.0,
               growth_factor=2.0, backoff_factor=0.5, growth_interval=2000):
    """One step in place. tensors: dicts with float32 arrays param, grad,
    exp_avg, exp_avg_sq and a float weight_decay. state: dict with loss_scale,
    growth_tracker, step (updated in place). Returns (skipped, norm, clip)."""
    f32 = np.float32
    inv = f32(1.0 / float(f32(state["loss_scale"])))
    unscaled = [t["grad"].astype(f32) * inv for t in tensors]
    sumsq = sum(float(np.sum(u.astype(np.float64) ** 2)) for u in unscaled)
    if not np.isfinite(sumsq):
        state["loss_scale"] = float(f32(state["loss_scale"]) * f32(backoff_factor))
        state["growth_tracker"] = 0
        return True, float(np.sqrt(sumsq)), 0.0
    norm = np.sqrt(sumsq)
    clip = f32(min(1.0, max_grad_norm / (norm + 1e-6))) if max_grad_norm > 0 else f32(1.0)
    state["step"] += 1
    t_ = state["step"]
    step_size = f32(lr / (1.0 - beta1 ** t_))
    bc2_sqrt = f32(np.sqrt(1.0 - beta2 ** t_))
    for t, u in zip(tensors, unscaled):
        g = u * clip
        p, m, v = t["param"], t["exp_avg"], t["exp_avg_sq"]
        p *= f32(1.0 - lr * t["weight_decay"])
        m += f32(1.0 - beta1) * (g - m)
        v *= f32(beta2)
        v += f32(1.0 - beta2) * (g * g)
        denom = np.sqrt(v) / bc2_sqrt + f32(eps)
        p -= step_size * (m / denom)
    if state["growth_tracker"] + 1 == growth_interval:
        state["loss_scale"] = float(f32(state["loss_scale"]) * f32(growth_factor))
        state["growth_tracker"] = 0
    else:
        state["growth_tracker"] += 1
    return False, float(norm), float(clip)

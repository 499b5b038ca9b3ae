"""Pins the CPU oracle (CPU only, no GPU): against the committed golden fixtures
(PyTorch float64 operators, tests/golden/make_golden.py), against closed forms
and exact cases the reference's tests use, and against planted mistakes, so
that a dropped term, a wrong sign or a transposed operand in the oracle fails
here before the oracle is trusted to judge the kernels."""

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")


def close(a, b, tol):
    return oracle.rel_max_err(a, b) <= tol


# ------------------------------------------------------------------ GELU


def test_gelu_against_golden():
    s = GOLDEN["gelu_in"]
    assert close(oracle.gelu64(s), GOLDEN["gelu_out"], 1e-12)
    assert close(oracle.gelu_grad64(s), GOLDEN["gelu_grad"], 1e-10)


def test_gelu_limits_and_identities():
    assert oracle.gelu64(np.inf) == np.inf
    assert np.isnan(oracle.gelu64(-np.inf))
    assert oracle.gelu_grad64(np.inf) == 1.0 and oracle.gelu_grad64(-np.inf) == 0.0
    assert np.isnan(oracle.gelu_grad64(np.nan))
    assert oracle.gelu_grad64(0.0) == 0.5
    # The x / (1 + exp(-2u)) form the kernel evaluates is the same function.
    s = np.linspace(-8, 8, 1001)
    u = np.sqrt(2 / np.pi) * (s + 0.044715 * s ** 3)
    assert close(s / (1 + np.exp(-2 * u)), oracle.gelu64(s), 1e-13)
    # Finite differences pin the derivative (a dropped term fails this).
    h = 1e-6
    fd = (oracle.gelu64(s + h) - oracle.gelu64(s - h)) / (2 * h)
    assert close(oracle.gelu_grad64(s), fd, 1e-7)


# ------------------------------------------------------------------ GEMM


def test_gemm_epilogues_against_golden():
    x, w, b, r = (GOLDEN[k] for k in ("gemm_x", "gemm_w", "gemm_b", "gemm_r"))
    s = oracle.gemm64(x, w, "nt")
    assert close(s, GOLDEN["gemm_nt"], 1e-14)
    assert close(oracle.gemm_epilogue64(s, "bias", bias=b), GOLDEN["gemm_bias"], 1e-14)
    y, pre = oracle.gemm_epilogue64(s, "bias_gelu", bias=b)
    assert close(y, GOLDEN["gemm_gelu"], 1e-12) and close(pre, GOLDEN["gemm_bias"], 1e-14)
    assert close(oracle.gemm_epilogue64(s, "bias_residual", bias=b, residual=r),
                 GOLDEN["gemm_residual"], 1e-14)
    # Layouts: NN of w^T and TN of x^T are the same product.
    assert close(oracle.gemm64(x, w.T, "nn"), s, 1e-14)
    assert close(oracle.gemm64(x.T, w.T, "tn"), s, 1e-14)
    assert not close(oracle.gemm64(x, w.T, "nn").T[: s.shape[0], : s.shape[0]],
                     s[:, : s.shape[0]], 1e-3)


# ------------------------------------------------------------------ LayerNorm


def test_layernorm_forward_against_golden():
    x, gm, bt = GOLDEN["ln_x"], GOLDEN["ln_gamma"], GOLDEN["ln_beta"]
    y64, mu64, rs64 = oracle.layernorm64(x, gm, bt, 1e-5)
    assert close(y64, GOLDEN["ln_y"], 1e-12)
    y, mu, rs = oracle.layernorm_forward(x.astype(np.float32), gm, bt, 1e-5)
    assert close(y, GOLDEN["ln_y"], 1e-3)
    assert close(mu, mu64, 1e-7) and close(rs, rs64, 1e-6)


def test_layernorm_forward_exact_cases():
    """Constant rows give beta exactly; a single column gives beta (var 0)
    (ref tests/test_layernorm.py:342-411)."""
    beta = np.linspace(-1, 1, 64).astype(np.float32)
    gamma = np.ones(64, np.float32)
    y, mu, rs = oracle.layernorm_forward(np.full((3, 64), 7.5, np.float32), gamma, beta, 1e-5)
    assert np.array_equal(y, beta.astype(np.float16)[None].repeat(3, 0))
    assert np.all(mu == 7.5)
    y1, _, _ = oracle.layernorm_forward(np.array([[5.0]], np.float32), np.ones(1, np.float32),
                                        np.array([0.25], np.float32), 1e-5)
    assert y1[0, 0] == np.float16(0.25)


def test_layernorm_backward_against_golden():
    x, gm = GOLDEN["ln_x"], GOLDEN["ln_gamma"]
    _, mu, rs = oracle.layernorm64(x, gm, GOLDEN["ln_beta"], 1e-5)
    dy = GOLDEN["ln_dy"]
    dx64, dg64, db64 = oracle.layernorm_backward64(dy, x, mu, rs, gm)
    assert close(dx64, GOLDEN["ln_dx"], 1e-10)
    assert close(dg64, GOLDEN["ln_dgamma"], 1e-10)
    assert close(db64, GOLDEN["ln_dbeta"], 1e-12)
    dx, dg, db = oracle.layernorm_backward(dy.astype(np.float16), x.astype(np.float32),
                                           mu.astype(np.float32), rs.astype(np.float32), gm)
    assert close(dx, GOLDEN["ln_dx"], 1e-3)
    assert close(dg, GOLDEN["ln_dgamma"], 1e-5)
    assert close(db, GOLDEN["ln_dbeta"], 1e-6)
    # accumulate: one FP32 add onto the old values.
    old = np.ones_like(dx)
    dxa, dga, dba = oracle.layernorm_backward(dy.astype(np.float16), x.astype(np.float32),
                                              mu.astype(np.float32), rs.astype(np.float32), gm,
                                              old, old[0], old[0])
    assert np.array_equal(dxa, (old + dx).astype(np.float32))
    assert np.array_equal(dba, (old[0] + db).astype(np.float32))


# ------------------------------------------------------------------ bias gradient


def test_bias_gradient_is_nearly_correctly_rounded():
    rng = np.random.default_rng(0)
    dy = rng.standard_normal((1000, 64)).astype(np.float16)
    dy[:, 3] += np.float16(3000)
    exact = dy.astype(np.float64).sum(0)
    got = oracle.bias_gradient(dy)
    assert np.mean(got == exact.astype(np.float32)) >= 0.95
    assert close(got, exact, 1e-7)
    # A plain FP32 running sum (the mistake compensation guards against) is worse.
    plain = np.zeros(64, np.float32)
    for r in range(dy.shape[0]):
        plain = plain + dy[r].astype(np.float32)
    assert np.abs(plain - exact).max() > np.abs(got - exact).max()


def test_bias_gradient_nonfinite():
    dy = np.zeros((300, 8), np.float16)
    dy[5, 0] = np.inf
    dy[7, 1] = np.nan
    got = oracle.bias_gradient(dy)
    assert got[0] == np.inf and np.isnan(got[1]) and np.all(got[2:] == 0)


# ------------------------------------------------------------------ softmax


def test_softmax_against_golden():
    s, t = GOLDEN["sm_s"], GOLDEN["sm_s"].shape[-1]
    p64 = oracle.causal_softmax64(s, t)
    assert close(p64, GOLDEN["sm_p"].reshape(-1, t), 1e-13)
    p = oracle.softmax_forward(s.astype(np.float16), t)
    assert close(p, GOLDEN["sm_p"].reshape(-1, t), 1e-3)
    ds64 = oracle.causal_softmax_backward64(GOLDEN["sm_p"], GOLDEN["sm_dp"], t, 0.125)
    assert close(ds64, GOLDEN["sm_ds"].reshape(-1, t), 1e-12)
    ds = oracle.softmax_backward(GOLDEN["sm_p"].astype(np.float16), GOLDEN["sm_dp"], t, 0.125)
    ref = oracle.causal_softmax_backward64(GOLDEN["sm_p"].astype(np.float16), GOLDEN["sm_dp"], t,
                                           0.125)
    assert close(ds, ref, 1e-3)


def test_softmax_equal_scores():
    """Equal scores give RN16(1/(t+1)) (ref tests/test_softmax.py:470-497)."""
    t = 48
    p = oracle.softmax_forward(np.full((t, t), 2.0, np.float16), t)
    for i in range(t):
        assert np.all(p[i, : i + 1] == np.float16(np.float32(1) / np.float32(i + 1)))
        assert np.all(p[i, i + 1:] == 0)


# ------------------------------------------------------------------ cross-entropy


def test_cross_entropy_against_golden():
    lg, tg, vocab = GOLDEN["ce_logits"], GOLDEN["ce_targets"], int(GOLDEN["ce_vocab"])
    scale = float(GOLDEN["ce_scale"])
    loss64, d64 = oracle.cross_entropy64(lg, tg, vocab, scale)
    assert close(loss64, GOLDEN["ce_loss"], 1e-12)
    assert close(d64, GOLDEN["ce_dlogits"], 1e-12)
    loss, d = oracle.cross_entropy(lg.astype(np.float16), tg, vocab, scale)
    assert close(loss, GOLDEN["ce_loss"], 1e-5)
    assert close(d, GOLDEN["ce_dlogits"], 1e-3)
    assert np.all(d[:, vocab:] == 0)


def test_cross_entropy_exact_cases():
    """Equal logits: loss log(vocab); vocab 1: loss 0 (ref tests/test_cross_entropy.py:891-933)."""
    lg = np.full((2, 64), 0.5, np.float16)
    loss, _ = oracle.cross_entropy(lg, np.array([3, 9]), 50, 1.0)
    assert np.allclose(loss, np.log(50), rtol=1e-6)
    loss1, d1 = oracle.cross_entropy(lg, np.array([0, 0]), 1, 1.0)
    assert np.all(loss1 == 0) and np.all(d1[:, 0] == 0)
    # A sign slip in the target term would make the target's gradient positive.
    _, d = oracle.cross_entropy(lg, np.array([3, 9]), 50, 1.0)
    assert d[0, 3] < 0 and d[1, 9] < 0 and np.all(d[0, :3] > 0)


# ------------------------------------------------------------------ embedding


def test_embedding_backward_against_golden():
    seqs, length, vocab, width = (int(v) for v in GOLDEN["emb_shape"])
    dwte, dwpe = oracle.embedding_backward(GOLDEN["emb_dx"].astype(np.float32),
                                           GOLDEN["emb_tokens"], seqs, length, vocab, width)
    assert close(dwte, GOLDEN["emb_dwte"], 1e-6)
    assert close(dwpe, GOLDEN["emb_dwpe"], 1e-6)


def test_rel_max_err_metric():
    assert oracle.rel_max_err(np.array([1.0, 2.0]), np.array([1.0, 2.002])) == pytest.approx(
        0.002 / 2.002)


# ---- the shape-only summation orders against the reference's own emulations
#
# tests/golden/reference_orders.npz holds inputs and the outputs of the
# reference's numpy emulations of its kernels' arithmetic (written by
# tests/golden/make_reference_orders.py from the reference checkout). The C
# oracle restates those orders independently; here it must reproduce every
# output bit (values compared as integers, so -0/+0 and NaN payloads count).
# The GPU kernels are checked against the C oracle bit for bit in
# test_reductions.py and test_support.py, which closes the chain.

REF_ORDERS = Path(__file__).resolve().parent / "golden" / "reference_orders.npz"


def _bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    view = np.uint32 if a.dtype == np.float32 else np.uint16
    return np.array_equal(a.view(view), b.view(view))


@pytest.fixture(scope="module")
def ref_orders():
    return dict(np.load(REF_ORDERS))


def test_bias_gradient_order_is_the_references(ref_orders):
    r = ref_orders
    assert _bits_equal(oracle.bias_gradient(r["bias_dy"]), r["bias_out"])
    assert _bits_equal(oracle.bias_gradient(r["bias_dy"], r["bias_old"]), r["bias_out_acc"])
    assert _bits_equal(oracle.bias_gradient(r["bias_dy2"]), r["bias_out2"])


def test_layernorm_backward_order_is_the_references(ref_orders):
    r = ref_orders
    args = (r["ln_dy"], r["ln_x"], r["ln_mean"], r["ln_rstd"], r["ln_gamma"])
    dx, dgamma, dbeta = oracle.layernorm_backward(*args)
    assert _bits_equal(dx, r["ln_dx"])
    assert _bits_equal(dgamma, r["ln_dgamma"])
    # dbeta is the bias gradient of dy.
    assert _bits_equal(dbeta, oracle.bias_gradient(r["ln_dy"]))
    dx_acc, _, _ = oracle.layernorm_backward(*args, dx_old=r["ln_dx_old"])
    assert _bits_equal(dx_acc, r["ln_dx_acc"])


def test_softmax_backward_order_is_the_references(ref_orders):
    r = ref_orders
    t = r["sm_p"].shape[-1]
    ds = oracle.softmax_backward(r["sm_p"], r["sm_dp"], t, 0.125).reshape(r["sm_ds"].shape)
    assert _bits_equal(ds, r["sm_ds"])


def test_embedding_backward_order_is_the_references(ref_orders):
    r = ref_orders
    vocab, width = r["emb_dwte"].shape
    length = r["emb_dwpe"].shape[0]
    seqs = r["emb_dx"].shape[0] // length
    dwte, dwpe = oracle.embedding_backward(r["emb_dx"], r["emb_tokens"], seqs, length, vocab, width)
    assert _bits_equal(dwte, r["emb_dwte"])
    assert _bits_equal(dwpe, r["emb_dwpe"])


def test_a_plain_sum_would_not_match_the_references_order(ref_orders):
    """The fixtures can tell orders apart: plain FP32 column sums of the mixed
    case differ from the reference's compensated chunked sums."""
    r = ref_orders
    plain = r["bias_dy2"].astype(np.float32).sum(axis=0, dtype=np.float32)
    assert not _bits_equal(plain, r["bias_out2"])

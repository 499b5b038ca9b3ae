"""Fused causal attention (include/flint/flint_attention.h) against PyTorch on
the CPU: the forward output and its log-sum-exp, and the three gradients, from
the same FP16 inputs computed in float64 (max|err| / max|ref| within the
north star's 2e-3 for products; 1e-3 relative for the log-sum-exp).

Beside the tolerance, the library's own materialised path (scores and
probabilities stored in FP16, then the causal softmax: what the reference's
model computes, ref src/api/gpt2.cpp:511-514) is run on the same inputs, and the
fused kernels must be at least as close to float64 (they keep scores and
probabilities in FP32 until the products). Runs are deterministic."""

import math

import numpy as np
import pytest
import torch

from inputs import normal, rel_err

pytestmark = pytest.mark.gpu

HD = 64
TOL = 2e-3


def reference(q, k, v, dout, scale):
    """float64 causal attention and its gradients (CPU autograd)."""
    q64, k64, v64 = (t.double().requires_grad_(True) for t in (q, k, v))
    length = q.shape[1]
    s = scale * q64 @ k64.transpose(1, 2)
    mask = torch.triu(torch.ones(length, length, dtype=torch.bool), 1)
    s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    o = torch.softmax(s, dim=-1) @ v64
    o.backward(dout.double())
    return o.detach(), lse.detach(), q64.grad, k64.grad, v64.grad


def run(flint, cuda, q, k, v, dout, scale):
    b, length, _ = q.shape
    dq_, dk_, dv_, do_ = (t.to(cuda) for t in (q, k, v, dout))
    o = torch.full((b, length, HD), float("nan"), dtype=torch.float16, device=cuda)
    lse = torch.full((b, length), float("nan"), device=cuda)
    flint.attention_forward(o, lse, dq_, dk_, dv_, b, length, HD, scale)
    dq = torch.full_like(o, float("nan"))
    dk = torch.full_like(o, float("nan"))
    dv = torch.full_like(o, float("nan"))
    flint.attention_backward(dq, dk, dv, do_, dq_, dk_, dv_, o, lse, b, length, HD, scale)
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu(), dq.cpu(), dk.cpu(), dv.cpu()


def inputs(batches, length, seed):
    q = normal((batches, length, HD), seed, 1.0, torch.float16)
    k = normal((batches, length, HD), seed + 1, 1.0, torch.float16)
    v = normal((batches, length, HD), seed + 2, 1.0, torch.float16)
    dout = normal((batches, length, HD), seed + 3, 1e-2, torch.float16)
    return q, k, v, dout


@pytest.mark.parametrize("batches,length", [(1, 1), (3, 7), (2, 64), (2, 100), (4, 128), (3, 200),
                                            (2, 1024)])
def test_matches_float64(flint, cuda, batches, length):
    q, k, v, dout = inputs(batches, length, 80 + length)
    scale = 1.0 / math.sqrt(HD)
    got = run(flint, cuda, q, k, v, dout, scale)
    ref = reference(q, k, v, dout, scale)
    for name, g, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        assert bool(torch.isfinite(g).all()), name
        tol = 1e-3 if name == "lse" else TOL
        err = rel_err(g, r)
        print(f"{batches}x{length} {name}: {err:.2e}")
        assert err <= tol, (name, err)


@pytest.mark.parametrize("batches,length,scale", [(3, 200, -0.125), (2, 100, -1.0), (2, 64, 0.0)])
def test_any_finite_scale(flint, cuda, batches, length, scale):
    """The forward takes the block max of c s as c max(s) (c min(s) for a
    negative scale): negative and zero scales against float64."""
    q, k, v, dout = inputs(batches, length, 70 + length)
    got = run(flint, cuda, q, k, v, dout, scale)
    ref = reference(q, k, v, dout, scale)
    for name, g, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        assert bool(torch.isfinite(g).all()), name
        err = rel_err(g, r)
        print(f"{batches}x{length} scale {scale} {name}: {err:.2e}")
        assert err <= (1e-3 if name == "lse" else TOL), (name, err)


def test_gpt2_shape_sampled(flint, cuda):
    """96 x 1024 (GPT-2 124M: 8 sequences x 12 heads), the first and last 4
    batches checked against float64."""
    batches, length = 96, 1024
    q, k, v, dout = inputs(batches, length, 90)
    scale = 0.125
    got = run(flint, cuda, q, k, v, dout, scale)
    pick = list(range(4)) + list(range(batches - 4, batches))
    ref = reference(q[pick], k[pick], v[pick], dout[pick], scale)
    for name, g, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        assert bool(torch.isfinite(g).all()), name
        err = rel_err(g[pick], r)
        print(f"96x1024 {name}: {err:.2e}")
        assert err <= (1e-3 if name == "lse" else TOL), (name, err)


def test_no_less_accurate_than_the_materialised_path(flint, cuda):
    """Scores S = RN16(scale q k^T) through the batched GEMM, P by the causal
    softmax, O = RN16(P v): the fused output must be at least as close to
    float64."""
    batches, length = 4, 512
    q, k, v, dout = inputs(batches, length, 95)
    scale = 0.125
    fused = run(flint, cuda, q, k, v, dout, scale)[0]
    s = torch.empty((batches, length, length), dtype=torch.float16, device=cuda)
    p = torch.empty_like(s)
    o = torch.empty((batches, length, HD), dtype=torch.float16, device=cuda)
    flint.gemm_nt_batched(s, q.to(cuda), k.to(cuda), batches, length, length, HD, scale)
    flint.causal_softmax_forward(p, s, batches, length)
    flint.gemm_nn_batched(o, p, v.to(cuda), batches, length, HD, length)
    torch.cuda.synchronize()
    ref = reference(q, k, v, dout, scale)[0]
    e_fused, e_mat = rel_err(fused, ref), rel_err(o.cpu(), ref)
    print(f"fused {e_fused:.2e}, materialised {e_mat:.2e}")
    assert e_fused <= e_mat * 1.05


def test_two_runs_are_bit_identical(flint, cuda):
    q, k, v, dout = inputs(12, 384, 97)
    a = run(flint, cuda, q, k, v, dout, 0.125)
    b = run(flint, cuda, q, k, v, dout, 0.125)
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.float16 else x.view(torch.int32),
                           y.view(torch.int16) if y.dtype == torch.float16 else y.view(torch.int32))


def test_the_first_query_sees_only_the_first_key(flint, cuda):
    """Row 0 of o is v[0] exactly (one visible key, probability 1), and its
    lse is scale q0 . k0."""
    q, k, v, dout = inputs(2, 130, 99)
    got = run(flint, cuda, q, k, v, dout, 0.125)
    assert torch.equal(got[0][:, 0], v[:, 0])
    expect = 0.125 * (q[:, 0].double() * k[:, 0].double()).sum(-1)
    assert torch.allclose(got[1][:, 0].double(), expect, rtol=1e-5, atol=1e-5)

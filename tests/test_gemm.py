"""GEMM family parity on the GPU, through the C ABI, against a PyTorch FP32 CPU
reference (the north star's: max|err| / max|ref| <= 2e-3) and the exact
contracts of the reference's tests (ref tests/test_gemm*.py)."""

import numpy as np
import pytest
import torch

from inputs import normal, rel_err, uniform

pytestmark = pytest.mark.gpu

TOL = 2e-3


def ref_nt(x, w):
    return x.float() @ w.float().T


def ref_nn(x, w):
    return x.float() @ w.float()


def ref_tn(x, w):
    return x.float().T @ w.float()


# Odd shapes (edge tiles, k tails), whole-tile shapes, and GPT-2 shapes.
NT_SHAPES = [(1, 1, 8), (37, 53, 24), (200, 136, 72), (256, 192, 128), (1024, 768, 768),
             (8192, 2304, 768)]
NN_SHAPES = [(1, 8, 8), (37, 56, 24), (200, 136, 72), (256, 192, 128), (8192, 768, 3072)]


@pytest.mark.parametrize("m,n,k", NT_SHAPES)
def test_nt(flint, cuda, m, n, k):
    x = uniform((m, k), 1)
    w = uniform((n, k), 2)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
    flint.gemm_nt(y, x.to(cuda), w.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), ref_nt(x, w)) <= TOL


@pytest.mark.parametrize("m,n,k", [(37, 53, 24), (256, 192, 128), (8192, 2304, 768)])
def test_nt_bias(flint, cuda, m, n, k):
    x = uniform((m, k), 3)
    w = normal((n, k), 4, 0.02, torch.float16)
    b = normal((n,), 5, 0.02)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt_bias(y, x.to(cuda), w.to(cuda), b.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), ref_nt(x, w) + b) <= TOL


@pytest.mark.parametrize("m,n,k", [(37, 53, 24), (256, 192, 128), (8192, 3072, 768)])
def test_nt_bias_gelu(flint, cuda, m, n, k):
    x = uniform((m, k), 6)
    w = normal((n, k), 7, 0.02, torch.float16)
    b = normal((n,), 8, 0.02)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    pre = torch.empty_like(y)
    flint.gemm_nt_bias_gelu(y, pre, x.to(cuda), w.to(cuda), b.to(cuda), m, n, k)
    torch.cuda.synchronize()
    s = ref_nt(x, w) + b
    assert rel_err(pre.cpu(), s) <= TOL
    gelu = torch.nn.functional.gelu(s.double(), approximate="tanh")
    assert rel_err(y.cpu(), gelu) <= TOL
    # pre is bit for bit gemm_nt_bias's output (ref tests/test_gemm_bias_gelu.py:129-138).
    yb = torch.empty_like(y)
    flint.gemm_nt_bias(yb, x.to(cuda), w.to(cuda), b.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(yb.cpu().view(torch.int16), pre.cpu().view(torch.int16))


@pytest.mark.parametrize("m,n,k", [(37, 54, 24), (256, 192, 128), (8192, 768, 768),
                                   (8192, 768, 3072)])
def test_nt_bias_residual(flint, cuda, m, n, k):
    x = uniform((m, k), 9)
    w = normal((n, k), 10, 0.02, torch.float16)
    b = normal((n,), 11, 0.02)
    r = normal((m, n), 12)
    y = torch.empty((m, n), dtype=torch.float32, device=cuda)
    flint.gemm_nt_bias_residual(y, x.to(cuda), w.to(cuda), b.to(cuda), r.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), r + (ref_nt(x, w) + b)) <= TOL
    # A -0 residual reproduces gemm_nt_bias's FP32 sums before rounding: check
    # that y - residual rounds to gemm_nt_bias bit for bit
    # (ref tests/test_gemm_bias_residual.py:330).
    z = torch.full((m, n), -0.0, dtype=torch.float32, device=cuda)
    flint.gemm_nt_bias_residual(y, x.to(cuda), w.to(cuda), b.to(cuda), z, m, n, k)
    yb = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt_bias(yb, x.to(cuda), w.to(cuda), b.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y.half().cpu().view(torch.int16), yb.cpu().view(torch.int16))


@pytest.mark.parametrize("m,n,k", NN_SHAPES)
def test_nn(flint, cuda, m, n, k):
    x = uniform((m, k), 13)
    w = uniform((k, n), 14)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nn(y, x.to(cuda), w.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), ref_nn(x, w)) <= TOL


@pytest.mark.parametrize("m,n,k", [(37, 56, 24), (256, 192, 128), (8192, 3072, 768)])
def test_nn_dgelu(flint, cuda, m, n, k):
    x = normal((m, k), 15, 1e-2, torch.float16)
    w = normal((k, n), 16, 0.02, torch.float16)
    pre = normal((m, n), 17, 1.0, torch.float16)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nn_dgelu(y, x.to(cuda), w.to(cuda), pre.to(cuda), m, n, k)
    torch.cuda.synchronize()
    from oracle.oracle import gelu_grad64

    dg = torch.from_numpy(gelu_grad64(pre.float().numpy()))
    assert rel_err(y.cpu(), ref_nn(x, w).double() * dg) <= TOL


def test_nn_dgelu_limits(flint, cuda):
    """pre = +inf gives gemm_nn, -inf gives 0 (ref tests/test_gemm_dgelu.py:422-465)."""
    m, n, k = 64, 64, 64
    x = uniform((m, k), 18)
    w = uniform((k, n), 19)
    plain = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nn(plain, x.to(cuda), w.to(cuda), m, n, k)
    for value, expect in ((float("inf"), plain), (float("-inf"), torch.zeros_like(plain))):
        pre = torch.full((m, n), value, dtype=torch.float16, device=cuda)
        y = torch.empty_like(plain)
        flint.gemm_nn_dgelu(y, x.to(cuda), w.to(cuda), pre, m, n, k)
        torch.cuda.synchronize()
        assert torch.equal(y.cpu().float(), expect.cpu().float())


TN_SHAPES = [(8, 8, 1), (8, 8, 16384), (136, 120, 3000), (296, 200, 2049), (768, 768, 8192),
             (3072, 768, 8192), (2304, 768, 1024)]


@pytest.mark.parametrize("m,n,k", TN_SHAPES)
@pytest.mark.parametrize("accumulate", [False, True])
def test_tn(flint, cuda, m, n, k, accumulate):
    x = normal((k, m), 20, 1e-2, torch.float16)
    w = uniform((k, n), 21)
    y0 = normal((m, n), 22)
    y = y0.clone().to(cuda)
    flint.gemm_tn(y, x.to(cuda), w.to(cuda), m, n, k, accumulate=accumulate)
    torch.cuda.synchronize()
    ref = ref_tn(x, w) + (y0 if accumulate else 0)
    assert rel_err(y.cpu(), ref) <= TOL
    if accumulate:
        # Accumulating equals y0 + the plain result bit for bit (ref tests/test_gemm_tn.py:304).
        plain = torch.empty((m, n), device=cuda)
        flint.gemm_tn(plain, x.to(cuda), w.to(cuda), m, n, k, accumulate=False)
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), y0 + plain.cpu())


def test_tn_workspace_contract(flint, cuda):
    """Workspace sizes the reference's tests pin (ref tests/test_gemm_tn.py:193-237)."""
    for m, n, k in [(64, 64, 1000), (50304, 768, 65536), (4096, 4096, 65536), (2304, 768, 1024)]:
        assert flint.gemm_tn_workspace(m, n, k) == 0, (m, n, k)
    for m, n, k in [(8, 8, 16384), (136, 120, 3000), (296, 200, 2049), (1032, 8, 4096),
                    (2056, 16, 8192)]:
        b = flint.gemm_tn_workspace(m, n, k)
        assert b > 0 and b % (m * n * 4) == 0 and b // (m * n * 4) <= 16, (m, n, k, b)


def test_integer_exact(flint, cuda):
    """Inputs in {-1, 0, 1} at k = 2^16 sum exactly (ref tests/test_gemm.py:522-534)."""
    m, n, k = 64, 64, 65536
    g = torch.Generator().manual_seed(23)
    x = torch.randint(-1, 2, (m, k), generator=g).half()
    w = torch.randint(-1, 2, (n, k), generator=g).half()
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt(y, x.to(cuda), w.to(cuda), m, n, k)
    torch.cuda.synchronize()
    exact = (x.double() @ w.double().T).half()
    assert torch.equal(y.cpu(), exact)
    xt = x.T.contiguous()
    yt = torch.empty((m, n), device=cuda)
    flint.gemm_tn(yt, xt.to(cuda), w.T.contiguous().to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(yt.cpu(), (x.double() @ w.double().T).float())


@pytest.mark.parametrize("batches,m,n,k", [(3, 40, 56, 24), (96, 1024, 1024, 64)])
def test_nt_batched(flint, cuda, batches, m, n, k):
    x = uniform((batches, m, k), 24)
    w = uniform((batches, n, k), 25)
    y = torch.empty((batches, m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt_batched(y, x.to(cuda), w.to(cuda), batches, m, n, k, 0.125)
    torch.cuda.synchronize()
    ref = torch.bmm(x.float(), w.float().transpose(1, 2).contiguous()) * 0.125
    assert rel_err(y.cpu(), ref) <= TOL
    # Scale 1 equals gemm_nt per batch bit for bit (ref tests/test_gemm_batched.py:390).
    flint.gemm_nt_batched(y, x.to(cuda), w.to(cuda), batches, m, n, k, 1.0)
    one = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt(one, x[-1].contiguous().to(cuda), w[-1].contiguous().to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y[-1].cpu().view(torch.int16), one.cpu().view(torch.int16))


@pytest.mark.parametrize("batches,m,n,k", [(3, 40, 56, 24), (96, 1024, 64, 1024)])
def test_nn_batched(flint, cuda, batches, m, n, k):
    x = uniform((batches, m, k), 26)
    w = uniform((batches, k, n), 27)
    y = torch.empty((batches, m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nn_batched(y, x.to(cuda), w.to(cuda), batches, m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), torch.bmm(x.float(), w.float())) <= TOL


@pytest.mark.parametrize("batches,m,n,k", [(3, 40, 56, 24), (96, 1024, 64, 1024)])
def test_tn_batched(flint, cuda, batches, m, n, k):
    x = uniform((batches, k, m), 28)
    w = uniform((batches, k, n), 29)
    y = torch.empty((batches, m, n), dtype=torch.float16, device=cuda)
    flint.gemm_tn_batched(y, x.to(cuda), w.to(cuda), batches, m, n, k)
    torch.cuda.synchronize()
    ref = torch.bmm(x.float().transpose(1, 2).contiguous(), w.float())
    assert rel_err(y.cpu(), ref) <= TOL


def test_logits_head(flint, cuda):
    """Config 4's NT 8192 x 50304 x 768, with the padding columns of w zero."""
    m, n, k, vocab = 8192, 50304, 768, 50257
    x = uniform((m, k), 30)
    w = normal((n, k), 31, 0.02, torch.float16)
    w[vocab:] = 0
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt(y, x.to(cuda), w.to(cuda), m, n, k)
    torch.cuda.synchronize()
    rows = torch.arange(0, m, 97)
    ref = x[rows].float() @ w.float().T
    assert rel_err(y.cpu()[rows], ref) <= TOL
    assert torch.all(y[:, vocab:] == 0).item()


def test_overflow_gives_inf(flint, cuda):
    """Each output rounds once: sums past FP16's range give inf (ref tests/test_gemm.py:359-389)."""
    m, n, k = 32, 32, 64
    x = torch.full((m, k), 60.0, dtype=torch.float16)
    w = torch.full((n, k), 60.0, dtype=torch.float16)
    w[1] = -60.0
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nt(y, x.to(cuda), w.to(cuda), m, n, k)
    torch.cuda.synchronize()
    yc = y.cpu().float()
    assert torch.all(yc[:, 0] == float("inf")) and torch.all(yc[:, 1] == float("-inf"))


def test_deterministic(flint, cuda):
    m, n, k = 1024, 768, 3072
    x = uniform((m, k), 32).to(cuda)
    w = uniform((n, k), 33).to(cuda)
    a = torch.empty((m, n), dtype=torch.float16, device=cuda)
    b = torch.full((m, n), 7.0, dtype=torch.float16, device=cuda)
    flint.gemm_nt(a, x, w, m, n, k)
    flint.gemm_nt(b, x, w, m, n, k)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


# Every configuration of the one-wave-per-SIMD NT pipeline (gemm_pipe.hip),
# forced through FLINT_GEMM_PIPE, with every epilogue it serves: edge tiles in
# m and n, fewer k-steps than stages, and more tiles than CUs (each workgroup
# then walks several, the next one's loads streaming under this one's stores).
PIPE_CONFIGS = ["256,256,3", "256,192,4", "128,192,4", "256,64,4", "128,64,4", "128,192,3,64",
                "256,128,3,64", "256,256,2,64", "256,192,2,64", "128,192,3,64,4,1",
                "256,128,3,64,4,1", "128,64,3,64", "256,64,3,64"]
PIPE_SHAPES = [(300, 200, 64), (4315, 4600, 96), (1100, 968, 448)]
# The NT layout also has an 8-wave configuration (two waves per SIMD).
NT_PIPE_CONFIGS = PIPE_CONFIGS + ["256,192,2,64,8"]


@pytest.mark.parametrize("cfg", NT_PIPE_CONFIGS)
@pytest.mark.parametrize("m,n,k", PIPE_SHAPES)
@pytest.mark.parametrize("epi", ["none", "bias", "gelu", "residual"])
def test_nt_pipe_forced(flint, cuda, tune, cfg, m, n, k, epi):
    tune("gemm_pipe", cfg)
    x = uniform((m, k), 40)
    w = normal((n, k), 41, 0.05, torch.float16)
    b = normal((n,), 42, 0.02)
    s = ref_nt(x, w)
    xd, wd, bd = x.to(cuda), w.to(cuda), b.to(cuda)
    if epi == "none":
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
        flint.gemm_nt(y, xd, wd, m, n, k)
        torch.cuda.synchronize()
        assert rel_err(y.cpu(), s) <= TOL
    elif epi == "bias":
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
        flint.gemm_nt_bias(y, xd, wd, bd, m, n, k)
        torch.cuda.synchronize()
        assert rel_err(y.cpu(), s + b) <= TOL
    elif epi == "gelu":
        y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
        pre = torch.full_like(y, float("nan"))
        flint.gemm_nt_bias_gelu(y, pre, xd, wd, bd, m, n, k)
        torch.cuda.synchronize()
        assert rel_err(pre.cpu(), s + b) <= TOL
        gelu = torch.nn.functional.gelu((s + b).double(), approximate="tanh")
        assert rel_err(y.cpu(), gelu) <= TOL
    else:
        r = normal((m, n), 43)
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device=cuda)
        flint.gemm_nt_bias_residual(y, xd, wd, bd, r.to(cuda), m, n, k)
        torch.cuda.synchronize()
        assert rel_err(y.cpu(), r + (s + b)) <= TOL


@pytest.mark.parametrize("cfg", NT_PIPE_CONFIGS)
def test_nt_batched_pipe_forced(flint, cuda, tune, cfg):
    tune("gemm_pipe", cfg)
    batches, m, n, k = 5, 264, 200, 64
    x = uniform((batches, m, k), 44)
    w = uniform((batches, n, k), 45)
    y = torch.full((batches, m, n), float("nan"), dtype=torch.float16, device=cuda)
    flint.gemm_nt_batched(y, x.to(cuda), w.to(cuda), batches, m, n, k, 0.125)
    torch.cuda.synchronize()
    ref = torch.bmm(x.float(), w.float().transpose(1, 2).contiguous()) * 0.125
    assert rel_err(y.cpu(), ref) <= TOL


# The pipeline's k-major operand paths (NN's w, TN's x and w through the
# transposing LDS reads), forced per configuration: edge tiles, a k-range
# shorter than the stages, splits of TN (whose workspace plan is the ABI's).
@pytest.mark.parametrize("cfg", PIPE_CONFIGS)
@pytest.mark.parametrize("m,n,k", [(300, 200, 64), (1100, 1096, 320)])
def test_nn_pipe_forced(flint, cuda, tune, cfg, m, n, k):
    tune("gemm_pipe", cfg)
    x = uniform((m, k), 46)
    w = normal((k, n), 47, 0.05, torch.float16)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
    flint.gemm_nn(y, x.to(cuda), w.to(cuda), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), ref_nn(x, w)) <= TOL
    pre = normal((m, n), 48, 1.0, torch.float16)
    flint.gemm_nn_dgelu(y, x.to(cuda), w.to(cuda), pre.to(cuda), m, n, k)
    torch.cuda.synchronize()
    from oracle.oracle import gelu_grad64

    dg = torch.from_numpy(gelu_grad64(pre.float().numpy()))
    assert rel_err(y.cpu(), ref_nn(x, w).double() * dg) <= TOL


@pytest.mark.parametrize("cfg", PIPE_CONFIGS)
@pytest.mark.parametrize("m,n,k", [(296, 200, 2048), (1032, 264, 4096), (768, 768, 8192)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_tn_pipe_forced(flint, cuda, tune, cfg, m, n, k, accumulate):
    tune("gemm_pipe", cfg)
    x = normal((k, m), 49, 1e-2, torch.float16)
    w = uniform((k, n), 50)
    y0 = normal((m, n), 51)
    y = y0.clone().to(cuda)
    flint.gemm_tn(y, x.to(cuda), w.to(cuda), m, n, k, accumulate=accumulate)
    torch.cuda.synchronize()
    ref = ref_tn(x, w) + (y0 if accumulate else 0)
    assert rel_err(y.cpu(), ref) <= TOL
    if accumulate:
        plain = torch.empty((m, n), device=cuda)
        flint.gemm_tn(plain, x.to(cuda), w.to(cuda), m, n, k, accumulate=False)
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), y0 + plain.cpu())


@pytest.mark.parametrize("cfg", PIPE_CONFIGS)
def test_batched_nn_tn_pipe_forced(flint, cuda, tune, cfg):
    tune("gemm_pipe", cfg)
    batches, m, n, k = 5, 264, 72, 96
    x = uniform((batches, m, k), 52)
    w = uniform((batches, k, n), 53)
    y = torch.full((batches, m, n), float("nan"), dtype=torch.float16, device=cuda)
    flint.gemm_nn_batched(y, x.to(cuda), w.to(cuda), batches, m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), torch.bmm(x.float(), w.float())) <= TOL
    xt = uniform((batches, k, m), 54)
    y2 = torch.full((batches, m, n), float("nan"), dtype=torch.float16, device=cuda)
    flint.gemm_tn_batched(y2, xt.to(cuda), w.to(cuda), batches, m, n, k)
    torch.cuda.synchronize()
    ref = torch.bmm(xt.float().transpose(1, 2).contiguous(), w.float())
    assert rel_err(y2.cpu(), ref) <= TOL


# the logits head's backward GEMMs at their full size. Both take the
# 824 MB dlogits as an operand (NN as x, 8192 x 50304 row-major; TN as x, read
# k-major), the largest buffers on the path; rows / columns are sampled for the
# FP32 CPU reference.
LOGITS_ROWS, LOGITS_VOCAB, LOGITS_WIDTH = 8192, 50304, 768


def _sampled(count, total, seed):
    g = torch.Generator().manual_seed(seed)
    pick = torch.randperm(total, generator=g)[:count].sort().values
    # The first and last rows of the output are always in: the largest offsets.
    return torch.unique(torch.cat([pick, torch.tensor([0, total - 1])]))


def test_logits_dx_nn_8192x768x50304(flint, cuda):
    m, n, k = LOGITS_ROWS, LOGITS_WIDTH, LOGITS_VOCAB
    dlogits = normal((m, k), 40, 1e-2, torch.float16)
    wte = normal((k, n), 41, 0.02, torch.float16)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=cuda)
    flint.gemm_nn(y, dlogits.to(cuda), wte.to(cuda), m, n, k)
    torch.cuda.synchronize()
    rows = _sampled(96, m, 42)
    got = y.cpu()
    assert bool(torch.isfinite(got).all())
    assert rel_err(got[rows], ref_nn(dlogits[rows], wte)) <= TOL


def test_logits_dw_tn_50304x768x8192_accumulates(flint, cuda):
    m, n, k = LOGITS_VOCAB, LOGITS_WIDTH, LOGITS_ROWS
    dlogits = normal((k, m), 43, 1e-2, torch.float16)       # x: k x m, read transposed
    h = uniform((k, n), 44)                                   # w: the final LayerNorm's output
    y0 = normal((m, n), 45)
    y = y0.to(cuda)
    flint.gemm_tn(y, dlogits.to(cuda), h.to(cuda), m, n, k, accumulate=True)
    torch.cuda.synchronize()
    rows = _sampled(96, m, 46)
    got = y.cpu()
    assert bool(torch.isfinite(got).all())
    ref = dlogits[:, rows].float().T @ h.float() + y0[rows]
    assert rel_err(got[rows], ref) <= TOL
    # Every column of every sampled row moved off y0 (a skipped tile would not).
    assert bool(((got[rows] - y0[rows]) != 0).float().mean() > 0.999)


# Memory safety of the stores: every output of every entry point is placed 16,
# 32 or 48 bytes into an allocation filled with a 16-bit pattern, with 4 KiB of
# pattern after it; nothing outside the output may change. The shapes leave
# partial tiles on both edges, and each pipeline configuration is forced in
# turn (the edge handling differs between tile sizes).
GUARD = 0x7C5A                      # an FP16 NaN pattern no kernel writes
GUARD_AFTER = 2048                  # halves


def _guarded(count_halves, offset_bytes, cuda):
    """(allocation, view of count_halves halves offset_bytes in)."""
    off = offset_bytes // 2
    buf = torch.full((off + count_halves + GUARD_AFTER,), GUARD - 65536 if GUARD > 32767 else GUARD,
                     dtype=torch.int16, device=cuda)
    return buf, buf[off:off + count_halves], off


def _assert_guards(name, buf, off, count):
    b = buf.cpu()
    pattern = GUARD - 65536 if GUARD > 32767 else GUARD
    assert bool((b[:off] == pattern).all()), f"{name} wrote before its output"
    assert bool((b[off + count:] == pattern).all()), f"{name} wrote past its output"


GUARD_CASES = ["nt", "nt_bias", "nt_bias_gelu", "nt_bias_residual", "nn", "nn_dgelu", "tn", "tn_acc"]


@pytest.mark.parametrize("force", [None, "128,192,3,64", "256,128,3,64", "256,256,3", "256,64,4",
                                   "256,192,2,64,8", "128,192,3,64,4,1"])
@pytest.mark.parametrize("offset", [16, 32, 48])
@pytest.mark.parametrize("case", GUARD_CASES)
def test_outputs_stay_inside_their_buffers(flint, cuda, tune, case, offset, force):
    if force is not None:
        tune("gemm_pipe", force)
    m, n, k = (264, 200, 96) if not case.startswith("tn") else (264, 200, 1000)
    x = uniform((m, k) if not case.startswith("tn") else (k, m), 50).to(cuda)
    w_shape = (n, k) if case.startswith("nt") else (k, n)
    w = uniform(w_shape, 51, -0.1, 0.1).to(cuda)
    b = normal((n,), 52, 0.02).to(cuda)
    f32_out = case in ("nt_bias_residual", "tn", "tn_acc")
    halves = m * n * (2 if f32_out else 1)
    ybuf, yh, yoff = _guarded(halves, offset, cuda)
    y = yh.view(torch.float32 if f32_out else torch.float16).view(m, n)
    if case == "tn_acc":
        y.copy_(normal((m, n), 53).to(cuda))
    pbuf, ph, poff = _guarded(m * n, offset, cuda)
    pre = ph.view(torch.float16).view(m, n)
    if case == "nn_dgelu":
        pre.copy_(normal((m, n), 54, 1.0, torch.float16).to(cuda))
    if case == "nt":
        flint.gemm_nt(y, x, w, m, n, k)
        ref = ref_nt(x.cpu(), w.cpu())
    elif case == "nt_bias":
        flint.gemm_nt_bias(y, x, w, b, m, n, k)
        ref = ref_nt(x.cpu(), w.cpu()) + b.cpu()
    elif case == "nt_bias_gelu":
        flint.gemm_nt_bias_gelu(y, pre, x, w, b, m, n, k)
        s = ref_nt(x.cpu(), w.cpu()) + b.cpu()
        ref = torch.nn.functional.gelu(s.double(), approximate="tanh")
    elif case == "nt_bias_residual":
        r = normal((m, n), 55).to(cuda)
        flint.gemm_nt_bias_residual(y, x, w, b, r, m, n, k)
        ref = r.cpu() + (ref_nt(x.cpu(), w.cpu()) + b.cpu())
    elif case == "nn":
        flint.gemm_nn(y, x, w, m, n, k)
        ref = ref_nn(x.cpu(), w.cpu())
    elif case == "nn_dgelu":
        flint.gemm_nn_dgelu(y, x, w, pre, m, n, k)
        p = pre.cpu().double()
        t = torch.tanh(0.7978845608028654 * (p + 0.044715 * p ** 3))
        gp = 0.5 * (1 + t) + 0.5 * p * (1 - t * t) * 0.7978845608028654 * (1 + 3 * 0.044715 * p * p)
        ref = ref_nn(x.cpu(), w.cpu()).double() * gp
    else:
        y0 = y.cpu().clone()
        flint.gemm_tn(y, x, w, m, n, k, accumulate=case == "tn_acc")
        ref = ref_tn(x.cpu(), w.cpu()) + (y0 if case == "tn_acc" else 0)
    torch.cuda.synchronize()
    _assert_guards(case, ybuf, yoff, halves)
    if case in ("nt_bias_gelu", "nn_dgelu"):
        _assert_guards(case + " pre", pbuf, poff, m * n)
    assert rel_err(y.cpu(), ref) <= TOL


@pytest.mark.parametrize("case", ["nt", "nn", "tn"])
@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "default-stream"])
def test_gemm_is_ordered_on_the_given_stream(flint, cuda, case, side):
    """A GEMM queued behind a long kernel and an input fill on the same stream
    sees the filled input: the product then equals k exactly."""
    m = n = k = 64
    x = torch.zeros((m, k), dtype=torch.float16, device=cuda)
    w = torch.ones((n, k), dtype=torch.float16, device=cuda)
    y = torch.zeros((m, n), dtype=torch.float32 if case == "tn" else torch.float16, device=cuda)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream() if side else torch.cuda.current_stream()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(50_000_000)
        x.fill_(1)
        if case == "nt":
            flint.gemm_nt(y, x, w, m, n, k, stream=stream)
        elif case == "nn":
            flint.gemm_nn(y, x, w, m, n, k, stream=stream)
        else:
            flint.gemm_tn(y, x, w, m, n, k, stream=stream)
    stream.synchronize()
    assert bool((y.float() == k).all())


# ---- exact-rounding contracts of the GELU and dGELU epilogues
#
# With sums made exact (a zero x for GELU, so s is the bias; a one-hot w for
# dGELU, so the sum is dh), every output is one FP16 rounding of a known real
# number. Within one FP16 ulp of the correctly rounded value everywhere, and
# equal to it wherever the exact value lies farther from a rounding boundary
# than the FP32 evaluation's error can move it. With t = s (c0 + c1 s^2) the
# exponential's argument in log2 units, an FP32 error of about 2^-22 |t| ln 2
# relative in exp2(t) reaches the result where the exponential dominates
# (t > 0, i.e. s < 0); where it is small against 1 (s > 0) it does not. So
# 2^-21 (2 + max(t, 0) ln 2), plus a few FP32 ulps, is taken as the bound.

def _ordered(h):
    """FP16 values to integers in value order, +0 and -0 both 0 (ulp distance)."""
    u = np.asarray(h, dtype=np.float16).view(np.uint16).astype(np.int64)
    return np.where(u & 0x8000, -(u & 0x7FFF), u)


def _safe(v, rel, absolute=0.0):
    """Whether float64 values v lie farther from the nearest FP16 rounding
    boundary (the midpoint between the FP16 neighbours around v) than an
    error of rel |v| + absolute can move them."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        h = v.astype(np.float16)
        up = np.nextafter(h, np.float16(np.inf)).astype(np.float64)
        dn = np.nextafter(h, np.float16(-np.inf)).astype(np.float64)
        hf = h.astype(np.float64)
        d = np.minimum(np.abs(v - (hf + up) / 2), np.abs(v - (hf + dn) / 2))
        d = np.where(np.isfinite(d), d, np.inf)
        return d > rel * np.abs(v) + absolute


def _exponent_arg(s):
    s = np.asarray(s, dtype=np.float64)
    return s * (-2.3022082 - 0.10294324 * s * s)


def _gelu_sweep():
    rng = np.random.default_rng(7)
    grid = np.linspace(-12.0, 12.0, 32768)
    rand = rng.random(16384) * 24 - 12
    mags = [1e-40, 1e-30, 2.0**-25, 6e-8, 1e-5, 20.0, 30.0, 100.0, 1000.0, 1e4, 65000.0, 65504.0,
            65519.0, 65520.0, 65536.0, 1e5, 1e30, 3.4028234e38]
    ext = [0.0] + [sg * m for m in mags for sg in (1, -1)]
    s = np.concatenate([grid, rand, ext]).astype(np.float32)
    pad = (-len(s)) % 64
    return np.concatenate([s, np.zeros(pad, np.float32)])


def test_gelu_epilogue_is_the_correctly_rounded_gelu(flint, cuda):
    from oracle import oracle

    bias = _gelu_sweep()
    n, m, k = len(bias), 2, 64
    x = torch.zeros((m, k), dtype=torch.float16, device=cuda)
    w = torch.ones((n, k), dtype=torch.float16, device=cuda)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    pre = torch.empty_like(y)
    flint.gemm_nt_bias_gelu(y, pre, x, w, torch.from_numpy(bias).to(cuda), m, n, k)
    torch.cuda.synchronize()
    y, pre = y.cpu().numpy(), pre.cpu().numpy()
    assert np.array_equal(pre[0].view(np.uint16), bias.astype(np.float16).view(np.uint16))
    assert np.array_equal(y[0].view(np.uint16), y[1].view(np.uint16))
    with np.errstate(all="ignore"):
        exact64 = oracle.gelu64(bias.astype(np.float64))
    exact = exact64.astype(np.float16)
    dist = np.abs(_ordered(y[0]) - _ordered(exact))
    assert dist.max() <= 1, (dist.max(), bias[dist.argmax()])
    safe = _safe(exact64, 2.0**-21 * (2 + np.log(2) * np.maximum(_exponent_arg(bias), 0)))
    assert safe.mean() > 0.95
    wrong = safe & (_ordered(y[0]) != _ordered(exact))
    assert not wrong.any(), (int(wrong.sum()), bias[wrong][:3])
    # GELU of the FP32 sum, not of its FP16 rounding: at safe points the two
    # differ often, so the bit-exact match above tells them apart.
    with np.errstate(all="ignore"):
        from_pre = oracle.gelu64(bias.astype(np.float16).astype(np.float64)).astype(np.float16)
    assert (safe & (_ordered(from_pre) != _ordered(exact))).sum() > 1000


def test_dgelu_epilogue_over_every_finite_fp16_pre(flint, cuda):
    from oracle import oracle

    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    s = allbits[np.isfinite(allbits)]
    n = len(s)
    assert n == 63488
    dhs = [1.0, 1000.0, 2.0**-10, -1.0, -3.0, float(np.float16(0.1))]
    m, k = len(dhs), 8
    x = torch.zeros((m, k), dtype=torch.float16)
    x[:, 0] = torch.tensor(dhs, dtype=torch.float16)
    w = torch.zeros((k, n), dtype=torch.float16)
    w[0] = 1
    pre = torch.from_numpy(np.broadcast_to(s, (m, n)).copy())
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nn_dgelu(y, x.to(cuda), w.to(cuda), pre.to(cuda), m, n, k)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    with np.errstate(all="ignore"):
        g = oracle.gelu_grad64(s.astype(np.float64))
    v = np.asarray(dhs)[:, None] * g[None, :]
    with np.errstate(over="ignore"):
        exact = v.astype(np.float16)
    root = -0.7517916243
    near_root = np.abs(s.astype(np.float64) - root) < 0.25
    dist = np.abs(_ordered(y) - _ordered(exact))
    close = np.abs(y.astype(np.float64) - v) <= np.abs(np.asarray(dhs))[:, None] * 1e-7
    bad = (dist > 1) & ~(near_root[None, :] & close)
    assert not bad.any(), int(bad.sum())
    rel = 2.0**-21 * (2 + np.log(2) * np.maximum(_exponent_arg(s), 0))
    absb = np.where(near_root[None, :], np.abs(np.asarray(dhs))[:, None] * 1e-7, 0.0)
    safe = _safe(v, rel[None, :], absb)
    assert safe.mean() > 0.95
    wrong = safe & (_ordered(y) != _ordered(exact))
    assert not wrong.any(), int(wrong.sum())


# ---- Reads stay inside the operands ------------------------------------------
# Each operand below ends at the last byte of a device allocation of its own
# (a fresh segment of whole 2 MiB pieces: torch's caching allocator hands
# such a request its own hipMalloc when nothing cached fits), so a load past
# its end would leave the allocation. Buffer range checks cover the vector
# offset only; these cases are the ones whose tiles run past an operand's
# end: the bias of an edge column tile (read 256 columns a wave into LDS),
# and a k-major operand's last k rows at an edge tile (NN's w, TN's x and w).


def _at_allocation_end(t):
    """A device copy of t whose last byte ends its allocation."""
    nbytes = t.numel() * t.element_size()
    piece = 2 << 20
    total = (nbytes + piece - 1) // piece * piece + piece
    torch.cuda.empty_cache()
    buf = torch.empty(total, dtype=torch.uint8, device="cuda")
    out = buf[total - nbytes:].view(t.dtype).view(t.shape)
    out.copy_(t.to("cuda"))
    return out


@pytest.mark.parametrize("m,n,k", [(512, 3072, 768), (300, 2312, 128), (256, 200, 64)])
def test_bias_ending_at_its_allocation(flint, cuda, m, n, k):
    x = uniform((m, k), 90)
    w = normal((n, k), 91, 0.02, torch.float16)
    b = normal((n,), 92, 0.02)
    bd = _at_allocation_end(b)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    pre = torch.empty_like(y)
    flint.gemm_nt_bias_gelu(y, pre, x.to(cuda), w.to(cuda), bd, m, n, k)
    torch.cuda.synchronize()
    assert rel_err(pre.cpu(), ref_nt(x, w) + b) <= TOL
    flint.gemm_nt_bias(y, x.to(cuda), w.to(cuda), bd, m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), ref_nt(x, w) + b) <= TOL


@pytest.mark.parametrize("m,n,k", [(200, 136, 512), (520, 200, 256)])
def test_k_major_operands_ending_at_their_allocation(flint, cuda, m, n, k):
    # NN: w is k x n (k-major); TN: x is k x m and w is k x n.
    x_nn = uniform((m, k), 93)
    w_nn = uniform((k, n), 94)
    y = torch.empty((m, n), dtype=torch.float16, device=cuda)
    flint.gemm_nn(y, x_nn.to(cuda), _at_allocation_end(w_nn), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(y.cpu(), ref_nn(x_nn, w_nn)) <= TOL
    x_tn = uniform((k, m), 95)
    w_tn = uniform((k, n), 96)
    yt = torch.empty((m, n), dtype=torch.float32, device=cuda)
    flint.gemm_tn(yt, _at_allocation_end(x_tn), _at_allocation_end(w_tn), m, n, k)
    torch.cuda.synchronize()
    assert rel_err(yt.cpu(), ref_tn(x_tn, w_tn)) <= 1e-4

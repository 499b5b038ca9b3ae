"""LayerNorm, bias gradient, causal softmax and softmax + cross-entropy parity on
the GPU through the C ABI. Tolerances are the north star's (1e-3 relative for
LayerNorm, softmax and loss); where the reference fixes a shape-only
summation order, the C oracle restates it and the kernel must match it bit
for bit. Target gathers are bit-exact."""

import numpy as np
import pytest
import torch

from inputs import normal, rel_err, targets, uniform
from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _bits(t):
    return t.cpu().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 3), (33, 768), (8192, 768), (7, 1000),
                                       (64, 4096), (3, 8000)])
def test_layernorm_forward(flint, cuda, rows, cols):
    x = normal((rows, cols), 1)
    x[:, ::97] += 3000.0  # GPT-2-like outlier channels
    gamma = 1 + normal((cols,), 2, 0.1)
    beta = normal((cols,), 3, 0.1)
    y = torch.empty((rows, cols), dtype=torch.float16, device=cuda)
    mean = torch.empty(rows, device=cuda)
    rstd = torch.empty(rows, device=cuda)
    flint.layernorm_forward(y, mean, rstd, x.to(cuda), gamma.to(cuda), beta.to(cuda), rows, cols)
    torch.cuda.synchronize()
    ref_y, ref_mu, ref_rs = oracle.layernorm64(x.numpy(), gamma.numpy(), beta.numpy(), 1e-5)
    assert rel_err(y.cpu(), torch.from_numpy(ref_y)) <= TOL
    assert np.allclose(mean.cpu().numpy(), ref_mu, rtol=1e-6, atol=1e-6)
    assert np.allclose(rstd.cpu().numpy(), ref_rs, rtol=1e-5)
    ey, emu, ers = oracle.layernorm_forward(x.numpy(), gamma.numpy(), beta.numpy(), 1e-5)
    # The compensated sums make the order nearly irrelevant: >= 99.9% equal bits.
    same = (y.cpu().numpy().view(np.int16) == ey.view(np.int16)).mean()
    assert same >= 0.999


def test_layernorm_exact_cases(flint, cuda):
    """Constant rows give y = beta; gamma = 0 gives beta (ref tests/test_layernorm.py:342-411)."""
    rows, cols = 4, 768
    x = torch.full((rows, cols), 3.25)
    gamma = normal((cols,), 4)
    beta = normal((cols,), 5)
    y = torch.empty((rows, cols), dtype=torch.float16, device=cuda)
    mean = torch.empty(rows, device=cuda)
    rstd = torch.empty(rows, device=cuda)
    flint.layernorm_forward(y, mean, rstd, x.to(cuda), gamma.to(cuda), beta.to(cuda), rows, cols)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), beta.half().expand(rows, cols))
    assert torch.all(mean.cpu() == 3.25)


@pytest.mark.parametrize("rows,cols", [(1, 8), (300, 24), (8192, 768), (1000, 3072), (517, 2056)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_bias_gradient(flint, cuda, rows, cols, accumulate):
    dy = normal((rows, cols), 6, 1.0, torch.float16)
    old = normal((cols,), 7)
    out = old.clone().to(cuda)
    flint.bias_gradient(out, dy.to(cuda), rows, cols, accumulate=accumulate)
    torch.cuda.synchronize()
    expect = oracle.bias_gradient(dy.numpy(), old.numpy() if accumulate else None)
    assert np.array_equal(out.cpu().numpy().view(np.int32), expect.view(np.int32))
    ref = dy.double().sum(0) + (old.double() if accumulate else 0)
    assert rel_err(out.cpu(), ref) <= 1e-5


def test_bias_gradient_past_65535_chunks(flint, cuda):
    """More chunks of 256 rows than a grid's y dimension holds (the reference's limits
    cover rows up to 2^31 - 1 chunks): small-integer dy, so every sum is exact."""
    rows, cols = 65536 * 256 + 77, 8
    vals = (np.arange(rows * cols, dtype=np.int64) % 7 - 3).reshape(rows, cols)
    vals[::3] *= -2
    dy = torch.from_numpy(vals.astype(np.float16))
    out = torch.full((cols,), float("nan"), device=cuda)
    flint.bias_gradient(out, dy.to(cuda), rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), vals.sum(0).astype(np.float32))


# 1 to 4 pieces of 8 columns per lane of the dx kernel and past them (1,032 and
# 4,096 columns); a last chunk whose phases 1..7 hold no row (257 rows). Both
# launch plans: partials and dx in one launch then the merge (default), and
# partials then dx with the merge (FLINT_LN_FUSED=0); 4,096 columns take the
# second either way.
@pytest.mark.parametrize("rows,cols", [(3, 8), (300, 24), (257, 512), (8192, 768), (1000, 1024),
                                       (9, 1032), (100, 4096)])
@pytest.mark.parametrize("acc", [False, True])
@pytest.mark.parametrize("fused", ["1", "0"])
def test_layernorm_backward(flint, cuda, tune, rows, cols, acc, fused):
    tune("ln_fused", fused)
    x = normal((rows, cols), 8)
    gamma = 1 + normal((cols,), 9, 0.1)
    beta = normal((cols,), 10, 0.1)
    dy = normal((rows, cols), 11, 1.0, torch.float16)
    y = torch.empty((rows, cols), dtype=torch.float16, device=cuda)
    mean = torch.empty(rows, device=cuda)
    rstd = torch.empty(rows, device=cuda)
    flint.layernorm_forward(y, mean, rstd, x.to(cuda), gamma.to(cuda), beta.to(cuda), rows, cols)
    dx0 = normal((rows, cols), 12)
    dg0 = normal((cols,), 13)
    db0 = normal((cols,), 14)
    dx, dg, db = dx0.clone().to(cuda), dg0.clone().to(cuda), db0.clone().to(cuda)
    flint.layernorm_backward(dx, dg, db, dy.to(cuda), x.to(cuda), mean, rstd, gamma.to(cuda),
                             rows, cols, accumulate_dx=acc, accumulate_params=acc)
    torch.cuda.synchronize()
    mu, rs = mean.cpu().numpy(), rstd.cpu().numpy()
    edx, edg, edb = oracle.layernorm_backward(
        dy.numpy(), x.numpy(), mu, rs, gamma.numpy(),
        dx0.numpy() if acc else None, dg0.numpy() if acc else None, db0.numpy() if acc else None)
    for got, want in ((dx, edx), (dg, edg), (db, edb)):
        assert np.array_equal(got.cpu().numpy().view(np.int32), want.view(np.int32))
    rdx, rdg, rdb = oracle.layernorm_backward64(dy.numpy(), x.numpy(), mu, rs, gamma.numpy())
    if acc:
        rdx, rdg, rdb = rdx + dx0.numpy(), rdg + dg0.numpy(), rdb + db0.numpy()
    for got, want in ((dx, rdx), (dg, rdg), (db, rdb)):
        assert rel_err(got.cpu(), torch.from_numpy(want)) <= TOL


@pytest.mark.parametrize("batches,length", [(1, 8), (3, 40), (4, 1024), (96, 1024)])
def test_causal_softmax_forward(flint, cuda, batches, length):
    s = normal((batches, length, length), 15, 4.0, torch.float16)
    p = torch.full_like(s, float("nan")).to(cuda)
    flint.causal_softmax_forward(p, s.to(cuda), batches, length)
    torch.cuda.synchronize()
    pc = p.cpu()
    # Every batch, 8 at a time (the float64 reference of 96 x 1024 x 1024 at
    # once would hold 800 MB per array).
    same = 0
    for b0 in range(0, batches, 8):
        pick = slice(b0, min(batches, b0 + 8))
        ref = oracle.causal_softmax64(s[pick].numpy(), length).reshape(-1, length, length)
        assert rel_err(pc[pick], torch.from_numpy(ref)) <= TOL, b0
        emu = oracle.softmax_forward(s[pick].numpy(), length).reshape(-1, length, length)
        same += int((pc[pick].numpy().view(np.int16) == emu.view(np.int16)).sum())
    assert same >= 0.999 * batches * length * length
    upper = torch.triu(torch.ones(length, length, dtype=torch.bool), 1)
    assert torch.all(pc[:, upper] == 0) and not torch.any(torch.signbit(pc[:, upper]))


def test_causal_softmax_equal_scores(flint, cuda):
    """Equal scores give RN16(1 / (t + 1)) (ref tests/test_softmax.py:470-497)."""
    length = 64
    s = torch.full((1, length, length), 0.5, dtype=torch.float16)
    p = torch.empty_like(s).to(cuda)
    flint.causal_softmax_forward(p, s.to(cuda), 1, length)
    torch.cuda.synchronize()
    for t in range(length):
        want = torch.tensor(1.0 / (t + 1), dtype=torch.float32).half()
        assert torch.all(p[0, t, : t + 1].cpu() == want), t


@pytest.mark.parametrize("batches,length", [(1, 8), (3, 40), (96, 1024)])
@pytest.mark.parametrize("in_place", [False, True])
def test_causal_softmax_backward(flint, cuda, batches, length, in_place):
    s = normal((batches, length, length), 16, 4.0, torch.float16)
    p = torch.empty_like(s).to(cuda)
    flint.causal_softmax_forward(p, s.to(cuda), batches, length)
    dp = normal((batches, length, length), 17, 1.0, torch.float16)
    dpg = dp.clone().to(cuda)
    ds = dpg if in_place else torch.empty_like(dpg)
    flint.causal_softmax_backward(ds, p, dpg, batches, length, 0.125)
    torch.cuda.synchronize()
    pc, dsc = p.cpu(), ds.cpu()
    same = 0
    for b0 in range(0, batches, 8):     # every batch, 8 at a time
        pick = slice(b0, min(batches, b0 + 8))
        pn = pc[pick].numpy()
        ref = oracle.causal_softmax_backward64(pn, dp[pick].numpy(), length, 0.125)
        assert rel_err(dsc[pick], torch.from_numpy(ref.reshape(-1, length, length))) <= TOL, b0
        emu = oracle.softmax_backward(pn, dp[pick].numpy(), length, 0.125)
        # Values, not bits: where p underflowed to 0 the kernel may store +0 for -0.
        same += int((dsc[pick].numpy().reshape(-1, length) == emu).sum())
    assert same >= 0.999 * batches * length * length


@pytest.mark.parametrize("rows,vocab,cols", [(1, 1, 8), (7, 1001, 1032), (64, 50257, 50304),
                                             (8192, 50257, 50304), (3, 65536, 65536)])
def test_softmax_cross_entropy(flint, cuda, rows, vocab, cols):
    logits = normal((rows, cols), 18, 2.0, torch.float16)
    t32, t16 = targets(rows, vocab, 19)
    dl = torch.full((rows, cols), float("nan"), dtype=torch.float16, device=cuda)
    loss = torch.empty(rows, device=cuda)
    scale = 1024.0 / 8192.0
    flint.softmax_cross_entropy(dl, loss, logits.to(cuda), t16.to(cuda), scale, rows, vocab,
                                cols)
    torch.cuda.synchronize()
    # Every row, in blocks of 512 (the FP64 reference of all 8,192 rows at
    # once would hold 3.3 GB per array).
    got_loss, got_d = loss.cpu(), dl.cpu()
    same = 0
    for r0 in range(0, rows, 512):
        pick = torch.arange(r0, min(rows, r0 + 512))
        ref_loss, ref_d = oracle.cross_entropy64(logits[pick].numpy(), t32[pick].numpy(), vocab,
                                                 scale)
        assert rel_err(got_loss[pick], torch.from_numpy(ref_loss)) <= TOL, r0
        assert rel_err(got_d[pick], torch.from_numpy(ref_d)) <= TOL, r0
        el, ed = oracle.cross_entropy(logits[pick].numpy(), t32[pick].numpy(), vocab, scale)
        same += int((got_d[pick].numpy().view(np.int16) == ed.view(np.int16)).sum())
    assert same >= 0.999 * rows * cols
    pick = torch.arange(rows)
    # Bit-exact target gather: dlogits at the target carries p - 1 (negative)
    # and every other visible value is >= 0.
    d = dl.cpu()[pick].float()
    tcol = t32[pick].long()
    assert torch.all(d[torch.arange(len(pick)), tcol] <= 0)
    if cols > vocab:
        assert torch.all(dl.cpu()[:, vocab:] == 0)


def test_cross_entropy_target_gather_is_exact(flint, cuda):
    """Rows whose every logit but the maximum lies more than 104 below it: in
    FP32 each of their exponentials is exactly 0, so sum = 1, row_loss =
    max - l_t exactly, dlogits = +scale at the maximum, -scale at the target
    and 0 elsewhere. The logits of a row are all distinct, so reading any
    column but the target's gives another loss (ref cross_entropy.cu:145-147,
    :163-166)."""
    rows, vocab, cols = 4096, 50257, 50304
    g = torch.Generator().manual_seed(31)
    tgt = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int32)
    top = (tgt + 1 + torch.randint(0, vocab - 1, (rows,), generator=g, dtype=torch.int32)) % vocab
    col = torch.arange(cols, dtype=torch.float32)
    r = torch.arange(rows, dtype=torch.float32)[:, None]
    # q = (c + 7r) mod 2048 picks one of 2,048 distinct FP16 values: the
    # binade [128, 256) in steps of 1/8, then [256, 512) in steps of 1/4.
    q = torch.remainder(col[None, :] + 7 * r, 2048.0)
    logits = torch.where(q < 1024, -(128.0 + q / 8), -(256.0 + (q - 1024) / 4)).half()
    assert int((logits[0].float().unique()).numel()) == 2048
    logits[torch.arange(rows), top.long()] = 3.0
    dl = torch.empty((rows, cols), dtype=torch.float16, device=cuda)
    loss = torch.empty(rows, device=cuda)
    scale = 0.125
    flint.softmax_cross_entropy(dl, loss, logits.to(cuda), tgt.to(torch.int16).to(cuda), scale, rows,
                                vocab, cols)
    torch.cuda.synchronize()
    lt = logits[torch.arange(rows), tgt.long()].float()
    expect = 3.0 - lt                      # log(1) - (l_t - max), exact in FP32
    assert torch.equal(loss.cpu(), expect)
    d = dl.cpu().float()
    want = torch.zeros(rows, cols)
    want[torch.arange(rows), top.long()] = scale
    want[torch.arange(rows), tgt.long()] = -scale
    assert torch.equal(d, want)


def test_cross_entropy_special_values(flint, cuda):
    """NaN and infinities follow the reference's arithmetic (ref cross_entropy.cu:123-171):
    a NaN or +inf logit makes the row's loss and every visible dlogit NaN, -inf logits add
    exp(-inf) = 0, an all -inf row is NaN, and padding columns never matter."""
    rows, vocab, cols = 6, 1001, 1008
    logits = normal((rows, cols), 21, 2.0, torch.float16)
    logits[0, 5] = float("nan")
    logits[1, 17] = float("inf")
    logits[2, 1::3] = float("-inf")
    logits[3, :vocab] = float("-inf")
    logits[4, vocab:] = float("nan")
    logits[5, vocab - 1] = 30.0
    t32 = torch.tensor([3, 9, 0, 4, 1000, 1000], dtype=torch.int32)
    t16 = t32.to(torch.int16)
    dl = torch.empty((rows, cols), dtype=torch.float16, device=cuda)
    loss = torch.empty(rows, device=cuda)
    flint.softmax_cross_entropy(dl, loss, logits.to(cuda), t16.to(cuda), 0.125, rows, vocab, cols)
    torch.cuda.synchronize()
    el, ed = oracle.cross_entropy(logits.numpy(), t32.numpy(), vocab, 0.125)
    got_l = loss.cpu().numpy()
    got_d = dl.cpu().float().numpy()
    ed = ed.astype(np.float32)
    assert np.array_equal(np.isnan(got_l), np.isnan(el)), (got_l, el)
    assert np.isnan(got_l[[0, 1, 3]]).all() and np.isfinite(got_l[[2, 4, 5]]).all()
    fin = np.isfinite(el)
    assert np.allclose(got_l[fin], el[fin], rtol=1e-5, atol=0)
    assert np.array_equal(np.isnan(got_d), np.isnan(ed))
    assert (got_d[:, vocab:] == 0).all()
    fin = np.isfinite(ed)
    assert np.allclose(got_d[fin], ed[fin], rtol=2e-3, atol=6e-8)


def test_cross_entropy_exact_cases(flint, cuda):
    """Equal logits give loss log(vocab); vocab 1 gives loss 0
    (ref tests/test_cross_entropy.py:891-933)."""
    rows, cols, vocab = 4, 1024, 1000
    logits = torch.full((rows, cols), 1.5, dtype=torch.float16)
    _, t16 = targets(rows, vocab, 20)
    dl = torch.empty((rows, cols), dtype=torch.float16, device=cuda)
    loss = torch.empty(rows, device=cuda)
    flint.softmax_cross_entropy(dl, loss, logits.to(cuda), t16.to(cuda), 1.0, rows, vocab, cols)
    torch.cuda.synchronize()
    assert np.allclose(loss.cpu().numpy(), np.log(vocab), rtol=1e-6)
    flint.softmax_cross_entropy(dl, loss, logits.to(cuda), torch.zeros(rows, dtype=torch.int16,
                                device=cuda), 1.0, rows, 1, cols)
    torch.cuda.synchronize()
    assert torch.all(loss.cpu() == 0)
    assert torch.all(dl.cpu()[:, 0] == 0)

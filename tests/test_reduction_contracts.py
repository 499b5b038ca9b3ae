"""The reductions' edge contracts on the GPU, through the C ABI: non-finite
inputs, poison in the masked columns, every output element written and
nothing around it, stream order, overflow to +-inf, the 1-ulp bound against
the correctly rounded float64 result, and the batch limit. These follow the
reference's contracts (ref tests/test_layernorm.py:429-586,
tests/test_layernorm_backward.py:1156-1286, tests/test_bias_gradient.py:1011-1147,
tests/test_softmax.py:406-818, tests/test_softmax_backward.py:798-1125,
tests/test_cross_entropy.py:731-1368) with this file's own cases.

Correct rounding is judged with numpy: float64 -> float16 rounds once, to
nearest even. FP16 values are compared by ordinal (the integer order of the
finite values, -0 and +0 both 0), so a difference of 1 is one ulp."""

import math

import numpy as np
import pytest
import torch

from inputs import normal
from oracle import oracle

pytestmark = pytest.mark.gpu

NAN16, NNAN16, INF16, NINF16 = 0x7E00, 0xFE00, 0x7C00, 0xFC00
FILLS = (0xFFC0, 0x3C01)          # NaN in FP16 and FP32 halves; 1.000977 (FP16)


def _i16(bits):
    return bits - 65536 if bits > 32767 else bits


def _ordinal(h):
    """Ordinals of FP16 values (numpy float16 array), as int32."""
    b = np.asarray(h, dtype=np.float16).view(np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def _same_bits(a, b, what):
    ba, bb = _bits(a), _bits(b)
    assert torch.equal(ba, bb), f"{what}: {int((ba != bb).sum())} values differ"


def _mask(t):
    return torch.tril(torch.ones(t, t, dtype=torch.bool))


class Guarded:
    """A device buffer `offset` bytes into an allocation filled with a 16-bit
    pattern, with 4 KiB of the pattern after it."""

    def __init__(self, shape, dtype, offset, fill=FILLS[0]):
        self.count = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size() // 2
        self.off = offset // 2
        self.fill = _i16(fill)
        self.buf = torch.full((self.off + self.count + 2048,), self.fill, dtype=torch.int16,
                              device="cuda")
        self.t = self.buf[self.off:self.off + self.count].view(dtype).view(shape)

    def check(self, name):
        b = self.buf.cpu()
        assert bool((b[:self.off] == self.fill).all()), f"{name}: a write before the buffer"
        assert bool((b[self.off + self.count:] == self.fill).all()), f"{name}: a write past it"


def _softmax(flint, s, offset=0, fill=FILLS[0]):
    b, t, _ = s.shape
    p = Guarded((b, t, t), torch.float16, offset, fill)
    flint.causal_softmax_forward(p.t, s, b, t)
    torch.cuda.synchronize()
    p.check("p")
    return p.t


def _softmax64(s):
    """The float64 causal softmax of FP16 scores (device), on the CPU."""
    t = s.shape[-1]
    m = _mask(t).to(s.device)
    x = s.double().masked_fill(~m, -math.inf)
    return torch.softmax(x, dim=-1).masked_fill(~m, 0.0).cpu().numpy()


def _ulps(got, exact):
    """Per-element ulps between FP16 results and the correct rounding of exact."""
    with np.errstate(over="ignore"):    # past FP16's range rounds to +-inf
        ref = np.nan_to_num(exact).astype(np.float16)
    return np.abs(_ordinal(got.detach().cpu().numpy()) - _ordinal(ref)), ref


def _assert_rounded(got, exact, visible, what, min_count=20_000):
    diff, ref = _ulps(got, exact)
    d = diff[visible]
    nonzero = visible & (ref != 0)
    exact_share = (diff[nonzero] == 0).mean() if nonzero.any() else 1.0
    print(f"{what}: worst {d.max()} ulp, {exact_share:.6f} of {int(nonzero.sum())} exact")
    assert d.max() <= 1, f"{what}: {d.max()} ulps from the correct rounding"
    if nonzero.sum() >= min_count:
        assert exact_share >= 0.999, f"{what}: only {exact_share:.6f} correctly rounded"


def _scores(kind, b, t, seed, flint=None):
    g = torch.Generator(device="cuda").manual_seed(seed)
    if kind == "qk":
        q = torch.randn((b, t, 64), generator=g, device="cuda").half()
        k = torch.randn((b, t, 64), generator=g, device="cuda").half()
        s = torch.empty((b, t, t), dtype=torch.float16, device="cuda")
        flint.gemm_nt_batched(s, q, k, b, t, t, 64, 0.125)
        return s
    std = {"normal": 2.0, "wide": 8.0}[kind]
    return (torch.randn((b, t, t), generator=g, device="cuda") * std).half()


# ---- causal softmax forward --------------------------------------------------

SOFTMAX_SHAPES = [(3, 8), (2, 24), (5, 72), (4, 128), (12, 256), (3, 520), (2, 1016), (12, 1024)]


@pytest.mark.parametrize("b,t", SOFTMAX_SHAPES, ids=str)
@pytest.mark.parametrize("kind", ["normal", "wide", "qk"])
def test_softmax_is_within_an_ulp_of_the_correct_rounding(flint, cuda, kind, b, t):
    s = _scores(kind, b, t, 1, flint)
    p = _softmax(flint, s)
    visible = np.broadcast_to(_mask(t).numpy(), (b, t, t))
    _assert_rounded(p, _softmax64(s), visible, f"softmax {kind} {b}x{t}")
    assert bool((_bits(p)[:, ~_mask(t)] == 0).all())


@pytest.mark.parametrize("t", [72, 1016])
def test_softmax_non_finite_scores_spoil_only_their_rows(flint, cuda, t):
    # One batch per kind; every fourth row gets the value at a column that
    # varies with the row. NaN and +inf turn the row's visible outputs NaN;
    # -inf gets +0 and leaves the rest within an ulp of the softmax of the
    # others. Other rows are the clean run's bits; masked columns stay +0.
    base = _scores("normal", 1, t, 2)
    clean = _softmax(flint, base)
    rows = torch.arange(1, t, 4)
    cols = (rows * 7 + 3) % (rows + 1)
    kinds = [NAN16, NNAN16, INF16, NINF16]
    s = base.repeat(len(kinds), 1, 1)
    for i, bits in enumerate(kinds):
        s.view(torch.int16)[i, rows, cols] = _i16(bits)
    p = _softmax(flint, s).cpu()
    hit = torch.zeros(t, dtype=torch.bool)
    hit[rows] = True
    vis = _mask(t)
    for i, bits in enumerate(kinds):
        assert bool((_bits(p[i])[~vis] == 0).all())
        _same_bits(p[i][~hit], clean[0].cpu()[~hit], f"{bits:#x}: the other rows")
        if bits == NINF16:
            assert bool((_bits(p[i])[rows, cols] == 0).all())
            exact = _softmax64(s[i:i + 1])
            visible = np.broadcast_to(vis.numpy(), (1, t, t))
            _assert_rounded(p[i:i + 1], exact, visible, "-inf rows")
        else:
            assert bool(torch.isnan(p[i][rows][vis[rows]]).all()), f"{bits:#x}"


def test_softmax_rows_of_minus_inf(flint, cuda):
    # Rows 2 mod 5 see only -inf: NaN. Rows 3 mod 5 see one finite score,
    # which takes exactly 1.0.
    t = 72
    s = _scores("normal", 1, t, 3)
    clean = _softmax(flint, s).cpu()
    r = torch.arange(t)
    vis = _mask(t).cuda()
    all_inf = ((r % 5 == 2).cuda()[:, None]) & vis
    one = ((r % 5 == 3).cuda()[:, None]) & vis & (torch.arange(t, device="cuda")[None, :]
                                                  != (r // 2).cuda()[:, None])
    s[0][all_inf | one] = -math.inf
    p = _softmax(flint, s)[0].cpu()
    vc = vis.cpu()
    assert bool(torch.isnan(p[r % 5 == 2][vc[r % 5 == 2]]).all())
    rows3 = r[r % 5 == 3]
    expect = torch.zeros(len(rows3), t, dtype=torch.float16)
    expect[torch.arange(len(rows3)), rows3 // 2] = 1.0
    _same_bits(p[rows3], expect, "one finite score")
    other = (r % 5 != 2) & (r % 5 != 3)
    _same_bits(p[other], clean[0][other], "the other rows")


@pytest.mark.parametrize("first,second", [(INF16, NINF16), (NAN16, INF16), (NAN16, NINF16)])
def test_softmax_two_kinds_of_non_finite_give_nan(flint, cuda, first, second):
    t = 1016
    s = _scores("normal", 1, t, 4)
    clean = _softmax(flint, s).cpu()
    rows = torch.arange(3, t, 3)
    s.view(torch.int16)[0, rows, rows // 2] = _i16(first)
    s.view(torch.int16)[0, rows, rows] = _i16(second)
    p = _softmax(flint, s)[0].cpu()
    vis = _mask(t)
    assert bool(torch.isnan(p[rows][vis[rows]]).all())
    keep = torch.ones(t, dtype=torch.bool)
    keep[rows] = False
    _same_bits(p[keep], clean[0][keep], "the other rows")


@pytest.mark.parametrize("poison", ["random", NAN16, NNAN16, INF16, NINF16],
                         ids=["random", "nan", "-nan", "inf", "-inf"])
@pytest.mark.parametrize("b,t", [(2, 8), (3, 24), (2, 72), (2, 1016), (1, 1024)], ids=str)
def test_softmax_ignores_poison_in_the_masked_columns(flint, cuda, poison, b, t):
    s = _scores("normal", b, t, 5)
    vis = _mask(t).cuda()
    if poison == "random":
        g = torch.Generator(device="cuda").manual_seed(6)
        junk = torch.randint(-32768, 32768, s.shape, generator=g, device="cuda",
                             dtype=torch.int32).to(torch.int16).view(torch.float16)
        junk.view(torch.int16)[..., 1::11] = _i16(INF16)
    else:
        junk = torch.full_like(s.view(torch.int16), _i16(poison)).view(torch.float16)
    clean = torch.where(vis, s, torch.zeros_like(s))
    dirty = torch.where(vis, s, junk)
    _same_bits(_softmax(flint, dirty), _softmax(flint, clean), "poison in the masked columns")


@pytest.mark.parametrize("b,t,offset", [(1, 8, 16), (3, 16, 32), (2, 24, 48), (5, 40, 16),
                                        (2, 72, 32), (1, 1016, 48), (2, 1024, 16)])
def test_softmax_writes_every_element_and_nothing_else(flint, cuda, b, t, offset):
    s = _scores("normal", b, t, 7)
    s0 = s.clone()
    a = _softmax(flint, s, offset, FILLS[0])
    c = _softmax(flint, s, 0, FILLS[1])
    assert bool(torch.isfinite(a).all())
    _same_bits(a, c, "runs into two fills")
    _same_bits(s, s0, "s unchanged")


def test_softmax_65535_batches(flint, cuda):
    b, t = 65535, 8
    s = _scores("normal", b, t, 8)
    p = _softmax(flint, s)
    visible = np.broadcast_to(_mask(t).numpy(), (b, t, t))
    _assert_rounded(p, _softmax64(s), visible, "65,535 batches")
    for j in (0, 1, 255, 256, 4096, 32767, 32768, 65534):
        _same_bits(p[j:j + 1], _softmax(flint, s[j:j + 1].contiguous()), f"batch {j}")


def _sleep_then(stream, fill_fn):
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(50_000_000)
        fill_fn()


@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "current-stream"])
def test_softmax_runs_on_the_given_stream(flint, cuda, side):
    b, t = 3, 64
    s = torch.full((b, t, t), math.nan, dtype=torch.float16, device="cuda")
    p = torch.zeros_like(s)
    st = torch.cuda.Stream() if side else torch.cuda.current_stream()
    _sleep_then(st, lambda: s.fill_(0.0))
    with torch.cuda.stream(st):
        flint.causal_softmax_forward(p, s, b, t, stream=st)
    st.synchronize()
    _same_bits(p, _softmax(flint, torch.zeros_like(s)), "behind the fill")


@pytest.mark.parametrize("value", [0.0, 1.0, -3.5, 1000.0, -60000.0, 65504.0, 6e-8])
def test_softmax_equal_scores_give_the_correctly_rounded_reciprocal(flint, cuda, value):
    t = 1024
    p = _softmax(flint, torch.full((2, t, t), value, dtype=torch.float16, device="cuda"))
    n = np.arange(1, t + 1, dtype=np.float64)
    col = (1.0 / n).astype(np.float16)
    expect = np.where(_mask(t).numpy(), col[:, None], np.float16(0)).astype(np.float16)
    got = p.cpu().numpy()
    wrong = (got.view(np.int16) != expect.view(np.int16)[None]).any(-1)
    assert not wrong.any(), f"rows {np.nonzero(wrong.any(0))[0][:10]} differ from 1 / (t + 1)"


# ---- causal softmax backward -------------------------------------------------

def _backward(flint, p, dp, scale, offset=0, fill=FILLS[0], in_place=False):
    b, t, _ = p.shape
    if in_place:
        ds = Guarded((b, t, t), torch.float16, offset, fill)
        ds.t.copy_(dp)
        flint.causal_softmax_backward(ds.t, p, ds.t, b, t, scale)
    else:
        ds = Guarded((b, t, t), torch.float16, offset, fill)
        flint.causal_softmax_backward(ds.t, p, dp, b, t, scale)
    torch.cuda.synchronize()
    ds.check("ds")
    return ds.t


def _backward64(p, dp, scale):
    t = p.shape[-1]
    m = _mask(t).to(p.device)
    pd = p.double().masked_fill(~m, 0.0)
    dpd = dp.double().masked_fill(~m, 0.0)
    d = (pd * dpd).sum(-1, keepdim=True)
    return ((pd * (dpd - d)) * float(np.float32(scale))).masked_fill(~m, 0.0).cpu().numpy()


def _case(flint, b, t, seed, dp_std=1.0):
    p = _softmax(flint, _scores("normal", b, t, seed))
    g = torch.Generator(device="cuda").manual_seed(seed + 100)
    dp = (torch.randn(p.shape, generator=g, device="cuda") * dp_std).half()
    return p, dp


@pytest.mark.parametrize("b,t", SOFTMAX_SHAPES, ids=str)
@pytest.mark.parametrize("scale", [0.125, 1.0, 0.3])
def test_softmax_backward_is_within_an_ulp_of_the_correct_rounding(flint, cuda, b, t, scale):
    p, dp = _case(flint, b, t, 10)
    ds = _backward(flint, p, dp, scale)
    visible = np.broadcast_to(_mask(t).numpy(), (b, t, t))
    _assert_rounded(ds, _backward64(p, dp, scale), visible, f"backward {b}x{t} x{scale}")
    assert bool((_bits(ds)[:, ~_mask(t)] == 0).all())


def test_softmax_backward_signed_zeros_are_ieee(flint, cuda):
    """A zero probability times a negative (dp - D) is -0, as the reference's
    FP32 arithmetic then __float2half_rn gives; a positive one +0. (A
    mixed-precision fma with a +0 addend would turn the -0 into +0.)"""
    t = 16
    p = torch.zeros((1, t, t), dtype=torch.float16, device=cuda)
    dp = torch.zeros_like(p)
    for r in range(t):
        p[0, r, 0] = 1.0           # D = dp[r, 0] = 1 for every row
        dp[0, r, 0] = 1.0
        dp[0, r, 1:r + 1] = torch.where(torch.arange(1, r + 1, device=cuda) % 2 == 0, 3.0, -2.0)
    ds = _backward(flint, p, dp, 0.5).cpu()
    for r in range(t):
        for c in range(1, r + 1):
            want_negative = c % 2 == 1   # dp - D = -3 < 0 on odd columns
            assert float(ds[0, r, c]) == 0.0
            assert bool(torch.signbit(ds[0, r, c])) == want_negative, (r, c)


@pytest.mark.parametrize("target", ["p", "dp"])
@pytest.mark.parametrize("t", [72, 1016])
def test_softmax_backward_non_finite_values_reach_only_their_rows(flint, cuda, target, t):
    # NaN / +inf / -inf in p or dp at one column of every fourth row: NaN
    # and infinity sit where the C restatement of the reference's order and
    # an FP32 evaluation of the formula have them, finite values are within
    # an ulp of the restatement's (the kernel's 64-lane compensated sum is
    # another order of the same sum), the other rows are the clean run's
    # bits, masked columns stay +0.
    scale = 0.3
    p0, dp0 = _case(flint, 1, t, 11)
    clean = _backward(flint, p0, dp0, scale).cpu()
    rows = torch.arange(0, t, 4)
    cols = (rows * 5 + 1) % (rows + 1)
    kinds = [NAN16, INF16, NINF16]
    p, dp = p0.repeat(len(kinds), 1, 1), dp0.repeat(len(kinds), 1, 1)
    victim = p if target == "p" else dp
    for i, bits in enumerate(kinds):
        victim.view(torch.int16)[i, rows, cols] = _i16(bits)
    ds = _backward(flint, p, dp, scale).cpu()
    emu = oracle.softmax_backward(p.cpu().numpy(), dp.cpu().numpy(), t, scale)
    got = ds.numpy().reshape(-1, t)
    assert np.array_equal(np.isnan(got), np.isnan(emu))
    assert np.array_equal(np.isposinf(got), np.isposinf(emu))
    assert np.array_equal(np.isneginf(got), np.isneginf(emu))
    fin = np.isfinite(emu)
    diff = np.abs(_ordinal(got[fin]) - _ordinal(emu[fin].astype(np.float16)))
    assert diff.max() <= 1, "against the C restatement"
    vis = _mask(t)
    hit = torch.zeros(t, dtype=torch.bool)
    hit[rows] = True
    pf = torch.where(vis, p.float().cpu(), torch.zeros(()))
    dpf = torch.where(vis, dp.float().cpu(), torch.zeros(()))
    d = (pf * dpf).sum(-1, keepdim=True)
    ref = ((pf * (dpf - d)) * float(np.float32(scale))).half()

    def classes(x):
        return torch.where(torch.isnan(x), 1, torch.where(torch.isposinf(x), 2,
                                                          torch.where(torch.isneginf(x), 3, 0)))

    wrong = (classes(ds.float()) != classes(ref.float())) & vis
    assert not bool(wrong.any()), f"{int(wrong.sum())} NaN / inf places differ from FP32"
    for i in range(len(kinds)):
        assert bool((_bits(ds[i])[~vis] == 0).all())
        _same_bits(ds[i][~hit], clean[0][~hit], "the other rows")


@pytest.mark.parametrize("y,z,expected", [(-32752.0, -32752.0, 65504.0),
                                          (-32752.0, -32768.0, math.inf),
                                          (32752.0, 32768.0, -math.inf),
                                          (32768.0, 32768.0, -math.inf)])
@pytest.mark.parametrize("t,row,cols", [(8, 2, (0, 1, 2)), (264, 263, (5, 100, 263))])
def test_softmax_backward_past_fp16_is_inf(flint, cuda, y, z, expected, t, row, cols):
    # p = 1 at three visible columns, dp = 0, y, z there: D = y + z exactly
    # and ds at the first column is -(y + z), at scale 1.
    p = torch.zeros((1, t, t), dtype=torch.float16, device="cuda")
    dp = torch.zeros_like(p)
    p[0, row, list(cols)] = 1.0
    dp[0, row, cols[1]], dp[0, row, cols[2]] = y, z
    ds = _backward(flint, p, dp, 1.0)
    assert ds[0, row, cols[0]].item() == expected


@pytest.mark.parametrize("b,t,offset", [(1, 8, 16), (3, 16, 32), (2, 24, 48), (2, 72, 16),
                                        (1, 1016, 32), (2, 1024, 48)])
@pytest.mark.parametrize("in_place", [False, True], ids=["separate", "in-place"])
def test_softmax_backward_writes_every_element_and_nothing_else(flint, cuda, b, t, offset,
                                                                  in_place):
    p, dp = _case(flint, b, t, 12)
    p0, dp0 = p.clone(), dp.clone()
    a = _backward(flint, p, dp, 0.125, offset, FILLS[0], in_place)
    c = _backward(flint, p, dp, 0.125, 0, FILLS[1], False)
    assert bool(torch.isfinite(a).all())
    _same_bits(a, c, "runs into two fills")
    _same_bits(p, p0, "p unchanged")
    _same_bits(dp, dp0, "dp unchanged")


def test_softmax_backward_65535_batches(flint, cuda):
    b, t = 65535, 8
    p, dp = _case(flint, b, t, 13)
    ds = _backward(flint, p, dp, 0.125)
    visible = np.broadcast_to(_mask(t).numpy(), (b, t, t))
    _assert_rounded(ds, _backward64(p, dp, 0.125), visible, "65,535 batches")
    for j in (0, 256, 32768, 65534):
        one = _backward(flint, p[j:j + 1].contiguous(), dp[j:j + 1].contiguous(), 0.125)
        _same_bits(ds[j:j + 1], one, f"batch {j}")


@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "current-stream"])
def test_softmax_backward_runs_on_the_given_stream(flint, cuda, side):
    b, t = 2, 64
    p = torch.full((b, t, t), math.nan, dtype=torch.float16, device="cuda")
    dp = torch.zeros_like(p)
    ds = torch.full_like(p, 5.0)
    st = torch.cuda.Stream() if side else torch.cuda.current_stream()
    _sleep_then(st, lambda: p.fill_(0.25))
    with torch.cuda.stream(st):
        flint.causal_softmax_backward(ds, p, dp, b, t, 1.0, stream=st)
    st.synchronize()
    assert bool((_bits(ds) == 0).all())


# ---- softmax + cross-entropy -------------------------------------------------

def _ce(flint, logits, tgt16, scale, vocab, offset=0, fill=FILLS[0]):
    rows, cols = logits.shape
    d = Guarded((rows, cols), torch.float16, offset, fill)
    loss = Guarded((rows,), torch.float32, offset, fill)
    flint.softmax_cross_entropy(d.t, loss.t, logits, tgt16, scale, rows, vocab, cols)
    torch.cuda.synchronize()
    d.check("dlogits")
    loss.check("row_loss")
    return d.t, loss.t


def _ce64(logits, targets, scale, vocab):
    """(dlogits, row_loss) in float64 on the CPU, from device inputs."""
    x = logits[:, :vocab].double()
    lse = torch.logsumexp(x, dim=-1)
    p = torch.softmax(x, dim=-1)
    onehot = torch.zeros_like(p)
    onehot[torch.arange(len(targets)), targets.long()] = 1.0
    loss = lse - x[torch.arange(len(targets)), targets.long()]
    return ((p - onehot) * float(np.float32(scale))).cpu().numpy(), loss.cpu().numpy()


def _logits(rows, cols, std, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn((rows, cols), generator=g, device="cuda") * std).half()


def _targets(rows, vocab, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    t = torch.randint(0, vocab, (rows,), generator=g, device="cuda", dtype=torch.int32)
    return t, t.to(torch.int16)


@pytest.mark.parametrize("rows,vocab,cols", [(5, 37, 40), (16, 257, 264), (32, 1023, 1024),
                                             (64, 50257, 50304), (128, 50257, 50304)], ids=str)
@pytest.mark.parametrize("std", [2.0, 8.0], ids=["normal", "wide"])
def test_cross_entropy_is_within_an_ulp_of_the_correct_rounding(flint, cuda, rows, vocab, cols,
                                                                 std):
    x = _logits(rows, cols, std, 20)
    t32, t16 = _targets(rows, vocab, 21)
    d, loss = _ce(flint, x, t16, 1.0, vocab)
    ref_d, ref_loss = _ce64(x, t32, 1.0, vocab)
    _assert_rounded(d[:, :vocab], ref_d, np.ones_like(ref_d, dtype=bool),
                    f"dlogits {rows}x{vocab} std {std}")
    assert bool((_bits(d)[:, vocab:] == 0).all())
    rl = np.abs(loss.cpu().numpy() - ref_loss) / np.maximum(np.abs(ref_loss), 1e-30)
    assert rl.max() <= 1e-5


NF_ROWS, NF_VOCAB, NF_COLS = 40, 1001, 1008


@pytest.mark.parametrize("bits", [NAN16, NNAN16, 0x7D00, INF16],
                         ids=["nan", "-nan", "snan", "inf"])
def test_cross_entropy_nan_or_inf_spoils_only_its_row(flint, cuda, bits):
    clean = _logits(NF_ROWS, NF_COLS, 2.0, 22)
    t32, t16 = _targets(NF_ROWS, NF_VOCAB, 23)
    cd, cl = _ce(flint, clean, t16, 0.5, NF_VOCAB)
    rows = torch.arange(1, NF_ROWS, 3, device="cuda")
    dirty = clean.clone()
    dirty.view(torch.int16)[rows, (rows * 97) % NF_VOCAB] = _i16(bits)
    hit = torch.zeros(NF_ROWS, dtype=torch.bool, device="cuda")
    hit[rows] = True
    for scale in (0.5, 0.0, -0.5):
        d, loss = _ce(flint, dirty, t16, scale, NF_VOCAB)
        assert torch.equal(torch.isnan(loss), hit)
        assert torch.equal(torch.isnan(d[:, :NF_VOCAB]).all(-1), hit)
        assert torch.equal(torch.isnan(d[:, :NF_VOCAB]).any(-1), hit)
        assert bool((_bits(d)[:, NF_VOCAB:] == 0).all())
        if scale == 0.5:
            _same_bits(d[~hit], cd[~hit], "the other rows' dlogits")
            _same_bits(loss[~hit], cl[~hit], "the other rows' loss")


def test_cross_entropy_minus_inf_gets_p_0(flint, cuda):
    scale = 0.5
    clean = _logits(NF_ROWS, NF_COLS, 2.0, 24)
    t32, t16 = _targets(NF_ROWS, NF_VOCAB, 25)
    cd, cl = _ce(flint, clean, t16, scale, NF_VOCAB)
    rows = torch.arange(0, NF_ROWS, 2, device="cuda")
    cols = (rows * 31 + 5) % NF_VOCAB
    cols = torch.where(cols == t32[rows].long(), (cols + 1) % NF_VOCAB, cols)
    on_target = rows % 4 == 0          # every other injected row: at its target
    cols = torch.where(on_target, t32[rows].long(), cols)
    dirty = clean.clone()
    dirty[rows, cols] = -math.inf
    d, loss = _ce(flint, dirty, t16, scale, NF_VOCAB)
    keep = torch.ones(NF_ROWS, dtype=torch.bool, device="cuda")
    keep[rows] = False
    _same_bits(d[keep], cd[keep], "the other rows")
    plain, hit = rows[~on_target], rows[on_target]
    assert bool((_bits(d[plain, cols[~on_target]]) == 0).all())
    assert bool((loss[hit] == math.inf).all())
    assert bool((d[hit, cols[on_target]] == -scale).all())
    assert bool(torch.isfinite(d[:, :NF_VOCAB]).all())
    ref_d, _ = _ce64(dirty[plain], t32[plain], scale, NF_VOCAB)
    _assert_rounded(d[plain, :NF_VOCAB], np.nan_to_num(ref_d),
                    np.ones_like(ref_d, dtype=bool), "-inf rows")


@pytest.mark.parametrize("vocab,cols", [(1, 8), (37, 40), (1023, 1024)])
def test_cross_entropy_row_of_only_minus_inf_is_nan(flint, cuda, vocab, cols):
    rows = 10
    clean = _logits(rows, cols, 2.0, 26)
    _, t16 = _targets(rows, vocab, 27)
    cd, cl = _ce(flint, clean, t16, 1.0, vocab)
    dirty = clean.clone()
    dirty[::2, :vocab] = -math.inf
    nan_rows = torch.zeros(rows, dtype=torch.bool, device="cuda")
    nan_rows[::2] = True
    d, loss = _ce(flint, dirty, t16, 1.0, vocab)
    assert torch.equal(torch.isnan(loss), nan_rows)
    assert torch.equal(torch.isnan(d[:, :vocab]).all(-1), nan_rows)
    assert bool((_bits(d)[:, vocab:] == 0).all())
    _same_bits(d[~nan_rows], cd[~nan_rows], "the other rows")
    _same_bits(loss[~nan_rows], cl[~nan_rows], "the other rows' loss")


@pytest.mark.parametrize("first,second", [(INF16, NINF16), (NAN16, INF16), (NAN16, NINF16)])
def test_cross_entropy_two_kinds_of_non_finite_give_nan(flint, cuda, first, second):
    clean = _logits(NF_ROWS, NF_COLS, 2.0, 28)
    _, t16 = _targets(NF_ROWS, NF_VOCAB, 29)
    cd, _ = _ce(flint, clean, t16, 1.0, NF_VOCAB)
    rows = torch.arange(3, NF_ROWS, 3, device="cuda")
    dirty = clean.clone()
    dirty.view(torch.int16)[rows, (rows * 7) % NF_VOCAB] = _i16(first)
    dirty.view(torch.int16)[rows, (rows * 7 + 501) % NF_VOCAB] = _i16(second)
    d, loss = _ce(flint, dirty, t16, 1.0, NF_VOCAB)
    hit = torch.zeros(NF_ROWS, dtype=torch.bool, device="cuda")
    hit[rows] = True
    assert torch.equal(torch.isnan(loss), hit)
    assert torch.equal(torch.isnan(d[:, :NF_VOCAB]).all(-1), hit)
    _same_bits(d[~hit], cd[~hit], "the other rows")


@pytest.mark.parametrize("scale", [1e6, -1e6, 1e5])
@pytest.mark.parametrize("std", [8.0, 0.5], ids=["wide", "narrow"])
def test_cross_entropy_overflow_gives_inf_and_no_nan(flint, cuda, scale, std):
    rows, vocab, cols = 64, 1000, 1000
    x = _logits(rows, cols, std, 30)
    t32, t16 = _targets(rows, vocab, 31)
    scale = float(np.float32(scale))
    d, loss = _ce(flint, x, t16, scale, vocab)
    ref_d, _ = _ce64(x, t32, scale, vocab)
    out = d[:, :vocab].cpu()
    assert not bool(torch.isnan(out).any()) and not bool(torch.isnan(loss).any())
    diff, _ = _ulps(out, ref_d)
    assert diff.max() <= 1
    over = np.abs(ref_d) >= 65520.0 * (1 + 1e-5)
    under = np.abs(ref_d) <= 65520.0 * (1 - 1e-5)
    o = out.numpy()
    assert over.any() and np.isinf(o[over]).all() and (np.sign(o[over]) == np.sign(ref_d[over])).all()
    assert np.isfinite(o[under]).all()


@pytest.mark.parametrize("rows,vocab,cols,offset", [(1, 1, 8, 16), (3, 37, 40, 32),
                                                    (7, 1001, 1032, 48), (9, 50257, 50304, 16)])
def test_cross_entropy_writes_every_element_and_nothing_else(flint, cuda, rows, vocab, cols,
                                                             offset):
    x = _logits(rows, cols, 2.0, 32)
    x0 = x.clone()
    _, t16 = _targets(rows, vocab, 33)
    a = _ce(flint, x, t16, 0.125, vocab, offset, FILLS[0])
    c = _ce(flint, x, t16, 0.125, vocab, 0, FILLS[1])
    for u, v, name in zip(a, c, ("dlogits", "row_loss")):
        assert bool(torch.isfinite(u).all()), name
        _same_bits(u, v, name + ": runs into two fills")
    _same_bits(x, x0, "logits unchanged")


@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "current-stream"])
def test_cross_entropy_runs_on_the_given_stream(flint, cuda, side):
    rows, vocab, cols = 4, 64, 64
    x = torch.full((rows, cols), math.nan, dtype=torch.float16, device="cuda")
    t16 = torch.zeros(rows, dtype=torch.int16, device="cuda")
    d = torch.empty_like(x)
    loss = torch.empty(rows, device="cuda")
    st = torch.cuda.Stream() if side else torch.cuda.current_stream()
    _sleep_then(st, lambda: x.fill_(0.0))
    with torch.cuda.stream(st):
        flint.softmax_cross_entropy(d, loss, x, t16, 1.0, rows, vocab, cols, stream=st)
    st.synchronize()
    assert np.allclose(loss.cpu().numpy(), math.log(vocab), rtol=1e-6)


# ---- LayerNorm forward -------------------------------------------------------

def _layernorm(flint, x, gamma, beta, offset=0, fill=FILLS[0]):
    rows, cols = x.shape
    y = Guarded((rows, cols), torch.float16, offset, fill)
    mean = Guarded((rows,), torch.float32, offset, fill)
    rstd = Guarded((rows,), torch.float32, offset, fill)
    flint.layernorm_forward(y.t, mean.t, rstd.t, x, gamma, beta, rows, cols)
    torch.cuda.synchronize()
    for g, n in ((y, "y"), (mean, "mean"), (rstd, "rstd")):
        g.check(n)
    return y.t, mean.t, rstd.t


def _ln_inputs(rows, cols, seed):
    return (normal((rows, cols), seed).cuda(), (1 + normal((cols,), seed + 1, 0.1)).cuda(),
            normal((cols,), seed + 2, 0.1).cuda())


@pytest.mark.parametrize("cols", [768, 1001])
def test_layernorm_non_finite_input_makes_only_its_row_nan(flint, cuda, cols):
    rows = 21
    x, gamma, beta = _ln_inputs(rows, cols, 40)
    clean = _layernorm(flint, x, gamma, beta)
    bad = {0: [(0, math.inf)], 5: [(cols // 2, -math.inf)], 9: [(1, math.inf), (2, -math.inf)],
           14: [(cols - 1, math.nan)], 20: [(3, math.nan)]}
    xb = x.clone()
    for r, entries in bad.items():
        for c, v in entries:
            xb[r, c] = v
    dirty = _layernorm(flint, xb, gamma, beta)
    hit = torch.zeros(rows, dtype=torch.bool, device="cuda")
    hit[list(bad)] = True
    for name, out, c in zip(("y", "mean", "rstd"), dirty, clean):
        assert bool(torch.isnan(out[hit]).all()), name
        assert bool(torch.isfinite(out[~hit]).all()), name
        _same_bits(out[~hit], c[~hit], name + ": the other rows")


@pytest.mark.parametrize("rows,cols", [(150, 133), (64, 768)])
def test_layernorm_overflow_gives_inf_with_the_right_sign(flint, cuda, rows, cols):
    x, _, beta = _ln_inputs(rows, cols, 41)
    gamma = (30000.0 * normal((cols,), 44)).cuda()
    y, mean, rstd = _layernorm(flint, x, gamma, beta)
    ref, _, _ = oracle.layernorm64(x.cpu().numpy(), gamma.cpu().numpy(), beta.cpu().numpy(), 1e-5)
    yc = y.cpu().numpy().astype(np.float64)
    assert not np.isnan(yc).any()
    over = np.abs(ref) >= 65520.0 * (1 + 1e-4)
    fits = np.abs(ref) <= 65520.0 * (1 - 1e-4)
    assert (over & (ref > 0)).any() and (over & (ref < 0)).any()
    assert (yc[over] == np.where(ref[over] > 0, np.inf, -np.inf)).all()
    assert np.isfinite(yc[fits]).all()


@pytest.mark.parametrize("rows,offset", [(1, 16), (7, 32), (9, 48), (17, 16), (33, 32)])
@pytest.mark.parametrize("cols", [33, 100, 768])
def test_layernorm_writes_every_element_and_nothing_else(flint, cuda, rows, cols, offset):
    x, gamma, beta = _ln_inputs(rows, cols, 42)
    a = _layernorm(flint, x, gamma, beta, offset, FILLS[0])
    c = _layernorm(flint, x, gamma, beta, 0, FILLS[1])
    for u, v, n in zip(a, c, ("y", "mean", "rstd")):
        assert bool(torch.isfinite(u).all()), n
        _same_bits(u, v, n)


@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "current-stream"])
def test_layernorm_runs_on_the_given_stream(flint, cuda, side):
    rows, cols = 16, 64
    x = torch.full((rows, cols), math.nan, device="cuda")
    gamma = torch.ones(cols, device="cuda")
    beta = torch.full((cols,), 0.5, device="cuda")
    y = torch.zeros((rows, cols), dtype=torch.float16, device="cuda")
    mean, rstd = torch.zeros(rows, device="cuda"), torch.zeros(rows, device="cuda")
    st = torch.cuda.Stream() if side else torch.cuda.current_stream()
    _sleep_then(st, lambda: x.fill_(2.5))
    with torch.cuda.stream(st):
        flint.layernorm_forward(y, mean, rstd, x, gamma, beta, rows, cols, stream=st)
    st.synchronize()
    assert bool((y == 0.5).all()) and bool((mean == 2.5).all())


# ---- LayerNorm backward and bias gradient ------------------------------------

NF_BROWS, NF_BCOLS = 300, 264


def _ln_backward(flint, dy, x, mean, rstd, gamma, offset=0, fill=FILLS[0], extra=0):
    rows, cols = x.shape
    dx = Guarded((rows, cols), torch.float32, offset, fill)
    dg = Guarded((cols,), torch.float32, offset, fill)
    db = Guarded((cols,), torch.float32, offset, fill)
    need = flint.layernorm_backward_workspace(rows, cols)
    ws = Guarded((need + extra,), torch.uint8, offset, fill)
    flint.layernorm_backward(dx.t, dg.t, db.t, dy, x, mean, rstd, gamma, rows, cols,
                             workspace=ws.t, workspace_bytes=need)
    torch.cuda.synchronize()
    for g, n in ((dx, "dx"), (dg, "dgamma"), (db, "dbeta")):
        g.check(n)
    wb = ws.buf.cpu()
    assert bool((wb[ws.off + (need + 1) // 2:] == ws.fill).all()), "workspace: past its size"
    assert bool((wb[:ws.off] == ws.fill).all()), "workspace: before it"
    return dx.t, dg.t, db.t


def _ln_backward_case(flint, seed, rows=NF_BROWS, cols=NF_BCOLS):
    x, gamma, beta = _ln_inputs(rows, cols, seed)
    dy = normal((rows, cols), seed + 3, 1.0, torch.float16).cuda()
    y = torch.empty((rows, cols), dtype=torch.float16, device="cuda")
    mean, rstd = torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")
    flint.layernorm_forward(y, mean, rstd, x, gamma, beta, rows, cols)
    return dy, x, mean, rstd, gamma


def _ln_emulation(dy, x, mean, rstd, gamma):
    return oracle.layernorm_backward(dy.cpu().numpy(), x.cpu().numpy(), mean.cpu().numpy(),
                                     rstd.cpu().numpy(), gamma.cpu().numpy())


def _equal_or_both_nan(got, want, what):
    g = got.cpu().numpy()
    assert np.array_equal(np.isnan(g), np.isnan(want)), what
    f = ~np.isnan(want)
    assert np.array_equal(g[f].view(np.int32), want[f].astype(np.float32).view(np.int32)), what


@pytest.mark.parametrize("value", [math.inf, -math.inf, math.nan], ids=["inf", "-inf", "nan"])
@pytest.mark.parametrize("row,col", [(0, 0), (130, 100), (256, 3), (299, 263)], ids=str)
def test_layernorm_backward_non_finite_x(flint, cuda, value, row, col):
    dy, x, mean, rstd, gamma = _ln_backward_case(flint, 50)
    clean = _ln_backward(flint, dy, x, mean, rstd, gamma)
    xb = x.clone()
    xb[row, col] = value
    y = torch.empty(x.shape, dtype=torch.float16, device="cuda")
    mb, rb = torch.empty_like(mean), torch.empty_like(rstd)
    flint.layernorm_forward(y, mb, rb, xb, gamma, torch.zeros_like(gamma), *x.shape)
    dx, dg, db = _ln_backward(flint, dy, xb, mb, rb, gamma)
    assert bool(torch.isnan(dx[row]).all()) and bool(torch.isnan(dg).all())
    keep = torch.arange(x.shape[0], device="cuda") != row
    _same_bits(dx[keep], clean[0][keep], "the other rows of dx")
    _same_bits(db, clean[2], "dbeta")
    for got, want, n in zip((dx, dg, db), _ln_emulation(dy, xb, mb, rb, gamma),
                            ("dx", "dgamma", "dbeta")):
        _equal_or_both_nan(got, want, n + " against the C restatement")


@pytest.mark.parametrize("col", [0, 7, 131, 263])
def test_layernorm_backward_nan_gamma(flint, cuda, col):
    dy, x, mean, rstd, gamma = _ln_backward_case(flint, 51)
    clean = _ln_backward(flint, dy, x, mean, rstd, gamma)
    gb = gamma.clone()
    gb[col] = math.nan
    dx, dg, db = _ln_backward(flint, dy, x, mean, rstd, gb)
    assert bool(torch.isnan(dx).all())
    _same_bits(dg, clean[1], "dgamma")
    _same_bits(db, clean[2], "dbeta")


@pytest.mark.parametrize("offset", [16, 32, 48])
def test_layernorm_backward_writes_nothing_around_outputs_or_workspace(flint, cuda, offset):
    dy, x, mean, rstd, gamma = _ln_backward_case(flint, 52, 513, 264)
    got = _ln_backward(flint, dy, x, mean, rstd, gamma, offset, FILLS[0], extra=4096)
    for g, want, n in zip(got, _ln_emulation(dy, x, mean, rstd, gamma), ("dx", "dgamma", "dbeta")):
        _equal_or_both_nan(g, want, n)


@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "current-stream"])
def test_layernorm_backward_runs_on_the_given_stream(flint, cuda, side):
    rows, cols = 300, 64
    dy = torch.full((rows, cols), math.nan, dtype=torch.float16, device="cuda")
    x = normal((rows, cols), 53).cuda()
    gamma = torch.ones(cols, device="cuda")
    mean, rstd = x.mean(1), torch.rsqrt(x.var(1, unbiased=False) + 1e-5)
    dx, dg, db = (torch.zeros((rows, cols), device="cuda"), torch.zeros(cols, device="cuda"),
                  torch.zeros(cols, device="cuda"))
    ws = torch.empty(flint.layernorm_backward_workspace(rows, cols), dtype=torch.uint8,
                     device="cuda")
    st = torch.cuda.Stream() if side else torch.cuda.current_stream()
    _sleep_then(st, lambda: dy.fill_(1.0))
    with torch.cuda.stream(st):
        flint.layernorm_backward(dx, dg, db, dy, x, mean, rstd, gamma, rows, cols,
                                 workspace=ws, stream=st)
    st.synchronize()
    assert bool((db == rows).all())


def _bias(flint, dy, old=None, offset=0, fill=FILLS[0], extra=0):
    rows, cols = dy.shape
    out = Guarded((cols,), torch.float32, offset, fill)
    if old is not None:
        out.t.copy_(old)
    need = flint.bias_gradient_workspace(rows, cols)
    ws = Guarded((need + extra,), torch.uint8, offset, fill)
    flint.bias_gradient(out.t, dy, rows, cols, accumulate=old is not None, workspace=ws.t,
                        workspace_bytes=need)
    torch.cuda.synchronize()
    out.check("dbias")
    wb = ws.buf.cpu()
    assert bool((wb[ws.off + (need + 1) // 2:] == ws.fill).all()), "workspace: past its size"
    assert bool((wb[:ws.off] == ws.fill).all()), "workspace: before it"
    return out.t


@pytest.mark.parametrize("accumulate", [False, True], ids=["overwrite", "accumulate"])
def test_bias_gradient_non_finite_reaches_only_its_column(flint, cuda, accumulate):
    dy = normal((NF_BROWS, NF_BCOLS), 60, 1.0, torch.float16).cuda()
    old = (100 * normal((NF_BCOLS,), 61)).cuda() if accumulate else None
    clean = _bias(flint, dy, old)
    cases = {3: [(0, INF16)], 40: [(7, NINF16)], 99: [(255, NAN16)],
             130: [(10, INF16), (200, INF16)], 200: [(1, INF16), (299, NINF16)],
             263: [(256, NNAN16), (5, INF16)]}
    expect = {3: math.inf, 40: -math.inf, 99: math.nan, 130: math.inf, 200: math.nan,
              263: math.nan}
    bad = dy.clone()
    for col, entries in cases.items():
        for row, bits in entries:
            bad.view(torch.int16)[row, col] = _i16(bits)
    got = _bias(flint, bad, old)
    for col, want in expect.items():
        v = got[col].item()
        assert (math.isnan(v) if math.isnan(want) else v == want), (col, v)
    keep = torch.ones(NF_BCOLS, dtype=torch.bool, device="cuda")
    keep[list(cases)] = False
    _same_bits(got[keep], clean[keep], "the other columns")
    emu = oracle.bias_gradient(bad.cpu().numpy(), old.cpu().numpy() if accumulate else None)
    _equal_or_both_nan(got, emu, "against the C restatement")


@pytest.mark.parametrize("offset", [16, 32, 48])
def test_bias_gradient_writes_nothing_around_dbias_or_workspace(flint, cuda, offset):
    dy = normal((513, 264), 62, 1.0, torch.float16).cuda()
    got = _bias(flint, dy, None, offset, FILLS[0], extra=4096)
    _equal_or_both_nan(got, oracle.bias_gradient(dy.cpu().numpy()), "dbias")


@pytest.mark.parametrize("side", [True, False], ids=["side-stream", "current-stream"])
def test_bias_gradient_accumulates_on_the_given_stream(flint, cuda, side):
    rows, cols = 1000, 64
    dy = torch.full((rows, cols), math.nan, dtype=torch.float16, device="cuda")
    out = torch.full((cols,), 7.0, device="cuda")
    ws = torch.empty(flint.bias_gradient_workspace(rows, cols), dtype=torch.uint8,
                     device="cuda")
    st = torch.cuda.Stream() if side else torch.cuda.current_stream()
    _sleep_then(st, lambda: dy.fill_(0.5))
    with torch.cuda.stream(st):
        flint.bias_gradient(out, dy, rows, cols, accumulate=True, workspace=ws, stream=st)
    st.synchronize()
    assert bool((out == 7.0 + 0.5 * rows).all())


# ---- GEMM at the ABI's m and n limit -----------------------------------------

def test_gemm_at_the_largest_m_and_n(flint, cuda):
    """m (then n) of 8,388,480, the ABI's limit: small-integer operands, so
    every output is exact; sampled rows and columns checked."""
    big = 8_388_480
    k = 16
    g = torch.Generator(device="cuda").manual_seed(70)
    x = torch.randint(-2, 3, (big, k), generator=g, device="cuda").half()
    w = torch.randint(-2, 3, (8, k), generator=g, device="cuda").half()
    y = torch.empty((big, 8), dtype=torch.float16, device="cuda")
    flint.gemm_nt(y, x, w, big, 8, k)
    torch.cuda.synchronize()
    pick = torch.cat([torch.arange(0, 4096), torch.arange(big - 4096, big),
                      torch.randint(0, big, (4096,), generator=torch.Generator().manual_seed(71))])
    pick = pick.cuda()
    ref = x[pick].float() @ w.float().T
    assert torch.equal(y[pick].float(), ref)
    del x, y
    # n at the limit: w's rows repeat the 8 of the small operand, so column j
    # of y is column j % 8 of w w^T.
    yn = torch.empty((8, big), dtype=torch.float16, device="cuda")
    flint.gemm_nt(yn, w, w.repeat(big // 8, 1), 8, big, k)
    torch.cuda.synchronize()
    ref = (w.float() @ w.float().T)[:, pick % 8]
    assert torch.equal(yn[:, pick].float(), ref)

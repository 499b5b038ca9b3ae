"""The support callees of the GPT-2 step through the C ABI: flint_embedding_forward,
flint_embedding_backward, flint_heads_split / flint_heads_merge, flint_fp32_to_fp16
and flint_copy (ref tests/test_embedding.py, test_embedding_backward.py,
test_heads.py, test_convert.py, test_copy.py for the contracts).

All of it is exact work with one right answer: gathers and moves are compared bit
for bit with PyTorch's indexing, the conversion with numpy's round-to-nearest-even
astype(float16), and the embedding's backward sums with the C oracle's
restatement of the reference's order (ascending rows per token, TwoSum; dwpe as
the bias gradient's column sums), also bit for bit."""

import numpy as np
import pytest
import torch

from inputs import normal, targets, uniform
from oracle import oracle

pytestmark = pytest.mark.gpu


def _i32(t):
    return t.cpu().contiguous().view(torch.int32)


# ----------------------------------------------------------------- embedding


@pytest.mark.parametrize("sequences,length,vocab,width", [
    (8, 1024, 50257, 768), (1, 8, 1, 8), (3, 40, 1000, 24), (2, 64, 65536, 16)])
def test_embedding_forward_matches_pytorch_bitwise(flint, cuda, sequences, length, vocab, width):
    rows = sequences * length
    wte = normal((vocab, width), 1, 0.02)
    wte[::7] *= 3000.0   # outlier rows
    wpe = normal((length + 5, width), 2, 0.01)
    t32, t16 = targets(rows, vocab, 3)
    t32[0], t32[-1] = 0, vocab - 1
    t16 = t32.to(torch.int16)
    x = torch.full((rows + 2, width), float("nan"), device=cuda)
    flint.embedding_forward(x, t16.to(cuda), wte.to(cuda), wpe.to(cuda), sequences, length,
                            vocab, width)
    torch.cuda.synchronize()
    pos = torch.arange(rows) % length
    expect = wte[t32.long()] + wpe[pos]
    assert torch.equal(_i32(x[:rows]), expect.view(torch.int32))
    assert torch.isnan(x[rows:]).all()   # nothing written past x


@pytest.mark.parametrize("sequences,length,vocab,width,kind", [
    (2, 64, 1000, 64, "uniform"), (3, 40, 200, 24, "few"), (1, 2048, 50, 8, "one"),
    (2, 1500, 5000, 16, "zipf"), (4, 256, 65536, 8, "uniform"), (9, 16, 300, 16, "zipf"),
    (300, 8, 100, 8, "uniform"), (3, 4000, 65536, 8, "uniform"), (5, 1700, 3000, 8, "zipf")])
@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("together", ["1", "0"])   # position sums in the token rows' launch, or after
@pytest.mark.parametrize("scan", ["1", "0"])       # token rows by the scan (accumulating), or sorted
def test_embedding_backward_matches_the_oracle_bitwise(flint, cuda, tune, together, scan,
                                                       sequences, length, vocab,
                                                       width, kind, accumulate):
    tune("emb_together", together)
    tune("emb_scan", scan)
    rows = sequences * length
    g = torch.Generator().manual_seed(4)
    if kind == "uniform":
        tok = torch.randint(0, vocab, (rows,), generator=g)
    elif kind == "few":
        tok = torch.randint(0, 3, (rows,), generator=g) * (vocab // 3)
    elif kind == "one":
        tok = torch.full((rows,), vocab - 1)
    else:
        u = torch.rand(rows, generator=g)
        tok = (u.pow(-1.2) - 1).long().clamp(0, vocab - 1)   # Zipf-like: token 0 most often
    dx = normal((rows, width), 5)
    dx[:, ::5] *= 3000.0
    old_wte = normal((vocab, width), 6) if accumulate else None
    old_wpe = normal((length, width), 7) if accumulate else None
    dwte = (old_wte.clone() if accumulate else torch.full((vocab, width), float("nan"))).to(cuda)
    dwpe = (old_wpe.clone() if accumulate else torch.full((length, width), float("nan"))).to(cuda)
    t16 = tok.to(torch.int32).to(torch.int16)
    flint.embedding_backward(dwte, dwpe, dx.to(cuda), t16.to(cuda), sequences, length, vocab,
                             width, accumulate_wte=accumulate, accumulate_wpe=accumulate)
    torch.cuda.synchronize()
    ewte, ewpe = oracle.embedding_backward(
        dx.numpy(), tok.numpy().astype(np.uint16), sequences, length, vocab, width,
        old_wte.numpy() if accumulate else None, old_wpe.numpy() if accumulate else None)
    assert np.array_equal(dwte.cpu().numpy().view(np.int32), ewte.view(np.int32))
    assert np.array_equal(dwpe.cpu().numpy().view(np.int32), ewpe.view(np.int32))
    # And the sums themselves, against FP64.
    ref = torch.zeros(vocab, width, dtype=torch.float64).index_add_(0, tok, dx.double())
    if accumulate:
        ref += old_wte.double()
    assert torch.allclose(dwte.cpu().double(), ref, rtol=1e-6, atol=1e-3)


@pytest.mark.parametrize("sequences,length", [(3, 700), (1, 13), (5, 1637)])
def test_embedding_backward_rows_past_whole_words(flint, cuda, sequences, length):
    """Row counts that are not a multiple of 8 (the sort-free path reads the
    tokens in 16-byte words and the last few one by one, and masks the scan's
    last block at the row count): the oracle's bits."""
    vocab, width = 300, 24
    rows = sequences * length
    g = torch.Generator().manual_seed(12)
    tok = torch.randint(0, vocab, (rows,), generator=g)
    tok[-1] = tok[0]   # a run that ends at the last row
    dx = normal((rows, width), 13)
    old_wte, old_wpe = normal((vocab, width), 14), normal((length, width), 15)
    dwte, dwpe = old_wte.clone().to(cuda), old_wpe.clone().to(cuda)
    flint.embedding_backward(dwte, dwpe, dx.to(cuda), tok.to(torch.int16).to(cuda), sequences,
                             length, vocab, width, accumulate_wte=True, accumulate_wpe=True)
    torch.cuda.synchronize()
    ewte, ewpe = oracle.embedding_backward(dx.numpy(), tok.numpy().astype(np.uint16), sequences,
                                           length, vocab, width, old_wte.numpy(), old_wpe.numpy())
    assert np.array_equal(dwte.cpu().numpy().view(np.int32), ewte.view(np.int32))
    assert np.array_equal(dwpe.cpu().numpy().view(np.int32), ewpe.view(np.int32))


def test_embedding_backward_at_gpt2_shape_against_fp64(flint, cuda):
    """GPT-2's 8 x 1024 tokens over 50,257 x 768 (too large for the scalar oracle):
    every row a token reaches holds its FP64 sum to FP32 rounding, every other row
    +0, and dwpe the FP64 column sums."""
    sequences, length, vocab, width = 8, 1024, 50257, 768
    rows = sequences * length
    tok, t16 = targets(rows, vocab, 8)
    dx = normal((rows, width), 9, 1e-2)
    dwte = torch.full((vocab, width), float("nan"), device=cuda)
    dwpe = torch.full((length, width), float("nan"), device=cuda)
    flint.embedding_backward(dwte, dwpe, dx.to(cuda), t16.to(cuda), sequences, length, vocab,
                             width)
    torch.cuda.synchronize()
    ref = torch.zeros(vocab, width, dtype=torch.float64).index_add_(0, tok.long(), dx.double())
    got = dwte.cpu().double()
    assert torch.allclose(got, ref, rtol=1e-6, atol=1e-9)
    seen = torch.zeros(vocab, dtype=torch.bool)
    seen[tok.long()] = True
    assert (got[~seen] == 0).all()
    pref = dx.double().reshape(sequences, length, width).sum(0)
    assert torch.allclose(dwpe.cpu().double(), pref, rtol=1e-6, atol=1e-9)


# --------------------------------------------------------------------- heads


@pytest.mark.parametrize("batches,length,heads,hw,row_width,first", [
    (8, 1024, 12, 64, 2304, 0), (8, 1024, 12, 64, 2304, 768), (8, 1024, 12, 64, 2304, 1536),
    (2, 24, 3, 8, 40, 8), (1, 8, 1, 16, 16, 0)])
def test_heads_split_and_merge_move_bits(flint, cuda, batches, length, heads, hw, row_width,
                                         first):
    rows = batches * length
    x = uniform((rows, row_width), 10).view(torch.int16)
    x[::3, ::7] = torch.tensor(0x7E01, dtype=torch.int16)   # a NaN payload moves unchanged
    xd = x.to(cuda)
    y = torch.full((batches * heads * length * hw + 8,), -1, dtype=torch.int16, device=cuda)
    flint.heads_split(y, xd, batches, length, heads, hw, row_width, first)
    torch.cuda.synchronize()
    block = x[:, first:first + heads * hw].reshape(batches, length, heads, hw)
    expect = block.permute(0, 2, 1, 3).reshape(-1)
    assert torch.equal(y[:expect.numel()].cpu(), expect)
    assert (y[expect.numel():].cpu() == -1).all()
    # Merge back into a buffer holding other columns: only the block changes.
    z = torch.full((rows, row_width), 0x1234, dtype=torch.int16, device=cuda)
    flint.heads_merge(z, y, batches, length, heads, hw, row_width, first)
    torch.cuda.synchronize()
    want = torch.full((rows, row_width), 0x1234, dtype=torch.int16)
    want[:, first:first + heads * hw] = x[:, first:first + heads * hw]
    assert torch.equal(z.cpu(), want)


# ------------------------------------------------------------------- convert


def test_fp32_to_fp16_edge_values_round_to_nearest_even(flint, cuda):
    f16 = np.float16
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, float("inf"),
            float("-inf"), 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26,
            2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11), 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11,
            -(1 + 2.0 ** -11), 1e-10, -1e-10]
    x = np.array(vals, np.float32)
    bits = np.concatenate([x.view(np.uint32),
                           np.array([0x7F800001, 0x7FC00000, 0xFFFFFFFF, 0x7F802000],
                                    np.uint32)])
    xs = torch.from_numpy(bits.view(np.int32).copy()).view(torch.float32)
    y = torch.empty(len(bits), dtype=torch.float16, device=cuda)
    flint.fp32_to_fp16(y, xs.to(cuda), len(bits))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    with np.errstate(over="ignore"):   # values past FP16's range round to inf
        expect = bits.view(np.float32).astype(f16)
    finite = ~np.isnan(expect)
    assert np.array_equal(got[finite].view(np.uint16), expect[finite].view(np.uint16))
    assert np.isnan(got[~finite]).all()


@pytest.mark.parametrize("count", [1, 3, 4, 5, 8, 1023, 4097, 124_475_904])
def test_fp32_to_fp16_matches_numpy_at_every_count(flint, cuda, count):
    g = torch.Generator().manual_seed(count % 1000)
    x = torch.randn(count, generator=g) * torch.exp2(torch.randint(-30, 18, (count,),
                                                                   generator=g).float())
    y = torch.full((count + 8,), -1, dtype=torch.int16, device=cuda)
    flint.fp32_to_fp16(y, x.to(cuda), count)
    torch.cuda.synchronize()
    with np.errstate(over="ignore"):   # values past FP16's range round to inf
        expect = x.numpy().astype(np.float16).view(np.int16)
    got = y.cpu().numpy()
    assert np.array_equal(got[:count], expect)
    assert (got[count:] == -1).all()


# ---------------------------------------------------------------------- copy


@pytest.mark.parametrize("n,src_off,dst_off", [(1, 0, 0), (15, 1, 3), (16, 0, 0),
                                              (4097, 7, 2), (1 << 24, 0, 0), (12345677, 5, 11)])
def test_copy_is_bitwise(flint, cuda, n, src_off, dst_off):
    src = torch.randint(0, 256, (n + src_off,), dtype=torch.uint8,
                        generator=torch.Generator().manual_seed(n)).to(cuda)
    dst = torch.full((n + dst_off + 64,), 0xAB, dtype=torch.uint8, device=cuda)
    flint.copy(dst.data_ptr() + dst_off, src.data_ptr() + src_off, n)
    torch.cuda.synchronize()
    d = dst.cpu()
    assert torch.equal(d[dst_off:dst_off + n], src.cpu()[src_off:])
    assert (d[:dst_off] == 0xAB).all() and (d[dst_off + n:] == 0xAB).all()

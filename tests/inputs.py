"""Seeded synthetic inputs (CPU torch tensors) shared by the tests and bench.py."""

import torch


def gen(seed):
    return torch.Generator().manual_seed(seed)


def uniform(shape, seed, lo=-1.0, hi=1.0, dtype=torch.float16):
    g = gen(seed)
    return (torch.rand(shape, generator=g, dtype=torch.float32) * (hi - lo) + lo).to(dtype)


def normal(shape, seed, std=1.0, dtype=torch.float32):
    g = gen(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)


def targets(rows, vocab, seed):
    """int32 U[0, vocab) narrowed to the ABI's uint16 (held in an int16 tensor)."""
    g = gen(seed)
    t = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int32)
    assert int(t.max()) < 65536
    return t, t.to(torch.int16)


def rel_err(got, ref):
    got = got.double()
    ref = ref.double()
    denom = ref.abs().max().item()
    diff = (got - ref).abs().max().item()
    return diff / denom if denom > 0 else diff

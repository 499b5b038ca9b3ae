"""flint_bias_gradient_noalloc (include/flint/flint_noalloc.h): the bias
gradient with the library's per-device scratch array in place of a workspace.
On the GPU it must equal flint_bias_gradient bit for bit, call after call, a
larger input followed by a smaller one (the scratch keeps the first call's
partials, which the second must not read). On the CPU: sizes whose partials
exceed the scratch are refused before any device work."""

import pytest
import torch

from flint_amd.flint_lib import FlintError
from inputs import normal


def test_sizes_beyond_the_scratch_are_refused(flint):
    # ceil(rows / 256) * cols * 8 bytes: 8,192 x 16,392 needs 4,196,352 > 4 MiB.
    with pytest.raises(FlintError, match="needs 4196352 bytes of scratch"):
        flint.check(flint.lib.flint_bias_gradient_noalloc(16, 32, 8192, 16392, 0, None))


def test_argument_checks_match_the_workspace_version(flint):
    with pytest.raises(FlintError, match="cols .* must be a multiple of 8"):
        flint.check(flint.lib.flint_bias_gradient_noalloc(16, 32, 8, 12, 0, None))
    with pytest.raises(FlintError, match="dbias is null"):
        flint.check(flint.lib.flint_bias_gradient_noalloc(None, 32, 8, 16, 0, None))


@pytest.mark.gpu
@pytest.mark.parametrize("accumulate", [False, True])
def test_equals_the_workspace_version_call_after_call(flint, cuda, accumulate):
    cases = [(8192, 3072, 60), (1000, 768, 61)]       # the second is smaller
    for rows, cols, seed in cases:
        print(f"noalloc bias gradient {rows}x{cols} accumulate={accumulate}", flush=True)
        dy = normal((rows, cols), seed, 1.0, torch.float16).to(cuda)
        start = normal((cols,), seed + 100).to(cuda)
        want = start.clone()
        got = start.clone()
        flint.bias_gradient(want, dy, rows, cols, accumulate=accumulate)
        flint.bias_gradient_noalloc(got, dy, rows, cols, accumulate=accumulate)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (rows, cols)
    # The largest size the scratch holds: 8,192 rows x 16,384 columns.
    rows, cols = 8192, 16384
    dy = normal((rows, cols), 62, 1.0, torch.float16).to(cuda)
    want = torch.empty(cols, device=cuda)
    got = torch.empty(cols, device=cuda)
    flint.bias_gradient(want, dy, rows, cols)
    flint.bias_gradient_noalloc(got, dy, rows, cols)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))

"""flint_gpt2: the assembled GPT-2 forward and backward passes through the C ABI
(ref tests/test_gpt2.py, tests/test_gpt2_backward.py for the strategy).

The whole-model gate follows the reference's: from identical FP32 master weights,
with the FP32 CPU model (tests/gpt2_model.py) as the reference and an FP16 peer
(the same model rounded to FP16 where the library stores FP16) beside it, the
library's error against the reference must be at most 2x the peer's, by relative
L2 and by max-abs (3x for the weight gradients), with a small absolute floor for
outputs the peer gets almost exactly. It covers logits below vocab, each row's
loss, dlogits and every master weight's gradient. The assembly's own checks follow:
parameter names, order and shapes; mean_loss as the exact FP64 mean of row_loss;
two runs bit-identical; one allocation and separate buffers giving the same bits;
padded vocabulary rows getting zero gradient; accumulate adding one pass to the
old gradients."""

import numpy as np
import pytest
import torch

import gpt2_model as G
from flint_amd.flint_lib import FlintError, Gpt2

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, heads=2, width=64, block_size=64, vocab=1000, padded_vocab=1024)
ODD = dict(layers=1, heads=3, width=96, block_size=48, vocab=997, padded_vocab=1000)


def _rel_l2(a, b):
    return float(torch.linalg.vector_norm((a - b).double()) /
                 max(float(torch.linalg.vector_norm(b.double())), 1e-30))


def _rel_max(a, b):
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-30))


def _gate(name, got, ref, peer, factor, floor):
    """got's error against ref within factor x peer's, by both measures."""
    for measure in (_rel_l2, _rel_max):
        e_got = measure(got, ref)
        e_peer = measure(peer, ref)
        bound = max(factor * e_peer, floor)
        print(f"{name} {measure.__name__}: flint {e_got:.3e} peer {e_peer:.3e} bound {bound:.3e}")
        assert e_got <= bound, f"{name}: {measure.__name__} {e_got:.3e} > {bound:.3e}"


def _make(flint, cfg, sequences, length, separate=False, backward=True, fused=False):
    return Gpt2(flint, cfg["layers"], cfg["heads"], cfg["width"], cfg["block_size"],
                cfg["vocab"], cfg["padded_vocab"], sequences, length, separate, backward, fused)


def _load(model, params):
    for name, address, rows, cols in model.parameters():
        t = params[name]
        assert tuple(t.shape) == (rows, cols), name
        model.write(address, t.contiguous().cuda())
    model.sync_weights()


def _tokens(cfg, sequences, length, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, cfg["vocab"], (sequences, length), generator=g)
    tgt = torch.randint(0, cfg["vocab"], (sequences, length), generator=g)
    return idx, tgt


def _dev16(t):
    return t.to(torch.int32).to(torch.int16).reshape(-1).cuda()


def _run(flint, cfg, sequences, length, params, idx, tgt, scale, separate=False, fused=False):
    """(logits, row_loss, dlogits, grads, mean_loss) from the library, on the CPU."""
    with _make(flint, cfg, sequences, length, separate, fused=fused) as model:
        _load(model, params)
        tok, trg = _dev16(idx), _dev16(tgt)
        model.forward(tok, trg, scale)
        model.backward(tok)
        lg, dl, rl = model.outputs()
        rows = sequences * length
        pv = cfg["padded_vocab"]
        logits = model.read(lg, (rows, pv), torch.float16).float().cpu()
        dlogits = model.read(dl, (rows, pv), torch.float16).float().cpu()
        row_loss = model.read(rl, (rows,), torch.float32).cpu()
        grads = {n: model.read(a, (r, c), torch.float32).cpu()
                 for n, a, r, c in model.gradients()}
        mean = model.mean_loss()
        torch.cuda.synchronize()
    return logits, row_loss, dlogits, grads, mean


def _reference(params, idx, tgt, cfg, scale, fp16, device):
    """G.gradients on `device` (FP32 arithmetic either way), returned on the CPU."""
    if device == "cpu":
        return G.gradients(params, idx, tgt, cfg, scale, fp16=fp16)
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = {n: t.to(device) for n, t in params.items()}
    out = G.gradients(dev, idx.to(device), tgt.to(device), cfg, scale, fp16=fp16)
    return (out[0].cpu(), out[1].cpu(), out[2].cpu(), {n: g.cpu() for n, g in out[3].items()})


def _gate_case(flint, cfg, sequences, length, trained, idx=None, tgt=None, fused=False,
               ref_device="cpu"):
    """The whole-model gate (forward outputs and every gradient) for one
    configuration and batch. ref_device "cuda" computes the FP32 reference and
    the FP16 peer with torch on the GPU (the sizes of configs[4]'s batch)."""
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=5, trained=trained)
    # Start from FP16-representable masters, so the FP16 copies equal them.
    params = {n: t.half().float() for n, t in params.items()}
    if idx is None:
        idx, tgt = _tokens(cfg, sequences, length, 6)
    rows = sequences * length
    scale = 1024.0 / rows
    ref = _reference(params, idx, tgt, cfg, scale, False, ref_device)
    peer = _reference(params, idx, tgt, cfg, scale, True, ref_device)
    logits, row_loss, dlogits, grads, mean = _run(flint, cfg, sequences, length, params, idx,
                                                  tgt, scale, fused=fused)
    v = cfg["vocab"]
    _gate("logits", logits[:, :v], ref[0], peer[0], 2.0, 1e-3)
    _gate("row_loss", row_loss, ref[1], peer[1], 2.0, 1e-4)
    _gate("dlogits", dlogits[:, :v], ref[2], peer[2], 2.0, 1e-3)
    for name, g in grads.items():
        _gate(name, g, ref[3][name], peer[3][name], 3.0, 2e-3)
    # Padded vocabulary: zero logits from zero wte rows, zero dlogits and gradient rows.
    assert (logits[:, v:] == 0).all() and (dlogits[:, v:] == 0).all()
    assert (grads["wte.weight"][v:] == 0).all()
    # Rows of wpe past length get +0.
    assert (grads["wpe.weight"][length:] == 0).all()
    # mean_loss is the FP64 mean of row_loss.
    assert mean == pytest.approx(float(row_loss.double().mean()), rel=1e-15, abs=0)
    assert abs(mean - float(ref[1].double().mean())) <= 1e-3 * abs(float(ref[1].mean()))


@pytest.mark.parametrize("cfg,sequences,length", [(TINY, 2, 64), (TINY, 3, 32), (ODD, 2, 48)],
                         ids=["tiny-2x64", "tiny-3x32", "odd-2x48"])
@pytest.mark.parametrize("trained", [False, True], ids=["init", "trained"])
def test_forward_and_backward_pass_the_gate(flint, cuda, cfg, sequences, length, trained):
    _gate_case(flint, cfg, sequences, length, trained)


# Head width 64: flint_gpt2_create (the reference's stored scores and
# probabilities) and flint_gpt2_create_fused (the fused causal attention of
# flint_attention.h) both pass the gate; the fused path keeps scores and
# probabilities in FP32 longer, so its forward error is no larger.
HEAD64 = dict(layers=2, heads=2, width=128, block_size=128, vocab=1000, padded_vocab=1024)


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "stored"])
@pytest.mark.parametrize("trained", [False, True], ids=["init", "trained"])
def test_head64_passes_the_gate_fused_and_stored(flint, cuda, fused, trained):
    _gate_case(flint, HEAD64, 2, 128, trained, fused=fused)


def test_fused_attention_forward_error_is_no_larger(flint, cuda):
    cfg, sequences, length = HEAD64, 3, 96
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=21, trained=True)
    params = {n: t.half().float() for n, t in params.items()}
    idx, tgt = _tokens(cfg, sequences, length, 22)
    ref = G.gradients(params, idx, tgt, cfg, 1.0)
    errs = {}
    for fused in (True, False):
        out = _run(flint, cfg, sequences, length, params, idx, tgt, 1.0, fused=fused)
        errs[fused] = _rel_l2(out[0][:, :cfg["vocab"]], ref[0])
    print(f"logits rel L2: fused {errs[True]:.3e} stored {errs[False]:.3e}")
    assert errs[True] <= errs[False] * 1.05


# GPT-2 124M itself (configs[4]'s model), at the reference's gate shapes (ref
# tests/test_gpt2.py:686, :712-715; gradients ref tests/test_gpt2_backward.py:651-653).
GPT2 = dict(layers=12, heads=12, width=768, block_size=1024, vocab=50257, padded_vocab=50304)


@pytest.mark.parametrize("sequences,length", [(2, 256), (1, 1024), (8, 64)],
                         ids=["2x256", "1x1024", "8x64"])
@pytest.mark.parametrize("trained", [False, True], ids=["init", "trained"])
def test_gpt2_124m_passes_the_gate(flint, cuda, sequences, length, trained):
    _gate_case(flint, GPT2, sequences, length, trained)


@pytest.mark.parametrize("sequences", [8, 16], ids=["8x1024", "16x1024"])
def test_gpt2_124m_passes_the_gate_at_full_batch(flint, cuda, sequences):
    """configs[4]'s own batch (8 x 1024) and the reference's micro-batch
    (16 x 1024, ref tests/test_gpt2.py:744-755): every output and gradient
    through the gate, with the FP32 reference and the FP16 peer computed by
    torch on the GPU (FP32 matmuls, no TF32)."""
    _gate_case(flint, GPT2, sequences, 1024, trained=sequences == 16, ref_device="cuda")


def test_gpt2_124m_full_batch_is_deterministic(flint, cuda):
    """configs[4]'s batch run twice: every output, gradient and the mean loss
    equal bit for bit, every gradient finite and somewhere nonzero."""
    cfg, sequences, length = GPT2, 8, 1024
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=15, trained=False)
    params = {n: t.half().float() for n, t in params.items()}
    idx, tgt = _tokens(cfg, sequences, length, 16)
    scale = 1024.0 / (sequences * length)
    a = _run(flint, cfg, sequences, length, params, idx, tgt, scale)
    b = _run(flint, cfg, sequences, length, params, idx, tgt, scale)
    for x in a[:3]:
        assert bool(torch.isfinite(x).all())
    for n, g in a[3].items():
        assert bool(torch.isfinite(g).all()), n
        assert bool((g != 0).any()), n
    for x, y in zip(a[:3], b[:3]):
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x.view(torch.int16),
                           y.view(torch.int32) if y.dtype == torch.float32 else y.view(torch.int16))
    for n in a[3]:
        assert torch.equal(a[3][n].view(torch.int32), b[3][n].view(torch.int32)), n
    assert a[4] == b[4]


def test_a_token_file_batch_runs_through_the_model(flint, cuda, tmp_path):
    """FLINTTOK -> DataLoader -> flint_gpt2_forward/backward: the loader's uint16
    rows go to the device as they are (two bytes a token, the ABI's type) and
    the model passes the gate on them."""
    from flint_amd.tokens import DataLoader, write_token_file

    cfg, sequences, length = TINY, 2, 64
    g = torch.Generator().manual_seed(17)
    stream = torch.randint(0, cfg["vocab"], (3 * sequences * length + 1,), generator=g)
    write_token_file(tmp_path / "shard.bin", stream.numpy())
    loader = DataLoader([tmp_path / "shard.bin"], sequences, length)
    loader.next_batch()
    tokens, targets = loader.next_batch()         # the second batch: offset 128
    assert tokens.dtype == np.uint16 and tokens.shape == (sequences, length)
    idx = torch.from_numpy(tokens.astype(np.int64))
    tgt = torch.from_numpy(targets.astype(np.int64))
    assert torch.equal(idx.reshape(-1), stream[128:256]) and torch.equal(tgt.reshape(-1), stream[129:257])
    # The device copy of the loader's own bytes is what _dev16 makes of idx.
    assert torch.equal(torch.from_numpy(tokens.view(np.int16).copy()).reshape(-1).cuda(), _dev16(idx))
    _gate_case(flint, cfg, sequences, length, True, idx, tgt)


def test_parameters_are_named_in_order(flint, cuda):
    cfg = TINY
    with _make(flint, cfg, 2, 64) as model:
        got = [(n, r, c) for n, _, r, c in model.parameters()]
        assert got == G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                         cfg["padded_vocab"])
        assert [(n, r, c) for n, _, r, c in model.gradients()] == got


def test_run_twice_and_separate_buffers_give_the_same_bits(flint, cuda):
    cfg, sequences, length = TINY, 2, 64
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=7, trained=True)
    idx, tgt = _tokens(cfg, sequences, length, 8)
    a = _run(flint, cfg, sequences, length, params, idx, tgt, 0.125)
    b = _run(flint, cfg, sequences, length, params, idx, tgt, 0.125)
    c = _run(flint, cfg, sequences, length, params, idx, tgt, 0.125, separate=True)
    for other in (b, c):
        for x, y in zip(a[:3], other[:3]):
            assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x,
                               y.view(torch.int32) if y.dtype == torch.float32 else y)
        for n in a[3]:
            assert torch.equal(a[3][n].view(torch.int32), other[3][n].view(torch.int32)), n
        assert a[4] == other[4]


@pytest.mark.parametrize("length", [1024, 320])
@pytest.mark.parametrize("force", [None, "128,64,4", "128,192,3,64", "256,128,3,64", "256,256,3"])
def test_causal_attention_products_change_no_bits(flint, cuda, tune, length, force):
    """The attention GEMMs skip the tiles and k-ranges above the diagonal
    (FLINT_ATTN_CAUSAL unset); computing everything (=0) must give the same
    bits in every output and gradient, whichever tiles the pipeline uses."""
    cfg = dict(layers=1, heads=4, width=256, block_size=1024, vocab=1000, padded_vocab=1024)
    sequences = 2
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=11, trained=True)
    params = {n: t.half().float() for n, t in params.items()}
    idx, tgt = _tokens(cfg, sequences, length, 12)
    if force is not None:
        tune("gemm_pipe", force)
    # The stored scores and probabilities (flint_gpt2_create's model).
    tune("attn_causal", "0")
    full = _run(flint, cfg, sequences, length, params, idx, tgt, 0.25)
    tune("attn_causal", None)
    causal = _run(flint, cfg, sequences, length, params, idx, tgt, 0.25)
    for x, y in zip(full[:3], causal[:3]):
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x,
                           y.view(torch.int32) if y.dtype == torch.float32 else y)
    for n in full[3]:
        assert torch.equal(full[3][n].view(torch.int32), causal[3][n].view(torch.int32)), n
    assert full[4] == causal[4]
    assert bool(torch.isfinite(full[1]).all())


@pytest.mark.parametrize("length", [1024, 320, 32])
@pytest.mark.parametrize("causal", ["1", "0"], ids=["causal", "full"])
def test_fused_scores_and_softmax_change_no_bits(flint, cuda, tune, length, causal):
    """The stored-probability model computes P = softmax(scale q kᵀ) and
    dS = softmax_backward(p, dO vᵀ) in one launch each, the scores kept in
    LDS; the two-launch sequence (attn_scores=0: the batched product, then
    the softmax pass) must give the same bits in every output and gradient,
    with the causal products or the full ones."""
    cfg = dict(layers=1, heads=4, width=256, block_size=1024, vocab=1000, padded_vocab=1024)
    sequences = 2
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=13, trained=True)
    params = {n: t.half().float() for n, t in params.items()}
    idx, tgt = _tokens(cfg, sequences, length, 14)
    if causal == "0":
        tune("attn_causal", "0")
    tune("attn_scores", "0")
    two = _run(flint, cfg, sequences, length, params, idx, tgt, 0.25)
    tune("attn_scores", None)
    one = _run(flint, cfg, sequences, length, params, idx, tgt, 0.25)
    for x, y in zip(two[:3], one[:3]):
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x,
                           y.view(torch.int32) if y.dtype == torch.float32 else y)
    for n in two[3]:
        assert torch.equal(two[3][n].view(torch.int32), one[3][n].view(torch.int32)), n
    assert two[4] == one[4]
    assert bool(torch.isfinite(one[1]).all())


@pytest.mark.parametrize("length", [1024, 320, 96, 32])
@pytest.mark.parametrize("causal", ["1", "0"], ids=["causal", "full"])
def test_head_views_change_no_bits(flint, cuda, tune, length, causal):
    """In one allocation the stored-probability model reads q, k, v and dO and
    writes O, dQ, dK and dV as heads views of the token rows, with no split or
    merge copies; separate buffers (q, k, v not back to back) run the copies
    and the [batches][length][64] products. Every output and gradient must be
    the same bits."""
    cfg = dict(layers=2, heads=3, width=192, block_size=1024, vocab=1000, padded_vocab=1024)
    sequences = 2
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=17, trained=True)
    params = {n: t.half().float() for n, t in params.items()}
    idx, tgt = _tokens(cfg, sequences, length, 18)
    if causal == "0":
        tune("attn_causal", "0")
    views = _run(flint, cfg, sequences, length, params, idx, tgt, 0.25)
    copies = _run(flint, cfg, sequences, length, params, idx, tgt, 0.25, separate=True)
    for x, y in zip(copies[:3], views[:3]):
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x,
                           y.view(torch.int32) if y.dtype == torch.float32 else y)
    for n in copies[3]:
        assert torch.equal(copies[3][n].view(torch.int32), views[3][n].view(torch.int32)), n
    assert copies[4] == views[4]
    assert bool(torch.isfinite(views[1]).all())


WIDE = dict(layers=1, heads=4, width=256, block_size=1024, vocab=1000, padded_vocab=1024)


@pytest.mark.parametrize("cfg,sequences,length", [(TINY, 8, 64), (ODD, 2, 48), (WIDE, 2, 520)],
                         ids=["tiny-8x64", "odd-2x48", "wide-2x520"])
def test_fused_column_sums_change_no_bits(flint, cuda, tune, cfg, sequences, length):
    """The model's LayerNorm backward runs its chunk partials and dx rows in
    one launch and leaves the dbeta / dgamma merge to the next linear layer's
    finish (FLINT_FUSED_SUMS and FLINT_LN_DEFER unset); the merge in a launch
    of its own (FLINT_LN_DEFER=0) and flint_layernorm_backward plus a
    conversion (FLINT_FUSED_SUMS=0) must give the same bits."""
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=13, trained=True)
    idx, tgt = _tokens(cfg, sequences, length, 14)
    tune("fused_sums", "0")
    plain = _run(flint, cfg, sequences, length, params, idx, tgt, 0.5)
    tune("fused_sums", None)
    tune("ln_defer", "0")
    in_place = _run(flint, cfg, sequences, length, params, idx, tgt, 0.5)
    tune("ln_defer", None)
    fused = _run(flint, cfg, sequences, length, params, idx, tgt, 0.5)
    for other in (in_place, fused):
        for n in plain[3]:
            assert torch.equal(plain[3][n].view(torch.int32), other[3][n].view(torch.int32)), n
        assert plain[4] == other[4]


@pytest.mark.parametrize("cfg,sequences,length", [(TINY, 8, 64), (ODD, 2, 48), (WIDE, 2, 520)],
                         ids=["tiny-8x64", "odd-2x48", "wide-2x520"])
def test_fused_linear_grads_change_no_bits(flint, cuda, tune, cfg, sequences, length):
    """The model finishes each linear layer's weight and bias gradients in one
    launch (FLINT_FUSED_GRADS unset); flint_gemm_tn and flint_bias_gradient
    called one after the other (=0) must give the same bits, after a fresh
    backward and after a second, accumulating one."""
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=15, trained=True)
    idx, tgt = _tokens(cfg, sequences, length, 16)

    def grads_twice():
        with _make(flint, cfg, sequences, length) as model:
            _load(model, params)
            tok, trg = _dev16(idx), _dev16(tgt)
            model.forward(tok, trg, 0.5)
            model.backward(tok)
            fresh = {n: model.read(a, (r, c), torch.float32).cpu()
                     for n, a, r, c in model.gradients()}
            model.backward(tok, accumulate=True)
            twice = {n: model.read(a, (r, c), torch.float32).cpu()
                     for n, a, r, c in model.gradients()}
            torch.cuda.synchronize()
        return fresh, twice

    tune("fused_grads", "0")
    plain = grads_twice()
    tune("fused_grads", None)
    fused = grads_twice()
    for a, b in zip(plain, fused):
        assert a.keys() == b.keys()
        for n in a:
            assert torch.equal(a[n].view(torch.int32), b[n].view(torch.int32)), n


def test_backward_accumulate_adds_one_pass(flint, cuda):
    """accumulate: every gradient gets this pass's added with one FP32 add, wte
    with two (old + output layer's part) + the embedding's part, so only wte may
    differ from old + fresh in the last bit (ref flint.h:530-545)."""
    cfg, sequences, length = TINY, 2, 32
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=9, trained=True)
    idx, tgt = _tokens(cfg, sequences, length, 10)
    with _make(flint, cfg, sequences, length) as model:
        _load(model, params)
        tok, trg = _dev16(idx), _dev16(tgt)
        model.forward(tok, trg, 0.25)
        model.backward(tok)
        fresh = {n: model.read(a, (r, c), torch.float32) for n, a, r, c in model.gradients()}
        model.backward(tok, accumulate=True)
        twice = {n: model.read(a, (r, c), torch.float32) for n, a, r, c in model.gradients()}
        torch.cuda.synchronize()
    for n in fresh:
        expect = fresh[n] + fresh[n]
        if n == "wte.weight":
            assert torch.allclose(twice[n], expect, rtol=1e-6, atol=1e-12), n
        elif n == "wpe.weight":
            # Rows past length are left as they are (+0 from the first pass).
            assert torch.equal(twice[n][:length], expect[:length]), n
            assert (twice[n][length:] == 0).all()
        else:
            assert torch.equal(twice[n], expect), n


def test_backward_needs_a_backward_model(flint, cuda):
    cfg = TINY
    with _make(flint, cfg, 1, 8, backward=False) as model:
        tok = torch.zeros(8, dtype=torch.int16, device=cuda)
        with pytest.raises(FlintError) as e:
            model.backward(tok)
        assert e.value.status == 1


def test_mean_loss_of_equal_logits_is_log_vocab(flint, cuda):
    """All-zero weights: every logit is 0, so each row's loss is log(vocab) exactly
    as the kernel computes it (ref tests/test_cross_entropy.py:891-933)."""
    cfg, sequences, length = TINY, 1, 16
    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    params = {n: torch.zeros(r, c) for n, r, c in shapes}
    for n in params:
        if n.endswith("ln_1.weight") or n.endswith("ln_2.weight") or n == "ln_f.weight":
            params[n] += 1
    idx, tgt = _tokens(cfg, sequences, length, 11)
    _, row_loss, _, _, mean = _run(flint, cfg, sequences, length, params, idx, tgt, 1.0)
    assert np.allclose(row_loss.numpy(), np.log(cfg["vocab"]), rtol=1e-6)
    assert mean == pytest.approx(np.log(cfg["vocab"]), rel=1e-6)


# ---- The assembly equals the public kernels called one by one --------------
# (ref tests/test_gpt2.py:1114-1123, ref tests/test_gpt2_backward.py:896-950)

# The reference's TINY model (ref scripts/gpt2_torch.py:34): heads of width 64.
REF_TINY = dict(layers=2, heads=2, width=128, block_size=64, vocab=50257, padded_vocab=50304)


def _model_passes(flint, cfg, sequences, length, params, tok, trg, scale, fused, old=None):
    """flint_gpt2_forward + flint_gpt2_backward; (logits, dlogits, row_loss,
    grads) on the device."""
    rows, pv = sequences * length, cfg["padded_vocab"]
    with _make(flint, cfg, sequences, length, fused=fused) as model:
        for name, address, _, _ in model.parameters():
            model.write(address, params[name].contiguous())
        model.sync_weights()
        if old is not None:
            for name, address, _, _ in model.gradients():
                model.write(address, old[name].contiguous())
        model.forward(tok, trg, scale)
        model.backward(tok, accumulate=old is not None)
        lg, dl, rl = model.outputs()
        out = (model.read(lg, (rows, pv), torch.float16), model.read(dl, (rows, pv), torch.float16),
               model.read(rl, (rows,), torch.float32),
               {n: model.read(a, (r, c), torch.float32) for n, a, r, c in model.gradients()})
        torch.cuda.synchronize()
    return out


def _same_bits(a, b, what):
    ia = a.view(torch.int16 if a.dtype == torch.float16 else torch.int32)
    ib = b.view(torch.int16 if b.dtype == torch.float16 else torch.int32)
    differ = int((ia != ib).sum())
    assert differ == 0, f"{what}: {differ} of {a.numel()} values differ"


def _compare_with_hand(flint, cfg, sequences, length, fused, accumulate, seed):
    import compose

    shapes = G.parameter_shapes(cfg["layers"], cfg["width"], cfg["block_size"],
                                cfg["padded_vocab"])
    # FP32 masters off FP16's grid, so the FP16 copies round.
    params = {n: t.cuda() for n, t in
              G.init_params(shapes, cfg["layers"], cfg["vocab"], seed=seed, trained=True).items()}
    idx, tgt = _tokens(cfg, sequences, length, seed + 1)
    tok, trg = _dev16(idx), _dev16(tgt)
    scale = 1024.0 / (sequences * length)
    old = None
    if accumulate:
        g = torch.Generator().manual_seed(seed + 2)
        old = {n: (0.01 * torch.randn(r, c, generator=g)).cuda() for n, r, c in shapes}
    by_model = _model_passes(flint, cfg, sequences, length, params, tok, trg, scale, fused, old)
    by_hand = compose.passes(flint, cfg, sequences, length, params, tok, trg, scale,
                             fused=fused, old=old)
    for what, a, b in zip(("logits", "dlogits", "row_loss"), by_model[:3], by_hand[:3]):
        _same_bits(a, b, what)
    assert by_model[3].keys() == by_hand[3].keys()
    for n in by_model[3]:
        _same_bits(by_model[3][n], by_hand[3][n], n)


@pytest.mark.parametrize("sequences,length", [(1, 8), (3, 64), (2, 32)], ids=str)
@pytest.mark.parametrize("fused", [False, True], ids=["stored", "fused"])
def test_the_assembly_equals_the_kernels_called_by_hand(flint, cuda, fused, sequences, length):
    _compare_with_hand(flint, REF_TINY, sequences, length, fused, False, 31)


@pytest.mark.parametrize("fused", [False, True], ids=["stored", "fused"])
def test_the_accumulating_assembly_equals_the_kernels_called_by_hand(flint, cuda, fused):
    _compare_with_hand(flint, REF_TINY, 2, 32, fused, True, 41)


@pytest.mark.parametrize("cfg,sequences,length", [(TINY, 2, 64), (ODD, 2, 48)],
                         ids=["heads-of-32", "heads-of-32-odd-vocab"])
def test_other_head_widths_equal_the_kernels_called_by_hand(flint, cuda, cfg, sequences, length):
    _compare_with_hand(flint, cfg, sequences, length, False, False, 51)


def test_gpt2_124m_equals_the_kernels_called_by_hand(flint, cuda):
    _compare_with_hand(flint, GPT2, 1, 256, False, False, 61)

"""The training-step extension (include/flint/flint_train.h): AdamW with global
gradient clipping and a dynamic loss scale.

CPU: the oracle (oracle.adamw_step) is pinned against PyTorch's own step on the
CPU, as the reference runs it (ref scripts/gpt2_torch.py:161-192): GradScaler
unscale_/step/update, clip_grad_norm_ and torch.optim.AdamW with the
reference's parameter groups; and the C ABI's argument checks.
GPU: flint_adamw_step against the oracle over several steps, with a skipped
(non-finite) step, loss-scale growth and backoff, tails of every length, and a
tensor without an FP16 copy; the FP16 copy is checked bit for bit against the
kernel's own FP32 weights, and two runs from the same start must agree bit for
bit."""

import ctypes

import numpy as np
import pytest
import torch

from flint_amd.flint_lib import AdamwOptions, FlintError, TrainState
from oracle import oracle

# Element counts: one chunk is 8,192 values; tails of 0-3 past a float4 and
# several chunks per tensor.
COUNTS = [768 * 4, 1, 3, 16384 * 2 + 7, 50304 + 2, 768, 16384, 5]


def make_tensors(seed, counts=COUNTS, scale=1024.0):
    rng = np.random.default_rng(seed)
    out = []
    for i, n in enumerate(counts):
        out.append({
            "param": rng.normal(0, 0.02, n).astype(np.float32),
            "grad": (rng.normal(0, 0.01, n) * scale).astype(np.float32),
            "exp_avg": np.zeros(n, np.float32),
            "exp_avg_sq": np.zeros(n, np.float32),
            "weight_decay": 0.1 if i % 2 == 0 else 0.0,
        })
    return out


def new_grads(tensors, seed, scale, inf_at=None):
    rng = np.random.default_rng(seed)
    for i, t in enumerate(tensors):
        t["grad"] = (rng.normal(0, 0.01 * (1 + i), t["param"].size) * scale).astype(np.float32)
    if inf_at is not None:
        tensors[inf_at]["grad"][0] = np.inf


# ------------------------------------------------------------------ CPU: the oracle against PyTorch

def test_oracle_matches_torch_adamw_clip_and_grad_scaler():
    tensors = make_tensors(1, counts=[64, 5, 300, 7])
    params = [torch.nn.Parameter(torch.from_numpy(t["param"].copy())) for t in tensors]
    groups = [{"params": [p for p, t in zip(params, tensors) if t["weight_decay"] > 0], "weight_decay": 0.1},
              {"params": [p for p, t in zip(params, tensors) if t["weight_decay"] == 0], "weight_decay": 0.0}]
    opt = torch.optim.AdamW(groups, lr=6e-4, betas=(0.9, 0.95), eps=1e-8, foreach=False)
    scaler = torch.amp.GradScaler("cpu", init_scale=1024.0, growth_interval=2)
    state = {"loss_scale": 1024.0, "growth_tracker": 0, "step": 0}
    # Step 3 has a non-finite gradient; growth_interval 2 makes the scale grow.
    for step in range(6):
        scale = state["loss_scale"]
        new_grads(tensors, 100 + step, scale, inf_at=1 if step == 3 else None)
        scaler.scale(torch.ones(()))   # the scaler's per-iteration bookkeeping
        for p, t in zip(params, tensors):
            p.grad = torch.from_numpy(t["grad"].copy())
        scaler.unscale_(opt)
        torch.nn.utils.clip_grad_norm_(params, 1.0)
        scaler.step(opt)
        scaler.update()
        skipped, _, _ = oracle.adamw_step(tensors, state, growth_interval=2)
        assert skipped == (step == 3)
        assert state["loss_scale"] == scaler.get_scale()
        for p, t in zip(params, tensors):
            np.testing.assert_allclose(t["param"], p.detach().numpy(), rtol=1e-6, atol=1e-9)
            if p in opt.state:
                np.testing.assert_allclose(t["exp_avg"], opt.state[p]["exp_avg"].numpy(), rtol=1e-6, atol=1e-9)
                np.testing.assert_allclose(t["exp_avg_sq"], opt.state[p]["exp_avg_sq"].numpy(), rtol=1e-6,
                                           atol=1e-15)
    assert state["step"] == 5


def test_oracle_clip_factor_is_the_closed_form():
    # One tensor of n equal gradients g: norm = |g| sqrt(n); the first step's
    # update is lr * sign(g) for every element (m/sqrt(v) = 1 after bias
    # correction), whatever the clip factor, and m = (1 - beta1) c g.
    n, g = 400, 0.5
    t = [{"param": np.zeros(n, np.float32), "grad": np.full(n, g * 8, np.float32),
          "exp_avg": np.zeros(n, np.float32), "exp_avg_sq": np.zeros(n, np.float32), "weight_decay": 0.0}]
    state = {"loss_scale": 8.0, "growth_tracker": 0, "step": 0}
    skipped, norm, clip = oracle.adamw_step(t, state)
    assert not skipped
    assert norm == pytest.approx(g * np.sqrt(n))
    assert clip == pytest.approx(1.0 / (g * np.sqrt(n) + 1e-6), rel=1e-6)
    np.testing.assert_allclose(t[0]["exp_avg"], 0.1 * clip * g, rtol=1e-5)
    np.testing.assert_allclose(t[0]["param"], -6e-4, rtol=1e-4)


# ------------------------------------------------------------------ CPU: ABI checks (no GPU call)

def test_defaults_are_the_references_constants(flint):
    o = flint.adamw_defaults()
    assert (o.lr, o.beta1, o.beta2, o.eps, o.max_grad_norm) == pytest.approx((6e-4, 0.9, 0.95, 1e-8, 1.0))
    assert (o.growth_factor, o.backoff_factor, o.growth_interval) == (2.0, 0.5, 2000)


def test_state_is_32_bytes():
    assert ctypes.sizeof(TrainState) == 32


@pytest.mark.parametrize("field, value, text", [
    ("beta1", 1.0, "betas"), ("beta2", -0.1, "betas"), ("eps", 0.0, "eps"), ("lr", float("nan"), "lr"),
    ("growth_interval", 0, "growth_interval"), ("backoff_factor", 2.0, "backoff_factor"),
])
def test_bad_options_rejected(flint, field, value, text):
    o = flint.adamw_defaults()
    setattr(o, field, value)
    t = [{"param": 16, "grad": 32, "exp_avg": 48, "exp_avg_sq": 64, "count": 4, "weight_decay": 0.0}]
    with pytest.raises(FlintError, match=text):
        flint.check(flint.lib.flint_adamw_step(flint.adamw_tensors(t), 1, 4096, ctypes.byref(o), 8192, 1 << 20, None))


def test_workspace_and_its_check(flint):
    t = [{"param": 0, "grad": 0, "exp_avg": 0, "exp_avg_sq": 0, "count": 16384 * 3 + 1, "weight_decay": 0.0},
         {"param": 0, "grad": 0, "exp_avg": 0, "exp_avg_sq": 0, "count": 10, "weight_decay": 0.1}]
    need = flint.adamw_workspace(t)
    chunks = -(-(16384 * 3 + 1) // 8192) + 1   # 8,192-value chunks
    assert need == (chunks * 8 + 255) // 256 * 256 + 256   # FP64 partials, then the decision
    o = flint.adamw_defaults()
    with pytest.raises(FlintError, match="needs .* bytes of workspace"):
        flint.check(flint.lib.flint_adamw_step(flint.adamw_tensors(t), 2, 4096, ctypes.byref(o), 8192, need - 1, None))
    bad = [dict(t[0], weight_decay=-1.0)]
    with pytest.raises(FlintError, match="weight_decay"):
        flint.adamw_workspace(bad)


def test_misaligned_and_overlapping_buffers_rejected(flint):
    o = flint.adamw_defaults()
    base = 1 << 20
    t = [{"param": base + 8, "grad": base + 4096, "exp_avg": base + 8192, "exp_avg_sq": base + 12288, "count": 16}]
    with pytest.raises(FlintError, match="param"):
        flint.check(flint.lib.flint_adamw_step(flint.adamw_tensors(t), 1, 4096, ctypes.byref(o), 1 << 19, 1024, None))
    t = [{"param": base, "grad": base + 32, "exp_avg": base + 8192, "exp_avg_sq": base + 12288, "count": 16}]
    with pytest.raises(FlintError, match="overlap"):
        flint.check(flint.lib.flint_adamw_step(flint.adamw_tensors(t), 1, 4096, ctypes.byref(o), 1 << 19, 1024, None))


def test_tensors_sharing_memory_are_rejected(flint):
    """A tensor listed twice, or two tensors whose buffers overlap, would be
    stepped twice or race on their moments: the step refuses them before any
    device work (the addresses below are never dereferenced)."""
    o = flint.adamw_defaults()
    base = 1 << 24

    def tensor(at, count=64):
        return {"param": at, "grad": at + 4096, "exp_avg": at + 8192, "exp_avg_sq": at + 12288,
                "count": count, "weight_decay": 0.0}

    state, ws = 4096, 1 << 22

    def step(ts):
        flint.check(flint.lib.flint_adamw_step(flint.adamw_tensors(ts), len(ts), state, ctypes.byref(o),
                                               ws, 1 << 16, None))

    with pytest.raises(FlintError, match="tensor 0's param and tensor 1's param overlap"):
        step([tensor(base), tensor(base)])
    # Tensor 1's grad lands inside tensor 0's exp_avg_sq; its other buffers are far away.
    other = dict(tensor(base + (1 << 20)), grad=base + 12288 + 128)
    with pytest.raises(FlintError, match="tensor 0's exp_avg_sq and tensor 1's grad overlap"):
        step([tensor(base), other])
    # Adjacent tensors (no shared byte) are not run here: the addresses are
    # not device memory. The GPU tests step real adjacent tensors.


# ------------------------------------------------------------------ GPU: parity with the oracle

def to_dev(tensors, cuda, half_skip=2):
    dev = []
    for i, t in enumerate(tensors):
        d = {k: torch.from_numpy(t[k].copy()).to(cuda) for k in ("param", "grad", "exp_avg", "exp_avg_sq")}
        d["param_half"] = None if i == half_skip else torch.empty(t["param"].size, dtype=torch.float16, device=cuda)
        d["weight_decay"] = t["weight_decay"]
        dev.append(d)
    return dev


def read_state(state):
    raw = state.cpu().numpy().tobytes()
    return TrainState.from_buffer_copy(raw)


@pytest.mark.gpu
def test_adamw_step_matches_the_oracle(flint, cuda):
    host = make_tensors(7)
    dev = to_dev(host, cuda)
    o = flint.adamw_defaults()
    o.growth_interval = 2
    state = torch.zeros(8, dtype=torch.float32, device=cuda)   # 32 bytes
    flint.train_state_init(state, 1024.0)
    ws = torch.empty(flint.adamw_workspace(dev), dtype=torch.uint8, device=cuda)
    ostate = {"loss_scale": 1024.0, "growth_tracker": 0, "step": 0}
    for step in range(6):
        inf_at = 4 if step == 2 else None
        new_grads(host, 500 + step, ostate["loss_scale"], inf_at=inf_at)
        for d, h in zip(dev, host):
            d["grad"].copy_(torch.from_numpy(h["grad"]))
        flint.adamw_step(dev, state, o, ws)
        skipped, norm, clip = oracle.adamw_step(host, ostate, growth_interval=2)
        torch.cuda.synchronize()
        s = read_state(state)
        print(f"step {step}: skipped {skipped}, norm {norm:.6g}, clip {clip:.6g}, scale {s.loss_scale}", flush=True)
        assert bool(s.found_inf) == skipped
        assert (s.loss_scale, s.growth_tracker, s.step) == (ostate["loss_scale"], ostate["growth_tracker"],
                                                             ostate["step"])
        if not skipped:
            assert s.grad_norm == pytest.approx(norm, rel=1e-12)
            assert s.clip_coef == pytest.approx(clip, rel=1e-7)
        for i, (d, h) in enumerate(zip(dev, host)):
            p = d["param"].cpu().numpy()
            np.testing.assert_allclose(p, h["param"], rtol=2e-6, atol=1e-9, err_msg=f"param {i}")
            np.testing.assert_allclose(d["exp_avg"].cpu().numpy(), h["exp_avg"], rtol=2e-6, atol=1e-9)
            np.testing.assert_allclose(d["exp_avg_sq"].cpu().numpy(), h["exp_avg_sq"], rtol=2e-6, atol=1e-15)
            if d["param_half"] is not None:
                assert np.array_equal(d["param_half"].cpu().numpy().view(np.uint16),
                                      p.astype(np.float16).view(np.uint16)), f"half {i}"
    assert s.step == 5


@pytest.mark.gpu
def test_adamw_step_is_deterministic(flint, cuda):
    results = []
    for _ in range(2):
        host = make_tensors(9)
        dev = to_dev(host, cuda)
        o = flint.adamw_defaults()
        state = torch.zeros(8, dtype=torch.float32, device=cuda)
        flint.train_state_init(state, 1024.0)
        ws = torch.empty(flint.adamw_workspace(dev), dtype=torch.uint8, device=cuda)
        for step in range(3):
            flint.adamw_step(dev, state, o, ws)
        torch.cuda.synchronize()
        results.append([d["param"].cpu().numpy().tobytes() for d in dev] + [state.cpu().numpy().tobytes()])
    assert results[0] == results[1]


@pytest.mark.gpu
def test_adamw_step_over_gpt2_parameters(flint, cuda):
    """The 124M-parameter model's tensors (PyTorch named_parameters shapes):
    one step from zero moments moves every weight by lr g / (|g| + eps), and
    the norm equals the FP64 norm of the same unscaled gradients."""
    shapes = [(50257, 768), (1024, 768)]
    for _ in range(12):
        shapes += [(768,), (768,), (2304, 768), (2304,), (768, 768), (768,), (768,), (768,), (3072, 768),
                   (3072,), (768, 3072), (768,)]
    shapes += [(768,), (768,)]
    gen = torch.Generator(device=cuda).manual_seed(3)
    dev = []
    for shp in shapes:
        n = int(np.prod(shp))
        dev.append({"param": torch.randn(n, device=cuda, generator=gen) * 0.02,
                    "grad": torch.randn(n, device=cuda, generator=gen) * 1024 * 1e-4,
                    "exp_avg": torch.zeros(n, device=cuda), "exp_avg_sq": torch.zeros(n, device=cuda),
                    "param_half": torch.empty(n, dtype=torch.float16, device=cuda),
                    "weight_decay": 0.1 if len(shp) == 2 else 0.0})
    before = [d["param"].clone() for d in dev]
    o = flint.adamw_defaults()
    state = torch.zeros(8, dtype=torch.float32, device=cuda)
    flint.train_state_init(state, 1024.0)
    ws = torch.empty(flint.adamw_workspace(dev), dtype=torch.uint8, device=cuda)
    flint.adamw_step(dev, state, o, ws)
    torch.cuda.synchronize()
    s = read_state(state)
    want = torch.sqrt(sum(((d["grad"].double() / 1024) ** 2).sum() for d in dev)).item()
    assert s.grad_norm == pytest.approx(want, rel=1e-9)
    assert s.step == 1 and s.found_inf == 0
    for d, b, shp in zip(dev, before, shapes):
        decayed = b * (1 - 6e-4 * (0.1 if len(shp) == 2 else 0.0))
        moved = (decayed - d["param"]).double()
        # First step from zero moments: m_hat = g, sqrt(v_hat) = |g|, so each
        # element moves by lr g / (|g| + eps), g the unscaled, clipped gradient.
        g = d["grad"].double() / 1024 * s.clip_coef
        want = 6e-4 * g / (g.abs() + 1e-8)
        assert torch.allclose(moved, want, rtol=1e-3, atol=1e-8)

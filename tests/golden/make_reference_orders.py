"""Writes tests/golden/reference_orders.npz: inputs and outputs of the
reference's own emulations of the shape-only summation orders, for the C
oracle's restatement to be checked against bit for bit.

The emulations are the reference's numpy transcriptions of its kernels'
arithmetic (ref tests/test_bias_gradient.py:239 `emulate`,
tests/test_layernorm_backward.py:148 `emulate_dx` and :238 `emulate_dgamma`,
tests/test_softmax_backward.py:120 `emulate`, tests/test_embedding_backward.py:322
`emulate_all`). This script imports them from the reference checkout, so it
runs only where that checkout is (the build container): the GPU box and the
tests read the committed .npz alone. Inputs are generated here from fixed
seeds; none of the reference's code or text is stored, only the vectors.

    python tests/golden/make_reference_orders.py [/path/to/reference]
"""

import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "reference_orders.npz"


def main(ref_root):
    sys.path.insert(0, str(Path(ref_root) / "tests"))
    import test_bias_gradient as bg                # noqa: E402
    import test_embedding_backward as eb           # noqa: E402
    import test_layernorm_backward as lb           # noqa: E402
    import test_softmax_backward as sb             # noqa: E402

    rng = np.random.default_rng(20261202)
    out = {}

    # Bias gradient: 600 rows (3 chunks, the last partial) x 136 columns, plain
    # and accumulating into an old value; a second case with large and tiny
    # magnitudes mixed so that the compensation matters.
    dy = rng.standard_normal((600, 136)).astype(np.float16)
    old = rng.standard_normal(136).astype(np.float32)
    out["bias_dy"] = dy
    out["bias_old"] = old
    out["bias_out"] = np.asarray(bg.emulate(dy), dtype=np.float32)
    out["bias_out_acc"] = np.asarray(bg.emulate(dy, old), dtype=np.float32)
    mixed = (rng.standard_normal((520, 64)) * np.where(rng.random((520, 64)) < 0.05, 3e3, 1e-2))
    out["bias_dy2"] = mixed.astype(np.float16)
    out["bias_out2"] = np.asarray(bg.emulate(out["bias_dy2"]), dtype=np.float32)

    # LayerNorm backward: 300 rows x 72 columns.
    rows, cols = 300, 72
    x = (rng.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
    mean = x.astype(np.float64).mean(axis=1).astype(np.float32)
    var = x.astype(np.float64).var(axis=1)
    rstd = (1.0 / np.sqrt(var + 1e-5)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    ldy = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float16)
    dx_old = rng.standard_normal((rows, cols)).astype(np.float32)
    out.update(ln_dy=ldy, ln_x=x, ln_mean=mean, ln_rstd=rstd, ln_gamma=gamma, ln_dx_old=dx_old)
    out["ln_dx"] = np.asarray(lb.emulate_dx(ldy, x, mean, rstd, gamma), dtype=np.float32)
    out["ln_dx_acc"] = np.asarray(lb.emulate_dx(ldy, x, mean, rstd, gamma, dx_old), dtype=np.float32)
    dgamma = lb.emulate_dgamma(ldy, x, mean, rstd)
    out["ln_dgamma"] = np.asarray(dgamma[0] if isinstance(dgamma, tuple) else dgamma, dtype=np.float32)

    # Causal softmax backward: 2 batches of 80 x 80 (p a causal softmax of
    # random scores, zero above the diagonal), scale 1/8.
    b, t = 2, 80
    s = rng.standard_normal((b, t, t)) * 2
    mask = np.triu(np.ones((t, t), dtype=bool), 1)
    s[:, mask] = -np.inf
    e = np.exp(s - s.max(axis=2, keepdims=True))
    p = (e / e.sum(axis=2, keepdims=True)).astype(np.float16)
    dp = (rng.standard_normal((b, t, t)) * 0.1).astype(np.float16)
    out.update(sm_p=p, sm_dp=dp)
    out["sm_ds"] = np.asarray(sb.emulate(p, dp, 0.125), dtype=np.float16)

    # Embedding backward: 2 sequences x 40 positions, width 64, vocabulary 50
    # (tokens repeat, so rows of dwte sum several rows of dx).
    seqs, length, vocab, width = 2, 40, 50, 64
    edx = rng.standard_normal((seqs * length, width)).astype(np.float32)
    tok = rng.integers(0, vocab, seqs * length).astype(np.uint16)
    exp = eb.emulate_all(edx, tok, seqs, length, vocab)
    out.update(emb_dx=edx, emb_tokens=tok)
    out["emb_dwte"] = np.asarray(exp[0], dtype=np.float32)
    out["emb_dwpe"] = np.asarray(exp[1], dtype=np.float32)

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

"""Writes tests/golden/golden.npz: small seeded inputs and the outputs that
PyTorch's own CPU float64 operators give for them (F.gelu(tanh) and its
autograd derivative, F.layer_norm and its autograd backward, masked softmax
and its backward, F.cross_entropy and its logit gradient, a float64 index_add
for the embedding gradient). PyTorch is an implementation independent of
both the reference and this repository's oracle, so the fixtures pin the
oracle; they are data, regenerated with `python tests/golden/make_golden.py`."""

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "golden.npz"


def main():
    g = torch.Generator().manual_seed(1234)
    d = {}
    # GELU and its derivative over a spread of FP16 inputs.
    s = (torch.randn(4096, generator=g) * 4).half().double()
    s.requires_grad_(True)
    y = F.gelu(s, approximate="tanh")
    (gs,) = torch.autograd.grad(y.sum(), s)
    d["gelu_in"] = s.detach().numpy()
    d["gelu_out"] = y.detach().numpy()
    d["gelu_grad"] = gs.numpy()

    # LayerNorm forward / backward.
    rows, cols = 24, 200
    x = (torch.randn(rows, cols, generator=g) + 2).double()
    x[:, 5] += 3000
    gamma = (1 + 0.1 * torch.randn(cols, generator=g)).double()
    beta = (0.1 * torch.randn(cols, generator=g)).double()
    dy = torch.randn(rows, cols, generator=g).half().double()
    xr = x.clone().requires_grad_(True)
    gr = gamma.clone().requires_grad_(True)
    br = beta.clone().requires_grad_(True)
    ln = F.layer_norm(xr, (cols,), gr, br, eps=1e-5)
    dx, dgamma, dbeta = torch.autograd.grad(ln, (xr, gr, br), dy)
    d.update(ln_x=x.numpy(), ln_gamma=gamma.numpy(), ln_beta=beta.numpy(), ln_y=ln.detach().numpy(),
             ln_dy=dy.numpy(), ln_dx=dx.numpy(), ln_dgamma=dgamma.numpy(), ln_dbeta=dbeta.numpy())

    # Causal softmax forward / backward (scale 1/8).
    b, t = 3, 40
    sc = (torch.randn(b, t, t, generator=g) * 3).half().double()
    mask = torch.tril(torch.ones(t, t, dtype=torch.bool))
    sr = sc.clone().requires_grad_(True)
    p = torch.softmax(sr.masked_fill(~mask, float("-inf")), dim=-1)
    dp = torch.randn(b, t, t, generator=g).half().double()
    (dsv,) = torch.autograd.grad(p, sr, dp)
    d.update(sm_s=sc.numpy(), sm_p=p.detach().numpy(), sm_dp=dp.numpy(),
             sm_ds=(dsv * 0.125).masked_fill(~mask, 0).numpy())

    # Softmax + cross-entropy over the first vocab columns.
    rows, cols, vocab = 16, 136, 129
    logits = (torch.randn(rows, cols, generator=g) * 2).half().double()
    tg = torch.randint(0, vocab, (rows,), generator=g)
    lr = logits[:, :vocab].clone().requires_grad_(True)
    loss = F.cross_entropy(lr, tg, reduction="none")
    (dl,) = torch.autograd.grad(loss.sum() * 0.125, lr)
    dfull = torch.zeros(rows, cols, dtype=torch.float64)
    dfull[:, :vocab] = dl
    d.update(ce_logits=logits.numpy(), ce_targets=tg.numpy().astype(np.int64), ce_vocab=vocab,
             ce_loss=loss.detach().numpy(), ce_dlogits=dfull.numpy(), ce_scale=0.125)

    # Embedding backward: dwte via index_add, dwpe as a sum over sequences.
    seqs, length, vocab_e, width = 3, 16, 50, 24
    tok = torch.randint(0, vocab_e, (seqs * length,), generator=g)
    dxe = torch.randn(seqs * length, width, generator=g).double()
    dwte = torch.zeros(vocab_e, width, dtype=torch.float64).index_add_(0, tok, dxe)
    dwpe = dxe.view(seqs, length, width).sum(0)
    d.update(emb_tokens=tok.numpy().astype(np.int64), emb_dx=dxe.numpy(), emb_dwte=dwte.numpy(),
             emb_dwpe=dwpe.numpy(), emb_shape=np.array([seqs, length, vocab_e, width]))

    # GEMM with each epilogue, small.
    m, n, k = 20, 24, 32
    xg = (torch.rand(m, k, generator=g) * 2 - 1).half().double()
    wg = (torch.randn(n, k, generator=g) * 0.5).half().double()
    bg = torch.randn(n, generator=g).float().double()
    rg = torch.randn(m, n, generator=g).float().double()
    sg = xg @ wg.T
    d.update(gemm_x=xg.numpy(), gemm_w=wg.numpy(), gemm_b=bg.numpy(), gemm_r=rg.numpy(),
             gemm_nt=sg.numpy(), gemm_bias=(sg + bg).numpy(),
             gemm_gelu=F.gelu(sg + bg, approximate="tanh").numpy(),
             gemm_residual=(rg + (sg + bg)).numpy())
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()

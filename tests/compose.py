"""The GPT-2 passes rebuilt from the public entry points, one call at a time,
on fresh buffers: the contract that flint_gpt2_forward and flint_gpt2_backward
are exactly these calls in this order (ref tests/test_gpt2.py:1114-1123 for the
forward, ref tests/test_gpt2_backward.py:896-950 for the backward, whose call
order ref src/api/gpt2.cpp:495-618 and :721-813 define).

`passes(flint, cfg, sequences, length, params, tokens, targets, scale,
fused=False, old=None)` returns (logits, dlogits, row_loss, grads) as device
tensors. cfg is the model's config dict; params maps each master name to its
FP32 tensor on the device; tokens and targets are device int16 tensors of
sequences * length ids. With fused=True each block's attention is
flint_heads_split -> flint_attention_forward / _backward -> flint_heads_merge
(the model of flint_gpt2_create_fused); otherwise the stored scores and
probabilities of the reference's sequence. With old (name -> gradient) the
backward accumulates into copies of those gradients, else it writes
gradients that start as NaN (a missed write shows)."""

import math

import numpy as np
import torch


def _half(*shape):
    return torch.empty(*shape, dtype=torch.float16, device="cuda")


def _single(*shape):
    return torch.empty(*shape, dtype=torch.float32, device="cuda")


def _bytes(n):
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device="cuda")


def passes(flint, cfg, sequences, length, params, tokens, targets, scale, fused=False, old=None):
    W, H, S, T = cfg["width"], cfg["heads"], sequences, length
    V, PV = cfg["vocab"], cfg["padded_vocab"]
    rows, hw, nb = S * T, W // H, S * H
    heads_elems = nb * T * hw
    sscale = float(np.float32(1.0) / np.sqrt(np.float32(hw)))

    def fp16_of(name):
        m = params[name].contiguous().reshape(-1)
        y = _half(m.numel())
        flint.fp32_to_fp16(y, m, m.numel())
        return y

    copies = {n: fp16_of(n) for n in params
              if n == "wte.weight" or n.endswith(("c_attn.weight", "c_proj.weight", "c_fc.weight"))}

    def vec(name):
        return params[name].reshape(-1)

    def layer_norm(x, prefix):
        y, mean, rstd = _half(rows, W), _single(rows), _single(rows)
        flint.layernorm_forward(y, mean, rstd, x, vec(prefix + ".weight"), vec(prefix + ".bias"),
                                rows, W)
        return y, mean, rstd

    # ---- forward, every block's activations kept
    x = _single(rows, W)
    flint.embedding_forward(x, tokens, params["wte.weight"], params["wpe.weight"], S, T, PV, W)
    kept = []
    for i in range(cfg["layers"]):
        p = f"blocks.{i}."
        a = {"x_in": x}
        a["h1"], a["mean1"], a["rstd1"] = layer_norm(x, p + "ln_1")
        qkv = _half(rows, 3 * W)
        flint.gemm_nt_bias(qkv, a["h1"], copies[p + "attn.c_attn.weight"],
                           vec(p + "attn.c_attn.bias"), rows, 3 * W, W)
        a["q"], a["k"], a["v"] = (_half(heads_elems) for _ in range(3))
        for j, part in enumerate((a["q"], a["k"], a["v"])):
            flint.heads_split(part, qkv, S, T, H, hw, 3 * W, j * W)
        a["o"] = _half(heads_elems)
        if fused:
            a["lse"] = _single(nb * T)
            flint.attention_forward(a["o"], a["lse"], a["q"], a["k"], a["v"], nb, T, hw, sscale)
        else:
            scores, a["p"] = _half(nb, T, T), _half(nb, T, T)
            flint.gemm_nt_batched(scores, a["q"], a["k"], nb, T, T, hw, sscale)
            flint.causal_softmax_forward(a["p"], scores, nb, T)
            flint.gemm_nn_batched(a["o"], a["p"], a["v"], nb, T, hw, T)
        a["attn"] = _half(rows, W)
        flint.heads_merge(a["attn"], a["o"], S, T, H, hw, W, 0)
        a["x_mid"] = _single(rows, W)
        flint.gemm_nt_bias_residual(a["x_mid"], a["attn"], copies[p + "attn.c_proj.weight"],
                                    vec(p + "attn.c_proj.bias"), x, rows, W, W)
        a["h2"], a["mean2"], a["rstd2"] = layer_norm(a["x_mid"], p + "ln_2")
        a["gelu"], a["pre"] = _half(rows, 4 * W), _half(rows, 4 * W)
        flint.gemm_nt_bias_gelu(a["gelu"], a["pre"], a["h2"], copies[p + "mlp.c_fc.weight"],
                                vec(p + "mlp.c_fc.bias"), rows, 4 * W, W)
        x = _single(rows, W)
        flint.gemm_nt_bias_residual(x, a["gelu"], copies[p + "mlp.c_proj.weight"],
                                    vec(p + "mlp.c_proj.bias"), a["x_mid"], rows, W, 4 * W)
        kept.append(a)
    x_final = x
    h_f, mean_f, rstd_f = layer_norm(x_final, "ln_f")
    logits = _half(rows, PV)
    flint.gemm_nt(logits, h_f, copies["wte.weight"], rows, PV, W)
    dlogits, row_loss = _half(rows, PV), _single(rows)
    flint.softmax_cross_entropy(dlogits, row_loss, logits, targets, scale, rows, V, PV)

    # ---- backward
    acc = old is not None
    grads = {}
    for name, t in params.items():
        grads[name] = (old[name].clone() if acc
                       else torch.full(tuple(t.shape), math.nan, device="cuda"))
    if not acc:
        grads["wpe.weight"][T:] = 0   # positions past length are never seen

    def weight_grad(name, dy, xin, m, n):
        ws = _bytes(flint.gemm_tn_workspace(m, n, rows))
        flint.gemm_tn(grads[name], dy, xin, m, n, rows, accumulate=acc, workspace=ws)

    def bias_grad(name, dy, cols):
        flint.bias_gradient(grads[name], dy, rows, cols, accumulate=acc,
                            workspace=_bytes(flint.bias_gradient_workspace(rows, cols)))

    def norm_grad(prefix, dres, dh, xin, mean, rstd, acc_dx):
        flint.layernorm_backward(dres, grads[prefix + ".weight"], grads[prefix + ".bias"], dh, xin,
                                 mean, rstd, vec(prefix + ".weight"), rows, W,
                                 accumulate_dx=acc_dx, accumulate_params=acc,
                                 workspace=_bytes(flint.layernorm_backward_workspace(rows, W)))

    def half_of(dres):
        g = _half(rows, W)
        flint.fp32_to_fp16(g, dres, rows * W)
        return g

    weight_grad("wte.weight", dlogits, h_f, PV, W)
    dh = _half(rows, W)
    flint.gemm_nn(dh, dlogits, copies["wte.weight"], rows, W, PV)
    dres = _single(rows, W)
    norm_grad("ln_f", dres, dh, x_final, mean_f, rstd_f, False)
    for i in reversed(range(cfg["layers"])):
        p, a = f"blocks.{i}.", kept[i]
        g = half_of(dres)
        weight_grad(p + "mlp.c_proj.weight", g, a["gelu"], W, 4 * W)
        bias_grad(p + "mlp.c_proj.bias", g, W)
        dpre = _half(rows, 4 * W)
        flint.gemm_nn_dgelu(dpre, g, copies[p + "mlp.c_proj.weight"], a["pre"], rows, 4 * W, W)
        weight_grad(p + "mlp.c_fc.weight", dpre, a["h2"], 4 * W, W)
        bias_grad(p + "mlp.c_fc.bias", dpre, 4 * W)
        dh = _half(rows, W)
        flint.gemm_nn(dh, dpre, copies[p + "mlp.c_fc.weight"], rows, W, 4 * W)
        norm_grad(p + "ln_2", dres, dh, a["x_mid"], a["mean2"], a["rstd2"], True)

        g = half_of(dres)
        weight_grad(p + "attn.c_proj.weight", g, a["attn"], W, W)
        bias_grad(p + "attn.c_proj.bias", g, W)
        d_attn = _half(rows, W)
        flint.gemm_nn(d_attn, g, copies[p + "attn.c_proj.weight"], rows, W, W)
        d_o = _half(heads_elems)
        flint.heads_split(d_o, d_attn, S, T, H, hw, W, 0)
        dq, dk, dv = (_half(heads_elems) for _ in range(3))
        if fused:
            flint.attention_backward(dq, dk, dv, d_o, a["q"], a["k"], a["v"], a["o"], a["lse"],
                                     nb, T, hw, sscale)
        else:
            flint.gemm_tn_batched(dv, a["p"], d_o, nb, T, hw, T)
            ds = _half(nb, T, T)   # dP, then dS in place
            flint.gemm_nt_batched(ds, d_o, a["v"], nb, T, T, hw, 1.0)
            flint.causal_softmax_backward(ds, a["p"], ds, nb, T, sscale)
            flint.gemm_nn_batched(dq, ds, a["k"], nb, T, hw, T)
            flint.gemm_tn_batched(dk, ds, a["q"], nb, T, hw, T)
        dqkv = _half(rows, 3 * W)
        for j, part in enumerate((dq, dk, dv)):
            flint.heads_merge(dqkv, part, S, T, H, hw, 3 * W, j * W)
        weight_grad(p + "attn.c_attn.weight", dqkv, a["h1"], 3 * W, W)
        bias_grad(p + "attn.c_attn.bias", dqkv, 3 * W)
        dh = _half(rows, W)
        flint.gemm_nn(dh, dqkv, copies[p + "attn.c_attn.weight"], rows, W, 3 * W)
        norm_grad(p + "ln_1", dres, dh, a["x_in"], a["mean1"], a["rstd1"], True)
    flint.embedding_backward(grads["wte.weight"], grads["wpe.weight"], dres, tokens, S, T, PV, W,
                             accumulate_wte=True, accumulate_wpe=acc,
                             workspace=_bytes(flint.embedding_backward_workspace(S, T, PV, W)))
    torch.cuda.synchronize()
    return logits, dlogits, row_loss, grads

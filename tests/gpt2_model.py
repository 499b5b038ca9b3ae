"""GPT-2 in plain PyTorch on the CPU: the reference the assembled flint_gpt2 is
checked against (the model of ref scripts/gpt2_torch.py:45-137, written here as
functions over a name -> tensor dict in named_parameters order).

`forward(params, idx, targets, cfg, fp16=False)` returns (logits over vocab,
per-row loss). With fp16=True every tensor the library stores in FP16 is rounded
to FP16 where the library rounds it (LayerNorm outputs, GEMM outputs, the
attention scores and probabilities, GELU's input and output), while sums stay
FP32 and the residual stream stays FP32: that is the "peer", an FP16 computation
with the library's storage precisions, whose error against the FP32 model sets
the scale of the gate."""

import math

import torch
import torch.nn.functional as F


def parameter_shapes(layers, width, block_size, padded_vocab):
    """(name, rows, cols) in PyTorch's named_parameters order; vectors have 1 row."""
    c = width
    out = [("wte.weight", padded_vocab, c), ("wpe.weight", block_size, c)]
    for i in range(layers):
        p = f"blocks.{i}."
        out += [(p + "ln_1.weight", 1, c), (p + "ln_1.bias", 1, c),
                (p + "attn.c_attn.weight", 3 * c, c), (p + "attn.c_attn.bias", 1, 3 * c),
                (p + "attn.c_proj.weight", c, c), (p + "attn.c_proj.bias", 1, c),
                (p + "ln_2.weight", 1, c), (p + "ln_2.bias", 1, c),
                (p + "mlp.c_fc.weight", 4 * c, c), (p + "mlp.c_fc.bias", 1, 4 * c),
                (p + "mlp.c_proj.weight", c, 4 * c), (p + "mlp.c_proj.bias", 1, c)]
    out += [("ln_f.weight", 1, c), ("ln_f.bias", 1, c)]
    return out


def init_params(shapes, layers, vocab, seed, trained=False):
    """GPT-2's init (N(0, 0.02) weights, residual projections scaled by
    1/sqrt(2 layers), zero biases, unit LayerNorm gains, zero padded wte rows).
    trained=True moves biases and LayerNorm parameters off their init, as
    mid-training weights are."""
    g = torch.Generator().manual_seed(seed)
    params = {}
    for name, rows, cols in shapes:
        if name.endswith("ln_1.weight") or name.endswith("ln_2.weight") or name == "ln_f.weight":
            t = torch.ones(rows, cols)
            if trained:
                t += 0.1 * torch.randn(rows, cols, generator=g)
        elif rows == 1:
            t = torch.zeros(rows, cols)
            if trained:
                t += 0.02 * torch.randn(rows, cols, generator=g)
        else:
            std = 0.02
            if name.endswith("c_proj.weight"):
                std = 0.02 / math.sqrt(2 * layers)
            t = std * torch.randn(rows, cols, generator=g)
            if name == "wte.weight":
                t[vocab:] = 0
        params[name] = t
    return params


def _h(t, fp16):
    return t.half().float() if fp16 else t


def _layer_norm(x, w, b, fp16):
    return _h(F.layer_norm(x, (x.shape[-1],), w.reshape(-1), b.reshape(-1), eps=1e-5), fp16)


def _linear(x, w, b, fp16):
    y = x @ _h(w, fp16).T
    return y + b.reshape(-1) if b is not None else y


def forward(params, idx, targets, cfg, fp16=False):
    """(logits [rows, vocab], row_loss [rows]) for idx, targets of shape
    [sequences, length] (int64)."""
    layers, heads, width, vocab = cfg["layers"], cfg["heads"], cfg["width"], cfg["vocab"]
    seqs, length = idx.shape
    hd = width // heads
    x = params["wte.weight"][idx] + params["wpe.weight"][:length]
    mask = torch.triu(torch.ones(length, length, dtype=torch.bool, device=x.device), 1)
    for i in range(layers):
        p = f"blocks.{i}."
        h = _layer_norm(x, params[p + "ln_1.weight"], params[p + "ln_1.bias"], fp16)
        qkv = _h(_linear(h, params[p + "attn.c_attn.weight"], params[p + "attn.c_attn.bias"],
                         fp16), fp16)
        q, k, v = qkv.split(width, dim=-1)
        q, k, v = (t.reshape(seqs, length, heads, hd).transpose(1, 2) for t in (q, k, v))
        s = _h((q @ k.transpose(-1, -2).contiguous()) / math.sqrt(hd), fp16)
        a = _h(torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1), fp16)
        o = _h(a @ v, fp16).transpose(1, 2).reshape(seqs, length, width)
        x = x + _linear(o, params[p + "attn.c_proj.weight"], params[p + "attn.c_proj.bias"],
                        fp16)
        h = _layer_norm(x, params[p + "ln_2.weight"], params[p + "ln_2.bias"], fp16)
        pre = _h(_linear(h, params[p + "mlp.c_fc.weight"], params[p + "mlp.c_fc.bias"], fp16),
                 fp16)
        u = _h(F.gelu(pre, approximate="tanh"), fp16)
        x = x + _linear(u, params[p + "mlp.c_proj.weight"], params[p + "mlp.c_proj.bias"], fp16)
    xf = _layer_norm(x, params["ln_f.weight"], params["ln_f.bias"], fp16).reshape(-1, width)
    logits = _h(_linear(xf, params["wte.weight"], None, fp16), fp16)[:, :vocab]
    row_loss = F.cross_entropy(logits, targets.reshape(-1), reduction="none")
    return logits, row_loss


def gradients(params, idx, targets, cfg, scale, fp16=False):
    """(logits, row_loss, dlogits, grads): grads of scale * sum(row_loss), FP32."""
    leaves = {n: t.clone().requires_grad_(True) for n, t in params.items()}
    logits, row_loss = forward(leaves, idx, targets, cfg, fp16)
    logits.retain_grad()
    (scale * row_loss.sum()).backward()
    grads = {n: t.grad.detach() for n, t in leaves.items()}
    return logits.detach(), row_loss.detach(), logits.grad.detach(), grads

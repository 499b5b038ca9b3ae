"""ctypes binding of libflint.so's C ABI (include/flint/flint.h).

Mirrors the interface of the reference's test bridge (ref tests/flint_lib.py:
`SIGNATURES` table :57-408, `Flint` wrapper :440-870): the same method names,
argument order and meaning, so tests written against the reference read the
same here. Pointer arguments take a torch tensor (its data pointer), an int
address, or None for null; stream arguments take a torch.cuda.Stream, an int
handle, or None for torch's current stream.

The library path comes from FLINT_LIB, else build/release/bin/libflint.so at
the repository root (the path the reference's loader defaults to). Loading
fails loudly when the library is missing: there is no fallback.
"""

import ctypes
import os
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "flint" / "flint.h"
TRAIN_HEADER = ROOT / "include" / "flint" / "flint_train.h"
NOALLOC_HEADER = ROOT / "include" / "flint" / "flint_noalloc.h"
ATTENTION_HEADER = ROOT / "include" / "flint" / "flint_attention.h"
TUNING_HEADER = ROOT / "include" / "flint" / "flint_tuning.h"
LIBRARY = ROOT / "build" / "release" / "bin" / "libflint.so"

OK = 0
ERROR_INVALID_ARGUMENT = 1
ERROR_CUDA = 2

P = ctypes.c_void_p
Z = ctypes.c_size_t
I = ctypes.c_int
F = ctypes.c_float


class Gpt2Config(ctypes.Structure):
    """flint_gpt2_config (ref flint.h:455-466)."""

    _fields_ = [
        ("layers", Z), ("heads", Z), ("width", Z), ("block_size", Z), ("vocab", Z),
        ("padded_vocab", Z), ("sequences", Z), ("length", Z),
        ("separate_buffers", I), ("backward", I),
    ]


class Gpt2ParameterInfo(ctypes.Structure):
    """flint_gpt2_parameter_info (ref flint.h:470-475)."""

    _fields_ = [("name", ctypes.c_char_p), ("data", P), ("rows", Z), ("cols", Z)]


# Every function flint.h declares: name -> (restype, argtypes).
class AdamwTensor(ctypes.Structure):
    """flint_adamw_tensor (include/flint/flint_train.h)."""
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("exp_avg", ctypes.c_void_p),
                ("exp_avg_sq", ctypes.c_void_p), ("param_half", ctypes.c_void_p), ("count", ctypes.c_size_t),
                ("weight_decay", ctypes.c_float)]


class AdamwOptions(ctypes.Structure):
    """flint_adamw_options (include/flint/flint_train.h)."""
    _fields_ = [("lr", ctypes.c_float), ("beta1", ctypes.c_float), ("beta2", ctypes.c_float),
                ("eps", ctypes.c_float), ("max_grad_norm", ctypes.c_float), ("growth_factor", ctypes.c_float),
                ("backoff_factor", ctypes.c_float), ("growth_interval", ctypes.c_int)]


class TrainState(ctypes.Structure):
    """flint_train_state (include/flint/flint_train.h), 32 bytes."""
    _fields_ = [("loss_scale", ctypes.c_float), ("growth_tracker", ctypes.c_int), ("step", ctypes.c_int),
                ("found_inf", ctypes.c_int), ("grad_norm", ctypes.c_double), ("clip_coef", ctypes.c_double)]


SIGNATURES = {
    "flint_version": (ctypes.c_char_p, []),
    "flint_status_string": (ctypes.c_char_p, [I]),
    "flint_last_error": (ctypes.c_char_p, []),
    "flint_copy": (I, [P, P, Z, P]),
    "flint_adamw_defaults": (I, [ctypes.POINTER(AdamwOptions)]),
    "flint_train_state_init": (I, [P, ctypes.c_float, P]),
    "flint_adamw_workspace": (I, [ctypes.POINTER(AdamwTensor), Z, ctypes.POINTER(Z)]),
    "flint_adamw_step": (I, [ctypes.POINTER(AdamwTensor), Z, P, ctypes.POINTER(AdamwOptions), P, Z, P]),
    "flint_gemm_nt": (I, [P, P, P, Z, Z, Z, P]),
    "flint_gemm_nt_bias": (I, [P, P, P, P, Z, Z, Z, P]),
    "flint_gemm_nt_bias_gelu": (I, [P, P, P, P, P, Z, Z, Z, P]),
    "flint_gemm_nt_bias_residual": (I, [P, P, P, P, P, Z, Z, Z, P]),
    "flint_gemm_nn": (I, [P, P, P, Z, Z, Z, P]),
    "flint_gemm_nn_dgelu": (I, [P, P, P, P, Z, Z, Z, P]),
    "flint_gemm_tn": (I, [P, P, P, Z, Z, Z, I, P, Z, P]),
    "flint_gemm_tn_workspace": (I, [Z, Z, Z, ctypes.POINTER(Z)]),
    "flint_bias_gradient": (I, [P, P, Z, Z, I, P, Z, P]),
    "flint_bias_gradient_workspace": (I, [Z, Z, ctypes.POINTER(Z)]),
    # flint_noalloc.h (no counterpart in the reference)
    "flint_bias_gradient_noalloc": (I, [P, P, Z, Z, I, P]),
    # flint_attention.h (no counterpart in the reference's ABI)
    "flint_attention_forward": (I, [P, P, P, P, P, Z, Z, Z, F, P]),
    "flint_attention_backward_workspace": (I, [Z, Z, Z, ctypes.POINTER(Z)]),
    "flint_attention_backward": (I, [P, P, P, P, P, P, P, P, P, Z, Z, Z, F, P, Z, P]),
    "flint_gpt2_bytes_fused": (I, [ctypes.POINTER(Gpt2Config), ctypes.POINTER(Z)]),
    "flint_gpt2_create_fused": (I, [ctypes.POINTER(Gpt2Config), ctypes.POINTER(P)]),
    # flint_tuning.h (no counterpart in the reference)
    "flint_set_tuning": (I, [ctypes.c_char_p, ctypes.c_char_p]),
    "flint_gemm_nt_batched": (I, [P, P, P, Z, Z, Z, Z, F, P]),
    "flint_gemm_nn_batched": (I, [P, P, P, Z, Z, Z, Z, P]),
    "flint_gemm_tn_batched": (I, [P, P, P, Z, Z, Z, Z, P]),
    "flint_layernorm_forward": (I, [P, P, P, P, P, P, Z, Z, F, P]),
    "flint_layernorm_backward": (I, [P, P, P, P, P, P, P, P, Z, Z, I, I, P, Z, P]),
    "flint_layernorm_backward_workspace": (I, [Z, Z, ctypes.POINTER(Z)]),
    "flint_embedding_forward": (I, [P, P, P, P, Z, Z, Z, Z, P]),
    "flint_embedding_backward": (I, [P, P, P, P, Z, Z, Z, Z, I, I, P, Z, P]),
    "flint_embedding_backward_workspace": (I, [Z, Z, Z, Z, ctypes.POINTER(Z)]),
    "flint_fp32_to_fp16": (I, [P, P, Z, P]),
    "flint_heads_split": (I, [P, P, Z, Z, Z, Z, Z, Z, P]),
    "flint_heads_merge": (I, [P, P, Z, Z, Z, Z, Z, Z, P]),
    "flint_causal_softmax_forward": (I, [P, P, Z, Z, P]),
    "flint_causal_softmax_backward": (I, [P, P, P, Z, Z, F, P]),
    "flint_softmax_cross_entropy": (I, [P, P, P, P, F, Z, Z, Z, P]),
    "flint_gpt2_bytes": (I, [ctypes.POINTER(Gpt2Config), ctypes.POINTER(Z)]),
    "flint_gpt2_create": (I, [ctypes.POINTER(Gpt2Config), ctypes.POINTER(P)]),
    "flint_gpt2_destroy": (None, [P]),
    "flint_gpt2_parameter_count": (Z, [P]),
    "flint_gpt2_parameter": (I, [P, Z, ctypes.POINTER(Gpt2ParameterInfo)]),
    "flint_gpt2_sync_weights": (I, [P, P]),
    "flint_gpt2_forward": (I, [P, P, P, F, P]),
    "flint_gpt2_backward": (I, [P, P, I, P]),
    "flint_gpt2_gradient": (I, [P, Z, ctypes.POINTER(Gpt2ParameterInfo)]),
    "flint_gpt2_outputs": (I, [P, ctypes.POINTER(P), ctypes.POINTER(P), ctypes.POINTER(P)]),
    "flint_gpt2_mean_loss": (I, [P, P, ctypes.POINTER(ctypes.c_double)]),
}


class FlintError(RuntimeError):
    """A call returned a status other than FLINT_OK."""

    def __init__(self, status, message):
        super().__init__(message)
        self.status = status


def pointer(value):
    if value is None or isinstance(value, int):
        return value
    return value.data_ptr()


def stream_handle(stream):
    if isinstance(stream, int):
        return stream
    import torch

    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream


def library_path():
    override = os.environ.get("FLINT_LIB")
    return Path(override) if override else LIBRARY


class Flint:
    """The loaded library with every C signature declared."""

    def __init__(self, path=None):
        self.path = Path(path) if path else library_path()
        if not self.path.is_file():
            raise FileNotFoundError(
                f"{self.path} not found; build it with `python -c 'import __graft_entry__ as g; "
                "g.build()'` or `make -C flint_amd`"
            )
        self.lib = ctypes.CDLL(str(self.path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.restype = restype
            fn.argtypes = argtypes

    # -- status -------------------------------------------------------------
    def version(self):
        return self.lib.flint_version().decode()

    def status_string(self, status):
        return self.lib.flint_status_string(status).decode()

    def last_error(self):
        return self.lib.flint_last_error().decode()

    def check(self, status):
        if status != OK:
            message = f"{self.status_string(status)} (status {status})"
            detail = self.last_error()
            raise FlintError(status, f"{message}: {detail}" if detail else message)

    # -- GEMMs ----------------------------------------------------------------
    def set_tuning(self, name, value):
        """Forces (value a string) or clears (None) one plan override."""
        self.check(self.lib.flint_set_tuning(
            name.encode(), None if value is None else str(value).encode()))

    def tuned(self, **overrides):
        """A context in which the given plan overrides hold; each is cleared on
        exit (the library starts with none set)."""
        import contextlib

        @contextlib.contextmanager
        def scope():
            try:
                for name, value in overrides.items():
                    self.set_tuning(name, value)
                yield self
            finally:
                for name in overrides:
                    self.set_tuning(name, None)

        return scope()

    def copy(self, dst, src, nbytes, stream=None):
        self.check(self.lib.flint_copy(pointer(dst), pointer(src), nbytes, stream_handle(stream)))

    # -- training step (flint_train.h) -------------------------------------------
    def adamw_defaults(self):
        o = AdamwOptions()
        self.check(self.lib.flint_adamw_defaults(ctypes.byref(o)))
        return o

    @staticmethod
    def adamw_tensors(tensors):
        """dicts of param, grad, exp_avg, exp_avg_sq (FP32 tensors or addresses),
        optional param_half, count and weight_decay -> a flint_adamw_tensor array."""
        arr = (AdamwTensor * max(len(tensors), 1))()
        for i, t in enumerate(tensors):
            arr[i] = AdamwTensor(pointer(t["param"]), pointer(t["grad"]), pointer(t["exp_avg"]),
                                 pointer(t["exp_avg_sq"]), pointer(t.get("param_half")),
                                 t["count"] if "count" in t else t["param"].numel(), t.get("weight_decay", 0.0))
        return arr

    def train_state_init(self, state, loss_scale, stream=None):
        self.check(self.lib.flint_train_state_init(pointer(state), loss_scale, stream_handle(stream)))

    def adamw_workspace(self, tensors):
        out = Z(0)
        self.check(self.lib.flint_adamw_workspace(self.adamw_tensors(tensors), len(tensors), ctypes.byref(out)))
        return out.value

    def adamw_step(self, tensors, state, options, workspace, workspace_bytes=None, stream=None):
        nbytes = workspace.numel() * workspace.element_size() if workspace_bytes is None else workspace_bytes
        self.check(self.lib.flint_adamw_step(self.adamw_tensors(tensors), len(tensors), pointer(state),
                                             ctypes.byref(options), pointer(workspace), nbytes,
                                             stream_handle(stream)))

    def gemm_nt(self, y, x, w, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nt(pointer(y), pointer(x), pointer(w), m, n, k,
                                          stream_handle(stream)))

    def gemm_nt_bias(self, y, x, w, bias, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nt_bias(pointer(y), pointer(x), pointer(w), pointer(bias),
                                               m, n, k, stream_handle(stream)))

    def gemm_nt_bias_gelu(self, y, pre, x, w, bias, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nt_bias_gelu(pointer(y), pointer(pre), pointer(x),
                                                    pointer(w), pointer(bias), m, n, k,
                                                    stream_handle(stream)))

    def gemm_nt_bias_residual(self, y, x, w, bias, residual, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nt_bias_residual(pointer(y), pointer(x), pointer(w),
                                                        pointer(bias), pointer(residual), m, n, k,
                                                        stream_handle(stream)))

    def gemm_nn(self, y, x, w, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nn(pointer(y), pointer(x), pointer(w), m, n, k,
                                          stream_handle(stream)))

    def gemm_nn_dgelu(self, y, x, w, pre, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nn_dgelu(pointer(y), pointer(x), pointer(w), pointer(pre),
                                                m, n, k, stream_handle(stream)))

    def gemm_tn_workspace(self, m, n, k):
        out = Z(0)
        self.check(self.lib.flint_gemm_tn_workspace(m, n, k, ctypes.byref(out)))
        return out.value

    def gemm_tn(self, y, x, w, m, n, k, accumulate=False, workspace=None, workspace_bytes=None,
                stream=None):
        """y (+)= x^T w. Allocates the workspace with torch when none is given."""
        if workspace is None:
            need = self.gemm_tn_workspace(m, n, k)
            if need:
                import torch

                workspace = torch.empty(need, dtype=torch.uint8, device="cuda")
        if workspace_bytes is None:
            workspace_bytes = 0 if workspace is None or isinstance(workspace, int) else (
                workspace.numel() * workspace.element_size())
        self.check(self.lib.flint_gemm_tn(pointer(y), pointer(x), pointer(w), m, n, k,
                                          int(bool(accumulate)), pointer(workspace),
                                          workspace_bytes, stream_handle(stream)))

    def gemm_nt_batched(self, y, x, w, batches, m, n, k, scale=1.0, stream=None):
        self.check(self.lib.flint_gemm_nt_batched(pointer(y), pointer(x), pointer(w), batches, m,
                                                  n, k, scale, stream_handle(stream)))

    def gemm_nn_batched(self, y, x, w, batches, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_nn_batched(pointer(y), pointer(x), pointer(w), batches, m,
                                                  n, k, stream_handle(stream)))

    def gemm_tn_batched(self, y, x, w, batches, m, n, k, stream=None):
        self.check(self.lib.flint_gemm_tn_batched(pointer(y), pointer(x), pointer(w), batches, m,
                                                  n, k, stream_handle(stream)))

    # -- reductions -----------------------------------------------------------
    def bias_gradient_workspace(self, rows, cols):
        out = Z(0)
        self.check(self.lib.flint_bias_gradient_workspace(rows, cols, ctypes.byref(out)))
        return out.value

    def attention_forward(self, o, lse, q, k, v, batches, length, head_width, scale, stream=None):
        self.check(self.lib.flint_attention_forward(pointer(o), pointer(lse), pointer(q), pointer(k),
                                                    pointer(v), batches, length, head_width, scale,
                                                    stream_handle(stream)))

    def attention_backward_workspace(self, batches, length, head_width):
        out = Z(0)
        self.check(self.lib.flint_attention_backward_workspace(batches, length, head_width,
                                                               ctypes.byref(out)))
        return out.value

    def attention_backward(self, dq, dk, dv, dout, q, k, v, o, lse, batches, length, head_width,
                           scale, workspace=None, workspace_bytes=None, stream=None):
        if workspace is None:
            import torch

            workspace = torch.empty(max(self.attention_backward_workspace(batches, length,
                                                                          head_width), 16),
                                    dtype=torch.uint8, device="cuda")
        if workspace_bytes is None:
            workspace_bytes = workspace.numel() * workspace.element_size()
        self.check(self.lib.flint_attention_backward(
            pointer(dq), pointer(dk), pointer(dv), pointer(dout), pointer(q), pointer(k),
            pointer(v), pointer(o), pointer(lse), batches, length, head_width, scale,
            pointer(workspace), workspace_bytes, stream_handle(stream)))

    def bias_gradient_noalloc(self, dbias, dy, rows, cols, accumulate=False, stream=None):
        """flint_bias_gradient with the library's own scratch array (no workspace)."""
        self.check(self.lib.flint_bias_gradient_noalloc(pointer(dbias), pointer(dy), rows, cols,
                                                        int(bool(accumulate)), stream_handle(stream)))

    def bias_gradient(self, dbias, dy, rows, cols, accumulate=False, workspace=None,
                      workspace_bytes=None, stream=None):
        if workspace is None:
            import torch

            workspace = torch.empty(max(self.bias_gradient_workspace(rows, cols), 16),
                                    dtype=torch.uint8, device="cuda")
        if workspace_bytes is None:
            workspace_bytes = workspace.numel() * workspace.element_size()
        self.check(self.lib.flint_bias_gradient(pointer(dbias), pointer(dy), rows, cols,
                                                int(bool(accumulate)), pointer(workspace),
                                                workspace_bytes, stream_handle(stream)))

    def layernorm_forward(self, y, mean, rstd, x, gamma, beta, rows, cols, eps=1e-5,
                          stream=None):
        self.check(self.lib.flint_layernorm_forward(pointer(y), pointer(mean), pointer(rstd),
                                                    pointer(x), pointer(gamma), pointer(beta),
                                                    rows, cols, eps, stream_handle(stream)))

    def layernorm_backward_workspace(self, rows, cols):
        out = Z(0)
        self.check(self.lib.flint_layernorm_backward_workspace(rows, cols, ctypes.byref(out)))
        return out.value

    def layernorm_backward(self, dx, dgamma, dbeta, dy, x, mean, rstd, gamma, rows, cols,
                           accumulate_dx=False, accumulate_params=False, workspace=None,
                           workspace_bytes=None, stream=None):
        if workspace is None:
            import torch

            workspace = torch.empty(max(self.layernorm_backward_workspace(rows, cols), 16),
                                    dtype=torch.uint8, device="cuda")
        if workspace_bytes is None:
            workspace_bytes = workspace.numel() * workspace.element_size()
        self.check(self.lib.flint_layernorm_backward(
            pointer(dx), pointer(dgamma), pointer(dbeta), pointer(dy), pointer(x), pointer(mean),
            pointer(rstd), pointer(gamma), rows, cols, int(bool(accumulate_dx)),
            int(bool(accumulate_params)), pointer(workspace), workspace_bytes,
            stream_handle(stream)))

    def causal_softmax_forward(self, p, s, batches, length, stream=None):
        self.check(self.lib.flint_causal_softmax_forward(pointer(p), pointer(s), batches, length,
                                                         stream_handle(stream)))

    def causal_softmax_backward(self, ds, p, dp, batches, length, scale=1.0, stream=None):
        self.check(self.lib.flint_causal_softmax_backward(pointer(ds), pointer(p), pointer(dp),
                                                          batches, length, scale,
                                                          stream_handle(stream)))

    def softmax_cross_entropy(self, dlogits, row_loss, logits, targets, scale, rows, vocab, cols,
                              stream=None):
        self.check(self.lib.flint_softmax_cross_entropy(pointer(dlogits), pointer(row_loss),
                                                        pointer(logits), pointer(targets), scale,
                                                        rows, vocab, cols, stream_handle(stream)))

    # -- data movement --------------------------------------------------------
    def fp32_to_fp16(self, y, x, count, stream=None):
        self.check(self.lib.flint_fp32_to_fp16(pointer(y), pointer(x), count,
                                               stream_handle(stream)))

    def heads_split(self, y, x, batches, length, heads, head_width, row_width, first,
                    stream=None):
        self.check(self.lib.flint_heads_split(pointer(y), pointer(x), batches, length, heads,
                                              head_width, row_width, first, stream_handle(stream)))

    def heads_merge(self, y, x, batches, length, heads, head_width, row_width, first,
                    stream=None):
        self.check(self.lib.flint_heads_merge(pointer(y), pointer(x), batches, length, heads,
                                              head_width, row_width, first, stream_handle(stream)))

    def embedding_forward(self, x, tokens, wte, wpe, sequences, length, vocab, width,
                          stream=None):
        self.check(self.lib.flint_embedding_forward(pointer(x), pointer(tokens), pointer(wte),
                                                    pointer(wpe), sequences, length, vocab, width,
                                                    stream_handle(stream)))

    def embedding_backward_workspace(self, sequences, length, vocab, width):
        out = Z(0)
        self.check(self.lib.flint_embedding_backward_workspace(sequences, length, vocab, width,
                                                               ctypes.byref(out)))
        return out.value

    def embedding_backward(self, dwte, dwpe, dx, tokens, sequences, length, vocab, width,
                           accumulate_wte=False, accumulate_wpe=False, workspace=None,
                           workspace_bytes=None, stream=None):
        if workspace is None:
            import torch

            need = self.embedding_backward_workspace(sequences, length, vocab, width)
            workspace = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
        if workspace_bytes is None:
            workspace_bytes = workspace.numel() * workspace.element_size()
        self.check(self.lib.flint_embedding_backward(
            pointer(dwte), pointer(dwpe), pointer(dx), pointer(tokens), sequences, length, vocab,
            width, int(bool(accumulate_wte)), int(bool(accumulate_wpe)), pointer(workspace),
            workspace_bytes, stream_handle(stream)))


class Gpt2:
    """A flint_gpt2 model through the C ABI (ref tests/flint_lib.py's Gpt2 helper):
    parameters and gradients are (name, device address, rows, cols) and move in
    and out of torch tensors with flint_copy. fused=True creates the model with
    the fused attention (flint_gpt2_create_fused, flint_attention.h)."""

    def __init__(self, flint, layers, heads, width, block_size, vocab, padded_vocab, sequences,
                 length, separate_buffers=False, backward=True, fused=False):
        self.flint = flint
        self.fused = bool(fused)
        self.config = Gpt2Config(layers, heads, width, block_size, vocab, padded_vocab,
                                 sequences, length, int(bool(separate_buffers)),
                                 int(bool(backward)))
        self.handle = P()
        create = flint.lib.flint_gpt2_create_fused if self.fused else flint.lib.flint_gpt2_create
        flint.check(create(ctypes.byref(self.config), ctypes.byref(self.handle)))

    def close(self):
        if self.handle:
            self.flint.lib.flint_gpt2_destroy(self.handle)
            self.handle = P()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def bytes(self):
        out = Z(0)
        fn = self.flint.lib.flint_gpt2_bytes_fused if self.fused else self.flint.lib.flint_gpt2_bytes
        self.flint.check(fn(ctypes.byref(self.config), ctypes.byref(out)))
        return out.value

    def _infos(self, fn):
        n = self.flint.lib.flint_gpt2_parameter_count(self.handle)
        out = []
        for i in range(n):
            info = Gpt2ParameterInfo()
            self.flint.check(fn(self.handle, i, ctypes.byref(info)))
            out.append((info.name.decode(), info.data, info.rows, info.cols))
        return out

    def parameters(self):
        return self._infos(self.flint.lib.flint_gpt2_parameter)

    def gradients(self):
        return self._infos(self.flint.lib.flint_gpt2_gradient)

    def write(self, address, tensor, stream=None):
        """Copies a contiguous device tensor to a model address."""
        self.flint.copy(address, tensor, tensor.numel() * tensor.element_size(), stream)

    def read(self, address, shape, dtype, stream=None):
        """A new device tensor holding a copy of model memory."""
        import torch

        out = torch.empty(shape, dtype=dtype, device="cuda")
        self.flint.copy(out, address, out.numel() * out.element_size(), stream)
        return out

    def sync_weights(self, stream=None):
        self.flint.check(self.flint.lib.flint_gpt2_sync_weights(self.handle,
                                                                stream_handle(stream)))

    def forward(self, tokens, targets, scale, stream=None):
        self.flint.check(self.flint.lib.flint_gpt2_forward(
            self.handle, pointer(tokens), pointer(targets), scale, stream_handle(stream)))

    def backward(self, tokens, accumulate=False, stream=None):
        self.flint.check(self.flint.lib.flint_gpt2_backward(
            self.handle, pointer(tokens), int(bool(accumulate)), stream_handle(stream)))

    def outputs(self):
        """(logits, dlogits, row_loss) device addresses."""
        lg, dl, rl = P(), P(), P()
        self.flint.check(self.flint.lib.flint_gpt2_outputs(
            self.handle, ctypes.byref(lg), ctypes.byref(dl), ctypes.byref(rl)))
        return lg.value, dl.value, rl.value

    def mean_loss(self, stream=None):
        out = ctypes.c_double(0.0)
        self.flint.check(self.flint.lib.flint_gpt2_mean_loss(self.handle, stream_handle(stream),
                                                             ctypes.byref(out)))
        return out.value


def declared_functions(header=None):
    """Names of every FLINT_API function a header declares; by default those of
    flint.h and of the training-step extension, flint_train.h."""
    import re

    headers = ([header] if header is not None
               else [HEADER, TRAIN_HEADER, NOALLOC_HEADER, ATTENTION_HEADER, TUNING_HEADER])
    text = "".join(Path(h).read_text() for h in headers)
    return re.findall(r"FLINT_API\s+[^;(]*?\b(flint_\w+)\s*\(", text)

"""libflint for MI355X: GPT-2's training hot path (GEMM family, LayerNorm,
softmax, cross-entropy) as gfx950 HIP kernels behind Flint's C ABI.

The product is the shared library build/release/bin/libflint.so (built from
flint_amd/csrc by flint_amd/Makefile); flint_amd.flint_lib binds it with
ctypes.
"""

"""The fused RBF-attention operator on MI355X.

Importing vectra_amd.kernels (or vectra_amd.kernels.custom_ops) loads the
native libraries and registers torch.ops.vectra.rbf_attention, as importing
vectra_kernels.custom_ops does in the reference
(kernels/vectra_kernels/__init__.py:17).
"""

from vectra_amd.kernels import custom_ops  # noqa: F401  (registers the op)

"""torch.ops.vectra.rbf_attention on MI355X.

Same operator as the reference's kernels/vectra_kernels/custom_ops.py:52-97 (op :52-72, 'cuda' kernel :75-85, fake :88-97):

  out = torch.ops.vectra.rbf_attention(q, k, v, scale, key_bias=None)

  q [B, H, Nq, D], k [B, H, Nk, D], v [B, H, Nk, Dv] (float32, float16 or
  bfloat16, one dtype, any strides); scale broadcastable to [B, H, 1, 1];
  key_bias optional, broadcastable to [B, 1|H, 1, Nk] (0 or -inf for padded
  keys); returns softmax(-scale * ||q - k||^2 + key_bias) @ v as a new
  contiguous [B, H, Nq, Dv] tensor in v's dtype.

The schema, the CUDA-key implementation (HIP tensors on ROCm; it calls
libvectra_rbf.so on the current stream) and the CPU implementation live in
the C++ extension vectra_amd/csrc/ext/rbf_op.cpp.  This module loads it and
registers the fake (meta) implementation used while tracing.
"""

import torch

from vectra_amd.kernels import _native

OP_NAME = 'vectra::rbf_attention'

_native.load_torch_extension()


def hip_available() -> bool:
    """Whether the fused HIP path can run here (a GPU is visible)."""
    return torch.cuda.is_available()


@torch.library.register_fake(OP_NAME)
def _rbf_attention_fake(q, k, v, scale, key_bias=None):
    """Shape and dtype only (custom_ops.py:88-97): (*q.shape[:-1], Dv), v.dtype."""
    del k, scale, key_bias  # Only the output shape matters while tracing.
    return q.new_empty((*q.shape[:-1], v.shape[-1]), dtype=v.dtype)


def overload() -> torch._ops.OpOverload:
    """The operator's default overload, the node target a graph rewrite
    emits (defined once this module has loaded the extension)."""
    return torch.ops.vectra.rbf_attention.default


def rbf_attention(q, k, v, scale, key_bias=None):
    """Python-level alias of torch.ops.vectra.rbf_attention."""
    return torch.ops.vectra.rbf_attention(q, k, v, scale, key_bias)

"""vectra_amd: MI355X-native (gfx950) fused RBF attention for Vectra.

Subpackages mirror the reference's packages on the operator's path:

* vectra_amd.kernels            -- kernels/vectra_kernels (the operator
  torch.ops.vectra.rbf_attention, backed by the HIP library libvectra_rbf.so);
* vectra_amd.compiler           -- compiler/vectra_compiler (the `vectra`
  TorchDynamo backend that rewrites eager RBF attention into the operator);
* vectra_amd.price_transformer  -- models/price_transformer (the model whose
  attention sites the backend rewrites);
* vectra_amd.benchmarks         -- kernels/benchmarks (analytic traffic model
  and timing helpers).

Importing vectra_amd.kernels registers the operator.
"""

__version__ = '0.1.0'

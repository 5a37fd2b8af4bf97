"""The compiler pass that injects the fused operator.

Importing vectra_amd.compiler.backend registers the `vectra` TorchDynamo
backend:

  model = torch.compile(model, backend='vectra')
"""

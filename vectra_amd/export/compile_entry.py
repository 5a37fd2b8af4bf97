"""Compiles a checkpoint for serving and writes a release bundle.

  python -m vectra_amd.export.compile_entry --checkpoint-dir ckpt --out bundle \\
      [--device cuda] [--batch-size 1024] [--block-dtype bfloat16]

Restates the reference's models/export/compile_entry.py:145-355 on this
build: the model is compiled with the `vectra` backend (one graph, every
attention site rewritten to vectra::rbf_attention, which runs the HIP
kernels on the GPU), and the compiled model must match the eager model
(allclose, rtol 1e-3 / atol 1e-3, on seeded serving-shape batches) before the
bundle is written.  torch.compile is a just-in-time compiler, so a bundle
holds the verified inputs to compilation -- weights, architecture, serving
shape and precision, toolchain versions -- with checksums; `load_bundle`
recompiles at start-up and re-runs the same gates before serving.
"""

import argparse
import dataclasses
import hashlib
import json
import os
import platform
import shutil
import time

import numpy as np
import torch

from vectra_amd.compiler import backend
from vectra_amd.price_transformer import checkpoint
from vectra_amd.price_transformer import model as model_lib

FORMAT_VERSION = 1
MANIFEST = 'compile_manifest.json'
# The numerics gate: compiled must match eager at rtol 1e-3.
RTOL = 1e-3
ATOL = 1e-3


class NumericsError(RuntimeError):
    """The compiled model disagrees with the eager model."""


@dataclasses.dataclass(frozen=True)
class ServingSpec:
    """The shape and precision the model is compiled for."""

    device: str
    batch_size: int
    block_dtype: str

    @property
    def dtype(self) -> torch.dtype:
        return getattr(torch, self.block_dtype)


def default_block_dtype(device: str) -> str:
    """float16 blocks on the GPU (the reference's default), float32 on CPU."""
    return 'float16' if torch.device(device).type == 'cuda' else 'float32'


def toolchain_versions() -> dict[str, str]:
    """Versions that must match between export and serving."""
    from vectra_amd.kernels import capi  # pylint: disable=import-outside-toplevel

    versions = {
        'python': platform.python_version(),
        'torch': torch.__version__,
        'numpy': np.__version__,
        'hip': str(torch.version.hip),
        'vectra_rbf_abi': '%d.%d' % capi.abi_version(),
    }
    try:
        import triton  # pylint: disable=import-outside-toplevel

        versions['triton'] = triton.__version__
    except ImportError:
        versions['triton'] = 'unavailable'
    return versions


def _sha256(path: str) -> str:
    digest = hashlib.sha256()
    with open(path, 'rb') as f:
        for block in iter(lambda: f.read(1 << 22), b''):
            digest.update(block)
    return digest.hexdigest()


def prepare(model: model_lib.PriceTransformer, spec: ServingSpec) -> model_lib.PriceTransformer:
    """Moves `model` to the serving device and block precision (in place)."""
    model = model.to(spec.device).eval()
    if spec.dtype != torch.float32:
        model.set_block_dtype(spec.dtype)
    return model


def max_abs_error(compiled, eager, config: model_lib.ModelConfig, spec: ServingSpec, batches: int,
                  reference=None) -> tuple[float, float]:
    """Gates compiled-vs-eager numerics on seeded serving-shape batches.

    Returns (worst |compiled - eager|, worst |compiled - reference|), the
    reference being the fp32 eager model (0.0 without one).  Raises
    NumericsError when compiled and eager disagree beyond RTOL / ATOL.
    """
    worst, drift = 0.0, 0.0
    with torch.no_grad():
        for seed in range(batches):
            inputs = model_lib.example_inputs(config, spec.batch_size, spec.device, seed=1000 + seed)
            got = compiled(*inputs).float()
            want = eager(*inputs).float()
            error = (got - want).abs().max().item()
            if not torch.allclose(got, want, rtol=RTOL, atol=ATOL):
                raise NumericsError(
                    f'compiled model differs from eager by up to {error:.3g} '
                    f'(rtol {RTOL}, atol {ATOL}) on seeded batch {seed}'
                )
            worst = max(worst, error)
            if reference is not None:
                drift = max(drift, (got - reference(*inputs).float()).abs().max().item())
    return worst, drift


def compile_model(model: model_lib.PriceTransformer, spec: ServingSpec):
    """(compiled model, CompileReport, compile seconds) for a prepared model."""
    inputs = model_lib.example_inputs(model.config, spec.batch_size, spec.device)
    start = time.perf_counter()
    compiled, report = backend.compile_for_serving(model, tuple(inputs),
                                                   expected_sites=model.config.num_layers)
    return compiled, report, time.perf_counter() - start


def _device_name(device: str) -> str:
    if torch.device(device).type == 'cuda':
        return torch.cuda.get_device_name(device)
    return platform.processor() or platform.machine()


def export_bundle(checkpoint_dir: str, out_dir: str, spec: ServingSpec, numerics_batches: int = 4) -> dict:
    """Compiles, verifies and writes `out_dir`; returns the manifest."""
    eager = prepare(checkpoint.load(checkpoint_dir), spec)
    compiled, report, seconds = compile_model(eager, spec)
    reference = checkpoint.load(checkpoint_dir, spec.device) if spec.dtype != torch.float32 else None
    worst, drift = max_abs_error(compiled, eager, eager.config, spec, numerics_batches, reference)
    os.makedirs(out_dir, exist_ok=True)
    files = {}
    for name in (checkpoint.WEIGHTS, checkpoint.CONFIG):
        shutil.copyfile(os.path.join(checkpoint_dir, name), os.path.join(out_dir, name))
        files[name] = _sha256(os.path.join(out_dir, name))
    manifest = {
        'format_version': FORMAT_VERSION,
        'files': files,
        'model': dataclasses.asdict(eager.config),
        'serving': dataclasses.asdict(spec) | {'device_name': _device_name(spec.device)},
        'compile': {
            'backend': backend.BACKEND_NAME,
            'expected_sites': eager.config.num_layers,
            'sites': report.sites,
            'matches': report.matches,
            'graph_count': report.graph_count,
            'graph_break_count': report.graph_break_count,
            'seconds': round(seconds, 3),
        },
        'numerics': {
            'rtol': RTOL,
            'atol': ATOL,
            'batches': numerics_batches,
            'max_abs_error_vs_eager': worst,
            'max_abs_error_vs_float32_eager': drift,
        },
        'versions': toolchain_versions(),
    }
    with open(os.path.join(out_dir, MANIFEST), 'w', encoding='utf-8') as f:
        json.dump(manifest, f, indent=2, sort_keys=True)
        f.write('\n')
    return manifest


class ServingModel:
    """A compiled model plus the padding that keeps its shape static.

    The model is compiled for exactly `batch_size` requests, so a smaller
    batch is padded with copies of its last request and a larger one is
    split; padding rows are dropped from the result.
    """

    def __init__(self, compiled, config: model_lib.ModelConfig, spec: ServingSpec, manifest: dict):
        self.compiled = compiled
        self.config = config
        self.spec = spec
        self.manifest = manifest

    def predict(self, inputs: model_lib.PricingInputs) -> torch.Tensor:
        """Predicted log prices [n] for a batch of any size n >= 1."""
        n = inputs.query_embedding.shape[0]
        b = self.spec.batch_size
        outputs = []
        with torch.no_grad():
            for start in range(0, n, b):
                chunk = [t[start:start + b].to(self.spec.device) for t in inputs]
                size = chunk[0].shape[0]
                if size < b:
                    chunk = [torch.cat([t, t[-1:].expand(b - size, *t.shape[1:])]) for t in chunk]
                outputs.append(self.compiled(*chunk)[:size].float())
        return torch.cat(outputs)


def load_bundle(bundle_dir: str, device: str | None = None, strict_versions: bool = True) -> ServingModel:
    """Recompiles a bundle and re-verifies it before serving.

    `device` overrides the bundle's device (its precision is then that
    device's default).  Raises ValueError for a corrupt bundle or a toolchain
    mismatch, NumericsError when the recompiled model disagrees with eager,
    and the compiler's PatternNotFoundError / GraphBreakError when the
    rewrite does not apply.
    """
    with open(os.path.join(bundle_dir, MANIFEST), encoding='utf-8') as f:
        manifest = json.load(f)
    if manifest.get('format_version') != FORMAT_VERSION:
        raise ValueError(f'unsupported bundle format in {bundle_dir}')
    for name, digest in manifest['files'].items():
        if _sha256(os.path.join(bundle_dir, name)) != digest:
            raise ValueError(f'{name} does not match its manifest checksum')
    exported = manifest['versions']
    if strict_versions and exported != toolchain_versions():
        raise ValueError(f'toolchain {toolchain_versions()} differs from the export toolchain '
                         f'{exported}; re-export the bundle')
    serving = manifest['serving']
    spec = ServingSpec(
        device=device or serving['device'],
        batch_size=serving['batch_size'],
        block_dtype=serving['block_dtype'] if device is None else default_block_dtype(device),
    )
    model = prepare(checkpoint.load(bundle_dir), spec)
    compiled, _, _ = compile_model(model, spec)
    max_abs_error(compiled, model, model.config, spec, batches=1)
    return ServingModel(compiled, model.config, spec, manifest)


def main(argv=None) -> None:
    p = argparse.ArgumentParser(description='Compile and verify a price-model checkpoint for serving.')
    p.add_argument('--checkpoint-dir', required=True)
    p.add_argument('--out', required=True)
    p.add_argument('--device', default='cuda' if torch.cuda.is_available() else 'cpu')
    p.add_argument('--batch-size', type=int, default=64)
    p.add_argument('--block-dtype', choices=['float32', 'float16', 'bfloat16'], default=None)
    p.add_argument('--numerics-batches', type=int, default=4)
    args = p.parse_args(argv)
    spec = ServingSpec(args.device, args.batch_size, args.block_dtype or default_block_dtype(args.device))
    manifest = export_bundle(args.checkpoint_dir, args.out, spec, args.numerics_batches)
    print(json.dumps({'out': args.out, 'compile': manifest['compile'], 'numerics': manifest['numerics']},
                     sort_keys=True))


if __name__ == '__main__':
    main()

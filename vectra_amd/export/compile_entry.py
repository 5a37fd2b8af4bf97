"""Release bundles for the price model: compile, prove, package, reload.

  python -m vectra_amd.export.compile_entry --checkpoint-dir ckpt --out bundle \\
      [--device cuda] [--batch-size 1024] [--block-dtype bfloat16]

A bundle is a directory holding the checkpoint's two files and a manifest:

  model.safetensors, model_config.json   the checkpoint, copied
  compile_manifest.json                  what was built and the evidence

torch.compile compiles just in time, so a bundle carries no compiled code.
It carries the inputs to compilation (weights, architecture, serving shape
and precision) and a toolchain fingerprint, each file with its SHA-256.  Two
gates decide whether a compiled model may serve, both when the bundle is
exported and again when a serving host loads it:

* the compile gate: TorchDynamo captures the model as one graph and the
  `vectra` backend rewrites one attention site per Transformer block to
  vectra::rbf_attention (the HIP kernels on the GPU);
* the numerics gate: on seeded batches of the serving shape, every output of
  the compiled model lies within |compiled - eager| <= ATOL + RTOL * |eager|
  of the eager model in the same precision.

Reference behaviour: models/export/compile_entry.py:145-355 (export, gates,
manifest fields, padded prediction).
"""

import argparse
import dataclasses
import hashlib
import json
import os
import platform
import tempfile
import time

import numpy as np
import torch

from vectra_amd.compiler import backend
from vectra_amd.price_transformer import checkpoint
from vectra_amd.price_transformer import model as model_lib

FORMAT_VERSION = 1
MANIFEST = 'compile_manifest.json'
RTOL = 1e-3
ATOL = 1e-3

# Seeds of the numerics gate's batches: batch i is example_inputs(seed=base + i).
_GATE_SEED_BASE = 1000
_BLOCK_DTYPES = {'float32': torch.float32, 'float16': torch.float16, 'bfloat16': torch.bfloat16}
_COPY_BLOCK = 4 << 20


class NumericsError(RuntimeError):
    """The compiled model's outputs leave the numerics gate."""


class BundleError(ValueError):
    """A bundle directory that must not be served as it is."""


@dataclasses.dataclass(frozen=True)
class ServingSpec:
    """Where and how the model is compiled: device, static batch, block dtype."""

    device: str
    batch_size: int
    block_dtype: str

    def __post_init__(self):
        if self.block_dtype not in _BLOCK_DTYPES:
            raise ValueError(f'block_dtype must be one of {sorted(_BLOCK_DTYPES)}, not {self.block_dtype!r}')
        if self.batch_size < 1:
            raise ValueError(f'batch_size must be positive, not {self.batch_size}')

    @classmethod
    def for_device(cls, device: str, batch_size: int, block_dtype: str | None = None) -> 'ServingSpec':
        return cls(device, batch_size, block_dtype or default_block_dtype(device))

    @property
    def dtype(self) -> torch.dtype:
        return _BLOCK_DTYPES[self.block_dtype]


def default_block_dtype(device: str) -> str:
    """Half-precision blocks on a GPU, full precision on the host."""
    return 'float16' if torch.device(device).type == 'cuda' else 'float32'


def toolchain_versions() -> dict[str, str]:
    """The fingerprint a serving host must share with the exporting host.

    Inductor generates code for the parts of the model around the attention
    sites (Triton on the GPU), so its version is part of the fingerprint as
    well as torch's, HIP's and the C ABI of the attention library.
    """
    from vectra_amd.kernels import capi  # pylint: disable=import-outside-toplevel

    try:
        import triton  # pylint: disable=import-outside-toplevel
        triton_version = triton.__version__
    except ImportError:
        triton_version = 'unavailable'
    major, minor = capi.abi_version()
    return {
        'python': platform.python_version(),
        'torch': torch.__version__,
        'numpy': np.__version__,
        'hip': str(torch.version.hip),
        'vectra_rbf_abi': f'{major}.{minor}',
        'triton': triton_version,
    }


def _file_digest(path: str) -> str:
    digest = hashlib.sha256()
    with open(path, 'rb') as f:
        while chunk := f.read(_COPY_BLOCK):
            digest.update(chunk)
    return digest.hexdigest()


def _copy_and_digest(src: str, dst: str) -> str:
    """Copies `src` to `dst` and returns the SHA-256 of the bytes written, in
    one pass over the data."""
    digest = hashlib.sha256()
    with open(src, 'rb') as fin, open(dst, 'wb') as fout:
        while chunk := fin.read(_COPY_BLOCK):
            digest.update(chunk)
            fout.write(chunk)
    return digest.hexdigest()


def _write_json_atomically(path: str, payload: dict) -> None:
    """The manifest appears complete or not at all: a half-written manifest
    would otherwise read as a corrupt bundle."""
    directory = os.path.dirname(os.path.abspath(path))
    fd, tmp = tempfile.mkstemp(prefix='.manifest-', dir=directory)
    try:
        with os.fdopen(fd, 'w', encoding='utf-8') as f:
            json.dump(payload, f, indent=2, sort_keys=True)
            f.write('\n')
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise


def prepare(model: model_lib.PriceTransformer, spec: ServingSpec) -> model_lib.PriceTransformer:
    """Puts `model` (in place) on the serving device, in eval mode, with its
    Transformer blocks in the serving precision."""
    model = model.to(spec.device).eval()
    if spec.dtype is not torch.float32:
        model.set_block_dtype(spec.dtype)
    return model


def _largest_gap(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a - b).abs().max()) if a.numel() else 0.0


def max_abs_error(compiled, eager, config: model_lib.ModelConfig, spec: ServingSpec, batches: int,
                  reference=None) -> tuple[float, float]:
    """Runs the numerics gate over `batches` seeded serving-shape batches.

    Returns (largest |compiled - eager|, largest |compiled - reference|); the
    second is 0.0 without a `reference` (the fp32 eager model, reported but
    not gated).  Raises NumericsError at the first batch where an output of
    `compiled` leaves ATOL + RTOL * |eager| (NaN never passes).
    """
    vs_eager = vs_reference = 0.0
    with torch.no_grad():
        for i in range(batches):
            inputs = model_lib.example_inputs(config, spec.batch_size, spec.device, seed=_GATE_SEED_BASE + i)
            got = compiled(*inputs).float()
            want = eager(*inputs).float()
            gap = _largest_gap(got, want)
            within = torch.isclose(got, want, rtol=RTOL, atol=ATOL)
            if not bool(within.all()):
                bad = int((~within).sum())
                raise NumericsError(
                    f'gate batch {i}: {bad} of {within.numel()} outputs of the compiled model differ from '
                    f'eager by more than {ATOL:g} + {RTOL:g}*|eager| (largest gap {gap:.3g})')
            vs_eager = max(vs_eager, gap)
            if reference is not None:
                vs_reference = max(vs_reference, _largest_gap(got, reference(*inputs).float()))
    return vs_eager, vs_reference


def compile_model(model: model_lib.PriceTransformer, spec: ServingSpec):
    """Compiles a prepared model at the serving shape through the compile
    gate; returns (compiled model, CompileReport, seconds spent)."""
    shape_inputs = tuple(model_lib.example_inputs(model.config, spec.batch_size, spec.device))
    began = time.perf_counter()
    compiled, report = backend.compile_for_serving(model, shape_inputs, expected_sites=model.config.num_layers)
    return compiled, report, time.perf_counter() - began


def _device_label(device: str) -> str:
    if torch.device(device).type == 'cuda':
        return torch.cuda.get_device_name(device)
    return platform.processor() or platform.machine()


def export_bundle(checkpoint_dir: str, out_dir: str, spec: ServingSpec, numerics_batches: int = 4) -> dict:
    """Compiles the checkpoint for `spec`, passes both gates, and writes the
    bundle to `out_dir`.  Returns the manifest that was written."""
    eager = prepare(checkpoint.load(checkpoint_dir), spec)
    compiled, report, seconds = compile_model(eager, spec)
    fp32 = checkpoint.load(checkpoint_dir, spec.device) if spec.dtype is not torch.float32 else None
    vs_eager, vs_fp32 = max_abs_error(compiled, eager, eager.config, spec, numerics_batches, fp32)

    os.makedirs(out_dir, exist_ok=True)
    digests = {name: _copy_and_digest(os.path.join(checkpoint_dir, name), os.path.join(out_dir, name))
               for name in (checkpoint.WEIGHTS, checkpoint.CONFIG)}
    manifest = {
        'format_version': FORMAT_VERSION,
        'files': digests,
        'model': dataclasses.asdict(eager.config),
        'serving': {**dataclasses.asdict(spec), 'device_name': _device_label(spec.device)},
        'compile': {
            'backend': backend.BACKEND_NAME,
            'expected_sites': eager.config.num_layers,
            'sites': report.sites,
            'matches': dict(report.matches),
            'graph_count': report.graph_count,
            'graph_break_count': report.graph_break_count,
            'seconds': round(seconds, 3),
        },
        'numerics': {
            'rtol': RTOL,
            'atol': ATOL,
            'batches': numerics_batches,
            'max_abs_error_vs_eager': vs_eager,
            'max_abs_error_vs_float32_eager': vs_fp32,
        },
        'versions': toolchain_versions(),
    }
    _write_json_atomically(os.path.join(out_dir, MANIFEST), manifest)
    return manifest


class ServingModel:
    """A compiled model behind a request-count-agnostic predict().

    The compiled graph takes exactly `spec.batch_size` rows.  predict() walks
    the requests in windows of that size; each window is gathered with one
    index_select per input field whose indices run past the last request
    clamped to it, so a short window is padded with copies of its last
    request and the padded rows are dropped from the result.
    """

    def __init__(self, compiled, config: model_lib.ModelConfig, spec: ServingSpec, manifest: dict):
        self.compiled = compiled
        self.config = config
        self.spec = spec
        self.manifest = manifest

    def predict(self, inputs: model_lib.PricingInputs) -> torch.Tensor:
        """Log prices [n] for n >= 1 requests, in request order."""
        n = int(inputs.query_embedding.shape[0])
        rows = self.spec.batch_size
        fields = [t.to(self.spec.device) for t in inputs]
        results = torch.empty(n, dtype=torch.float32, device=self.spec.device)
        with torch.no_grad():
            for first in range(0, n, rows):
                live = min(rows, n - first)
                index = torch.arange(first, first + rows, device=self.spec.device).clamp_(max=n - 1)
                window = [t.index_select(0, index) for t in fields]
                results[first:first + live] = self.compiled(*window)[:live].float()
        return results


def _read_manifest(bundle_dir: str) -> dict:
    path = os.path.join(bundle_dir, MANIFEST)
    try:
        with open(path, encoding='utf-8') as f:
            manifest = json.load(f)
    except (OSError, json.JSONDecodeError) as e:
        raise BundleError(f'{path} is missing or unreadable: {e}') from e
    if manifest.get('format_version') != FORMAT_VERSION:
        raise BundleError(f'{bundle_dir} has bundle format {manifest.get("format_version")!r}; '
                          f'this build reads format {FORMAT_VERSION}')
    return manifest


def _check_files(bundle_dir: str, manifest: dict) -> None:
    for name, recorded in sorted(manifest['files'].items()):
        path = os.path.join(bundle_dir, name)
        if not os.path.exists(path) or _file_digest(path) != recorded:
            raise BundleError(f'{name} in {bundle_dir} fails its manifest checksum (SHA-256)')


def _check_toolchain(manifest: dict) -> None:
    here, there = toolchain_versions(), manifest['versions']
    changed = {k: (there.get(k), here.get(k)) for k in sorted(set(here) | set(there)) if here.get(k) != there.get(k)}
    if changed:
        listed = ', '.join(f'{k}: {a} at export, {b} here' for k, (a, b) in changed.items())
        raise BundleError(f'toolchain differs from the one the bundle was exported with ({listed}); '
                          're-export the bundle or load it with strict_versions=False')


def load_bundle(bundle_dir: str, device: str | None = None, strict_versions: bool = True) -> ServingModel:
    """Checks a bundle, recompiles it and re-runs both gates before serving.

    `device` moves the bundle to another device, in that device's default
    block precision.  Raises BundleError (a ValueError) for an unknown format,
    a file that fails its checksum or, with strict_versions, a different
    toolchain; NumericsError when the recompiled model leaves the numerics
    gate; the compiler's PatternNotFoundError / GraphBreakError when the
    compile gate fails.
    """
    manifest = _read_manifest(bundle_dir)
    _check_files(bundle_dir, manifest)
    if strict_versions:
        _check_toolchain(manifest)
    recorded = manifest['serving']
    if device is None:
        spec = ServingSpec(recorded['device'], recorded['batch_size'], recorded['block_dtype'])
    else:
        spec = ServingSpec.for_device(device, recorded['batch_size'])
    model = prepare(checkpoint.load(bundle_dir), spec)
    compiled, _, _ = compile_model(model, spec)
    max_abs_error(compiled, model, model.config, spec, batches=1)
    return ServingModel(compiled, model.config, spec, manifest)


def main(argv=None) -> None:
    parser = argparse.ArgumentParser(description='Compile a price-model checkpoint, gate it and write a bundle.')
    parser.add_argument('--checkpoint-dir', required=True, help='directory written by checkpoint.save')
    parser.add_argument('--out', required=True, help='bundle directory to write')
    parser.add_argument('--device', default='cuda' if torch.cuda.is_available() else 'cpu')
    parser.add_argument('--batch-size', type=int, default=64, help='static serving batch')
    parser.add_argument('--block-dtype', choices=sorted(_BLOCK_DTYPES), default=None,
                        help='Transformer-block precision (default: float16 on a GPU, float32 on the host)')
    parser.add_argument('--numerics-batches', type=int, default=4, help='seeded batches the gate compares')
    args = parser.parse_args(argv)
    spec = ServingSpec.for_device(args.device, args.batch_size, args.block_dtype)
    manifest = export_bundle(args.checkpoint_dir, args.out, spec, args.numerics_batches)
    print(json.dumps({'bundle': args.out, 'compile': manifest['compile'], 'numerics': manifest['numerics']},
                     sort_keys=True))


if __name__ == '__main__':
    main()

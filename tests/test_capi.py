"""The C ABI library loads, exports what include/vectra_rbf.h declares, and
validates its arguments on the host.  No kernel is launched here."""

import ctypes
import os
import re

import pytest
import torch

from vectra_amd.kernels import _native
from vectra_amd.kernels import capi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'include', 'vectra_rbf.h')


def _declared_functions() -> set[str]:
    text = open(HEADER, encoding='utf-8').read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return set(re.findall(r'^\s*(?:const\s+)?\w+\s*\*?\s*(vectra_\w+)\s*\(', text, flags=re.M))


def test_header_declares_the_bound_functions():
    assert _declared_functions() == set(capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_native.HIP_LIBRARY)
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    assert capi.abi_version() == (1, 3)
    for status in range(9):
        assert capi.status_string(status)
    assert capi.status_string(capi.OK) == 'ok'
    assert capi.status_string(99) == 'unknown status'


def _fake_args(dtype=torch.bfloat16, b=4, h=8, n_q=1, n_k=64, d=32, dv=32, *,
               out_dtype=None, base=1 << 20, variant='auto', contiguous=True):
    """Arguments with fake (never dereferenced) device addresses."""
    a = capi.RbfArgs()
    a.struct_size = ctypes.sizeof(capi.RbfArgs)
    a.q, a.k, a.v, a.out, a.scale = base, base + (1 << 16), base + (2 << 16), base + (3 << 16), base + (4 << 16)
    a.key_bias = None
    a.in_dtype = capi.DTYPES[dtype]
    a.out_dtype = capi.DTYPES[out_dtype or dtype]
    a.scale_dtype = capi.F32
    a.bias_dtype = capi.F32
    a.batch, a.heads, a.n_q, a.n_k, a.head_dim, a.value_dim = b, h, n_q, n_k, d, dv
    if contiguous:
        a.q_stride = (ctypes.c_int64 * 4)(h * n_q * d, n_q * d, d, 1)
        a.k_stride = (ctypes.c_int64 * 4)(h * n_k * d, n_k * d, d, 1)
        a.v_stride = (ctypes.c_int64 * 4)(h * n_k * dv, n_k * dv, dv, 1)
    else:  # head-transposed views of a [B, N, 3*H*D] projection
        a.q_stride = (ctypes.c_int64 * 4)(n_q * 3 * h * d, d, 3 * h * d, 1)
        a.k_stride = (ctypes.c_int64 * 4)(n_k * 3 * h * d, d, 3 * h * d, 1)
        a.v_stride = (ctypes.c_int64 * 4)(n_k * 3 * h * d, d, 3 * h * d, 1)
    a.out_stride = (ctypes.c_int64 * 4)(h * n_q * dv, n_q * dv, dv, 1)
    a.scale_stride_b, a.scale_stride_h = 0, 1
    a.variant = capi.VARIANTS[variant]
    return a


def test_struct_layout_is_accepted():
    assert ctypes.sizeof(capi.RbfArgs) == 296
    assert capi.select_variant(_fake_args()) > 0
    bad = _fake_args()
    bad.struct_size -= 8
    assert capi.select_variant(bad) == -capi.ERR_BAD_STRUCT


@pytest.mark.parametrize(
    'kwargs,variant',
    [
        ({}, 'stream'),  # the serving shape
        ({'dtype': torch.float32, 'd': 16, 'dv': 16, 'n_k': 32}, 'stream'),  # config 1
        ({'out_dtype': torch.float32}, 'stream'),
        ({'d': 16, 'dv': 16, 'contiguous': False}, 'stream'),  # model views, 16-B rows
        ({'d': 24, 'dv': 24}, 'generic'),  # 3 chunks: not a power of two
        ({'d': 32, 'dv': 16}, 'generic'),  # D != Dv
        ({'d': 7, 'dv': 7}, 'generic'),
        ({'base': (1 << 20) + 2}, 'generic'),  # misaligned rows
        ({'n_q': 65, 'n_k': 65}, 'plane'),  # self-attention over a comparable set
        ({'n_q': 65, 'n_k': 65, 'dtype': torch.float32}, 'plane'),  # the same in fp32
        ({'n_q': 65, 'n_k': 65, 'dtype': torch.float16, 'out_dtype': torch.float32}, 'plane'),
        ({'n_q': 65, 'n_k': 65, 'd': 16, 'dv': 16, 'contiguous': False}, 'plane'),  # model sites
        ({'n_q': 100, 'n_k': 100}, 'tile'),  # past one plane tile for 32-dim heads
        ({'n_q': 100, 'n_k': 100, 'd': 16, 'dv': 16}, 'plane'),  # 16-dim heads: tiles of 128
        ({'n_q': 200, 'n_k': 200, 'd': 16, 'dv': 16}, 'mfma'),  # 16-dim heads past 128 rows
        ({'n_q': 100, 'n_k': 100, 'dtype': torch.float32}, 'mfma'),  # fp32 past one plane tile
        ({'n_q': 65, 'n_k': 65, 'dtype': torch.float32, 'out_dtype': torch.bfloat16}, 'generic'),
        ({'n_q': 65, 'n_k': 65, 'd': 64, 'dv': 64}, 'tile'),
        ({'n_q': 4096, 'n_k': 4096, 'd': 64, 'dv': 64}, 'tile'),  # long key axis
        ({'n_q': 4096, 'n_k': 4096, 'd': 64, 'dv': 64, 'dtype': torch.float32}, 'mfma'),
        ({'n_q': 65, 'n_k': 65, 'd': 48, 'dv': 48}, 'generic'),  # no MFMA tile for 48 dims
        ({'n_q': 15, 'n_k': 65}, 'stream'),  # under one query tile: rows stream two key tiles
    ],
)
def test_variant_selection(kwargs, variant):
    assert capi.VARIANT_NAMES[capi.select_variant(_fake_args(**kwargs))] == variant


def test_negative_key_row_strides_go_to_the_generic_kernel():
    """The stream, plane, tile and MFMA kernels address key rows through
    unsigned 32-bit offsets within a plane; K, V or bias rows walked
    backwards (negative strides, which the ABI accepts) take the kernel with
    64-bit signed addressing."""
    for n in (64, 65, 100):
        assert capi.VARIANT_NAMES[capi.select_variant(_fake_args(n_q=n if n > 64 else 1, n_k=n))] != 'generic'
        for name, dim in (('k_stride', 32), ('v_stride', 32)):
            a = _fake_args(n_q=n if n > 64 else 1, n_k=n)
            setattr(a, name, (ctypes.c_int64 * 4)(8 * n * dim, n * dim, -dim, 1))
            assert capi.VARIANT_NAMES[capi.select_variant(a)] == 'generic', (n, name)
        a = _fake_args(n_q=n if n > 64 else 1, n_k=n)
        a.key_bias, a.bias_stride_b, a.bias_stride_h, a.bias_stride_n = (1 << 20) + (5 << 16), n, 0, -1
        assert capi.VARIANT_NAMES[capi.select_variant(a)] == 'generic', (n, 'bias')
        for variant in ('stream', 'plane', 'tile', 'mfma'):
            a = _fake_args(n_q=n if n > 64 else 1, n_k=n, variant=variant)
            a.k_stride = (ctypes.c_int64 * 4)(8 * n * 32, n * 32, -32, 1)
            assert capi.select_variant(a) == -capi.ERR_BAD_VARIANT, (n, variant)


def test_plane_kernel_needs_disjoint_rows_within_32_bit_offsets():
    """The plane kernel reads K and V through buffer extents that end at the
    last row, so rows past Nk read as zeros only when rows do not overlap; and
    its offsets span up to 144 rows."""
    assert capi.VARIANT_NAMES[capi.select_variant(_fake_args(n_q=65, n_k=65))] == 'plane'
    h, n, d = 8, 65, 32
    for name, row_stride in (('k_stride', 0), ('v_stride', 0), ('k_stride', 16), ('v_stride', 24)):
        a = _fake_args(n_q=n, n_k=n)
        setattr(a, name, (ctypes.c_int64 * 4)(h * n * 64, n * 64, row_stride, 1))
        assert capi.VARIANT_NAMES[capi.select_variant(a)] != 'plane', (name, row_stride)
    a = _fake_args(n_q=n, n_k=n)
    far = 1 << 24  # 144 rows of 32 MiB overflow 32-bit offsets
    a.q_stride = (ctypes.c_int64 * 4)(h * n * far, n * far, far, 1)
    assert capi.VARIANT_NAMES[capi.select_variant(a)] != 'plane'


@pytest.mark.parametrize('n,variant', [(65, 'plane'), (100, 'tile')])
def test_output_views_past_4_gib_of_a_plane_go_to_64_bit_kernels(n, variant):
    """The plane and tile kernels store through 32-bit byte offsets from a
    plane's first output element, so they take a strided output only while
    its last element lies within 4 GiB of the first: at 2^30 elements for an
    fp32 output, 2^31 for a 16-bit one.  Larger views go to a kernel with
    64-bit addressing."""
    h, dv = 8, 32

    def with_out_rows(row, out_dtype):
        a = _fake_args(n_q=n, n_k=n, out_dtype=out_dtype)
        a.out_stride = (ctypes.c_int64 * 4)(h * n * row, n * row, row, 1)
        return capi.VARIANT_NAMES[capi.select_variant(a)]

    # Last element offset (n - 1) * row + dv - 1, in elements.
    fits_f32 = (((1 << 30) - dv) // (n - 1))  # below 2^30 elements
    past_f32 = -(-((1 << 30) - dv + 1) // (n - 1))  # at or past 2^30 elements
    assert (n - 1) * fits_f32 + dv - 1 < (1 << 30) <= (n - 1) * past_f32 + dv - 1
    assert with_out_rows(fits_f32, torch.float32) == variant
    assert with_out_rows(past_f32, torch.float32) not in ('plane', 'tile')
    assert with_out_rows(past_f32, torch.bfloat16) == variant  # 2-byte elements: 2^31
    past_16 = -(-((1 << 31) - dv + 1) // (n - 1))
    assert with_out_rows(past_16, torch.bfloat16) not in ('plane', 'tile')


def test_sizes_beyond_the_kernels_index_range_are_rejected():
    for field, value in (('batch', 1 << 31), ('n_k', 1 << 40), ('value_dim', 1 << 31)):
        a = _fake_args()
        setattr(a, field, value)
        assert capi.select_variant(a) == -capi.ERR_TOO_LARGE, field
    a = _fake_args(d=1 << 24, dv=(65535 * 256) + 1)  # one more 256-column slice than the grid holds
    assert capi.select_variant(a) == -capi.ERR_TOO_LARGE
    a = _fake_args(b=1 << 12, h=1 << 12, n_q=1 << 8)  # 2^32 rows
    assert capi.select_variant(a) == -capi.ERR_TOO_LARGE
    lib = _native.hip_library()
    strides = (ctypes.c_int64 * 4)(0, 0, 0, 1)
    big = 1 << 40
    assert lib.vectra_rbf_squared_norms(1, 0, big, big, 2, 1, strides, 1, None) == capi.ERR_TOO_LARGE


def test_forcing_a_variant_that_cannot_run_is_an_error():
    a = _fake_args(d=24, dv=24, variant='stream')
    assert capi.select_variant(a) == -capi.ERR_BAD_VARIANT
    assert capi.select_variant(_fake_args(variant='generic')) == capi.VARIANTS['generic']


@pytest.mark.parametrize(
    'field,value,status',
    [
        ('in_dtype', 3, capi.ERR_BAD_DTYPE),  # f64 q/k/v
        ('out_dtype', 9, capi.ERR_BAD_DTYPE),
        ('scale_dtype', -1, capi.ERR_BAD_DTYPE),
        ('n_k', -1, capi.ERR_BAD_SHAPE),
        ('q', None, capi.ERR_NULL_ARGUMENT),
        ('scale', None, capi.ERR_NULL_ARGUMENT),
        ('variant', 11, capi.ERR_BAD_VARIANT),
        ('flags', 2, capi.ERR_BAD_FLAGS),
        ('flags', -1, capi.ERR_BAD_FLAGS),
    ],
)
def test_invalid_arguments_are_rejected_before_any_launch(field, value, status):
    a = _fake_args()
    setattr(a, field, value)
    assert capi.select_variant(a) == -status
    lib = _native.hip_library()
    assert lib.vectra_rbf_attention_fwd(ctypes.byref(a), None) == status


def test_the_split_weights_flag_is_accepted_by_every_variant():
    for variant in ('auto', 'generic', 'stream'):
        a = _fake_args(variant=variant)
        a.flags = capi.FLAG_SPLIT_WEIGHTS
        assert capi.select_variant(a) > 0, variant


def test_empty_problems_are_a_no_op():
    lib = _native.hip_library()
    for field in ('batch', 'heads', 'n_q', 'value_dim'):
        a = _fake_args()
        setattr(a, field, 0)
        a.q = a.k = a.v = a.out = a.scale = None  # never touched
        assert lib.vectra_rbf_attention_fwd(ctypes.byref(a), None) == capi.OK
    assert lib.vectra_rbf_attention_fwd(None, None) == capi.ERR_NULL_ARGUMENT


def test_squared_norms_validates_on_the_host():
    lib = _native.hip_library()
    strides = (ctypes.c_int64 * 4)(0, 0, 0, 1)
    assert lib.vectra_rbf_squared_norms(None, 7, 1, 1, 1, 1, strides, None, None) == capi.ERR_BAD_DTYPE
    assert lib.vectra_rbf_squared_norms(None, 0, 1, -1, 1, 1, strides, None, None) == capi.ERR_BAD_SHAPE
    assert lib.vectra_rbf_squared_norms(None, 0, 0, 1, 1, 1, strides, None, None) == capi.OK
    assert lib.vectra_rbf_squared_norms(None, 0, 1, 1, 1, 1, strides, None, None) == capi.ERR_NULL_ARGUMENT



_MISSING_SCRIPT = r'''
import importlib
for module in ('vectra_amd.kernels', 'vectra_amd.kernels.capi'):
    try:
        importlib.import_module(module)
        print(module, 'imported')
    except ImportError as e:
        print(module, type(e).__name__, e)
'''


def test_a_missing_library_fails_loudly(tmp_path):
    """A copy of the Python package without the built libraries: neither the
    operator nor the C-ABI bindings import, so there is no CPU fallback to
    land on."""
    import shutil
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    shutil.copytree(os.path.join(root, 'vectra_amd'), tmp_path / 'vectra_amd',
                    ignore=shutil.ignore_patterns('lib', 'csrc', '__pycache__'))
    env = dict(os.environ, PYTHONPATH=str(tmp_path))
    env.pop('VECTRA_LIB_DIR', None)  # the copy's own (absent) library directory
    done = subprocess.run([sys.executable, '-c', _MISSING_SCRIPT], cwd=tmp_path, capture_output=True, text=True,
                          timeout=300, env=env)
    assert done.returncode == 0, done.stderr
    lines = done.stdout.strip().splitlines()
    assert len(lines) == 2, lines
    for line in lines:
        assert ' NativeLibraryMissing ' in line, line
        assert 'libvectra_torch.so is missing' in line and 'make -C vectra_amd/csrc' in line, line

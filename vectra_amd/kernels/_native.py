"""Locates and loads the native libraries built in-tree.

* ``libvectra_rbf.so``   -- the C-ABI HIP library (include/vectra_rbf.h);
* ``libvectra_torch.so`` -- the torch.library extension that registers
  ``vectra::rbf_attention`` and links the first one;
* ``libvectra_scan.so``  -- the C-ABI distance scans (include/vectra_scan.h),
  used by vectra_amd.index.

All are produced by ``make -C vectra_amd/csrc`` (``__graft_entry__.build()``).
There is no fallback: if one is missing, the code that needs it fails.

``VECTRA_LIB_DIR`` names another directory holding the libraries; the
host-sanitizer build (``make -C vectra_amd/csrc sanitize-test``) uses it.
"""

import ctypes
import functools
import os

import torch

LIB_DIR = os.environ.get('VECTRA_LIB_DIR') or os.path.join(
    os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'lib')
HIP_LIBRARY = os.path.join(LIB_DIR, 'libvectra_rbf.so')
TORCH_LIBRARY = os.path.join(LIB_DIR, 'libvectra_torch.so')
SCAN_LIBRARY = os.path.join(LIB_DIR, 'libvectra_scan.so')


class NativeLibraryMissing(ImportError):
    """The native libraries have not been built."""


def _require(path: str) -> str:
    if not os.path.exists(path):
        raise NativeLibraryMissing(
            f'{path} is missing; build it with `make -C vectra_amd/csrc` '
            '(or __graft_entry__.build()).'
        )
    return path


@functools.cache
def load_torch_extension() -> str:
    """Loads the operator registration (once per process); returns its path."""
    torch.ops.load_library(_require(TORCH_LIBRARY))
    return TORCH_LIBRARY


@functools.cache
def hip_library() -> ctypes.CDLL:
    """The C-ABI library as a ctypes handle (shared with the extension)."""
    lib = ctypes.CDLL(_require(HIP_LIBRARY))
    lib.vectra_rbf_attention_fwd.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.vectra_rbf_attention_fwd.restype = ctypes.c_int
    lib.vectra_rbf_select_variant.argtypes = [ctypes.c_void_p]
    lib.vectra_rbf_select_variant.restype = ctypes.c_int
    lib.vectra_rbf_squared_norms.argtypes = [
        ctypes.c_void_p,
        ctypes.c_int32,
        ctypes.c_int64,
        ctypes.c_int64,
        ctypes.c_int64,
        ctypes.c_int64,
        ctypes.POINTER(ctypes.c_int64),
        ctypes.c_void_p,
        ctypes.c_void_p,
    ]
    lib.vectra_rbf_squared_norms.restype = ctypes.c_int
    lib.vectra_rbf_status_string.argtypes = [ctypes.c_int]
    lib.vectra_rbf_status_string.restype = ctypes.c_char_p
    lib.vectra_rbf_abi_version.argtypes = []
    lib.vectra_rbf_abi_version.restype = ctypes.c_int
    return lib


@functools.cache
def scan_library() -> ctypes.CDLL:
    """The distance-scan library as a ctypes handle."""
    lib = ctypes.CDLL(_require(SCAN_LIBRARY))
    for name in ('vectra_scan_rows', 'vectra_pq_distance_tables', 'vectra_scan_pq_adc', 'vectra_scan_top_k'):
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        fn.restype = ctypes.c_int
    lib.vectra_scan_top_k_ws.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    lib.vectra_scan_top_k_ws.restype = ctypes.c_int
    lib.vectra_scan_top_k_no_alloc.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.vectra_scan_top_k_no_alloc.restype = ctypes.c_int
    lib.vectra_scan_top_k_workspace_bytes.argtypes = [ctypes.c_void_p]
    lib.vectra_scan_top_k_workspace_bytes.restype = ctypes.c_int64
    lib.vectra_scan_status_string.argtypes = [ctypes.c_int]
    lib.vectra_scan_status_string.restype = ctypes.c_char_p
    lib.vectra_scan_abi_version.argtypes = []
    lib.vectra_scan_abi_version.restype = ctypes.c_int
    return lib


def loaded_libraries() -> list[str]:
    """In-tree native libraries mapped into this process (for audits)."""
    with open('/proc/self/maps', encoding='utf-8') as maps:
        paths = {line.split()[-1] for line in maps if LIB_DIR in line}
    return sorted(paths)

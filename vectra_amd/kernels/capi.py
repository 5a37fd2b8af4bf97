"""ctypes binding of the C ABI (include/vectra_rbf.h).

This is the binding a non-torch caller would write; the parity tests and the
benchmark use it to call libvectra_rbf.so directly, which also lets them ask
for an fp32 output from the same kernel the operator runs in v.dtype.
Tensors only supply device pointers, sizes and strides here.
"""

import ctypes

import torch

from vectra_amd.kernels import _native

# vectra_dtype
F32, F16, BF16, F64 = 0, 1, 2, 3
DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float64: F64}

# Status codes.
OK = 0
ERR_NULL_ARGUMENT = 1
ERR_BAD_DTYPE = 2
ERR_BAD_SHAPE = 3
ERR_BAD_STRUCT = 4
ERR_TOO_LARGE = 5
ERR_LAUNCH = 6
ERR_BAD_VARIANT = 7
ERR_BAD_FLAGS = 8
FLAG_SPLIT_WEIGHTS = 1  # VECTRA_FLAG_SPLIT_WEIGHTS

# Kernel variants.
VARIANTS = {'auto': 0, 'generic': 1, 'stream': 2, 'mfma': 3, 'plane': 4, 'tile': 5}
VARIANT_NAMES = {v: k for k, v in VARIANTS.items()}

# Exported functions, as declared in include/vectra_rbf.h.
EXPORTS = (
    'vectra_rbf_attention_fwd',
    'vectra_rbf_squared_norms',
    'vectra_rbf_select_variant',
    'vectra_rbf_status_string',
    'vectra_rbf_abi_version',
)

_I64x4 = ctypes.c_int64 * 4


class RbfArgs(ctypes.Structure):
    """struct vectra_rbf_args."""

    _fields_ = [
        ('struct_size', ctypes.c_int64),
        ('q', ctypes.c_void_p),
        ('k', ctypes.c_void_p),
        ('v', ctypes.c_void_p),
        ('out', ctypes.c_void_p),
        ('scale', ctypes.c_void_p),
        ('key_bias', ctypes.c_void_p),
        ('in_dtype', ctypes.c_int32),
        ('out_dtype', ctypes.c_int32),
        ('scale_dtype', ctypes.c_int32),
        ('bias_dtype', ctypes.c_int32),
        ('batch', ctypes.c_int64),
        ('heads', ctypes.c_int64),
        ('n_q', ctypes.c_int64),
        ('n_k', ctypes.c_int64),
        ('head_dim', ctypes.c_int64),
        ('value_dim', ctypes.c_int64),
        ('q_stride', _I64x4),
        ('k_stride', _I64x4),
        ('v_stride', _I64x4),
        ('out_stride', _I64x4),
        ('scale_stride_b', ctypes.c_int64),
        ('scale_stride_h', ctypes.c_int64),
        ('bias_stride_b', ctypes.c_int64),
        ('bias_stride_h', ctypes.c_int64),
        ('bias_stride_n', ctypes.c_int64),
        ('variant', ctypes.c_int32),
        ('flags', ctypes.c_int32),
    ]


class CapiError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, status: int):
        self.status = status
        text = _native.hip_library().vectra_rbf_status_string(status).decode()
        super().__init__(f'vectra C ABI status {status}: {text}')


def status_string(status: int) -> str:
    return _native.hip_library().vectra_rbf_status_string(status).decode()


def abi_version() -> tuple[int, int]:
    v = _native.hip_library().vectra_rbf_abi_version()
    return v >> 16, v & 0xFFFF


def broadcast_operands(q, k, scale, key_bias):
    """Broadcast views of scale [B,H,1,1] and key_bias [B,H,1,Nk] (or None).

    Same rules and errors as the operator (spatial_rbf_attention.py:208-236).
    """
    batch, heads = q.shape[0], q.shape[1]
    n_k = k.shape[2]
    scale4 = scale.expand(batch, heads, 1, 1)
    bias4 = None
    if key_bias is not None:
        bias4 = key_bias
        while bias4.dim() < 4:
            bias4 = bias4.unsqueeze(0)
        if bias4.shape[-2] != 1:
            raise ValueError('key_bias must be constant across queries')
        bias4 = bias4.expand(batch, heads, 1, n_k)
    return scale4, bias4


def make_args(q, k, v, out, scale4, bias4, variant: str = 'auto', flags: int = 0) -> RbfArgs:
    """Fills struct vectra_rbf_args from tensors (pointers, sizes, strides)."""
    a = RbfArgs()
    a.struct_size = ctypes.sizeof(RbfArgs)
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.scale = scale4.data_ptr()
    a.key_bias = bias4.data_ptr() if bias4 is not None else None
    a.in_dtype = DTYPES[q.dtype]
    a.out_dtype = DTYPES[out.dtype]
    a.scale_dtype = DTYPES[scale4.dtype]
    a.bias_dtype = DTYPES[bias4.dtype] if bias4 is not None else F32
    a.batch, a.heads, a.n_q, a.head_dim = q.shape
    a.n_k = k.shape[2]
    a.value_dim = v.shape[3]
    a.q_stride = _I64x4(*q.stride())
    a.k_stride = _I64x4(*k.stride())
    a.v_stride = _I64x4(*v.stride())
    a.out_stride = _I64x4(*out.stride())
    a.scale_stride_b, a.scale_stride_h = scale4.stride(0), scale4.stride(1)
    if bias4 is not None:
        a.bias_stride_b, a.bias_stride_h = bias4.stride(0), bias4.stride(1)
        a.bias_stride_n = bias4.stride(3)
    a.variant = VARIANTS[variant]
    a.flags = flags
    return a


def select_variant(a: RbfArgs) -> int:
    """vectra_rbf_select_variant (host only); negative = -status."""
    return _native.hip_library().vectra_rbf_select_variant(ctypes.byref(a))


def launch(a: RbfArgs, stream=None) -> None:
    """vectra_rbf_attention_fwd on `stream` (default: torch's current stream)."""
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    status = _native.hip_library().vectra_rbf_attention_fwd(ctypes.byref(a), stream)
    if status != OK:
        raise CapiError(status)


def forward(
    q,
    k,
    v,
    scale,
    key_bias=None,
    *,
    out_dtype=None,
    out=None,
    variant: str = 'auto',
    split_weights: bool = False,
    stream=None,
):
    """Runs the fused kernel through the C ABI; returns `out`.

    Args:
      q, k, v, scale, key_bias: as torch.ops.vectra.rbf_attention (GPU tensors).
      out_dtype: output dtype (default v.dtype); ignored when `out` is given.
      out: optional preallocated [B, H, Nq, Dv] output (any strides).
      variant: 'auto', 'generic', 'stream', 'mfma', 'plane' or 'tile'.
      split_weights: VECTRA_FLAG_SPLIT_WEIGHTS (the tile kernel keeps hi + lo
        weights on long key axes instead of its fp16-weight pass).
      stream: hipStream_t as an int (default: torch's current stream).
    """
    if not q.is_cuda:
        raise ValueError('capi.forward needs GPU tensors')
    if scale.device != q.device:
        scale = scale.to(q.device)
    scale4, bias4 = broadcast_operands(q, k, scale, key_bias)
    if out is None:
        out = torch.empty(
            (*q.shape[:-1], v.shape[-1]),
            dtype=out_dtype or v.dtype,
            device=q.device,
        )
    flags = FLAG_SPLIT_WEIGHTS if split_weights else 0
    launch(make_args(q, k, v, out, scale4, bias4, variant, flags), stream)
    return out


def squared_norms(x, stream=None):
    """vectra_rbf_squared_norms: fp32 [B, H, N] row norms of x [B, H, N, D]."""
    out = torch.empty(x.shape[:3], dtype=torch.float32, device=x.device)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    strides = _I64x4(*x.stride())
    status = _native.hip_library().vectra_rbf_squared_norms(
        x.data_ptr(), DTYPES[x.dtype], *x.shape, strides, out.data_ptr(), stream
    )
    if status != OK:
        raise CapiError(status)
    return out

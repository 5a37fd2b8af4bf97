"""Batched GPU distance scans over the C ABI of include/vectra_scan.h.

Each function computes many calls of one reference function at once and
returns what those calls return, bit for bit (the kernels keep the
reference's order of floating-point operations):

=======================  ==================================================
function                 reference (engine/src/index/...)
=======================  ==================================================
l2_squared_distances     L2SquaredDistance (simd_distance.cc:36-51), as
                         called per node by ShardIndex::ExhaustiveSearch
                         (shard_index.cc:244-264) and the re-rank
                         (hnsw_searcher.cc:145-158)
inner_products           InnerProduct (simd_distance.cc:53-62)
squared_norms            SquaredNorm (simd_distance.cc:64-66), as
                         FlatVectorStore computes per row (flat_store.cc:46)
pq_distance_tables       ProductQuantizer::ComputeDistanceTable
                         (pq_codec.cc:208-217)
pq_adc_distances         PqAdcDistance (simd_distance.cc:68-81), per code
                         (hnsw_searcher.h:74; tests/tools/index_study.cc:82)
nearest                  ShardIndex::ExhaustiveSearch's results
                         (shard_index.cc:236-264): the k nearest by
                         L2SquaredDistance in CloserFirst order
=======================  ==================================================

Arguments are torch tensors on the GPU: float32 vectors as [count, dimension]
with unit stride along the dimension (any row stride), uint8 codes as
[count, subspaces] with unit stride along the code, candidate ids as int32 or
uint32 [n].  A candidate id at or past the row count yields NaN.  Work goes
to torch's current stream; nothing is synchronised.  There is no CPU path:
the functions raise if the library is missing or a tensor is not on a GPU.
"""

import ctypes

import torch

from vectra_amd.kernels import _native

L2_SQUARED, INNER_PRODUCT, SQUARED_NORM = 0, 1, 2
PQ_CENTROIDS = 256
MAX_K = 1024            # VECTRA_SCAN_MAX_K
NO_NODE = 0xFFFFFFFF    # VECTRA_SCAN_NO_NODE: an empty result slot
_OK, _INVALID = 0, 1


class ScanError(RuntimeError):
    """A scan kernel could not be launched."""


class _ScanArgs(ctypes.Structure):
    _fields_ = [
        ('metric', ctypes.c_int32), ('dimension', ctypes.c_int32),
        ('queries', ctypes.c_void_p), ('num_queries', ctypes.c_int64), ('query_stride', ctypes.c_int64),
        ('rows', ctypes.c_void_p), ('num_rows', ctypes.c_int64), ('row_stride', ctypes.c_int64),
        ('ids', ctypes.c_void_p), ('num_ids', ctypes.c_int64),
        ('out', ctypes.c_void_p), ('out_stride', ctypes.c_int64),
    ]


class _PqTableArgs(ctypes.Structure):
    _fields_ = [
        ('dimension', ctypes.c_int32), ('subspaces', ctypes.c_int32),
        ('queries', ctypes.c_void_p), ('num_queries', ctypes.c_int64), ('query_stride', ctypes.c_int64),
        ('codebooks', ctypes.c_void_p),
        ('tables', ctypes.c_void_p), ('table_stride', ctypes.c_int64),
    ]


class _PqAdcArgs(ctypes.Structure):
    _fields_ = [
        ('subspaces', ctypes.c_int32),
        ('tables', ctypes.c_void_p), ('num_queries', ctypes.c_int64), ('table_stride', ctypes.c_int64),
        ('codes', ctypes.c_void_p), ('num_codes', ctypes.c_int64), ('code_stride', ctypes.c_int64),
        ('ids', ctypes.c_void_p), ('num_ids', ctypes.c_int64),
        ('out', ctypes.c_void_p), ('out_stride', ctypes.c_int64),
    ]


class _TopKArgs(ctypes.Structure):
    _fields_ = [
        ('dimension', ctypes.c_int32), ('k', ctypes.c_int32),
        ('queries', ctypes.c_void_p), ('num_queries', ctypes.c_int64), ('query_stride', ctypes.c_int64),
        ('rows', ctypes.c_void_p), ('num_rows', ctypes.c_int64), ('row_stride', ctypes.c_int64),
        ('ids', ctypes.c_void_p), ('num_ids', ctypes.c_int64),
        ('distances', ctypes.c_void_p), ('nodes', ctypes.c_void_p), ('out_stride', ctypes.c_int64),
    ]


def _check(status: int) -> None:
    if status == _OK:
        return
    text = _native.scan_library().vectra_scan_status_string(status).decode()
    if status == _INVALID:
        raise ValueError(f'vectra scan: {text}')
    raise ScanError(f'vectra scan: {text} (status {status})')


def _on_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f'{name} must be on a GPU (there is no CPU path)')


def _matrix(t: torch.Tensor, name: str, dtype: torch.dtype) -> torch.Tensor:
    _on_gpu(t, name)
    if t.dtype != dtype:
        raise ValueError(f'{name} must be {dtype}, got {t.dtype}')
    if t.dim() != 2:
        raise ValueError(f'{name} must be 2-D [count, width], got shape {tuple(t.shape)}')
    if t.shape[1] > 1 and t.stride(1) != 1:
        raise ValueError(f'{name} must have unit stride along its last dimension')
    return t


def _row_stride(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def _ids(ids, like: torch.Tensor):
    if ids is None:
        return None
    _on_gpu(ids, 'ids')
    if ids.dtype not in (torch.int32, torch.uint32) or ids.dim() != 1:
        raise ValueError('ids must be a 1-D int32 or uint32 tensor')
    if ids.device != like.device:
        raise ValueError('ids must be on the same device as the rows')
    return ids.contiguous()


# A NULL `ids` means every row to the C ABI, and the data pointer of an empty
# tensor is NULL: an empty candidate list is passed as this one-element
# buffer with a count of 0 (the library reads none of it).
_EMPTY_IDS = {}


def _ids_ptr(ids):
    """The C ABI's `ids` for a candidate tensor (None: every row)."""
    if ids is None:
        return None
    if ids.numel() > 0:
        return ids.data_ptr()
    dev = ids.device
    if dev not in _EMPTY_IDS:
        _EMPTY_IDS[dev] = torch.zeros(1, dtype=torch.int32, device=dev)
    return _EMPTY_IDS[dev].data_ptr()


def _out(out, shape, device) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=torch.float32, device=device)
    _on_gpu(out, 'out')
    if out.dtype != torch.float32 or tuple(out.shape) != tuple(shape):
        raise ValueError(f'out must be float32 of shape {tuple(shape)}')
    if shape[1] > 1 and out.stride(1) != 1:
        raise ValueError('out must have unit stride along its last dimension')
    return out


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _scan_rows(metric, queries, rows, ids, out):
    rows = _matrix(rows, 'rows', torch.float32)
    dim = rows.shape[1]
    if metric == SQUARED_NORM:
        num_queries, q_ptr, q_stride = 1, None, 0
    else:
        queries = _matrix(queries, 'queries', torch.float32)
        if queries.shape[1] != dim:
            raise ValueError(f'queries have {queries.shape[1]} dimensions, rows {dim}')
        if queries.device != rows.device:
            raise ValueError('queries and rows must be on the same device')
        num_queries, q_ptr, q_stride = queries.shape[0], queries.data_ptr(), _row_stride(queries)
    ids = _ids(ids, rows)
    count = rows.shape[0] if ids is None else ids.shape[0]
    out = _out(out, (num_queries, count), rows.device)
    args = _ScanArgs(metric, dim, q_ptr, num_queries, q_stride, rows.data_ptr(), rows.shape[0], _row_stride(rows),
                     _ids_ptr(ids), 0 if ids is None else ids.shape[0],
                     out.data_ptr(), out.stride(0) if num_queries > 1 else max(count, 1))
    with torch.cuda.device(rows.device):
        _check(_native.scan_library().vectra_scan_rows(ctypes.byref(args), _stream(rows.device)))
    return out


def l2_squared_distances(queries: torch.Tensor, rows: torch.Tensor, ids=None, out=None) -> torch.Tensor:
    """[num_queries, n] float32: L2SquaredDistance(query q, row ids[i] (or row i), dimension)."""
    return _scan_rows(L2_SQUARED, queries, rows, ids, out)


def inner_products(queries: torch.Tensor, rows: torch.Tensor, ids=None, out=None) -> torch.Tensor:
    """[num_queries, n] float32: InnerProduct(query q, row ids[i] (or row i), dimension)."""
    return _scan_rows(INNER_PRODUCT, queries, rows, ids, out)


def squared_norms(rows: torch.Tensor, out=None) -> torch.Tensor:
    """[n] float32: SquaredNorm(row i, dimension)."""
    view = None if out is None else out.view(1, -1)
    return _scan_rows(SQUARED_NORM, None, rows, None, view).view(-1)


def pq_distance_tables(queries: torch.Tensor, codebooks: torch.Tensor, subspaces: int, out=None) -> torch.Tensor:
    """[num_queries, subspaces * 256] float32 ADC tables (ComputeDistanceTable).

    `codebooks` is float32 [subspaces, 256, dimension / subspaces] (or any
    contiguous tensor of that many elements), the layout of
    ProductQuantizer::codebooks()."""
    queries = _matrix(queries, 'queries', torch.float32)
    _on_gpu(codebooks, 'codebooks')
    dim = queries.shape[1]
    if codebooks.dtype != torch.float32 or not codebooks.is_contiguous() or codebooks.numel() != dim * PQ_CENTROIDS:
        raise ValueError(f'codebooks must be contiguous float32 with {dim} * 256 elements')
    entries = subspaces * PQ_CENTROIDS
    out = _out(out, (queries.shape[0], entries), queries.device)
    args = _PqTableArgs(dim, subspaces, queries.data_ptr(), queries.shape[0], _row_stride(queries),
                        codebooks.data_ptr(), out.data_ptr(), out.stride(0) if queries.shape[0] > 1 else entries)
    with torch.cuda.device(queries.device):
        _check(_native.scan_library().vectra_pq_distance_tables(ctypes.byref(args), _stream(queries.device)))
    return out


def pq_adc_distances(tables: torch.Tensor, codes: torch.Tensor, ids=None, out=None) -> torch.Tensor:
    """[num_queries, n] float32: PqAdcDistance(table q, code ids[i] (or code i), subspaces)."""
    codes = _matrix(codes, 'codes', torch.uint8)
    subspaces = codes.shape[1]
    tables = _matrix(tables, 'tables', torch.float32)
    if tables.shape[1] != subspaces * PQ_CENTROIDS:
        raise ValueError(f'tables must have subspaces * 256 = {subspaces * PQ_CENTROIDS} columns')
    ids = _ids(ids, codes)
    count = codes.shape[0] if ids is None else ids.shape[0]
    out = _out(out, (tables.shape[0], count), codes.device)
    args = _PqAdcArgs(subspaces, tables.data_ptr(), tables.shape[0], _row_stride(tables),
                      codes.data_ptr(), codes.shape[0], _row_stride(codes),
                      _ids_ptr(ids), 0 if ids is None else ids.shape[0],
                      out.data_ptr(), out.stride(0) if tables.shape[0] > 1 else max(count, 1))
    with torch.cuda.device(codes.device):
        _check(_native.scan_library().vectra_scan_pq_adc(ctypes.byref(args), _stream(codes.device)))
    return out


def _top_k_args(queries, rows, k, ids, out):
    queries = _matrix(queries, 'queries', torch.float32)
    rows = _matrix(rows, 'rows', torch.float32)
    if queries.shape[1] != rows.shape[1]:
        raise ValueError('queries and rows must have the same dimension')
    if not 1 <= k <= MAX_K:
        raise ValueError(f'k must be in [1, {MAX_K}]')
    ids = _ids(ids, rows)
    n_q = queries.shape[0]
    if out is None:
        distances = torch.empty((n_q, k), dtype=torch.float32, device=rows.device)
        nodes = torch.empty((n_q, k), dtype=torch.uint32, device=rows.device)
    else:
        distances, nodes = out
        for t, dtype in ((distances, torch.float32), (nodes, torch.uint32)):
            _on_gpu(t, 'out')
            if t.dtype != dtype or tuple(t.shape) != (n_q, k) or not t.is_contiguous():
                raise ValueError(f'out must be contiguous ({n_q}, {k}) float32 and uint32 tensors')
    args = _TopKArgs(rows.shape[1], k, queries.data_ptr(), n_q, _row_stride(queries),
                     rows.data_ptr(), rows.shape[0], _row_stride(rows),
                     _ids_ptr(ids), 0 if ids is None else ids.shape[0],
                     distances.data_ptr(), nodes.data_ptr(), k)
    # The tensors the arguments point into stay referenced with them.
    return args, (queries, rows, ids), distances, nodes


TOP_K_FORMS = ('split', 'single', 'no_alloc')


def workspace_bytes(queries: torch.Tensor, rows: torch.Tensor, k: int, ids=None) -> int:
    """Device workspace bytes nearest(form='split') uses for these inputs
    (vectra_scan_top_k_workspace_bytes; 0: none)."""
    args, _keep, _d, _n = _top_k_args(queries, rows, k, ids, None)
    return int(_native.scan_library().vectra_scan_top_k_workspace_bytes(ctypes.byref(args)))


def nearest(queries: torch.Tensor, rows: torch.Tensor, k: int, ids=None, out=None, form='split', workspace=None):
    """ExhaustiveSearch for each query: (distances [num_queries, k] float32,
    nodes [num_queries, k] uint32), nearest first by (distance, node id).

    Candidates are rows ids[i] (ids not below the row count are skipped,
    duplicates kept) or every row; slots past the number of candidates hold
    +inf and NO_NODE.  k is 1 .. MAX_K.  `out` may give the two output
    tensors (contiguous, of those shapes and dtypes).

    `form` picks the entry point, all with the same results: 'split'
    (vectra_scan_top_k_ws: below 64 queries a query's candidates are spread
    over several workgroups; `workspace` is a uint8 CUDA tensor of at least
    workspace_bytes(...) whose first 256 bytes are zero before its first use,
    or None to allocate a zeroed one), 'single' (vectra_scan_top_k, one
    workgroup per query) or 'no_alloc' (vectra_scan_top_k_no_alloc, the
    split form on the library's own scratch)."""
    if form not in TOP_K_FORMS:
        raise ValueError(f'form must be one of {TOP_K_FORMS}')
    args, _keep, distances, nodes = _top_k_args(queries, rows, k, ids, out)
    lib = _native.scan_library()
    device = distances.device
    with torch.cuda.device(device):
        stream = _stream(device)
        if form == 'single':
            _check(lib.vectra_scan_top_k(ctypes.byref(args), stream))
        elif form == 'no_alloc':
            _check(lib.vectra_scan_top_k_no_alloc(ctypes.byref(args), stream))
        else:
            need = int(lib.vectra_scan_top_k_workspace_bytes(ctypes.byref(args)))
            if workspace is None:
                workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=device)
            _on_gpu(workspace, 'workspace')
            if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
                raise ValueError('workspace must be a contiguous uint8 tensor')
            _check(lib.vectra_scan_top_k_ws(ctypes.byref(args), ctypes.c_void_p(workspace.data_ptr()),
                                            workspace.numel(), stream))
    return distances, nodes

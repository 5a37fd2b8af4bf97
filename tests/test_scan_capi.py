"""libvectra_scan.so loads, exports what include/vectra_scan.h declares, and
validates its arguments on the host.  No kernel is launched here: every call
either fails validation or has nothing to do."""

import ctypes
import os
import re
import shutil
import subprocess

import pytest
import torch

from vectra_amd.index import scan
from vectra_amd.kernels import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), 'include', 'vectra_scan.h')
OK, INVALID, TOO_LARGE = 0, 1, 2


def _declared_functions() -> set[str]:
    text = open(HEADER, encoding='utf-8').read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return set(re.findall(r'^\s*(?:const\s+)?\w+\s*\*?\s*(vectra_\w+)\s*\(', text, flags=re.M))


def test_library_exports_every_declared_symbol():
    declared = _declared_functions()
    assert declared == {'vectra_scan_rows', 'vectra_pq_distance_tables', 'vectra_scan_pq_adc',
                        'vectra_scan_top_k', 'vectra_scan_top_k_ws', 'vectra_scan_top_k_workspace_bytes',
                        'vectra_scan_top_k_no_alloc', 'vectra_scan_status_string', 'vectra_scan_abi_version'}
    lib = ctypes.CDLL(_native.SCAN_LIBRARY)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    lib = _native.scan_library()
    assert lib.vectra_scan_abi_version() == 3
    assert lib.vectra_scan_status_string(0) == b'ok'
    assert lib.vectra_scan_status_string(1) == b'invalid argument'
    assert lib.vectra_scan_status_string(99) == b'unknown status'


@pytest.mark.skipif(shutil.which('gcc') is None, reason='needs gcc')
def test_struct_layouts_match_the_header(tmp_path):
    # offsetof / sizeof of the three argument structs from the header itself.
    structs = {'vectra_scan_args': scan._ScanArgs, 'vectra_pq_table_args': scan._PqTableArgs,
               'vectra_pq_adc_args': scan._PqAdcArgs, 'vectra_scan_top_k_args': scan._TopKArgs}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "vectra_scan.h"', 'int main(void) {']
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ['  return 0;', '}']
    src = tmp_path / 'layout.c'
    src.write_text('\n'.join(lines))
    exe = tmp_path / 'layout'
    subprocess.run(['gcc', '-D__HIP_PLATFORM_AMD__=1', f'-I{os.path.dirname(HEADER)}', '-I/opt/rocm/include',
                    str(src), '-o', str(exe)], check=True)
    printed = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split('\n')
    for line in filter(None, printed):
        cname, field, value = line.split()
        cls = structs[cname]
        got = ctypes.sizeof(cls) if field == 'sizeof' else getattr(cls, field).offset
        assert got == int(value), line


FAKE = 0x1000  # never dereferenced: validation fails (or there is no work) first


def _rows_args(**over):
    fields = dict(metric=0, dimension=8, queries=FAKE, num_queries=2, query_stride=8, rows=FAKE, num_rows=10,
                  row_stride=8, ids=None, num_ids=0, out=FAKE, out_stride=10)
    fields.update(over)
    return scan._ScanArgs(**fields)


@pytest.mark.parametrize('over,status', [
    (dict(metric=3), INVALID),
    (dict(metric=-1), INVALID),
    (dict(dimension=-1), INVALID),
    (dict(num_queries=-1), INVALID),
    (dict(row_stride=7), INVALID),
    (dict(query_stride=7), INVALID),
    (dict(out_stride=9), INVALID),
    (dict(out=None), INVALID),
    (dict(rows=None), INVALID),
    (dict(queries=None), INVALID),
    (dict(metric=2, num_queries=2), INVALID),
    (dict(ids=FAKE, num_ids=-1), INVALID),
    (dict(ids=FAKE, num_ids=11, out_stride=10), INVALID),
    (dict(num_queries=65535 * 4 + 1, out_stride=10), TOO_LARGE),
    (dict(num_rows=1 << 40, row_stride=1 << 30, out_stride=1 << 40), TOO_LARGE),
])
def test_row_scan_rejects_bad_arguments(over, status):
    lib = _native.scan_library()
    assert lib.vectra_scan_rows(ctypes.byref(_rows_args(**over)), None) == status
    assert lib.vectra_scan_rows(None, None) == INVALID


@pytest.mark.parametrize('over', [dict(num_queries=0), dict(num_rows=0, out_stride=0),
                                  dict(ids=FAKE, num_ids=0, out_stride=0)])
def test_empty_row_scans_launch_nothing(over):
    assert _native.scan_library().vectra_scan_rows(ctypes.byref(_rows_args(**over)), None) == OK


def _table_args(**over):
    fields = dict(dimension=128, subspaces=16, queries=FAKE, num_queries=3, query_stride=128, codebooks=FAKE,
                  tables=FAKE, table_stride=16 * 256)
    fields.update(over)
    return scan._PqTableArgs(**fields)


@pytest.mark.parametrize('over,status', [
    (dict(subspaces=0), INVALID),
    (dict(subspaces=3), INVALID),          # 128 is not a multiple of 3 (FromCodebooks' rule)
    (dict(dimension=0), INVALID),
    (dict(query_stride=127), INVALID),
    (dict(table_stride=16 * 256 - 1), INVALID),
    (dict(codebooks=None), INVALID),
    (dict(tables=None), INVALID),
    (dict(num_queries=-2), INVALID),
    (dict(num_queries=1 << 20), TOO_LARGE),
    (dict(num_queries=0), OK),
])
def test_table_arguments(over, status):
    assert _native.scan_library().vectra_pq_distance_tables(ctypes.byref(_table_args(**over)), None) == status


def _adc_args(**over):
    fields = dict(subspaces=16, tables=FAKE, num_queries=2, table_stride=16 * 256, codes=FAKE, num_codes=100,
                  code_stride=16, ids=None, num_ids=0, out=FAKE, out_stride=100)
    fields.update(over)
    return scan._PqAdcArgs(**fields)


@pytest.mark.parametrize('over,status', [
    (dict(subspaces=0), INVALID),
    (dict(subspaces=257, table_stride=257 * 256, code_stride=257), INVALID),
    (dict(table_stride=100), INVALID),
    (dict(code_stride=15), INVALID),
    (dict(out_stride=99), INVALID),
    (dict(codes=None), INVALID),
    (dict(tables=None), INVALID),
    (dict(ids=FAKE, num_ids=-1), INVALID),
    (dict(num_queries=65536), TOO_LARGE),
    (dict(num_codes=0, out_stride=0), OK),
    (dict(num_queries=0), OK),
])
def test_adc_arguments(over, status):
    assert _native.scan_library().vectra_scan_pq_adc(ctypes.byref(_adc_args(**over)), None) == status


def _top_k_args(**over):
    fields = dict(dimension=8, k=10, queries=FAKE, num_queries=2, query_stride=8, rows=FAKE, num_rows=100,
                  row_stride=8, ids=None, num_ids=0, distances=FAKE, nodes=FAKE, out_stride=10)
    fields.update(over)
    return scan._TopKArgs(**fields)


@pytest.mark.parametrize('over,status', [
    (dict(k=0), INVALID),
    (dict(k=scan.MAX_K + 1, out_stride=scan.MAX_K + 1), INVALID),
    (dict(out_stride=9), INVALID),
    (dict(dimension=-1), INVALID),
    (dict(row_stride=7), INVALID),
    (dict(query_stride=7), INVALID),
    (dict(num_rows=-1), INVALID),
    (dict(ids=FAKE, num_ids=-1), INVALID),
    (dict(distances=None), INVALID),
    (dict(nodes=None), INVALID),
    (dict(rows=None), INVALID),
    (dict(queries=None), INVALID),
    (dict(num_rows=1 << 32, row_stride=8), TOO_LARGE),   # node ids are 32-bit, below NO_NODE
    (dict(num_queries=1 << 31), TOO_LARGE),
    (dict(num_queries=0), OK),
])
def test_top_k_arguments(over, status):
    lib = _native.scan_library()
    args = ctypes.byref(_top_k_args(**over))
    assert lib.vectra_scan_top_k(args, None) == status
    assert lib.vectra_scan_top_k_ws(args, None, 0, None) == status
    assert lib.vectra_scan_top_k_no_alloc(args, None) == status
    if status != OK:
        assert lib.vectra_scan_top_k_workspace_bytes(args) == 0
    assert lib.vectra_scan_top_k(None, None) == INVALID
    assert lib.vectra_scan_top_k_ws(None, None, 0, None) == INVALID
    assert lib.vectra_scan_top_k_no_alloc(None, None) == INVALID
    assert lib.vectra_scan_top_k_workspace_bytes(None) == 0


# (queries, candidates, k) -> ranges per query: below 64 queries, ranges of
# at least 64 candidates, at most 64 of them, ranges * k within 2048 keys.
@pytest.mark.parametrize('n_q,n_rows,k,splits', [
    (1, 2048, 10, 32), (1, 100, 10, 2), (1, 64, 10, 1), (1, 65, 10, 2), (63, 2048, 10, 32), (64, 2048, 10, 1),
    (1, 1 << 20, 10, 64), (3, 1 << 20, 100, 16), (2, 1 << 20, 1000, 2), (2, 1 << 20, 1024, 2), (1, 5000, 1, 64),
    (0, 2048, 10, 1),
])
def test_top_k_workspace_bytes(n_q, n_rows, k, splits):
    lib = _native.scan_library()
    args = _top_k_args(num_queries=n_q, num_rows=n_rows, k=k, out_stride=k)
    want = 0 if splits == 1 else 256 + n_q * splits * k * 8
    assert lib.vectra_scan_top_k_workspace_bytes(ctypes.byref(args)) == want
    # The library's own scratch holds the largest of them (63 queries of 2048 keys).
    assert want <= 256 + 64 * 2048 * 8
    # Candidates from an id list count the same way.
    ids = _top_k_args(num_queries=n_q, num_rows=10, ids=FAKE, num_ids=n_rows, k=k, out_stride=k)
    assert lib.vectra_scan_top_k_workspace_bytes(ctypes.byref(ids)) == want


def test_top_k_workspace_must_be_aligned():
    lib = _native.scan_library()
    args = ctypes.byref(_top_k_args(num_queries=1, num_rows=2048))
    # Refused before anything is launched.
    assert lib.vectra_scan_top_k_ws(args, FAKE + 8, 1 << 20, None) == INVALID


def test_wrappers_refuse_cpu_tensors():
    rows = torch.zeros(4, 8)
    with pytest.raises(ValueError, match='GPU'):
        scan.l2_squared_distances(torch.zeros(1, 8), rows)
    with pytest.raises(ValueError, match='GPU'):
        scan.squared_norms(rows)
    with pytest.raises(ValueError, match='GPU'):
        scan.pq_adc_distances(torch.zeros(1, 256), torch.zeros(4, 1, dtype=torch.uint8))
    with pytest.raises(ValueError, match='GPU'):
        scan.pq_distance_tables(torch.zeros(1, 8), torch.zeros(8 * 256), 2)

"""Matrix-core / vector-unit co-execution on one gfx950 SIMD, and the ceiling
it sets for a kernel that needs both.

Runs the probe loops of ``coexec_probe.hip`` (in ``libvectra_bench.so``) at
one and two waves per SIMD and derives, from the two-wave runs, an issue
model of the SIMD in shader-clock ticks:

* ``fma``: one fp32 FMA (FMAs alone);
* ``exp2``: one exp2 (8 exp2 + 24 FMAs, less the FMAs);
* ``mfma``: one 16x16x32 bf16 MFMA on the matrix pipe (MFMAs alone);
* ``mfma_valu_block``: vector-issue ticks one such MFMA takes away from the
  vector instructions beside it (one MFMA : four FMAs, less the FMAs).

For an instruction mix (``--mix VALU EXP2 MFMA``, counts of one unit of work,
e.g. one wave's 64-key tile of the long-key kernel), the model's floor is
max(vector side, matrix side), vector side = (VALU - EXP2) fma + EXP2 exp2 +
MFMA mfma_valu_block, matrix side = MFMA mfma.  The long-key kernel compares
its measured time per unit with that floor, as the HBM kernels compare with
the plain read of their bytes.

    python3 -m vectra_amd.benchmarks.coexec [--mix 281 64 80] [--json out.json]
"""

import argparse
import ctypes
import json
import os
import sys

import torch

from vectra_amd.kernels import _native

BENCH_LIBRARY = os.path.join(_native.LIB_DIR, 'libvectra_bench.so')


def _library():
    if not os.path.exists(BENCH_LIBRARY):
        raise _native.NativeLibraryMissing(f'{BENCH_LIBRARY} is missing; build with `make -C vectra_amd/csrc`')
    lib = ctypes.CDLL(BENCH_LIBRARY)
    lib.vectra_bench_coexec_variants.restype = ctypes.c_int
    lib.vectra_bench_coexec_describe.argtypes = [ctypes.c_int] + [ctypes.POINTER(ctypes.c_int)] * 4
    lib.vectra_bench_coexec.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_int)]
    return lib


def describe(lib, i):
    vals = [ctypes.c_int() for _ in range(4)]
    if lib.vectra_bench_coexec_describe(i, *[ctypes.byref(v) for v in vals]) != 0:
        raise ValueError(f'no probe variant {i}')
    mfma, valu, exp2, big = (v.value for v in vals)
    return {'mfma': mfma, 'valu': valu, 'exp2': bool(exp2), 'mfma_32x32x16': bool(big)}


def run_probes():
    """Ticks per loop iteration of every variant at 1 and 2 waves per SIMD."""
    lib = _library()
    ticks = torch.empty(4096, dtype=torch.int64, device='cuda')
    sink = torch.empty(2048 * 64, dtype=torch.float32, device='cuda')
    rows = []
    for i in range(lib.vectra_bench_coexec_variants()):
        row = describe(lib, i)
        for waves in (1, 2):
            per = ctypes.c_double()
            ratio = ctypes.c_double()
            iters = ctypes.c_int()
            status = lib.vectra_bench_coexec(i, waves, ticks.data_ptr(), sink.data_ptr(), ctypes.byref(per),
                                             ctypes.byref(ratio), ctypes.byref(iters))
            if status != 0:
                raise RuntimeError(f'vectra_bench_coexec({i}, {waves}) returned {status}')
            row[f'ticks_per_iter_{waves}w'] = per.value
            row[f'tick_ghz_{waves}w'] = 0.1 * ratio.value  # s_memrealtime runs at 100 MHz
        rows.append(row)
    return rows


def issue_model(rows):
    """SIMD ticks per instruction from the two-wave runs (see the module docstring)."""
    def find(mfma, valu, exp2, big=False):
        for r in rows:
            if (r['mfma'], r['valu'], r['exp2'], r['mfma_32x32x16']) == (mfma, valu, exp2, big):
                return r['ticks_per_iter_2w'] / 2.0  # two waves share the SIMD: per wave-iteration of SIMD time
        raise KeyError((mfma, valu, exp2, big))

    fma = find(0, 32, False) / 32
    exp2 = (find(0, 32, True) - 24 * fma) / 8
    mfma = find(8, 0, False) / 8
    block = (find(8, 32, False) - 32 * fma) / 8
    mfma32 = find(4, 0, False, True) / 4
    block32 = (find(4, 32, False, True) - 32 * fma) / 4
    return {'fma': fma, 'exp2': exp2, 'mfma': mfma, 'mfma_valu_block': block,
            'mfma_32x32x16': mfma32, 'mfma_32x32x16_valu_block': block32}


def floor_ticks(model, valu, exp2, mfma):
    """Issue-model floor of a mix (VALU includes the exp2s, excludes the MFMAs)."""
    vector = (valu - exp2) * model['fma'] + exp2 * model['exp2'] + mfma * model['mfma_valu_block']
    matrix = mfma * model['mfma']
    return {'vector_side': vector, 'matrix_side': matrix, 'floor': max(vector, matrix)}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split('\n\n')[0])
    ap.add_argument('--mix', nargs=3, type=float, metavar=('VALU', 'EXP2', 'MFMA'),
                    help='non-MFMA vector instructions (exp2 included), exp2s and 16x16x32 MFMAs of one unit of work')
    ap.add_argument('--json', default=None)
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit('coexec needs a GPU')
    rows = run_probes()
    print(f'{"MFMA":>5} {"VALU":>5} {"exp2":>5} {"32x32":>6} {"1 wave":>9} {"2 waves":>9}  (ticks per iteration)')
    for r in rows:
        print(f'{r["mfma"]:5d} {r["valu"]:5d} {str(r["exp2"]):>5} {str(r["mfma_32x32x16"]):>6} '
              f'{r["ticks_per_iter_1w"]:9.1f} {r["ticks_per_iter_2w"]:9.1f}')
    model = issue_model(rows)
    ghz = sorted(r['tick_ghz_2w'] for r in rows)[len(rows) // 2]
    print(f'shader clock ticks at {ghz:.3f} GHz (median over the two-wave runs)')
    print('issue model (SIMD ticks per instruction, two waves per SIMD): ' +
          ', '.join(f'{k} {v:.2f}' for k, v in model.items()))
    out = {'probe': rows, 'model_ticks': model, 'tick_ghz': ghz}
    if a.mix:
        valu, exp2, mfma = a.mix
        out['mix'] = {'valu': valu, 'exp2': exp2, 'mfma': mfma, **floor_ticks(model, valu, exp2, mfma)}
        print(f'mix {a.mix}: vector side {out["mix"]["vector_side"]:.0f}, matrix side {out["mix"]["matrix_side"]:.0f}, '
              f'floor {out["mix"]["floor"]:.0f} ticks')
    if a.json:
        with open(a.json, 'w') as f:
            json.dump(out, f, indent=1)
    return out


if __name__ == '__main__':
    sys.exit(0 if main() else 1)

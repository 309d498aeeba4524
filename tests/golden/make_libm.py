"""Writes `libm.json`: the checksums of the reference's ports of glibc 2.39's math routines
(include/cuju/libm/*.h), compiled by `oracle/Makefile` into `oracle/_ref/liblibm_ports.so`, over the
inputs of `tests/libm_cases.py`: every float bit pattern for the unary float routines, the fixed
samples for the others. It runs in the build container, where the reference sources are:

    make -C oracle && python tests/golden/make_libm.py
"""

from __future__ import annotations

import ctypes
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

import libm_cases  # noqa: E402

PORTS = os.path.join(ROOT, 'oracle', '_ref', 'liblibm_ports.so')
OUT = os.path.join(HERE, 'libm.json')


def ports():
    lib = ctypes.CDLL(PORTS)
    lib.oracle_libm_float_range.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_longlong, ctypes.c_void_p]
    lib.oracle_libm_float.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong]
    lib.oracle_libm_double.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong]
    return lib


def float_outputs(lib, which, x, y):
    out = np.empty_like(x)
    lib.oracle_libm_float(which, x.ctypes.data, y.ctypes.data, out.ctypes.data, len(x))
    return out


def double_outputs(lib, which, x, y):
    out = np.empty_like(x)
    lib.oracle_libm_double(which, x.ctypes.data, y.ctypes.data, out.ctypes.data, len(x))
    return out


def main():
    lib = ports()
    result = {'exhaustive': {}, 'sampled_float': {}, 'sampled_double': {}, 'samples': {}}
    for name, which in libm_cases.UNARY_FLOAT.items():
        start = time.time()
        result['exhaustive'][name] = libm_cases.exhaustive_digest(
            lambda first, out, w=which: lib.oracle_libm_float_range(w, first, len(out), out.ctypes.data),
            threads=os.cpu_count() or 8)
        print(f'{name}: {time.time() - start:.0f} s', flush=True)
    for name, which in libm_cases.SAMPLED_FLOAT.items():
        x, y = libm_cases.float_pairs(name)
        result['sampled_float'][name] = libm_cases.sample_digest(float_outputs(lib, which, x, y))
        result['samples'][name] = len(x)
    for name, which in libm_cases.SAMPLED_DOUBLE.items():
        x, y = libm_cases.double_pairs(name)
        result['sampled_double'][name] = libm_cases.sample_digest(double_outputs(lib, which, x, y))
        result['samples'][name] = len(x)
    with open(OUT, 'w') as f:
        json.dump(result, f, indent=1, sort_keys=True)
        f.write('\n')
    print(f'wrote {OUT}')


if __name__ == '__main__':
    main()

"""Builds the native libraries in-tree.

* ``lib/libcuju_amd.so``: the product, the engine compiled for gfx950 behind the C ABI of
  ``include/cuju_amd.h``.
* ``lib/libcuju_amd_host.so``: the same engine and C ABI on host threads, a debugging build that
  tests use to follow a match tick by tick. The package never loads it.
* ``lib/libcuju_amd_host_sanitized.so``, on request only (``python -m cuju_amd.build --sanitize``):
  the host build under AddressSanitizer and UndefinedBehaviorSanitizer. The host tests load it
  in place of the host build when ``CUJU_AMD_HOST_LIBRARY`` names it, with the sanitizer runtimes
  preloaded into Python (``LD_PRELOAD``).

Every source compiles with IEEE semantics and no contraction of multiply-adds, which the engine's
bit-exactness needs. ``python -m cuju_amd.build`` runs the same steps.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, 'csrc')
OUT = os.path.join(HERE, 'lib')
BUILD = os.path.join(HERE, 'lib', 'obj')
ARCH = 'gfx950'
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
CXX = os.environ.get('CXX', 'g++')

PRODUCT = os.path.join(OUT, 'libcuju_amd.so')
HOST = os.path.join(OUT, 'libcuju_amd_host.so')
HOST_SANITIZED = os.path.join(OUT, 'libcuju_amd_host_sanitized.so')
# The sanitized host build: g++ only, so no GPU code is built with a sanitizer.
SANITIZE = ['-O1', '-g', '-fno-omit-frame-pointer', '-fsanitize=address,undefined', '-fno-sanitize-recover=undefined']

HOST_SOURCES = ['host/assets.cpp', 'host/runtime.cpp', 'host/api.cpp', 'host/scenario.cpp']
COMMON = ['-std=c++17', '-O2', '-fPIC', '-ffp-contract=off', '-fno-fast-math', '-fvisibility=hidden', '-w']
# Packed FP32 instructions stay off: plain float code only. -O2 measured about 1% faster than -O3
# for the step kernel on gfx950 (289 against 292 ms per step at 16,384 environments). Runtime
# unrolling lets loops of unknown trip count issue several iterations' loads together, which the
# latency-bound step kernel gains about 3% from (331 against 343 ms per step after 100 steps).
# The instruction scheduler's max-ILP strategy spreads independent work between dependent loads:
# 276-279 against 280-283 ms per step; the memory-clause strategy and promoting stack arrays to
# registers measured no better. The step kernel is bounded to two wavefronts per SIMD
# (hip_device.hip); without AGPR spills it fits that bound in 254 VGPRs, with them it takes 257
# registers and one wavefront per SIMD.
HIP_FLAGS = ['-std=c++17', '-O2', '-fPIC', '-ffp-contract=off', '-fno-fast-math', '-fvisibility=hidden', '-w',
             f'--offload-arch={ARCH}', '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
             '-mllvm', '-unroll-runtime', '-mllvm', '-amdgpu-sched-strategy=max-ilp',
             '-mllvm', '-amdgpu-spill-vgpr-to-agpr=0']


# The device code is built once per group width (lanes per environment); the first build also
# holds the geometry choice, the static scratch and the math check kernel.
GROUP_WIDTHS = (4, 2, 8, 16, 32, 64)


def _variant_flags(lanes):
    return [f'-DENG_GROUP_LANES={lanes}', f'-DENG_DEVICE_FACTORY=MakeHipDevice{lanes}',
            f'-DENG_PRIMARY_VARIANT={1 if lanes == GROUP_WIDTHS[0] else 0}']


def _run(command):
    result = subprocess.run(command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if result.returncode != 0:
        raise RuntimeError('build failed: ' + ' '.join(command) + '\n' + result.stdout[-6000:])
    return result.stdout


def _object(source, tag):
    return os.path.join(BUILD, tag + '_' + os.path.basename(source).replace('.', '_') + '.o')


def build(host=True, product=True, jobs=8):
    """Compiles both libraries (each source every time) and returns their paths."""
    os.makedirs(BUILD, exist_ok=True)
    tasks = []
    if product:
        for s in HOST_SOURCES:
            tasks.append([CXX, *COMMON, '-c', os.path.join(SOURCE, s), '-o', _object(s, 'p')])
        for lanes in GROUP_WIDTHS:
            tasks.append([HIPCC, *HIP_FLAGS, *_variant_flags(lanes), '-c', os.path.join(SOURCE, 'hip_device.hip'),
                          '-o', _object(f'hip_device_{lanes}.hip', 'p')])
    if host:
        for s in HOST_SOURCES + ['host/host_library.cpp']:
            tasks.append([CXX, *COMMON, '-c', os.path.join(SOURCE, s), '-o', _object(s, 'h')])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(_run, t) for t in tasks]:
            f.result()
    built = []
    if product:
        objects = [_object(s, 'p') for s in HOST_SOURCES] + [_object(f'hip_device_{lanes}.hip', 'p') for lanes in GROUP_WIDTHS]
        _run([HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', PRODUCT, *objects])
        built.append(PRODUCT)
    if host:
        objects = [_object(s, 'h') for s in HOST_SOURCES + ['host/host_library.cpp']]
        _run([CXX, '-shared', '-fPIC', '-o', HOST, *objects, '-lpthread'])
        built.append(HOST)
    shutil.rmtree(BUILD, ignore_errors=True)
    return built


def build_sanitized(jobs=8):
    """Compiles the host build under the sanitizers and returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    flags = [f for f in COMMON if f != '-O2'] + SANITIZE
    sources = HOST_SOURCES + ['host/host_library.cpp']
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for f in [pool.submit(_run, [CXX, *flags, '-c', os.path.join(SOURCE, s), '-o', _object(s, 's')])
                  for s in sources]:
            f.result()
    _run([CXX, '-shared', '-fPIC', '-fsanitize=address,undefined', '-o', HOST_SANITIZED,
          *[_object(s, 's') for s in sources], '-lpthread'])
    shutil.rmtree(BUILD, ignore_errors=True)
    return HOST_SANITIZED


if __name__ == '__main__':
    for path in (build_sanitized(),) if '--sanitize' in sys.argv[1:] else build():
        print(path)
    sys.exit(0)

"""The device's math routines (the glibc 2.39 algorithms the step calls, with their tables read
from LDS as in the step) give the reference ports' bits: all 2**32 inputs of sinf, cosf, atanf,
acosf and asinf, and the fixed samples of powf, atan2f, sincosf and the double routines, reduced
to the checksums the ports wrote (`tests/golden/libm.json`, `tests/libm_cases.py`)."""

import concurrent.futures
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import libm_cases
from conftest import PRODUCT, ROOT

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


def golden():
    with open(os.path.join(ROOT, 'tests', 'golden', 'libm.json')) as f:
        return json.load(f)


def device_libm():
    from cuju_amd import library
    return library.load(PRODUCT)


def evaluate(kind, which, first, count, x, y, out):
    lib = device_libm()
    stream = torch.cuda.current_stream().cuda_stream
    status = lib.cuju_debug_libm_device(kind, which, first, count, None if x is None else x.data_ptr(),
                                        None if y is None else y.data_ptr(), out.data_ptr(), stream)
    assert status == 0, 'the math kernel did not launch'


@pytest.mark.parametrize('name', sorted(libm_cases.UNARY_FLOAT))
def test_device_unary_float_math_on_every_input(name):
    which = libm_cases.UNARY_FLOAT[name]
    out = torch.empty(CHUNK, dtype=torch.float32, device='cuda:0')
    per_chunk = CHUNK // libm_cases.BLOCK
    with concurrent.futures.ThreadPoolExecutor(max_workers=16) as pool:
        futures = []
        for chunk in range((1 << 32) // CHUNK):
            evaluate(0, which, chunk * CHUNK, CHUNK, None, None, out)
            values = out.cpu().numpy()
            for b in range(per_chunk):
                part = values[b * libm_cases.BLOCK:(b + 1) * libm_cases.BLOCK]
                futures.append(pool.submit(lambda p: hashlib.sha256(libm_cases.canonical(p)).digest(), part))
        digests = [f.result() for f in futures]
    assert libm_cases.block_digests_to_checksum(digests) == golden()['exhaustive'][name]


@pytest.mark.parametrize('name', sorted(libm_cases.SAMPLED_FLOAT))
def test_device_float_math_on_samples(name):
    x, y = libm_cases.float_pairs(name)
    dx, dy = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    out = torch.empty_like(dx)
    evaluate(1, libm_cases.SAMPLED_FLOAT[name], 0, len(x), dx, dy, out)
    assert libm_cases.sample_digest(out.cpu().numpy()) == golden()['sampled_float'][name]


@pytest.mark.parametrize('name', sorted(libm_cases.SAMPLED_DOUBLE))
def test_device_double_math_on_samples(name):
    x, y = libm_cases.double_pairs(name)
    dx, dy = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    out = torch.empty_like(dx)
    evaluate(2, libm_cases.SAMPLED_DOUBLE[name], 0, len(x), dx, dy, out)
    assert libm_cases.sample_digest(out.cpu().numpy()) == golden()['sampled_double'][name]


def test_device_math_kernel_refuses_bad_arguments():
    out = torch.empty(4, dtype=torch.float32, device='cuda:0')
    lib = device_libm()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.cuju_debug_libm_device(3, 0, 0, 4, None, None, out.data_ptr(), stream) == -1
    assert lib.cuju_debug_libm_device(0, 9, 0, 4, None, None, out.data_ptr(), stream) == -1
    assert lib.cuju_debug_libm_device(1, 2, 0, 4, None, None, out.data_ptr(), stream) == -1
    assert lib.cuju_debug_libm_device(2, 6, 0, 4, out.data_ptr(), out.data_ptr(), out.data_ptr(), stream) == -1

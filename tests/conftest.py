"""Shared fixtures. Tests marked `gpu` need the HIP device; the rest run on the CPU."""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

DATA = os.path.join(ROOT, 'cuju_amd', 'data')
PRODUCT = os.path.join(ROOT, 'cuju_amd', 'lib', 'libcuju_amd.so')
# CUJU_AMD_HOST_LIBRARY names another host build, such as the sanitized one.
HOST = os.environ.get('CUJU_AMD_HOST_LIBRARY') or os.path.join(ROOT, 'cuju_amd', 'lib', 'libcuju_amd_host.so')
REFERENCE = os.path.join(ROOT, 'oracle', '_ref', 'libcuju_cpu.so')


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (HIP device)')


def load_digests():
    with open(os.path.join(DATA, 'digests.json')) as f:
        return json.load(f)


def short_cases(formats=('simple115', 'simple115v2', 'extracted', 'raw')):
    """The reference's short digest cases whose representation this build emits."""
    digests = load_digests()
    out = []
    for name, case in sorted(digests['cases'].items()):
        if case['options'].get('representation', 'simple115v2') in formats:
            out.append((name, case))
    return out


def digest_actions(step, environments, agents, action_count):
    """The actions of the reference self-check: (7 step + 3 env + 5 agent) mod n."""
    e = np.arange(environments, dtype=np.int64)[:, None]
    a = np.arange(agents, dtype=np.int64)[None, :]
    return ((step * 7 + e * 3 + a * 5) % action_count).astype(np.int32)


def play(batch, steps, environments):
    """SHA-256 over the reset observation, every step's observation, reward and done, then every
    environment's state. `batch` exposes reset/step/get_state returning array-likes."""
    def raw(x):
        # A raw observation is a dictionary, hashed by sorted name as the reference's check does.
        if isinstance(x, dict):
            return b''.join(raw(x[name]) for name in sorted(x))
        x = x.detach().cpu().numpy() if hasattr(x, 'detach') else np.asarray(x)
        return np.ascontiguousarray(x).tobytes()
    digest = hashlib.sha256()
    digest.update(raw(batch.reset()))
    for step in range(steps):
        out = batch.step(digest_actions(step, environments, batch.agents, batch.action_count))
        for x in out[:3]:
            digest.update(raw(x))
    if batch.stack == 1:
        for index in range(environments):
            digest.update(batch.get_state(index))
    return digest.hexdigest()


@pytest.fixture(scope='session')
def digests():
    return load_digests()


@pytest.fixture(scope='session')
def reference_library():
    if not os.path.isfile(REFERENCE):
        pytest.skip('the reference CPU library is not built (oracle/Makefile)')
    return REFERENCE


@pytest.fixture(scope='session')
def host_library():
    if not os.path.isfile(HOST):
        pytest.fail('the host debugging library is not built: run `python -m cuju_amd.build`')
    return HOST

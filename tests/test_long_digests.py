"""The reference's long digests: full matches (3,010 steps) and long runs of drill episodes, with
the raw, SMM and checkpoint outputs (python/cuju/data/digests.json `long_cases`, played by the
reference's tests/test_long.py). The engine's host build plays them on the CPU; the HIP build
plays them in tests/test_gpu_long.py when CUJU_AMD_LONG=1."""

import pytest

from conftest import load_digests, play
from oracle import ref

LONG = sorted(load_digests()['long_cases'].items())


@pytest.mark.parametrize('name,case', LONG, ids=[n for n, _ in LONG])
def test_host_engine_reproduces_long_digest(name, case, digests, host_library):
    batch = ref.ReferenceBatch(case['assets'], environment_count=digests['environments'], seed=digests['seed'],
                               threads=4, library_path=host_library, **dict(case['options']))
    try:
        assert play(batch, case['steps'], digests['environments']) == case['digest']
    finally:
        batch.close()

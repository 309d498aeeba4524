"""The oracle: the reference CPU library, built from its own sources by oracle/Makefile, must
reproduce the digests that the reference ships (python/cuju/data/digests.json) before it checks
anything else."""

import pytest

from conftest import play, short_cases
from oracle import ref


@pytest.mark.parametrize('name,case', short_cases(), ids=[n for n, _ in short_cases()])
def test_reference_reproduces_shipped_digest(name, case, digests, reference_library):
    options = dict(case['options'])
    batch = ref.ReferenceBatch(case['assets'], environment_count=digests['environments'], seed=7,
                               threads=1, library_path=reference_library, **options)
    try:
        assert play(batch, digests['steps'], digests['environments']) == case['digest']
    finally:
        batch.close()

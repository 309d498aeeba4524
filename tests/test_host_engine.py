"""The engine's host build (the same sources as the gfx950 kernels, compiled for the CPU) against
the shipped digests and, tick by tick, against the reference library on the same seeds and
actions. The product never loads this build; it locates divergences on the CPU."""

import ctypes
import random

import numpy as np
import pytest

from conftest import digest_actions, play, short_cases
from oracle import ref


@pytest.mark.parametrize('name,case', short_cases(), ids=[n for n, _ in short_cases()])
def test_host_engine_reproduces_shipped_digest(name, case, digests, host_library):
    batch = ref.ReferenceBatch(case['assets'], environment_count=digests['environments'], seed=7,
                               threads=4, library_path=host_library, **dict(case['options']))
    try:
        assert play(batch, digests['steps'], digests['environments']) == case['digest']
    finally:
        batch.close()


@pytest.mark.parametrize('assets,steps', [('11_vs_11_hard_stochastic_l11_r0', 60),
                                          ('5_vs_5_l4_r4', 80),
                                          ('academy_counterattack_hard_l4_r0', 80)])
def test_host_engine_matches_reference_every_tick(assets, steps, reference_library, host_library):
    """One tick per step, so every tick's full state is compared, not just the step's end."""
    options = dict(environment_count=2, seed=11, physics_steps_per_frame=1, threads=2)
    mine = ref.ReferenceBatch(assets, library_path=host_library, **options)
    theirs = ref.ReferenceBatch(assets, library_path=reference_library, **options)
    try:
        assert np.array_equal(mine.reset().view(np.uint32), theirs.reset().view(np.uint32))
        for step in range(steps):
            actions = digest_actions(step, 2, mine.agents, mine.action_count)
            a = [x.copy() for x in mine.step(actions)]
            b = [x.copy() for x in theirs.step(actions)]
            for x, y in zip(a, b):
                assert x.tobytes() == y.tobytes(), f'outputs differ at tick {step}'
            for e in range(2):
                assert mine.raw_state(e) == theirs.raw_state(e), f'state of env {e} differs at tick {step}'
    finally:
        mine.close()
        theirs.close()


def test_masked_reset_and_explicit_seeds(reference_library, host_library):
    options = dict(environment_count=4, seed=3, threads=2)
    mine = ref.ReferenceBatch('academy_3_vs_1_with_keeper_l1_r0', library_path=host_library, **options)
    theirs = ref.ReferenceBatch('academy_3_vs_1_with_keeper_l1_r0', library_path=reference_library, **options)
    try:
        for batch in (mine, theirs):
            batch.reset()
        for step in range(30):
            actions = digest_actions(step, 4, mine.agents, mine.action_count)
            assert mine.step(actions)[0].tobytes() == theirs.step(actions)[0].tobytes()
            if step % 10 == 9:
                mask = np.array([1, 0, step % 20 == 9, 1], dtype=np.uint8)
                seeds = np.array([-1, 5, 123456789, 4294967295], dtype=np.int64)
                assert mine.reset(seeds=seeds, mask=mask).tobytes() == theirs.reset(seeds=seeds, mask=mask).tobytes()
        for e in range(4):
            assert mine.get_state(e) == theirs.get_state(e)
    finally:
        mine.close()
        theirs.close()


def test_episode_seeds_follow_cpython_random(host_library):
    """GRF draws each episode seed with CPython's `random.randint(0, 2000000000)` after
    `random.seed(seed * 2**32 + index)`: Python's own generator is the oracle."""
    lib = ctypes.CDLL(host_library)
    lib.cuju_debug_episode_seeds.argtypes = [ctypes.c_ulonglong, ctypes.c_uint, ctypes.c_int, ctypes.c_void_p]
    for seed, index in [(0, 0), (0, 1), (7, 3), (2**32 - 1, 2**32 - 1), (123456789012, 77), (2**63, 5)]:
        out = np.zeros(8, dtype=np.uint32)
        lib.cuju_debug_episode_seeds(seed, index, 8, out.ctypes.data)
        rng = random.Random(seed * 2**32 + index)
        assert out.tolist() == [rng.randint(0, 2000000000) for _ in range(8)]

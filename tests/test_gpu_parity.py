"""Parity on the MI355X: the HIP library, through `cuju_amd.BatchEnvironment`, must reproduce the
reference's shipped digests and match the reference CPU library byte for byte on the headline
scenario, with masked resets and automatic episode resets."""

import numpy as np
import pytest
import torch

import lockstep
from conftest import PRODUCT, digest_actions, short_cases
from oracle import ref

pytestmark = pytest.mark.gpu


def gpu_batch(assets, **options):
    import cuju_amd
    return cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', **options)


def host(x):
    return x.detach().cpu().numpy()


@pytest.fixture(scope='module')
def shipped_digests_on_device(digests):
    """Every short digest case played at once, each batch on a stream of its own."""
    runs = []
    try:
        with lockstep.one_match_per_wavefront():
            for name, case in short_cases():
                runs.append(lockstep.DigestRun(name, case, digests['environments'], digests['seed'], digests['steps']))
        lockstep.play(runs, label='short digests', every=0)
        return {r.name: r.hexdigest() for r in runs}
    finally:
        for r in runs:
            r.close()


@pytest.mark.parametrize('name,case', short_cases(), ids=[n for n, _ in short_cases()])
def test_gpu_reproduces_shipped_digest(name, case, shipped_digests_on_device):
    assert shipped_digests_on_device[name] == case['digest']


def test_gpu_matches_reference_on_headline_scenario(reference_library):
    """11 agents against the hard AI (the throughput configuration) on a slice of environments."""
    environments, steps = 48, 40
    mine = gpu_batch('11_vs_11_hard_stochastic_l11_r0', environment_count=environments, seed=0)
    theirs = ref.ReferenceBatch('11_vs_11_hard_stochastic_l11_r0', environment_count=environments, seed=0,
                                threads=0, library_path=reference_library)
    try:
        assert host(mine.reset()).tobytes() == theirs.reset().tobytes()
        rng = np.random.default_rng(0)
        for step in range(steps):
            actions = rng.integers(0, 19, size=(environments, 11), dtype=np.int32)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            for x, y in zip(a[:3], b):
                assert host(x).astype(y.dtype).tobytes() == y.tobytes(), f'step {step}'
        for e in range(0, environments, 7):
            assert mine.get_state(e) == theirs.get_state(e), f'state of environment {e}'
    finally:
        mine.close()
        theirs.close()


@pytest.mark.parametrize('matches,lanes', [(32, 2), (16, 4), (8, 8), (4, 16), (1, 16), (2, 32), (1, 64)])
def test_every_geometry_matches_the_reference(matches, lanes, reference_library, monkeypatch):
    """Each build of the kernels (2 to 64 lanes per environment) at the matches per wavefront it
    serves plays the headline scenario as the reference does: 48 environments, 40 steps, then every
    state. 8 matches of 8 lanes is the geometry of the headline batch of 16,384; the 32- and
    64-lane builds take a whole half or whole wavefront per match (CUJU_AMD_LANES)."""
    monkeypatch.setenv('CUJU_AMD_MATCHES', str(matches))
    monkeypatch.setenv('CUJU_AMD_LANES', str(lanes))
    environments, steps = 48, 40
    mine = gpu_batch('11_vs_11_hard_stochastic_l11_r0', environment_count=environments, seed=2)
    theirs = ref.ReferenceBatch('11_vs_11_hard_stochastic_l11_r0', environment_count=environments, seed=2,
                                threads=0, library_path=reference_library)
    try:
        assert mine.geometry == (matches, lanes)
        assert host(mine.reset()).tobytes() == theirs.reset().tobytes()
        for step in range(steps):
            actions = digest_actions(step, environments, 11, 19)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            for x, y in zip(a[:3], b):
                assert host(x).astype(y.dtype).tobytes() == y.tobytes(), f'step {step}'
        for e in range(environments):
            assert mine.get_state(e) == theirs.get_state(e), f'state of environment {e}'
    finally:
        mine.close()
        theirs.close()


def test_the_geometry_fills_the_simds():
    """Two wavefronts for each SIMD where the batch allows: 32 environments of 2 lanes at 65,536,
    16 of 4 lanes at 32,768, 8 of 8 lanes at 16,384, 4 of 16 lanes at 8,192, 2 of 32 lanes at
    4,096 and one of 64 lanes, a whole wavefront, for a small batch."""
    import cuju_amd
    slots = 2 * 4 * torch.cuda.get_device_properties(0).multi_processor_count
    expected = {32 * slots: (32, 2), 16 * slots: (16, 4), 8 * slots: (8, 8), 4 * slots: (4, 16), 2 * slots: (2, 32),
                64: (1, 64)}
    for environments, geometry in expected.items():
        batch = cuju_amd.BatchEnvironment('academy_empty_goal_close', library=PRODUCT, device='cuda:0',
                                          environment_count=environments)
        try:
            assert batch.geometry == geometry, environments
        finally:
            batch.close()


def test_gpu_masked_reset_and_episode_end(reference_library):
    """Short academy episodes end and reset automatically; a masked reset with explicit and drawn
    seeds restarts a subset."""
    environments = 16
    options = dict(environment_count=environments, seed=5)
    mine = gpu_batch('academy_empty_goal_close_l1_r0', **options)
    theirs = ref.ReferenceBatch('academy_empty_goal_close_l1_r0', threads=0, library_path=reference_library, **options)
    try:
        assert host(mine.reset()).tobytes() == theirs.reset().tobytes()
        ends = 0
        for step in range(120):
            actions = digest_actions(step, environments, 1, 19)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            ends += int(b[2].sum())
            for x, y in zip(a[:3], b):
                assert host(x).astype(y.dtype).tobytes() == y.tobytes(), f'step {step}'
            assert host(a[3]['final_observation']).tobytes() == theirs.final_observation().tobytes()
            if step % 40 == 39:
                mask = (np.arange(environments) % 3 == step % 3).astype(np.uint8)
                seeds = np.where(np.arange(environments) % 2 == 0, -1, np.arange(environments) * 1000003).astype(np.int64)
                got = mine.reset(seeds=seeds, mask=torch.as_tensor(mask.astype(bool)))
                assert host(got).tobytes() == theirs.reset(seeds=seeds, mask=mask).tobytes()
        assert ends > 0, 'no episode ended, so the automatic reset went unchecked'
        for e in range(environments):
            assert mine.get_state(e) == theirs.get_state(e)
    finally:
        mine.close()
        theirs.close()


def test_gpu_set_state_continues_as_the_reference(reference_library):
    """States of a reference batch (with checkpoint counts) load into the HIP batch through
    `set_state`, shuffled across environments; the outputs right after and every later step and
    state match the reference given the same states."""
    assets, environments, played, after = '11_vs_11_hard_stochastic_l11_r0', 4, 30, 15
    options = dict(environment_count=environments, rewards='scoring,checkpoints')
    source = ref.ReferenceBatch(assets, seed=7, threads=0, library_path=reference_library, **options)
    source.reset()
    for step in range(played):
        source.step(digest_actions(step, environments, source.agents, source.action_count))
    states = [source.get_state(i) for i in range(environments)]
    raw = [source.raw_state(i) for i in range(environments)]
    source.close()
    mine = gpu_batch(assets, seed=11, **options)
    theirs = ref.ReferenceBatch(assets, seed=11, threads=0, library_path=reference_library, **options)
    try:
        mine.reset()
        theirs.reset()
        for index in range(environments):
            mine.set_state(index, states[(index + 1) % environments])
            match, episode = raw[(index + 1) % environments]
            theirs.set_raw_state(index, match, episode)
        assert host(mine.observation()).tobytes() == theirs.observation().tobytes()
        for index in range(environments):
            assert mine.get_state(index) == states[(index + 1) % environments]
        for step in range(after):
            actions = digest_actions(step + 5, environments, theirs.agents, theirs.action_count)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            for x, y in zip(a[:3], b):
                assert host(x).astype(y.dtype).tobytes() == y.tobytes(), f'step {step}'
        for index in range(environments):
            assert mine.get_state(index) == theirs.get_state(index)
    finally:
        mine.close()
        theirs.close()


def _host_observation(x):
    if isinstance(x, dict):
        return {k: host(v) for k, v in x.items()}
    return host(x)


def _same(a, b):
    if isinstance(a, dict):
        return sorted(a) == sorted(b) and all(_same(a[k], b[k]) for k in a)
    return np.ascontiguousarray(a).tobytes() == np.ascontiguousarray(b).tobytes()


@pytest.mark.parametrize('representation,stacked,with_raw', [('extracted', False, True), ('extracted', True, False),
                                                             ('raw', False, False)])
def test_gpu_smm_and_raw_match_reference(representation, stacked, with_raw, reference_library):
    """The SMM (one frame and a stack of four) and the raw arrays on the device, with the final
    observations of episodes that end, byte for byte against the reference CPU library on short
    academy episodes mixed with 5-a-side games."""
    environments = 24
    assets = ['academy_empty_goal_close_l1_r0', '5_vs_5_l4_r4']
    options = dict(environment_count=environments, seed=5, representation=representation, stacked=stacked,
                   with_raw=with_raw, assignment=[0, 1] * (environments // 2))
    mine = gpu_batch(assets, **options)
    theirs = ref.ReferenceBatch(assets, threads=0, library_path=reference_library, **options)
    try:
        assert _same(_host_observation(mine.reset()), theirs.reset())
        ended = 0
        for step in range(70):
            actions = digest_actions(step, environments, mine.agents, mine.action_count)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            assert _same(_host_observation(a[0]), b[0]), f'observation at step {step}'
            assert host(a[1]).tobytes() == b[1].tobytes(), f'reward at step {step}'
            assert host(a[2]).astype(np.uint8).tobytes() == b[2].tobytes(), f'done at step {step}'
            if b[2].any():
                ended += 1
                assert _same(_host_observation(a[3]['final_observation']), theirs.final_observation()), f'final at {step}'
            if with_raw:
                assert _same(_host_observation(mine.raw()), theirs.raw()), f'raw at step {step}'
        assert ended > 0
    finally:
        mine.close()
        theirs.close()

"""The five benchmark configurations on the MI355X against the reference CPU library, at the
configuration's shape with fewer environments where it is large.

Each step compares the observations, rewards, done flags and final observations byte for byte;
a run ends by comparing every environment's GRF state (unstacked configurations). Actions, reset
masks and reset seeds come from one counter hash of (seed, step, environment, agent), so both
sides consume identical inputs:

1. `5_vs_5_l4_r0`, 64 environments, simple115 and simple115v2.
2. `11_vs_11_stochastic_l1_r0` (opponent difficulty 0.6), 128 environments.
3. `11_vs_11_hard_stochastic_l11_r0`, in test_gpu_parity.py.
4. `11_vs_11_stochastic_l11_r11`, both sides controlled, 4-frame stacked observations, 10% of the
   environments reset every 40 steps with fresh int64 seeds.
5. A mixed batch: half `academy_3_vs_1_with_keeper_l3_r0` drills, a quarter `5_vs_5_l4_r0`, a
   quarter `11_vs_11_stochastic_l1_r0`; and the same mix with the drills of a GRF scenario file
   (three attackers 25 m out), built by the scenario builder.
"""

import os

import numpy as np
import pytest
import torch

from conftest import PRODUCT, ROOT
from oracle import ref

pytestmark = pytest.mark.gpu

MASK = (1 << 64) - 1


def counter(seed, step, environments, width, modulo):
    """SplitMix64 of (seed, step, environment, column), reduced modulo `modulo` (uint64 math)."""
    e = np.arange(environments, dtype=np.uint64)[:, None]
    a = np.arange(width, dtype=np.uint64)[None, :]
    with np.errstate(over='ignore'):
        x = (np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15) + np.uint64(step) * np.uint64(0xBF58476D1CE4E5B9) +
             e * np.uint64(0x94D049BB133111EB) + a * np.uint64(0x2545F4914F6CDD1D))
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    return x % np.uint64(modulo)


def host(x):
    return x.detach().cpu().numpy()


def compare(assets, environments, steps, seed=0, reset_every=None, states=True, their_assets=None, matches=None,
            **options):
    """`matches` sets the environments per wavefront (and so the group width) of the device batch,
    the geometry the library chooses for the configuration's full batch: 2 of 16 lanes for
    configuration 2, 4 of 16 lanes for 4, 16 of 4 lanes for 5. By default the library chooses,
    which for these small batches is one environment of 16 lanes."""
    import cuju_amd
    before = os.environ.get('CUJU_AMD_MATCHES')
    if matches is not None:
        os.environ['CUJU_AMD_MATCHES'] = str(matches)
    try:
        mine = cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', environment_count=environments,
                                         seed=seed, **options)
    finally:
        if before is None:
            os.environ.pop('CUJU_AMD_MATCHES', None)
        else:
            os.environ['CUJU_AMD_MATCHES'] = before
    theirs = ref.ReferenceBatch(their_assets or assets, environment_count=environments, seed=seed, threads=0,
                                **options)
    try:
        assert host(mine.reset()).tobytes() == theirs.reset().tobytes(), 'reset'
        agents = theirs.agents
        for step in range(steps):
            actions = counter(seed, step, environments, agents, theirs.action_count).astype(np.int32)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            for x, y, name in zip(a[:3], b, ('observation', 'reward', 'done')):
                assert host(x).astype(y.dtype).tobytes() == y.tobytes(), f'{name} at step {step}'
            if b[2].any():
                assert host(a[3]['final_observation']).tobytes() == theirs.final_observation().tobytes(), f'final at {step}'
            if reset_every and step % reset_every == reset_every - 1:
                draw = counter(seed + 1, step, environments, 2, 1 << 32)
                mask = (draw[:, 0] % np.uint64(10) == 0).astype(np.uint8)
                seeds = draw[:, 1].astype(np.int64)
                got = mine.reset(seeds=seeds, mask=torch.as_tensor(mask.astype(bool)))
                assert host(got).tobytes() == theirs.reset(seeds=seeds, mask=mask).tobytes(), f'masked reset at {step}'
        if states:
            for e in range(environments):
                assert mine.get_state(e) == theirs.get_state(e), f'state of environment {e}'
    finally:
        mine.close()
        theirs.close()


@pytest.mark.parametrize('representation', ['simple115', 'simple115v2'])
def test_config1_five_a_side(representation, reference_library):
    compare('5_vs_5_l4_r0', 64, 150, representation=representation)


def test_config2_eleven_a_side_one_agent(reference_library):
    compare('11_vs_11_stochastic_l1_r0', 128, 120, matches=2)


def test_config4_self_play_stacked_with_masked_resets(reference_library):
    compare('11_vs_11_stochastic_l11_r11', 32, 120, seed=3, reset_every=40, stacked=True, states=False, matches=4)


def test_config5_mixed_batch(reference_library):
    assignment = [0, 0, 1, 2] * 16
    compare(['academy_3_vs_1_with_keeper_l3_r0', '5_vs_5_l4_r0', '11_vs_11_stochastic_l1_r0'], 64, 150,
            seed=5, assignment=assignment, matches=16)


def test_config5_drills_from_a_scenario_file(reference_library, tmp_path):
    from cuju_amd import scenarios
    source = os.path.join(ROOT, 'tests', 'golden', 'scenarios', 'drill_3_vs_1_with_keeper.py')
    bundle = scenarios.build_bundle(source, str(tmp_path / 'drill_l0_r0.cjb'))
    others = ['5_vs_5_l0_r0', '11_vs_11_stochastic_l0_r0']
    assignment = [0, 0, 1, 2] * 16
    compare([source] + others, 64, 150, seed=9, assignment=assignment, their_assets=[bundle] + others,
            agent_counts=[(3, 0), (4, 0), (1, 0)])


def test_difficulty_reports_and_overrides(reference_library):
    """`difficulty` takes one (left, right) pair per bundle, None keeping the scenario's, and
    `batch.difficulty` reports what each environment plays (tests/test_difficulty.py of the
    reference); the overridden batch then plays as the reference with the same difficulties."""
    import cuju_amd
    batch = cuju_amd.BatchEnvironment(['5_vs_5_l1_r0', '11_vs_11_easy_stochastic_l1_r0', '1_vs_1_easy_l1_r0'],
                                      library=PRODUCT, device='cuda:0', environment_count=3, assignment=[0, 1, 2])
    try:
        assert batch.difficulty.dtype == torch.float32
        assert torch.equal(batch.difficulty, torch.tensor([[0.05, 0.05], [1.0, 0.05], [0.0, 0.0]]))
    finally:
        batch.close()
    assets = ['11_vs_11_stochastic_l1_r0', '5_vs_5_l1_r0']
    assignment = [0, 1] * 16
    mine = cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', environment_count=32,
                                     assignment=assignment, difficulty=[(None, 0.25), (0.75, None)], seed=4)
    per_environment = np.array([[-1.0, 0.25], [0.75, -1.0]] * 16, dtype=np.float32)
    theirs = ref.ReferenceBatch(assets, environment_count=32, seed=4, threads=0, assignment=assignment,
                                difficulty=per_environment)
    try:
        assert torch.equal(mine.difficulty, torch.tensor([[1.0, 0.25], [0.75, 0.05]] * 16))
        assert host(mine.reset()).tobytes() == theirs.reset().tobytes()
        for step in range(80):
            actions = counter(4, step, 32, theirs.agents, theirs.action_count).astype(np.int32)
            a = mine.step(torch.as_tensor(actions, device='cuda:0'))
            b = theirs.step(actions)
            for x, y, name in zip(a[:3], b, ('observation', 'reward', 'done')):
                assert host(x).astype(y.dtype).tobytes() == y.tobytes(), f'{name} at step {step}'
        for e in range(32):
            assert mine.get_state(e) == theirs.get_state(e), f'state of environment {e}'
    finally:
        mine.close()
        theirs.close()


def test_smm_of_other_dimensions(reference_library):
    """`channel_dimensions` resizes the SMM on the device as on the reference, stacked."""
    compare('5_vs_5_l2_r1', 16, 60, seed=4, states=False, representation='extracted', stacked=True,
            channel_dimensions=(37, 21))

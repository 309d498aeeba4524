"""The batch's Python surface beyond the step itself, on the MI355X, after the reference's
python/cuju/_batch/environment.py:

* step observers (:722-815, :840-866): the calls after `reset`, masked `reset`, `step`,
  `step_async`/`step_wait`, `reset_done` and `close`, the removal of an observer that raises, the
  argument errors, and an observer that closes the batch during a step;
* `scenario_name` (:710-721) and `final_raw` (:1278-1284);
* the gym spaces (:1228-1266), which need gymnasium or gym: without either they raise
  `ModuleNotFoundError`; with a stand-in module the shapes, bounds and sizes come through;
* `digest` (python/cuju/action_log.py:104-145) against the shipped self-check digests.
"""

import logging
import sys
import types

import numpy as np
import pytest
import torch

from conftest import PRODUCT
from cuju_amd import workloads
from cuju_amd.errors import ArgumentError, ClosedError, ConfigurationError

pytestmark = pytest.mark.gpu

ASSETS = 'academy_empty_goal_l1_r0'


def gpu_batch(assets=ASSETS, **options):
    import cuju_amd
    options.setdefault('environment_count', 4)
    return cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', **options)


def device_actions(step, batch):
    return torch.as_tensor(workloads.actions(5, step, 0, batch.environment_count, batch.agents), device='cuda:0')


class Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, batch, done, information):
        self.calls.append((batch, None if done is None else done.clone(), dict(information)))


def test_observers_see_every_reset_step_and_close():
    batch = gpu_batch(auto_reset=False)
    seen = batch.add_observer(Recorder())
    assert batch.observers == (seen,)
    batch.reset()
    assert len(seen.calls) == 1
    call_batch, done, information = seen.calls[-1]
    assert call_batch is batch and done is None and information == {'reset': None}

    mask = [True, False, True, False]
    batch.reset(mask=mask)
    _, done, information = seen.calls[-1]
    assert done is None and information['reset'].tolist() == mask

    observation, reward, done, information = batch.step(device_actions(0, batch))
    _, seen_done, seen_information = seen.calls[-1]
    assert len(seen.calls) == 3
    assert torch.equal(seen_done, done)
    assert set(seen_information) == {'final_observation', 'score_reward', 'reward'}
    assert torch.equal(seen_information['reward'], reward)
    assert set(information) == {'final_observation', 'score_reward'}

    batch.step_async(device_actions(1, batch))
    assert len(seen.calls) == 3
    _, reward, done, _ = batch.step_wait()
    assert len(seen.calls) == 4
    assert torch.equal(seen.calls[-1][1], done)
    assert torch.equal(seen.calls[-1][2]['reward'], reward)

    before = done.clone()
    batch.reset_done()
    _, done, information = seen.calls[-1]
    assert len(seen.calls) == 5 and done is None
    assert torch.equal(information['reset'].cpu(), before.cpu())

    batch.close()
    _, done, information = seen.calls[-1]
    assert len(seen.calls) == 6 and done is None and information == {'close': True}
    assert batch.observers == ()
    batch.close()
    assert len(seen.calls) == 6


def test_an_observer_that_raises_is_removed_with_a_warning(caplog):
    batch = gpu_batch()
    try:
        def failing(_batch, _done, _information):
            raise ValueError('planted')

        kept = Recorder()
        batch.add_observer(failing)
        batch.add_observer(kept)
        with caplog.at_level(logging.WARNING, logger='cuju_amd'):
            batch.reset()
        assert batch.observers == (kept,)
        assert any('planted' in record.getMessage() for record in caplog.records)
        assert len(kept.calls) == 1
        batch.step(device_actions(0, batch))
        assert len(kept.calls) == 2
    finally:
        batch.close()


def test_observer_arguments_are_checked():
    batch = gpu_batch()
    observer = Recorder()
    try:
        with pytest.raises(ArgumentError):
            batch.add_observer(3)
        assert batch.add_observer(observer) is observer
        with pytest.raises(ArgumentError):
            batch.add_observer(observer)
        batch.remove_observer(observer)
        with pytest.raises(ArgumentError):
            batch.remove_observer(observer)
    finally:
        batch.close()
    with pytest.raises(ClosedError):
        batch.add_observer(Recorder())


def test_an_observer_that_closes_the_batch_makes_the_step_raise():
    batch = gpu_batch()
    batch.reset()

    def closing(current, done, information):
        if 'close' not in information:
            current.close()

    batch.add_observer(closing)
    with pytest.raises(ClosedError):
        batch.step(device_actions(0, batch))
    with pytest.raises(ClosedError):
        batch.reset()


def test_scenario_name_and_final_raw():
    batch = gpu_batch(with_raw=True)
    try:
        assert batch.scenario_name == ASSETS
        batch.reset()
        batch.step(device_actions(0, batch))
        raw, final = batch.raw(), batch.final_raw()
        assert set(raw) == set(final)
        for name in raw:
            assert raw[name].shape == final[name].shape and raw[name].dtype == final[name].dtype
            assert raw[name].data_ptr() != final[name].data_ptr()
    finally:
        batch.close()
    plain = gpu_batch()
    try:
        with pytest.raises(ConfigurationError):
            plain.final_raw()
    finally:
        plain.close()


def _stand_in_gym():
    """A module with gymnasium's names, whose spaces record their arguments."""
    gym = types.ModuleType('gymnasium')
    spaces = types.ModuleType('gymnasium.spaces')

    class Box:
        def __init__(self, low, high, shape, dtype):
            self.low, self.high, self.shape, self.dtype = low, high, shape, dtype

    class Discrete:
        def __init__(self, n):
            self.n = n

    class MultiDiscrete:
        def __init__(self, nvec):
            self.nvec = list(nvec)

    spaces.Box, spaces.Discrete, spaces.MultiDiscrete = Box, Discrete, MultiDiscrete
    vector = types.ModuleType('gymnasium.vector')
    utils = types.ModuleType('gymnasium.vector.utils')
    utils.batch_space = lambda space, n: ('batched', space, n)
    gym.spaces, gym.vector, vector.utils = spaces, vector, utils
    return {'gymnasium': gym, 'gymnasium.spaces': spaces, 'gymnasium.vector': vector,
            'gymnasium.vector.utils': utils}


def test_spaces(monkeypatch):
    batch = gpu_batch(environment_count=3)
    smm = gpu_batch(environment_count=2, representation='extracted', squeeze=True)
    try:
        for name in ('gymnasium', 'gym'):
            monkeypatch.setitem(sys.modules, name, None)
        with pytest.raises(ModuleNotFoundError):
            batch.action_space
        for name, module in _stand_in_gym().items():
            monkeypatch.setitem(sys.modules, name, module)
        box = batch.single_observation_space
        assert box.shape == (1, 115) and box.dtype == np.float32 and box.low == -np.inf
        assert batch.single_action_space.nvec == [19]
        batched = batch.observation_space
        assert batched[0] == 'batched' and batched[1].shape == (1, 115) and batched[2] == 3
        assert batch.action_space[2] == 3
        image = smm.single_observation_space
        assert image.shape == (72, 96, 4) and image.dtype == np.uint8 and image.high == 255
        assert smm.single_action_space.n == 19
    finally:
        batch.close()
        smm.close()


@pytest.mark.parametrize('name', ['5_vs_5/raw', '5_vs_5/stacked', '11_vs_11_stochastic/checkpoints',
                                  'academy_corner/simple115v2'])
def test_digest_reproduces_the_shipped_case(name, digests):
    """`cuju_amd.digest` plays the reference self-check's run and gives its shipped SHA-256."""
    import cuju_amd
    from conftest import short_cases
    case = dict(short_cases())[name]
    got = cuju_amd.digest(case['assets'], device='cuda:0', steps=digests['steps'], seed=digests['seed'],
                          environment_count=digests['environments'], library=PRODUCT, **dict(case['options']))
    assert got == case['digest']


def test_agent_counts_keep_a_side_left_as_none_and_squeeze_needs_one_agent():
    """python/cuju/_batch/environment.py:477-494 (a None count keeps what the name gives) and
    :631-635 (squeezing needs one agent in every environment)."""
    batch = gpu_batch('5_vs_5_l4_r4', environment_count=2, agent_counts=[(2, None)])
    try:
        assert batch.left_agents.tolist() == [2, 2] and batch.right_agents.tolist() == [4, 4]
        assert batch.agent_mask.shape == (2, batch.agents) and batch.agent_mask.sum().item() == 12
    finally:
        batch.close()
    with pytest.raises(ConfigurationError):
        gpu_batch('5_vs_5_l4_r4', environment_count=2, agent_counts=[(2,)])
    with pytest.raises(ConfigurationError):
        gpu_batch('5_vs_5_l4_r4', environment_count=2, squeeze=True)

"""Stacked states on the MI355X. A stacked batch's state pickles GRF's `FrameStack` (a deque of the
last four observations, oldest first) beside the episode logic and the engine bytes; loading it
restores the stack (the reference's surface: python/cuju/_batch/environment.py:1487-1620,
python/cuju/_batch/frame_stack.py). The checks here:

* a state carried from one batch into an environment of another batch, with another seed, makes
  that environment continue frame for frame as the original does, for one agent, several agents
  and the SMM;
* the pickle holds GRF's deque, with one agent's frames lacking the agent axis, and its frames
  concatenate to the observation;
* four foreign frames become the stack, and the next step shifts them by one frame;
* malformed stacks and mismatched `stacked` options are refused.
(The continuation against the reference library is in test_gpu_surface.py.)
"""

import collections
import pickle
import struct
import sys
import types

import numpy as np
import pytest
import torch

from conftest import PRODUCT
from cuju_amd import workloads

pytestmark = pytest.mark.gpu


@pytest.fixture
def grf_env_state(monkeypatch):
    """A module tree standing in for GRF's, so that `pickle` can load and dump whole states."""
    path = ('gfootball', 'gfootball.env', 'gfootball.env.football_env_core')
    state_class = type('EnvState', (), {'__module__': path[-1], '__qualname__': 'EnvState'})
    for name in path:
        module = types.ModuleType(name)
        if name == path[-1]:
            module.EnvState = state_class
        monkeypatch.setitem(sys.modules, name, module)
    return state_class


def make(assets, **options):
    import cuju_amd
    return cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', **options)


def parts(state):
    """(unpickled episode logic, engine bytes) of `get_state` bytes."""
    (length,) = struct.unpack_from('<i', state)
    return pickle.loads(state[4:4 + length]), state[4 + length:]


def assemble(unpickled, engine):
    data = pickle.dumps(unpickled, protocol=2)
    return struct.pack('<i', len(data)) + data + engine


def as_bytes(x):
    return x.detach().cpu().numpy().tobytes()


def advance(batch, seed, first, count):
    for step in range(first, first + count):
        batch.step(torch.as_tensor(workloads.actions(seed, step, 0, batch.environment_count, batch.agents),
                                   device='cuda:0'))


@pytest.mark.parametrize('assets,representation', [('5_vs_5_l1_r0', 'simple115v2'), ('5_vs_5_l2_r1', 'simple115'),
                                                   ('5_vs_5_l2_r0', 'extracted')])
def test_a_carried_state_continues_frame_for_frame(assets, representation):
    options = dict(environment_count=3, representation=representation, stacked=True)
    source, target = make(assets, seed=31, **options), make(assets, seed=32, **options)
    try:
        source.reset()
        target.reset()
        advance(source, 31, 0, 21)
        advance(target, 32, 0, 9)
        # Environment 1 of the source goes into environment 2 of the target.
        target.set_state(2, source.get_state(1, stacked=True), stacked=True)
        assert as_bytes(target.observation()[2]) == as_bytes(source.observation()[1])
        for step in range(15):
            actions = workloads.actions(40, step, 0, 3, source.agents)
            moved = actions.copy()
            moved[2] = actions[1]
            a = source.step(torch.as_tensor(actions, device='cuda:0'))[0]
            b = target.step(torch.as_tensor(moved, device='cuda:0'))[0]
            assert as_bytes(b[2]) == as_bytes(a[1]), f'step {step} after the load'
    finally:
        source.close()
        target.close()


@pytest.mark.parametrize('assets,representation,frame_shape', [('5_vs_5_l2_r1', 'simple115v2', (3, 115)),
                                                               ('5_vs_5_l1_r0', 'simple115v2', (115,)),
                                                               ('5_vs_5_l1_r0', 'extracted', (72, 96, 4))])
def test_the_pickle_holds_grf_frame_stack(assets, representation, frame_shape, grf_env_state):
    batch = make(assets, environment_count=1, stacked=True, representation=representation)
    try:
        batch.reset()
        advance(batch, 3, 0, 6)
        unpickled, _ = parts(batch.get_state(0, stacked=True))
        frames = unpickled['FrameStack']
        assert isinstance(frames, collections.deque) and frames.maxlen == 4 and len(frames) == 4
        assert {frame.shape for frame in frames} == {frame_shape}
        assert np.concatenate(list(frames), axis=-1).tobytes() == as_bytes(batch.observation()[0])
        assert isinstance(unpickled['FootballEnvCore'], grf_env_state)
    finally:
        batch.close()


def test_foreign_frames_become_the_stack_and_shift(grf_env_state):
    batch = make('5_vs_5_l1_r0', environment_count=1, stacked=True)
    try:
        batch.reset()
        advance(batch, 5, 0, 4)
        unpickled, engine = parts(batch.get_state(0, stacked=True))
        frames = [np.full(115, k, dtype=np.float32) + np.arange(115, dtype=np.float32) / 1000 for k in range(4)]
        unpickled['FrameStack'] = collections.deque(frames, maxlen=4)
        batch.set_state(0, assemble(unpickled, engine), stacked=True)
        assert as_bytes(batch.observation()[0]) == np.concatenate(frames).tobytes()
        observation = batch.step(torch.zeros((1, 1), dtype=torch.int32, device='cuda:0'))[0]
        # The oldest frame leaves; the other three move down one place.
        assert observation[0, 0, :345].cpu().numpy().tobytes() == np.concatenate(frames[1:]).tobytes()
    finally:
        batch.close()


def test_malformed_stacks_are_refused(grf_env_state):
    batch = make('5_vs_5_l1_r0', environment_count=1, stacked=True, representation='extracted')
    try:
        batch.reset()
        unpickled, engine = parts(batch.get_state(0, stacked=True))
        frames = list(unpickled['FrameStack'])

        def marked(frame_list):
            frame_list = [f.copy() for f in frame_list]
            frame_list[0][0, 0, 0] = 7  # GRF's minimap holds 0 or 255 only
            return frame_list

        cases = [
            (collections.deque(frames[:3], maxlen=4), ValueError, 'frames'),
            (collections.deque([f[:, :10] for f in frames], maxlen=4), ValueError, 'shape'),
            (collections.deque(marked(frames), maxlen=4), RuntimeError, 'minimap'),
            (None, ValueError, 'FrameStack'),
        ]
        for stack, error, message in cases:
            variant = dict(unpickled)
            if stack is None:
                del variant['FrameStack']
            else:
                variant['FrameStack'] = stack
            with pytest.raises(error, match=message):
                batch.set_state(0, assemble(variant, engine), stacked=True)
    finally:
        batch.close()


def test_the_stacked_option_must_match_the_batch():
    stacked = make('5_vs_5_l1_r0', environment_count=1, stacked=True)
    plain = make('5_vs_5_l1_r0', environment_count=1)
    try:
        stacked.reset()
        plain.reset()
        for call in (lambda: stacked.get_state(0), lambda: plain.get_state(0, stacked=True),
                     lambda: stacked.set_state(0, plain.get_state(0))):
            with pytest.raises(ValueError, match='stacked=True'):
                call()
        # An unstacked state's pickle holds no frame stack: its bytes are what the digests hash.
        (length,) = struct.unpack_from('<i', plain.get_state(0))
        assert b'FrameStack' not in plain.get_state(0)[4:4 + length]
    finally:
        stacked.close()
        plain.close()

"""GRF's frame stack in the pickle of a stacked state, on the CPU: the batch's stack through GRF's
deque of four frames and back, the globals such a pickle may name (under either numpy spelling of
the core modules), and the refusals."""

import collections
import io
import pickle

import numpy as np
import pytest

from cuju_amd import frame_stack


class _Loader(pickle.Unpickler):
    def find_class(self, module, name):
        found = frame_stack.find_class(module, name)
        if found is None:
            raise pickle.UnpicklingError(f'refused {module}.{name}')
        return found


def _load(data):
    return _Loader(io.BytesIO(data)).load()


@pytest.mark.parametrize('agents,shape,dtype', [(1, (115,), 'float32'), (3, (115,), 'float32'),
                                                (2, (72, 96, 4), 'uint8'), (1, (72, 96, 4), 'uint8')])
def test_a_stack_goes_through_grf_frames_and_back(agents, shape, dtype):
    rng = np.random.default_rng(agents)
    stack = rng.integers(0, 200, size=(agents, *shape[:-1], 4 * shape[-1])).astype(dtype)
    frames = frame_stack.frames_of(stack, agents)
    assert len(frames) == 4
    # Frame f holds channels [f * c, (f + 1) * c) of the stack; one agent drops the agent axis.
    c = shape[-1]
    for f, frame in enumerate(frames):
        expected = stack[..., f * c:(f + 1) * c]
        assert np.array_equal(frame, expected[0] if agents == 1 else expected)
    body = frame_stack.pickled_frames(frames)
    deque = _load(b'\x80\x02' + body + b'.')
    assert isinstance(deque, collections.deque) and deque.maxlen == 4
    assert frame_stack.stack_bytes(deque, agents, shape, dtype) == stack.tobytes()


def test_the_pickle_of_frames_is_what_protocol_2_writes():
    frames = [np.full((2, 115), f, np.float32) for f in range(4)]
    whole = pickle.dumps(collections.deque(frames, maxlen=4), protocol=2)
    assert b'\x80\x02' + frame_stack.pickled_frames(frames) + b'.' == whole


def test_only_the_globals_of_a_frame_pickle_resolve():
    assert frame_stack.find_class('collections', 'deque') is collections.deque
    assert frame_stack.find_class('builtins', 'bytes') is bytes
    assert frame_stack.find_class('numpy', 'ndarray') is np.ndarray
    # Both spellings of numpy's core modules give this numpy's object.
    one = frame_stack.find_class('numpy.core.multiarray', '_reconstruct')
    two = frame_stack.find_class('numpy._core.multiarray', '_reconstruct')
    assert one is two and callable(one)
    assert frame_stack.find_class('numpy.core.numeric', '_frombuffer') is \
        frame_stack.find_class('numpy._core.numeric', '_frombuffer')
    for module, name in [('os', 'system'), ('builtins', 'eval'), ('numpy', 'load'), ('numpy.core.multiarray', 'scalar'),
                         ('collections', 'OrderedDict')]:
        assert frame_stack.find_class(module, name) is None


def test_frames_of_the_wrong_count_shape_or_type_are_refused():
    good = [np.zeros(115, np.float32)] * 4
    assert len(frame_stack.stack_bytes(good, 1, (115,), 'float32')) == 4 * 115 * 4
    with pytest.raises(ValueError, match='4 frames'):
        frame_stack.stack_bytes(good[:3], 1, (115,), 'float32')
    with pytest.raises(ValueError, match='4 frames'):
        frame_stack.stack_bytes(np.zeros((4, 115), np.float32), 1, (115,), 'float32')
    with pytest.raises(ValueError, match='shape'):
        frame_stack.stack_bytes([np.zeros(114, np.float32)] * 4, 1, (115,), 'float32')
    with pytest.raises(ValueError, match='type'):
        frame_stack.stack_bytes([np.zeros(115, np.float64)] * 4, 1, (115,), 'float32')
    with pytest.raises(ValueError, match='shape'):
        frame_stack.stack_bytes([np.zeros(115, np.float32)] * 4, 2, (115,), 'float32')

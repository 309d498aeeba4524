"""GRF's `FrameStack` in the pickle of a stacked state: a deque of the last four observations, the
oldest first, each a numpy array as GRF's wrappers return it (python/cuju/_batch/frame_stack.py).
One agent's frames drop the agent axis, as GRF's single-agent wrappers do."""

from __future__ import annotations

import collections
import importlib
import pickle
import warnings

import numpy as np

FRAMES = 4

# The globals a pickled deque of numpy arrays names (protocol 2), under numpy 1 and numpy 2.
_ALLOWED = {
    ('collections', 'deque'), ('_codecs', 'encode'), ('builtins', 'bytes'), ('numpy', 'ndarray'),
    ('numpy', 'dtype'), ('numpy._core.multiarray', '_reconstruct'), ('numpy.core.multiarray', '_reconstruct'),
    ('numpy._core.numeric', '_frombuffer'), ('numpy.core.numeric', '_frombuffer'),
}


def frames_of(stack: np.ndarray, agents: int) -> list:
    """The four frames of one environment's stack `[agents, ..., 4 * n]`, oldest first."""
    width = stack.shape[-1] // FRAMES
    frames = [np.ascontiguousarray(stack[..., width * f:width * (f + 1)]) for f in range(FRAMES)]
    return [frame[0] if agents == 1 else frame for frame in frames]


def pickled_frames(frames: list) -> bytes:
    """The protocol-2 opcodes of GRF's deque of `frames`, without the protocol and stop opcodes, to
    stand as the value of a key in a pickle that keeps no memo of its own."""
    data = pickle.dumps(collections.deque(frames, maxlen=FRAMES), protocol=2)
    if data[:2] != b'\x80\x02' or data[-1:] != b'.':
        raise RuntimeError('unexpected pickle framing of the frame stack')
    return data[2:-1]


def find_class(module: str, name: str):
    """The global a pickled frame stack may name, or None for any other."""
    if (module, name) not in _ALLOWED:
        return None
    if not module.startswith('numpy'):
        return getattr(importlib.import_module(module), name)
    # A state pickled under the other numpy major version spells the core module differently.
    other = module.replace('numpy._core', 'numpy.core') if '._core' in module else module.replace('numpy.core', 'numpy._core')
    for candidate in (module, other):
        try:
            with warnings.catch_warnings():
                warnings.simplefilter('ignore')
                return getattr(importlib.import_module(candidate), name)
        except (ImportError, AttributeError):
            continue
    raise pickle.UnpicklingError(f'cannot resolve `{module}.{name}` with this numpy')


def stack_bytes(frames, agents: int, shape: tuple, dtype: str) -> bytes:
    """The batch's stack `[agents, *shape[:-1], 4 * shape[-1]]` from GRF's four frames; ValueError
    unless they are four observations of `shape` (with the agent axis for several agents)."""
    frames = list(frames) if isinstance(frames, (collections.deque, list, tuple)) else None
    expected = tuple(shape) if agents == 1 else (agents, *shape)
    if frames is None or len(frames) != FRAMES:
        raise ValueError(f'expected the {FRAMES} frames of GRF in the FrameStack of the state')
    arrays = []
    for frame in frames:
        array = np.asarray(frame)
        if array.shape != expected or array.dtype != np.dtype(dtype):
            raise ValueError(f'expected frames of the shape {expected} and the type {dtype} in the state, found '
                             f'{array.shape} and {array.dtype}')
        arrays.append(array.reshape((agents, *shape)))
    return np.ascontiguousarray(np.concatenate(arrays, axis=-1)).tobytes()

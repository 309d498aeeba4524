"""GRF's `FrameStack` inside the pickle of a stacked state.

GRF's frame-stack wrapper keeps `collections.deque(maxlen=4)` of the last four observations, the
oldest first, each a numpy array shaped as the wrapper's inner environment returns it: `[agents,
*shape]` for several agents, `shape` for one (GRF's single-agent wrappers drop the agent axis).
The batch keeps the same four frames side by side along the last axis, `[agents, *shape[:-1],
4 * shape[-1]]`; this module converts between the two (the reference's counterpart is
python/cuju/_batch/frame_stack.py).

A pickled deque of numpy arrays names a fixed set of globals under protocol 2. numpy 2 moved the
core modules from `numpy.core` to `numpy._core`, so a state written under one major version names
the other's modules; both spellings resolve to this interpreter's objects.
"""

from __future__ import annotations

import collections
import importlib
import pickle
import warnings

import numpy as np

FRAMES = 4

# (module, attribute) of the numpy objects such a pickle names, with the module as numpy 2 spells
# it; `numpy.core.*` is the numpy 1 spelling of the same module.
_NUMPY_NAMES = {
    ('numpy', 'ndarray'), ('numpy', 'dtype'),
    ('numpy._core.multiarray', '_reconstruct'), ('numpy._core.numeric', '_frombuffer'),
}
# The builtins the protocol-2 pickle of a deque of byte buffers names.
_PLAIN = {
    ('collections', 'deque'): collections.deque,
    ('_codecs', 'encode'): importlib.import_module('_codecs').encode,
    ('builtins', 'bytes'): bytes,
}


def _canonical(module: str) -> str:
    """numpy 2's spelling of a numpy module name."""
    if module == 'numpy.core' or module.startswith('numpy.core.'):
        return 'numpy._core' + module[len('numpy.core'):]
    return module


def _numpy_object(module: str, name: str):
    """`module.name` from whichever spelling of the module this numpy imports without error."""
    spellings = [module]
    if module.startswith('numpy._core'):
        spellings.append('numpy.core' + module[len('numpy._core'):])
    for spelling in spellings:
        with warnings.catch_warnings():
            # numpy 2 warns that numpy.core is deprecated; the object is the same.
            warnings.simplefilter('ignore')
            try:
                return getattr(importlib.import_module(spelling), name)
            except (ImportError, AttributeError):
                pass
    raise pickle.UnpicklingError(f'this numpy has no `{module}.{name}` for the frames of the state')


def frames_of(stack: np.ndarray, agents: int) -> list:
    """GRF's four frames, oldest first, of one environment's stack `[agents, ..., 4 * n]`."""
    parts = np.split(np.asarray(stack), FRAMES, axis=-1)
    if agents == 1:
        parts = [part[0] for part in parts]
    return [np.ascontiguousarray(part) for part in parts]


def pickled_frames(frames: list) -> bytes:
    """The protocol-2 opcodes of GRF's deque of `frames`, stripped of the PROTO header and the STOP
    opcode, so they can stand as the value of a key inside another pickle that keeps no memo."""
    body = pickle.dumps(collections.deque(frames, maxlen=FRAMES), protocol=2)
    header, stop = bytes((pickle.PROTO[0], 2)), pickle.STOP
    if not (body.startswith(header) and body.endswith(stop)):
        raise RuntimeError('the pickle of the frame stack is not framed as protocol 2')
    return body[len(header):-len(stop)]


def find_class(module: str, name: str):
    """The object for a global that a pickled frame stack may name; None for any other global."""
    if (module, name) in _PLAIN:
        return _PLAIN[module, name]
    if (_canonical(module), name) in _NUMPY_NAMES:
        return _numpy_object(_canonical(module), name)
    return None


def stack_bytes(frames, agents: int, shape: tuple, dtype: str) -> bytes:
    """The batch's stack, `[agents, *shape[:-1], 4 * shape[-1]]` as bytes, of GRF's four frames.

    Raises ValueError unless `frames` is a deque (or list or tuple) of four arrays of the frame's
    shape (with the agent axis for several agents) and type."""
    if not isinstance(frames, (collections.deque, list, tuple)) or len(frames) != FRAMES:
        raise ValueError(f'expected the {FRAMES} frames of GRF in the FrameStack of the state')
    frame_shape = tuple(shape) if agents == 1 else (agents, *shape)
    wanted = np.dtype(dtype)
    arrays = [np.asarray(frame) for frame in frames]
    for array in arrays:
        if array.shape != frame_shape or array.dtype != wanted:
            raise ValueError(f'expected frames of the shape {frame_shape} and the type {dtype} in the state, found '
                             f'{array.shape} and {array.dtype}')
    # [frame, agents, ..., c] -> [agents, ..., frame, c] -> [agents, ..., frame * c + c'].
    block = np.stack(arrays).reshape((FRAMES, agents, *shape))
    block = np.moveaxis(block, 0, -2)
    return np.ascontiguousarray(block).reshape((agents, *shape[:-1], FRAMES * shape[-1])).tobytes()

"""`torch.compile` support: the operator `cuju_amd::advance`, through which a compiled program steps
a batch, or restarts its ended environments, without a graph break (the reference's compiled-step
surface is python/cuju/_batch/environment.py:983-1056).

The operator carries no Python object. A batch is named by its native handle, the library's
pointer as an integer, and each output tensor by the library buffer it views: a location string,
`name` for a whole buffer (`simple115`, `reward`, ...) or `name@offset` for a raw array inside the
`raw` buffers. A call runs the library on the current stream. Functionalization hands the operator
stand-ins for its mutated arguments rather than the batch's own tensors, so after the call every
stand-in gets the bytes of the library buffer it names. The outputs are declared mutated, so the
compiler orders each later read of them after the call and never drops the call. Handles are
checked against the open batches: a compiled program that outlives its batch raises instead of
reaching freed memory.

`what` packs the call: bit 0 selects a reset of the ended environments over a step, bit 1 waits
for the device after the call (debug batches), bit 2 checks the action range first, and bits 8 and
up hold the action count that check uses.
"""

from __future__ import annotations

import ctypes

import torch

from .errors import ActionRangeError, ClosedError, from_library
from .library import DeviceArray

RESET_DONE = 1
SYNCHRONIZE = 2
CHECK_ACTIONS = 4

# The open batches: native handle -> the loaded library that made it.
_OPEN: dict[int, ctypes.CDLL] = {}


def opened(handle: int, lib) -> None:
    _OPEN[handle] = lib


def closed(handle: int) -> None:
    _OPEN.pop(handle, None)


def packed(reset_done: bool, synchronize: bool, check_actions: bool, action_count: int) -> int:
    return ((RESET_DONE if reset_done else 0) | (SYNCHRONIZE if synchronize else 0) |
            (CHECK_ACTIONS if check_actions else 0) | (action_count << 8))


_NAMESPACE = torch.library.Library('cuju_amd', 'DEF')
_NAMESPACE.define('advance(int handle, int what, Tensor actions, str[] locations, Tensor(a!)[] outputs) -> ()')


def _check(lib, status):
    if status == -2:
        raise ActionRangeError(lib.cuju_last_error().decode())
    if status != 0:
        raise from_library(lib.cuju_last_error().decode())


def _library_tensor(lib, handle, location, like):
    """The library buffer at `location`, viewed with the shape and type of `like`."""
    name, _, offset = location.partition('@')
    pointer = lib.cuju_environment_buffer(handle, name.encode())
    if not pointer:
        raise from_library(lib.cuju_last_error().decode())
    return torch.as_tensor(DeviceArray(pointer + int(offset or 0), like.shape, like.dtype, None), device=like.device)


def _advance(handle, what, actions, locations, outputs):
    lib = _OPEN.get(handle)
    if lib is None:
        raise ClosedError('the batch of this compiled call is closed')
    device = outputs[0].device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        if what & RESET_DONE:
            status = lib.cuju_environment_reset_done(handle, stream)
        else:
            count = what >> 8
            if what & CHECK_ACTIONS and bool(((actions < -count) | (actions >= count)).any()):
                raise ActionRangeError(f'expected action indices from {-count} to {count - 1}')
            status = lib.cuju_environment_step(handle, actions.data_ptr(), 1, stream, 0)
        _check(lib, status)
        if what & SYNCHRONIZE:
            _check(lib, lib.cuju_environment_synchronize(handle, stream))
    for location, given in zip(locations, outputs):
        own = _library_tensor(lib, handle, location, given)
        if given.data_ptr() != own.data_ptr():
            given.copy_(own)


_NAMESPACE.impl('advance', _advance, 'CUDA')


@torch.library.register_fake('cuju_amd::advance')
def _advance_fake(handle, what, actions, locations, outputs):
    return None

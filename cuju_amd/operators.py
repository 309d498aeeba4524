"""The `torch.library` operators through which `torch.compile` traces a step without a graph break
(python/cuju/_batch/operators.py).

`cuju_amd::step` and `cuju_amd::reset_done` find their batch by an integer key and declare the
batch's output tensors as mutated arguments, so the compiler orders every read of an output after
the call and never drops it. Each runs the library call the eager method runs.
"""

from __future__ import annotations

import itertools
import weakref

import torch

_BATCHES: weakref.WeakValueDictionary = weakref.WeakValueDictionary()
_KEYS = itertools.count(1)


def register(batch) -> int:
    """A new key under which the operators find `batch`; a dead batch drops out."""
    key = next(_KEYS)
    _BATCHES[key] = batch
    return key


def _batch(key: int):
    batch = _BATCHES.get(key)
    if batch is None:
        raise RuntimeError('the batch of this compiled step is gone')
    return batch


@torch.library.custom_op('cuju_amd::step', mutates_args=('outputs',))
def step(batch: int, actions: torch.Tensor, outputs: list[torch.Tensor]) -> None:
    """Steps the batch of key `batch` with device `actions` and writes its outputs into `outputs`."""
    _batch(batch)._operator_step(actions, outputs)


@step.register_fake
def _step_fake(batch, actions, outputs):
    return None


@torch.library.custom_op('cuju_amd::reset_done', mutates_args=('outputs',))
def reset_done(batch: int, outputs: list[torch.Tensor]) -> None:
    """Resets the ended environments of the batch of key `batch` and writes `outputs`."""
    _batch(batch)._operator_reset_done(outputs)


@reset_done.register_fake
def _reset_done_fake(batch, outputs):
    return None

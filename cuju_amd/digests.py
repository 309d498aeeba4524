"""Digests of a batch's outputs, as the reference's self-check computes them
(python/cuju/action_log.py:44-145): `Digest` hashes outputs, and `digest` plays a scenario with
fixed actions and returns the SHA-256 of everything it produced. The shipped `digests.json` holds
such digests, so a digest of this build equal to one there shows the same run bit for bit."""

from __future__ import annotations

import ctypes
import hashlib
from typing import Any

import torch

__all__ = ['Digest', 'digest']


class Digest:
    """The SHA-256 of a sequence of outputs: a tensor adds the bytes of its elements in order, on
    any device; a dictionary adds its values by sorted key; a list or tuple adds its items in order;
    bytes add as they are."""

    def __init__(self) -> None:
        self._hash = hashlib.sha256()

    def update(self, value: Any) -> None:
        if isinstance(value, torch.Tensor):
            tensor = value.detach().to('cpu').contiguous()
            self._hash.update(ctypes.string_at(tensor.data_ptr(), tensor.numel() * tensor.element_size()))
        elif isinstance(value, dict):
            for key in sorted(value):
                self.update(value[key])
        elif isinstance(value, (list, tuple)):
            for item in value:
                self.update(item)
        elif isinstance(value, (bytes, bytearray)):
            self._hash.update(value)
        else:
            raise TypeError(f'expected tensors, dictionaries, sequences or bytes, found {value!r}')

    def copy(self) -> Digest:
        """A digest of the same outputs that goes on apart."""
        other = Digest()
        other._hash = self._hash.copy()
        return other

    def hexdigest(self) -> str:
        return self._hash.hexdigest()


def digest_actions(step: int, environment_count: int, agents: int, action_count: int) -> torch.Tensor:
    """Agent `a` of environment `e` takes `(7 step + 3 e + 5 a) mod action_count`, [E, A] int32."""
    environments = torch.arange(environment_count, dtype=torch.int64)[:, None]
    slots = torch.arange(agents, dtype=torch.int64)[None, :]
    return ((step * 7 + environments * 3 + slots * 5) % action_count).to(torch.int32)


def digest(assets: Any, device: Any = 'cuda', steps: int = 100, seed: int = 7, environment_count: int = 4,
           **options: Any) -> str:
    """Plays a batch with `digest_actions` and returns the SHA-256 of the reset's observation, each
    step's observation, reward and done flags, then every environment's state unless the batch
    stacks its observations. The reference's self-check plays 100 steps of 4 environments with
    seed 7."""
    from .environment import BatchEnvironment
    batch = BatchEnvironment(assets, environment_count=environment_count, device=device, seed=seed, **options)
    try:
        value = Digest()
        value.update(batch.reset())
        for step in range(steps):
            actions = digest_actions(step, environment_count, batch.agents, batch.action_count)
            observation, reward, done, _ = batch.step(actions.to(batch.torch_device))
            value.update(observation)
            value.update(reward)
            value.update(done)
        if not batch.stacked:
            for index in range(environment_count):
                value.update(batch.get_state(index))
        return value.hexdigest()
    finally:
        batch.close()

"""Digests of a batch's outputs, as the reference's self-check computes them
(python/cuju/action_log.py:44-145): `Digest` hashes outputs, and `digest` plays a scenario with
fixed actions and returns the SHA-256 of everything it produced. The shipped `digests.json` holds
such digests, so a digest of this build equal to one there shows the same run bit for bit."""

from __future__ import annotations

import hashlib
from typing import Any, Iterator

import torch

__all__ = ['Digest', 'digest']


def _chunks(value: Any) -> Iterator[bytes]:
    """The bytes a value contributes to a digest, in order: a tensor its elements' bytes in
    row-major order (from any device), a dictionary its values by sorted key, a list or tuple its
    items, bytes themselves."""
    if isinstance(value, (bytes, bytearray)):
        yield bytes(value)
    elif isinstance(value, torch.Tensor):
        flat = value.detach().to('cpu').contiguous().reshape(-1)
        # Reinterpreting a one-dimensional tensor as bytes spreads each element over its width.
        yield flat.view(torch.uint8).numpy().tobytes() if flat.numel() else b''
    elif isinstance(value, dict):
        for key in sorted(value):
            yield from _chunks(value[key])
    elif isinstance(value, (list, tuple)):
        for item in value:
            yield from _chunks(item)
    else:
        raise TypeError(f'expected tensors, dictionaries, sequences or bytes, found {value!r}')


class Digest:
    """The SHA-256 of a sequence of outputs, each added as `_chunks` lays it out."""

    def __init__(self) -> None:
        self._hash = hashlib.sha256()

    def update(self, value: Any) -> None:
        # Every chunk is produced before any is hashed, so a value that raises adds nothing.
        for chunk in list(_chunks(value)):
            self._hash.update(chunk)

    def copy(self) -> Digest:
        """A digest of the same outputs that goes on apart."""
        other = Digest.__new__(Digest)
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

"""Per-environment digests of long episodes of the five benchmark workloads.

A sample of each workload's environments is played for thousands of steps: two ranges, one at
the start of the workload's index range and one at its end, each a batch of its own whose
`first_index` places it there. Inputs come from `cuju_amd.workloads`, so a
sampled environment plays exactly what it plays in the full batch.

The start range plays one environment to a wavefront (a step then takes the least time), the end
range at the geometry the full batch gets, several environments sharing each wavefront, as the
benchmark runs them.

The digest of one environment is SHA-256 over, in order:

* its observation after the reset;
* at every step, its observation, reward and done flag (uint8), then its final observation when
  its episode ended at that step (the automatic reset replaced the observation);
* after every masked reset of workload 4, its observation;
* at a checkpoint, its state: the `get_state` bytes for an unstacked batch (GRF's episode pickle
  and the engine bytes), the engine bytes alone for a stacked one.

`tests/golden/make_episodes.py` plays the sample on the reference CPU library and commits the
digests at each checkpoint; `tests/test_gpu_long.py` plays it on the device.
"""

from __future__ import annotations

import hashlib
import struct

import numpy as np

from cuju_amd import workloads

RANGE = 8
CHECKPOINTS = (3000, 5000, 10000)

# Environments per wavefront that the library gives each workload's full batch on an MI355X (256
# compute units, two wavefronts per SIMD): 1 x 64 lanes for 64 environments, 2 x 32 for 4,096,
# 8 x 8 for 16,384, 4 x 16 for 8,192 and 16 x 4 for 32,768.
PRODUCTION_MATCHES = {1: 1, 2: 2, 3: 8, 4: 4, 5: 16}
# Wavefronts of the end range, which plays at the full batch's geometry.
END_WAVEFRONTS = 4


def sample_ranges(workload):
    """(first index, count, environments per wavefront) of the sampled ranges: `RANGE`
    environments at the start of the index range, one to a wavefront, and the end of the index
    range in `END_WAVEFRONTS` full wavefronts of the geometry the full batch gets (at most half of
    the batch)."""
    n = workload.environments
    matches = PRODUCTION_MATCHES[workload.number]
    end = max(RANGE, min(n // 2, matches * END_WAVEFRONTS))
    return [(0, RANGE, 1), (n - end, end, matches)]


def seed_of(workload):
    return 1000 + workload.number


def observation_bytes(x) -> list:
    """Per-environment bytes of an observation array `[E][A][...]`."""
    x = np.ascontiguousarray(x)
    return [x[i].tobytes() for i in range(x.shape[0])]


def engine_bytes(state: bytes) -> bytes:
    """The engine bytes of `get_state` bytes: they follow the length-prefixed episode pickle."""
    (length,) = struct.unpack_from('<i', state, 0)
    return state[4 + length:]


class OracleSide:
    """The reference CPU library (test infrastructure only)."""

    def __init__(self, workload, first_index, count, drill_paths=None, library_path=None, threads=0):
        from oracle import ref
        options = workload.batch_options(first_index, count, drill_paths)
        assets = options.pop('assets')
        self.batch = ref.ReferenceBatch(assets, seed=seed_of(workload), threads=threads, library_path=library_path,
                                        **options)
        self.stacked = workload.stacked

    def reset(self):
        return np.array(self.batch.reset())

    def reset_masked(self, mask, seeds):
        return np.array(self.batch.reset(seeds=seeds, mask=mask))

    def launch(self, actions):
        self.out = self.batch.step(actions)

    def collect(self):
        obs, reward, done = self.out
        final = np.array(self.batch.final_observation()) if done.any() else None
        return np.array(obs), np.array(reward), np.array(done, dtype=np.uint8), final

    def state(self, index):
        if self.stacked:
            return self.batch.raw_state(index)[0]
        return self.batch.get_state(index)

    def close(self):
        self.batch.close()


class EpisodeRun:
    """Plays one range of a workload on a side, keeping each environment's running digest."""

    def __init__(self, workload, first_index, count, side, checkpoints=CHECKPOINTS):
        self.workload = workload
        self.first_index = first_index
        self.count = count
        self.side = side
        self.checkpoints = tuple(checkpoints)
        self.step = 0
        self.hashes = [hashlib.sha256() for _ in range(count)]
        self.digests = {}

    @property
    def name(self):
        return f'workload {self.workload.number} [{self.first_index}, {self.first_index + self.count})'

    def _absorb(self, parts, only=None):
        for i, part in enumerate(parts):
            if only is None or only[i]:
                self.hashes[i].update(part)

    def start(self):
        self._absorb(observation_bytes(self.side.reset()))

    def launch(self):
        w = self.workload
        self.side.launch(workloads.actions(seed_of(w), self.step, self.first_index, self.count, w.agents))

    def collect(self):
        obs, reward, done, final = self.side.collect()
        obs_parts, reward_parts = observation_bytes(obs), observation_bytes(reward)
        for i in range(self.count):
            self.hashes[i].update(obs_parts[i])
            self.hashes[i].update(reward_parts[i])
            self.hashes[i].update(bytes([int(done[i])]))
        if final is not None:
            self._absorb(observation_bytes(final), only=done)
        self.step += 1
        w = self.workload
        if w.reset_every and self.step % w.reset_every == 0:
            mask, seeds = workloads.masked_reset(seed_of(w), self.step, self.first_index, self.count, w.reset_percent)
            self._absorb(observation_bytes(self.side.reset_masked(mask, seeds)))
        if self.step in self.checkpoints:
            found = []
            for i in range(self.count):
                h = self.hashes[i].copy()
                h.update(self.side.state(i))
                found.append(h.hexdigest())
            self.digests[self.step] = found

    @property
    def done(self):
        return self.step >= max(self.checkpoints)

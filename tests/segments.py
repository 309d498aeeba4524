"""Ten thousand steps of a benchmark workload at its production geometry, in one batch.

A step of a few wavefronts takes the time of one match's step, so a 10,000-step episode played
from the start would take that long ten thousand times over. Instead the batch holds four blocks
of `M` environments, `M` the environments per wavefront that the workload's full batch gets, so
each block fills one wavefront of that geometry:

* block 0 plays environments first_index .. first_index + M - 1 of the workload from the reset;
* block b (1, 2, 3) starts from the states of those same environments at global step
  `STARTS[b]`, which the reference CPU library reaches by playing them from the reset, and plays
  their inputs (actions and masked resets of those environments at those global steps) from there.

Every block plays `SEGMENT` steps, so together the blocks cover global steps 0 to 10,000. The
reference library plays the same batch (same environments, states and inputs); each
environment's digest over its block's steps (the observation after the reset or the state load,
then every step's observation, reward, done flag and final observation, and the observations of
its masked resets) and its state at the end must be equal. Block 0 is the start of
`tests/golden/episodes.json`'s end range, so its digests at step 3,000 are also those goldens.

The oracle here is test infrastructure: it supplies the states the blocks start from and the
digests they must reach.
"""

from __future__ import annotations

import hashlib

import numpy as np
import torch

import episodes
from cuju_amd import workloads

STARTS = (0, 2500, 5000, 7000)
SEGMENT = 3000
BLOCKS = len(STARTS)


def first_index(workload):
    """The first environment of block 0: the start of the goldens' end range."""
    first, _, _ = episodes.sample_ranges(workload)[1]
    return first


def block_options(workload, drill_paths, blocks=BLOCKS):
    """Options of the batch of `blocks` blocks: the end range's first index, blocks x M
    environments, and for the mixed workload every block with the bundles of block 0's
    environments."""
    m = episodes.PRODUCTION_MATCHES[workload.number]
    f = first_index(workload)
    options = workload.batch_options(f, blocks * m, drill_paths)
    if workload.number == 5:
        options['assignment'] = np.tile(workload.assignment(f, m), blocks)
    return options


class Inputs:
    """The inputs of the blocks at each local step: block b plays block 0's environments' inputs at
    global step starts[b] + t."""

    def __init__(self, workload, m, starts=STARTS):
        self.w, self.m, self.f, self.seed = workload, m, first_index(workload), episodes.seed_of(workload)
        self.starts = tuple(starts)

    def actions(self, t):
        return np.concatenate([workloads.actions(self.seed, s + t, self.f, self.m, self.w.agents) for s in self.starts])

    def masked_reset(self, t):
        """After local step t (0-based): the mask, seeds and the environments whose block's
        schedule resets now, or None when no block's does."""
        w = self.w
        if not w.reset_every:
            return None
        n = len(self.starts) * self.m
        mask = np.zeros(n, np.uint8)
        seeds = np.zeros(n, np.int64)
        due = np.zeros(n, bool)
        for b, s in enumerate(self.starts):
            g = s + t + 1
            if g % w.reset_every == 0:
                bm, bs = workloads.masked_reset(self.seed, g, self.f, self.m, w.reset_percent)
                mask[b * self.m:(b + 1) * self.m] = bm
                seeds[b * self.m:(b + 1) * self.m] = bs
                due[b * self.m:(b + 1) * self.m] = True
        return (mask, seeds, due) if due.any() else None


def starting_states(workload, drill_paths, library_path=None, starts=STARTS):
    """The states of block 0's environments at starts[1:] on the reference library, each as the
    engine bytes, the episode words and (for a stacked batch) the observation stack."""
    from oracle import ref
    m = episodes.PRODUCTION_MATCHES[workload.number]
    f = first_index(workload)
    options = workload.batch_options(f, m, drill_paths)
    assets = options.pop('assets')
    batch = ref.ReferenceBatch(assets, seed=episodes.seed_of(workload), threads=0, library_path=library_path, **options)
    seed = episodes.seed_of(workload)
    states = {}
    try:
        batch.reset()
        for t in range(starts[-1]):
            batch.step(workloads.actions(seed, t, f, m, workload.agents))
            if workload.reset_every and (t + 1) % workload.reset_every == 0:
                mask, seeds = workloads.masked_reset(seed, t + 1, f, m, workload.reset_percent)
                batch.reset(seeds=seeds, mask=mask)
            if t + 1 in starts:
                stack = np.array(batch.observation()) if workload.stacked else None
                states[t + 1] = [(*batch.raw_state(j), None if stack is None else stack[j]) for j in range(m)]
    finally:
        batch.close()
    return states


class BlockRun:
    """Plays the four-block batch on a side (the device or the reference) and keeps each
    environment's running digest. A side has reset(), load(env, match, episode, stack),
    reset_masked(mask, seeds), launch(actions), ready(), collect() and state(env)."""

    def __init__(self, workload, side, states, starts=STARTS, segment=SEGMENT):
        self.workload, self.side, self.states = workload, side, states
        self.starts, self.segment = tuple(starts), segment
        self.m = episodes.PRODUCTION_MATCHES[workload.number]
        self.count = len(self.starts) * self.m
        self.inputs = Inputs(workload, self.m, self.starts)
        self.hashes = [hashlib.sha256() for _ in range(self.count)]
        self.step = 0
        self.digests = None

    @property
    def name(self):
        return f'workload {self.workload.number} in blocks from steps {list(self.starts)}'

    def start(self):
        obs = self.side.reset()
        for b in range(1, len(self.starts)):
            for j, (match, episode, stack) in enumerate(self.states[self.starts[b]]):
                self.side.load(b * self.m + j, match, episode, stack)
        obs = self.side.observation()
        for i, part in enumerate(episodes.observation_bytes(obs)):
            self.hashes[i].update(part)

    def launch(self):
        self.side.launch(self.inputs.actions(self.step))

    def ready(self):
        return self.side.ready()

    def collect(self):
        obs, reward, done, final = self.side.collect()
        obs_parts, reward_parts = episodes.observation_bytes(obs), episodes.observation_bytes(reward)
        for i in range(self.count):
            self.hashes[i].update(obs_parts[i])
            self.hashes[i].update(reward_parts[i])
            self.hashes[i].update(bytes([int(done[i])]))
        if final is not None:
            for i, part in enumerate(episodes.observation_bytes(final)):
                if done[i]:
                    self.hashes[i].update(part)
        due = self.inputs.masked_reset(self.step)
        self.step += 1
        if due is not None:
            mask, seeds, which = due
            for i, part in enumerate(episodes.observation_bytes(self.side.reset_masked(mask, seeds))):
                if which[i]:
                    self.hashes[i].update(part)
        if self.done:
            found = []
            for i in range(self.count):
                h = self.hashes[i].copy()
                h.update(self.side.state(i))
                found.append(h.hexdigest())
            self.digests = found

    @property
    def done(self):
        return self.step >= self.segment


class OracleBlocks:
    """The four-block batch on the reference CPU library."""

    def __init__(self, workload, drill_paths, library_path=None, blocks=BLOCKS):
        from oracle import ref
        options = block_options(workload, drill_paths, blocks)
        assets = options.pop('assets')
        self.batch = ref.ReferenceBatch(assets, seed=episodes.seed_of(workload), threads=0, library_path=library_path,
                                        **options)
        self.stacked = workload.stacked

    def reset(self):
        return np.array(self.batch.reset())

    def observation(self):
        return np.array(self.batch.observation())

    def load(self, env, match, episode, stack):
        self.batch.set_raw_state(env, match, episode)
        if stack is not None:
            self.batch.set_stack(env, 'simple115', stack)

    def reset_masked(self, mask, seeds):
        return np.array(self.batch.reset(seeds=seeds, mask=mask))

    def launch(self, actions):
        self.out = self.batch.step(actions)

    def ready(self):
        return True

    def collect(self):
        obs, reward, done = self.out
        final = np.array(self.batch.final_observation()) if done.any() else None
        return np.array(obs), np.array(reward), np.array(done, dtype=np.uint8), final

    def state(self, index):
        return self.batch.raw_state(index)[0] if self.stacked else self.batch.get_state(index)

    def close(self):
        self.batch.close()


def play_oracle(run):
    run.start()
    while not run.done:
        run.launch()
        run.collect()
    run.side.close()
    return run.digests


class DeviceBlocks:
    """The four-block batch on the device, on a stream of its own."""

    def __init__(self, workload, drill_paths, library, matches_per_wavefront, stream=None):
        import ctypes
        import cuju_amd
        import lockstep
        self.ctypes = ctypes
        options = block_options(workload, drill_paths)
        assets = options.pop('assets')
        with lockstep.matches_per_wavefront(matches_per_wavefront):
            self.batch = cuju_amd.BatchEnvironment(assets, library=library, device='cuda:0',
                                                   seed=episodes.seed_of(workload), **options)
        self.stream = stream or torch.cuda.Stream()
        self.stacked = workload.stacked
        self.geometry = self.batch.geometry

    def _host(self, x):
        return x.detach().cpu().numpy()

    def reset(self):
        with torch.cuda.stream(self.stream):
            obs = self.batch.reset()
        self.stream.synchronize()
        return self._host(obs)

    def observation(self):
        with torch.cuda.stream(self.stream):
            obs = self._host(self.batch.observation())
        return obs

    def load(self, env, match, episode, stack):
        ctypes = self.ctypes
        lib, handle = self.batch._lib, self.batch._handle()
        words = (ctypes.c_int * len(episode))(*episode)
        self.stream.synchronize()
        if lib.cuju_environment_set_state(handle, env, match, len(match), words) != 0:
            raise RuntimeError(lib.cuju_last_error().decode())
        if stack is not None:
            frames = np.ascontiguousarray(stack)
            if lib.cuju_environment_set_stack(handle, env, b'simple115', frames.ctypes.data, frames.nbytes) != 0:
                raise RuntimeError(lib.cuju_last_error().decode())

    def reset_masked(self, mask, seeds):
        with torch.cuda.stream(self.stream):
            obs = self.batch.reset(seeds=seeds, mask=torch.as_tensor(mask.astype(bool)))
        self.stream.synchronize()
        return self._host(obs)

    def launch(self, actions):
        with torch.cuda.stream(self.stream):
            self.out = self.batch.step(torch.as_tensor(actions, device='cuda:0'))

    def ready(self):
        return self.stream.query()

    def collect(self):
        self.stream.synchronize()
        obs, reward, done, info = self.out
        with torch.cuda.stream(self.stream):
            done = self._host(done).astype(np.uint8)
            final = self._host(info['final_observation']) if done.any() else None
            return self._host(obs), self._host(reward), done, final

    def state(self, index):
        state = self.batch.get_state(index, stacked=self.stacked)
        return episodes.engine_bytes(state) if self.stacked else state

    def close(self):
        self.batch.close()

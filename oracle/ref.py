"""Test infrastructure: a ctypes driver of the reference CPU library built into `oracle/_ref/`.

This module is the oracle's entry point for the whole GRF step. It loads
`oracle/_ref/libcuju_cpu.so`, which `oracle/Makefile` compiles from the reference's own sources
(`src/cuju_cpu.cpp`, `src/environment_state.cpp`), and drives it through the reference C ABI
(`src/environment_api.h:47-95` for the configuration, `:252-317` for reset and step, `:367-388` for
`get_state`). Only tests, the smoke check and the CPU-baseline leg of the benchmark may import it,
and only as the checker or the timed baseline; the product never loads it.

The digest follows the reference self-check (`tests/conftest.py:60-98`): SHA-256 over every
observation, reward and done flag of every step, then every environment's `get_state` bytes, which
carry GRF's pickle header (`python/cuju/_batch/state.py:38-77`).
"""

from __future__ import annotations

import ctypes
import hashlib
import os
import re
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, '_ref', 'libcuju_cpu.so')
DATA = os.path.join(os.path.dirname(HERE), 'cuju_amd', 'data')

REPRESENTATIONS = {'simple115': 1, 'simple115v2': 2, 'extracted': 4, 'raw': 8}
ACTION_SETS = {'default': 0, 'v2': 1, 'full': 2}
ACTION_COUNTS = {'default': 19, 'v2': 20, 'full': 33}
MAXIMUM_AGENTS = 22


class Configuration(ctypes.Structure):
    """The reference `cuju_configuration`, version 2 (`src/environment_api.h:49-95`)."""

    _fields_ = [
        ('version', ctypes.c_int),
        ('assets', ctypes.POINTER(ctypes.c_char_p)),
        ('asset_count', ctypes.c_int),
        ('assignment', ctypes.c_void_p),
        ('animations', ctypes.c_char_p),
        ('environment_count', ctypes.c_int),
        ('seed', ctypes.c_ulonglong),
        ('action_set', ctypes.c_int),
        ('observation', ctypes.c_int),
        ('checkpoints', ctypes.c_int),
        ('numpy_legacy', ctypes.c_int),
        ('auto_reset', ctypes.c_int),
        ('threads', ctypes.c_int),
        ('ticks_per_step', ctypes.c_int),
        ('smm_width', ctypes.c_int),
        ('smm_height', ctypes.c_int),
        ('stack', ctypes.c_int),
        ('fixed_seeds', ctypes.c_void_p),
        ('agent_counts', ctypes.c_void_p),
        ('episode_number', ctypes.c_int),
        ('first_index', ctypes.c_ulonglong),
        ('allocate', ctypes.c_void_p),
        ('release', ctypes.c_void_p),
        ('allocator_context', ctypes.c_void_p),
        ('pin_threads', ctypes.c_int),
        ('numa', ctypes.c_int),
        ('page_aligned', ctypes.c_int),
    ]


def available() -> bool:
    return os.path.isfile(LIBRARY)


_libraries = {}


def library(path=None):
    """The reference library, or another library with the same C ABI at `path` (the tests drive
    the engine's host debugging build through the same calls)."""
    path = path or LIBRARY
    if path not in _libraries:
        if not os.path.isfile(path):
            raise FileNotFoundError(f'the library is not built: {path}')
        lib = ctypes.CDLL(path)
        lib.cuju_last_error.restype = ctypes.c_char_p
        lib.cuju_environment_create.restype = ctypes.c_void_p
        lib.cuju_environment_create.argtypes = [ctypes.POINTER(Configuration)]
        for name in ('count', 'threads'):
            getattr(lib, f'cuju_environment_{name}').argtypes = [ctypes.c_void_p]
        lib.cuju_environment_agents.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.cuju_environment_players.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.cuju_environment_destroy.argtypes = [ctypes.c_void_p]
        lib.cuju_environment_reset.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p]
        lib.cuju_environment_reset_masked.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_int]
        lib.cuju_environment_step.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                              ctypes.c_void_p, ctypes.c_int]
        lib.cuju_environment_get_state.restype = ctypes.c_void_p
        lib.cuju_environment_get_state.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_ulonglong), ctypes.c_void_p]
        lib.cuju_environment_buffer.restype = ctypes.c_void_p
        lib.cuju_environment_buffer.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        lib.cuju_environment_set_difficulty.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.cuju_environment_raw_field.restype = ctypes.c_char_p
        lib.cuju_environment_raw_field.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                                   ctypes.c_void_p, ctypes.POINTER(ctypes.c_ulonglong)]
        lib.cuju_environment_set_state.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p,
                                                   ctypes.c_ulonglong, ctypes.c_void_p]
        lib.cuju_environment_set_stack.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p,
                                                   ctypes.c_ulonglong]
        lib.cuju_environment_episode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        _libraries[path] = lib
    return _libraries[path]


# By the type code of `cuju_environment_raw_field` (`src/environment_api.h:446-460`).
RAW_TYPES = (np.float32, np.int32, np.bool_, np.uint8)


def describe_raw(lib, handle, environments, agents):
    """Name, type, shape and byte offset of each raw array of a batch, empty without raw."""
    fields = []
    element_type, offset = ctypes.c_int(), ctypes.c_ulonglong()
    dimensions = (ctypes.c_int * 2)()
    for field in range(64):
        name = lib.cuju_environment_raw_field(handle, field, ctypes.byref(element_type), dimensions,
                                              ctypes.byref(offset))
        if name is None:
            break
        shape = (environments, agents, *(d for d in dimensions if d))
        fields.append((name.decode(), RAW_TYPES[element_type.value], shape, offset.value))
    return fields


def observation_bytes(observation):
    """The bytes a digest hashes of an observation: a raw dictionary by sorted name
    (`python/cuju/check.py:81-87`)."""
    if isinstance(observation, dict):
        return b''.join(np.ascontiguousarray(observation[name]).tobytes() for name in sorted(observation))
    return np.ascontiguousarray(observation).tobytes()


def resolve_asset(name: str):
    """`<scenario>_l<L>_r<R>` to the shipped bundle and the agents per side
    (`python/cuju/_batch/assets.py:39-68`): the bundle with the fewest agents serves any counts.
    The path of a bundle file keeps its own agents."""
    if os.path.isfile(name):
        return name, (-1, -1)
    directory = os.path.join(DATA, 'assets')
    shipped = os.path.join(directory, name + '.cjb')
    if os.path.isfile(shipped):
        return shipped, (-1, -1)
    match = re.fullmatch(r'(.+)_l(\d+)_r(\d+)', name)
    if match is None:
        return os.path.join(directory, name + '_l0_r0.cjb'), (1, 0)
    return (os.path.join(directory, match.group(1) + '_l0_r0.cjb'),
            (int(match.group(2)), int(match.group(3))))


def _pickle_string(value: str) -> bytes:
    data = value.encode()
    return b'X' + struct.pack('<I', len(data)) + data


def _pickle_integer(value: int) -> bytes:
    return b'J' + struct.pack('<i', value)


def episode_pickle(episode, collected=None) -> bytes:
    """GRF's state pickle of the episode logic (`python/cuju/_batch/state.py:45-77`)."""
    logic = b''.join(
        _pickle_string(key) + _pickle_integer(value)
        for key, value in zip(('previous_score_diff', 'previous_game_mode',
                               'prev_ball_owned_team'), episode))
    data = (b'\x80\x02}(' + _pickle_string('FootballEnvCore')
            + b'cgfootball.env.football_env_core\nEnvState\n' + b')\x81}(' + logic + b'ub')
    if collected is not None:
        data += (_pickle_string('CheckpointRewardWrapper') + b'}('
                 + b''.join(_pickle_integer(a) + _pickle_integer(c)
                            for a, c in enumerate(collected) if c) + b'u')
    return data + b'u.'


class ReferenceBatch:
    """A batch of the reference CPU library with the options of `cuju.BatchEnvironment`."""

    def __init__(self, assets, environment_count=4, seed=0, representation='simple115v2',
                 rewards='scoring', action_set='default', stacked=False, auto_reset=True,
                 threads=0, assignment=None, agent_counts=None, first_index=0,
                 difficulty=None, numpy_legacy=True, episode_number=0,
                 physics_steps_per_frame=10, game_engine_random_seed=None, library_path=None,
                 with_raw=False, channel_dimensions=(96, 72)):
        lib = library(library_path)
        self._lib = lib
        names = [assets] if isinstance(assets, str) else list(assets)
        resolved = [resolve_asset(n) for n in names]
        counts = [pair if agent_counts is None else agent_counts[i]
                  for i, (_, pair) in enumerate(resolved)]
        self._paths = (ctypes.c_char_p * len(names))(*(p.encode() for p, _ in resolved))
        self._counts = (ctypes.c_int * (2 * len(names)))(*(c for pair in counts for c in pair))
        self._assignment = None
        if assignment is not None:
            self._assignment = np.ascontiguousarray(assignment, dtype=np.int32)
        self._fixed = None
        if game_engine_random_seed is not None:
            self._fixed = np.ascontiguousarray(np.broadcast_to(
                np.asarray(game_engine_random_seed, dtype=np.int64), (environment_count,)))
        self.checkpoints = 'checkpoints' in rewards.split(',')
        self.stack = 4 if stacked else 1
        self.representation = representation
        self.channel_dimensions = tuple(channel_dimensions)
        cfg = Configuration(
            version=2, assets=self._paths, asset_count=len(names),
            assignment=None if self._assignment is None else self._assignment.ctypes.data,
            animations=os.path.join(DATA, 'animations.bin').encode(),
            environment_count=environment_count, seed=seed,
            action_set=ACTION_SETS[action_set],
            observation=REPRESENTATIONS[representation] | (REPRESENTATIONS['raw'] if with_raw else 0),
            checkpoints=int(self.checkpoints), numpy_legacy=int(numpy_legacy),
            auto_reset=int(auto_reset), threads=threads,
            ticks_per_step=physics_steps_per_frame, smm_width=channel_dimensions[0],
            smm_height=channel_dimensions[1],
            stack=self.stack,
            fixed_seeds=None if self._fixed is None else self._fixed.ctypes.data,
            agent_counts=ctypes.addressof(self._counts), episode_number=episode_number,
            first_index=first_index, allocate=None, release=None, allocator_context=None,
            pin_threads=0, numa=0, page_aligned=0)
        handle = lib.cuju_environment_create(ctypes.byref(cfg))
        if not handle:
            raise RuntimeError(lib.cuju_last_error().decode())
        self._handle = handle
        self.environment_count = environment_count
        self.threads = lib.cuju_environment_threads(handle)
        self.left_agents = np.zeros(environment_count, dtype=np.int32)
        self.right_agents = np.zeros(environment_count, dtype=np.int32)
        self.agents = lib.cuju_environment_agents(handle, self.left_agents.ctypes.data,
                                                  self.right_agents.ctypes.data)
        self.action_count = ACTION_COUNTS[action_set]
        if difficulty is not None:
            values = np.ascontiguousarray(difficulty, dtype=np.float32).reshape(
                environment_count, 2)
            self._check(lib.cuju_environment_set_difficulty(handle, values.ctypes.data))
        self.raw_fields = describe_raw(lib, handle, environment_count, self.agents)

    def _raw(self, name):
        pointer = self._lib.cuju_environment_buffer(self._handle, name.encode())
        out = {}
        for field, dtype, shape, offset in self.raw_fields:
            count = int(np.prod(shape))
            buffer = (ctypes.c_char * (count * np.dtype(dtype).itemsize)).from_address(pointer + offset)
            out[field] = np.frombuffer(buffer, dtype=dtype).reshape(shape)
        return out

    def _observation(self, final):
        prefix = 'final_' if final else ''
        if self.representation == 'raw':
            return self._raw(prefix + 'raw')
        if self.representation == 'extracted':
            width, height = self.channel_dimensions
            return self._array(prefix + 'smm', np.uint8, (self.environment_count, self.agents, height, width, 4 * self.stack))
        return self._array(prefix + 'simple115', np.float32,
                           (self.environment_count, self.agents, 115 * self.stack))

    def _check(self, status):
        if status != 0:
            raise RuntimeError(self._lib.cuju_last_error().decode())

    def _array(self, name, dtype, shape):
        pointer = self._lib.cuju_environment_buffer(self._handle, name.encode())
        if not pointer:
            return None
        count = int(np.prod(shape))
        buffer = (ctypes.c_char * (count * np.dtype(dtype).itemsize)).from_address(pointer)
        return np.frombuffer(buffer, dtype=dtype).reshape(shape)

    def observation(self):
        """The observation of the batch's representation: `[E][A][115 * stack]` float32, the SMM
        `[E][A][72][96][4 * stack]` uint8, or for `raw` a dictionary of `[E][A]...` arrays."""
        return self._observation(False)

    def reward(self):
        return self._array('reward', np.float32, (self.environment_count, self.agents))

    def done(self):
        return self._array('done', np.uint8, (self.environment_count,))

    def score_reward(self):
        return self._array('score_reward', np.int32, (self.environment_count,))

    def final_observation(self):
        return self._observation(True)

    def raw(self, final=False):
        """The raw arrays of a batch of the raw representation or made `with_raw`."""
        return self._raw('final_raw' if final else 'raw')

    def reset(self, seeds=None, mask=None):
        if mask is None and seeds is None:
            self._check(self._lib.cuju_environment_reset(self._handle, None, None, None))
        else:
            m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
            s = None if seeds is None else np.ascontiguousarray(seeds, dtype=np.int64)
            self._check(self._lib.cuju_environment_reset_masked(
                self._handle, None if m is None else m.ctypes.data, 1,
                None if s is None else s.ctypes.data, None, None, 1))
        return self.observation()

    def step(self, actions):
        actions = np.ascontiguousarray(actions, dtype=np.int32)
        status = self._lib.cuju_environment_step(self._handle, actions.ctypes.data, 1, None, 1)
        self._check(status)
        return self.observation(), self.reward(), self.done()

    def raw_state(self, index):
        """`get_state` bytes of the library and the episode words."""
        size = ctypes.c_ulonglong()
        episode = (ctypes.c_int * (3 + MAXIMUM_AGENTS))()
        pointer = self._lib.cuju_environment_get_state(self._handle, index, ctypes.byref(size),
                                                       episode)
        if not pointer:
            raise RuntimeError(self._lib.cuju_last_error().decode())
        return ctypes.string_at(pointer, size.value), list(episode)

    def set_raw_state(self, index, match, episode):
        """`cuju_environment_set_state` (`src/environment_api.h:392-404`) with engine bytes and
        the episode words `raw_state` returned."""
        words = (ctypes.c_int * (3 + MAXIMUM_AGENTS))(*episode[:3 + MAXIMUM_AGENTS])
        self._check(self._lib.cuju_environment_set_state(self._handle, index, match, len(match), words))

    def set_stack(self, index, name, frames):
        """`cuju_environment_set_stack` (`src/environment_api.h:406-419`): the observation stack of
        environment `index`, `[agents][115 * stack]` float32 or the SMM's uint8 frames."""
        frames = np.ascontiguousarray(frames)
        self._check(self._lib.cuju_environment_set_stack(self._handle, index, name.encode(), frames.ctypes.data,
                                                         frames.nbytes))

    def episode(self, index):
        """`cuju_environment_episode` (`src/environment_api.h:470-516`): 17 episode values and the
        played then the scenario's (left, right) difficulties."""
        values = np.zeros(17, dtype=np.int64)
        difficulty = np.zeros(4, dtype=np.float32)
        self._check(self._lib.cuju_environment_episode(self._handle, index, values.ctypes.data,
                                                       difficulty.ctypes.data))
        return values, difficulty

    def get_state(self, index):
        """`BatchEnvironment.get_state` bytes: pickle length, pickle, then the match bytes."""
        match, episode = self.raw_state(index)
        collected = episode[3:3 + self.agents] if self.checkpoints else None
        data = episode_pickle(episode[:3], collected)
        return struct.pack('<i', len(data)) + data + match

    def close(self):
        if self._handle:
            self._lib.cuju_environment_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def actions_at(step, environments, agents, action_count):
    """The digest actions of the reference self-check (`tests/conftest.py:60-66`)."""
    e = np.arange(environments, dtype=np.int64)[:, None]
    a = np.arange(agents, dtype=np.int64)[None, :]
    return ((step * 7 + e * 3 + a * 5) % action_count).astype(np.int32)


def play_digest(batch_factory, assets, steps, seed=7, environments=4, **options):
    """SHA-256 of a played batch as `tests/conftest.py:69-98` defines it. `batch_factory` builds
    either a `ReferenceBatch` or any object with the same methods."""
    batch = batch_factory(assets, environment_count=environments, seed=seed, **options)
    digest = hashlib.sha256()
    digest.update(observation_bytes(batch.reset()))
    for step in range(steps):
        actions = actions_at(step, environments, batch.agents, batch.action_count)
        observation, reward, done = batch.step(actions)
        digest.update(observation_bytes(observation))
        digest.update(np.ascontiguousarray(reward).tobytes())
        digest.update(np.ascontiguousarray(done).tobytes())
    if batch.stack == 1:
        for index in range(environments):
            digest.update(batch.get_state(index))
    batch.close()
    return digest.hexdigest()

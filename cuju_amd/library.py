"""Loads the native library and declares its C ABI (include/cuju_amd.h) for ctypes.

The package calls only the HIP library `lib/libcuju_amd.so`. Without it every call fails with
`MissingFileError`: there is no other implementation to fall back to.
"""

from __future__ import annotations

import ctypes
import os

from .errors import MissingFileError

HERE = os.path.dirname(os.path.abspath(__file__))
PRODUCT = os.path.join(HERE, 'lib', 'libcuju_amd.so')
DATA = os.path.join(HERE, 'data')


class Configuration(ctypes.Structure):
    """`struct cuju_configuration`, version 2."""

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


class ScenarioPlayer(ctypes.Structure):
    """`struct cuju_scenario_player` (src/scenario_api.h:22-28)."""
    _fields_ = [('x', ctypes.c_double), ('y', ctypes.c_double), ('role', ctypes.c_int), ('lazy', ctypes.c_int),
                ('controllable', ctypes.c_int)]


class ScenarioDescription(ctypes.Structure):
    """`struct cuju_scenario_description`, version 1 (src/scenario_api.h:30-47)."""
    _fields_ = [
        ('version', ctypes.c_int), ('ball_x', ctypes.c_double), ('ball_y', ctypes.c_double),
        ('left_team', ctypes.POINTER(ScenarioPlayer)), ('left_size', ctypes.c_int),
        ('right_team', ctypes.POINTER(ScenarioPlayer)), ('right_size', ctypes.c_int),
        ('use_magnet', ctypes.c_int), ('offsides', ctypes.c_int), ('real_time', ctypes.c_int),
        ('left_team_difficulty', ctypes.c_double), ('right_team_difficulty', ctypes.c_double),
        ('deterministic', ctypes.c_int), ('end_episode_on_score', ctypes.c_int),
        ('end_episode_on_possession_change', ctypes.c_int), ('end_episode_on_out_of_play', ctypes.c_int),
        ('game_duration', ctypes.c_int), ('second_half', ctypes.c_int), ('control_all_players', ctypes.c_int),
        ('game_engine_random_seed', ctypes.c_uint),
    ]


# Every entry point of include/cuju_amd.h: (name, result, arguments).
P, I, U64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_ulonglong
SIGNATURES = [
    ('cuju_last_error', ctypes.c_char_p, []),
    ('cuju_backend', ctypes.c_char_p, []),
    ('cuju_environment_create', P, [ctypes.POINTER(Configuration)]),
    ('cuju_memory_estimate', I, [ctypes.POINTER(Configuration), ctypes.POINTER(U64)]),
    ('cuju_local_memory_bytes', I, [ctypes.POINTER(U64)]),
    ('cuju_environment_memory_bytes', U64, [P]),
    ('cuju_environment_destroy', None, [P]),
    ('cuju_environment_count', I, [P]),
    ('cuju_environment_geometry', I, [P, P]),
    ('cuju_environment_threads', I, [P]),
    ('cuju_environment_agents', I, [P, P, P]),
    ('cuju_environment_players', I, [P, P, P]),
    ('cuju_environment_set_difficulty', I, [P, P]),
    ('cuju_environment_difficulty', None, [P, P]),
    ('cuju_environment_reset', I, [P, P, P, P]),
    ('cuju_environment_reset_masked', I, [P, P, I, P, P, P, I]),
    ('cuju_environment_reset_done', I, [P, P]),
    ('cuju_environment_step', I, [P, P, I, P, I]),
    ('cuju_environment_step_no_alloc', I, [P, P, P]),
    ('cuju_environment_step_async', I, [P, P, I, P]),
    ('cuju_environment_step_wait', I, [P]),
    ('cuju_environment_synchronize', I, [P, P]),
    ('cuju_environment_get_state', P, [P, I, ctypes.POINTER(U64), P]),
    ('cuju_environment_set_state', I, [P, I, ctypes.c_char_p, U64, P]),
    ('cuju_environment_set_stack', I, [P, I, ctypes.c_char_p, P, U64]),
    ('cuju_environment_raw_field', ctypes.c_char_p, [P, I, P, P, P]),
    ('cuju_environment_buffer', P, [P, ctypes.c_char_p]),
    ('cuju_environment_episode', I, [P, I, P, P]),
    ('cuju_environment_scenario', ctypes.c_char_p, [P, I]),
    ('cuju_scenario_build_bundle', I, [ctypes.POINTER(ScenarioDescription), ctypes.POINTER(ScenarioDescription),
                                       ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]),
    ('cuju_debug_libm_device', I, [I, I, ctypes.c_uint, ctypes.c_longlong, P, P, P, P]),
]

_loaded = {}


def library_path(device=None) -> str:
    """The library `BatchEnvironment` loads by default for `device` (python/cuju/_batch/library.py:82-95).
    This build has one, the HIP library, for `cuda`, `cuda:N`, a `torch.device` of type `cuda`, `auto`
    or None; another device names no library here."""
    name = 'cuda' if device is None else str(device)
    if name != 'auto' and name.split(':')[0] != 'cuda':
        from .errors import ChoiceError
        raise ChoiceError(f'expected the device cuda, cuda:N or auto for the HIP library, found {device!r}')
    return PRODUCT


def load(path: str | None = None):
    """The library at `path`, by default the in-tree HIP build, with its signatures declared."""
    path = os.path.abspath(path or PRODUCT)
    if path not in _loaded:
        if not os.path.isfile(path):
            raise MissingFileError(
                f'the HIP library is not built: {path} (run `python -m cuju_amd.build`)')
        lib = ctypes.CDLL(path)
        for name, result, arguments in SIGNATURES:
            # Another library with the reference ABI (the reference's own, for its scenario
            # builder) lacks this build's debugging entry points.
            if not hasattr(lib, name):
                continue
            function = getattr(lib, name)
            function.restype = result
            function.argtypes = arguments
        _loaded[path] = lib
    return _loaded[path]


class DeviceArray:
    """A device buffer of the library that `torch.as_tensor` views without a copy, through
    `__cuda_array_interface__`; `owner` stays alive as long as any view does."""

    TYPES = {'float32': '<f4', 'int32': '<i4', 'uint8': '|u1', 'bool': '|b1'}

    def __init__(self, pointer, shape, dtype, owner):
        self.owner = owner
        self.__cuda_array_interface__ = {'data': (pointer, False), 'shape': tuple(shape),
                                         'typestr': self.TYPES[str(dtype).replace('torch.', '')], 'version': 2,
                                         'strides': None}


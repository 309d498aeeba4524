"""GRF scenario files to asset bundles, without GRF (the reference's counterpart is
python/cuju/scenarios.py; the C side is include/cuju/assets/scenario_builder.h).

A scenario file defines `build_scenario(builder)` against GRF's `Scenario` API: `config()`,
`SetTeam`, `AddPlayer`, `SetBallPosition` and `EpisodeNumber`. Running it against `Builder`
records a `Description`: the config fields, the ball and the two formations, as GRF would hand
them to its engine. One bundle holds one template per parity of the episode number, so `describe`
records the scenario for a spread of episode numbers, refuses what one bundle cannot hold, and
returns the even and odd descriptions. `build_bundle` hands those to the library's
`cuju_scenario_build_bundle`, which writes the agentless (`l0_r0`) bundle a batch loads:

    from cuju_amd import scenarios
    scenarios.build_bundle('my_drill.py', 'my_drill_l0_r0.cjb')

`BatchEnvironment` also takes the path of a scenario file in place of a bundle and builds it at
creation (into `CUJU_BUNDLE_CACHE` when that is set). A scenario that GRF refuses, or that one
bundle cannot hold, raises `ScenarioError`.
"""

from __future__ import annotations

import ctypes
import dataclasses
import enum
import hashlib
import importlib.util
import os
import random
import sys
import tempfile
import types
import warnings
from typing import Callable, NamedTuple

from . import library as _library
from .errors import ConfigurationError, from_library

__all__ = ['Builder', 'Description', 'PlayerRole', 'ScenarioConfig', 'ScenarioError', 'Team', 'build_bundle',
           'cache_directory', 'cached_bundle', 'describe', 'load_scenario']


class PlayerRole(enum.IntEnum):
    """GRF's `e_PlayerRole` values."""
    e_PlayerRole_GK = 0
    e_PlayerRole_CB = 1
    e_PlayerRole_LB = 2
    e_PlayerRole_RB = 3
    e_PlayerRole_DM = 4
    e_PlayerRole_CM = 5
    e_PlayerRole_LM = 6
    e_PlayerRole_RM = 7
    e_PlayerRole_AM = 8
    e_PlayerRole_CF = 9


class Team(enum.IntEnum):
    """GRF's `e_Team` values."""
    e_Left = 0
    e_Right = 1


class ScenarioError(ConfigurationError):
    """A scenario that GRF refuses or that a bundle cannot hold. It is a `ValueError`."""


# ---- values as GRF's boost.python bindings convert them ---------------------------------------------

def _coerce(kind: str, name: str, value):
    """The value a `ScenarioConfig` field of `kind` stores for `value`, or ScenarioError."""
    if kind == 'flag':
        if value is None or isinstance(value, int):  # bool is an int
            return bool(value)
        raise ScenarioError(f'expected True or False for {name}, found {value!r}')
    if kind == 'number':
        if isinstance(value, (int, float)):
            return float(value)
        raise ScenarioError(f'expected a number for {name}, found {value!r}')
    low, high = (0, 2 ** 32 - 1) if kind == 'seed' else (-2 ** 31, 2 ** 31 - 1)
    if not isinstance(value, int):
        raise ScenarioError(f'expected an integer for {name}, found {value!r}')
    if not low <= value <= high:
        raise ScenarioError(f'expected {name} from {low} to {high}, found {value}')
    return int(value)


class _Field(NamedTuple):
    name: str
    default: object
    kind: str


# The fields of GRF's `ScenarioConfig` a scenario may set, with GRF's defaults.
FIELDS = (
    _Field('use_magnet', True, 'flag'), _Field('offsides', True, 'flag'), _Field('real_time', False, 'flag'),
    _Field('left_team_difficulty', 1.0, 'number'), _Field('right_team_difficulty', 0.6, 'number'),
    _Field('deterministic', False, 'flag'), _Field('end_episode_on_score', False, 'flag'),
    _Field('end_episode_on_possession_change', False, 'flag'), _Field('end_episode_on_out_of_play', False, 'flag'),
    _Field('game_duration', 3000, 'integer'), _Field('second_half', 999999999, 'integer'),
    _Field('control_all_players', False, 'flag'), _Field('game_engine_random_seed', 42, 'seed'),
    _Field('reverse_team_processing', False, 'flag'), _Field('left_agents', 1, 'integer'),
    _Field('right_agents', 0, 'integer'),
)
# Fields the environment's own configuration sets after `build_scenario`, so a bundle ignores them.
_SET_BY_ENVIRONMENT = ('left_agents', 'right_agents', 'real_time')


class Player(NamedTuple):
    """One `AddPlayer` call: start position, role and flags, as GRF's `FormationEntry` holds it."""
    x: float
    y: float
    role: int
    lazy: bool
    controllable: bool


# GRF's `Scenario._FakePlayersForEmptyTeam`: an empty team gets this lazy goalkeeper.
_STAND_IN_KEEPER = Player(-1.0, 0.42, int(PlayerRole.e_PlayerRole_GK), True, True)
_TEAM_LIMIT = 11  # formation slots and persons of a GRF team


class _ConfigField:
    """A typed field of `ScenarioConfig`: reads the stored value, converts what is assigned."""

    def __init__(self, field: _Field):
        self.field = field

    def __get__(self, config, owner=None):
        if config is None:
            return self
        return config._values[self.field.name]

    def __set__(self, config, value):
        config._values[self.field.name] = _coerce(self.field.kind, self.field.name, value)


class _ComputedField:
    """A field GRF computes at its first read and then keeps for the match. A bundle is built
    before the agents are known, so a scenario that reads one cannot be held."""

    def __init__(self, compute: Callable):
        self.compute = compute

    def __set_name__(self, owner, name):
        self.name = name

    def __get__(self, config, owner=None):
        if config is None:
            return self
        object.__setattr__(config, '_computed_read', True)
        return self.compute(config)

    def __set__(self, config, value):
        raise AttributeError(f"can't set attribute {self.name}")


class ScenarioConfig:
    """What `builder.config()` returns. Known fields convert as GRF's bindings do; an unknown name
    is kept and ignored, as a boost.python instance keeps it, with a warning."""

    def __init__(self):
        object.__setattr__(self, '_values', {f.name: f.default for f in FIELDS})
        object.__setattr__(self, '_computed_read', False)
        object.__setattr__(self, 'left_team', [])
        object.__setattr__(self, 'right_team', [])
        object.__setattr__(self, 'ball_position', [0.0, 0.0, 0.0])

    def __setattr__(self, name, value):
        if isinstance(getattr(type(self), name, None), (_ConfigField, _ComputedField)):
            object.__setattr__(self, name, value)
        elif name in ('left_team', 'right_team', 'ball_position'):
            raise ScenarioError(f'set {name} through AddPlayer or SetBallPosition')
        else:
            warnings.warn(f'the scenario sets {name!r}, which GRF does not know and ignores', stacklevel=2)
            object.__setattr__(self, name, value)

    controllable_left_players = _ComputedField(lambda c: sum(p.controllable for p in c.left_team))
    controllable_right_players = _ComputedField(lambda c: sum(p.controllable for p in c.right_team))
    # Whether agents choose their players as play goes: unless each side's agents control exactly
    # its controllable players, or that side has no agents.
    dynamic_player_selection = _ComputedField(
        lambda c: not all(agents == 0 or agents == sum(p.controllable for p in team)
                          for agents, team in ((c._values['left_agents'], c.left_team),
                                               (c._values['right_agents'], c.right_team))))


for _field in FIELDS:
    setattr(ScenarioConfig, _field.name, _ConfigField(_field))


class Builder:
    """The `builder` that `build_scenario` receives, behaving as GRF's `Scenario` does."""

    def __init__(self, episode_number: int):
        self._config = ScenarioConfig()
        self._team = Team.e_Left
        self._episode = episode_number

    def config(self):
        return self._config

    ScenarioConfig = config  # GRF exposes the config under both names

    def SetTeam(self, team):
        self._team = team

    def AddPlayer(self, x, y, role, lazy=False, controllable=True):
        if not isinstance(role, PlayerRole):
            raise ScenarioError(f'expected a role such as e_PlayerRole_GK, found {role!r}')
        player = Player(_coerce('number', 'x', x), _coerce('number', 'y', y), int(role), _coerce('flag', 'lazy', lazy),
                        _coerce('flag', 'controllable', controllable))
        team = self._config.left_team if self._team == Team.e_Left else self._config.right_team
        team.append(player)

    def SetBallPosition(self, ball_x, ball_y):
        self._config.ball_position[:2] = [_coerce('number', 'ball_x', ball_x), _coerce('number', 'ball_y', ball_y)]

    def EpisodeNumber(self):
        return self._episode


# ---- what one episode's run records, and what a bundle can hold ------------------------------------

@dataclasses.dataclass(frozen=True)
class Description:
    """The scenario GRF would build for one episode number: the config values a bundle stores
    (the environment sets the others), the ball's start and the two formations."""
    values: dict
    ball: tuple
    left: tuple
    right: tuple


def _random_states():
    numpy = sys.modules.get('numpy')
    numpy_state = None
    if numpy is not None:
        kind, keys, position, has_gauss, gauss = numpy.random.get_state()
        numpy_state = (kind, keys.tobytes(), position, has_gauss, gauss)
    return random.getstate(), numpy_state


def _record(build_scenario: Callable, episode: int) -> Description:
    """Runs `build_scenario` for one episode number and records what GRF would build."""
    python_before, numpy_before = _random_states()
    builder = Builder(episode)
    build_scenario(builder)
    python_after, numpy_after = _random_states()
    if python_after != python_before:
        raise ScenarioError('the scenario draws from the random module of Python; GRF draws the seed of every '
                            'episode from that generator right after the scenario, so a bundle cannot hold it')
    if numpy_after != numpy_before:
        raise ScenarioError('the scenario draws from the global random generator of NumPy')
    config = builder.config()
    if config._computed_read:
        raise ScenarioError('the scenario reads controllable_left_players, controllable_right_players or '
                            'dynamic_player_selection, which GRF computes once at that read, before it sets the '
                            'agents, and keeps for the match, so a bundle cannot hold it')
    teams = []
    for side, team in (('left', config.left_team), ('right', config.right_team)):
        team = list(team) or [_STAND_IN_KEEPER]
        if len(team) > _TEAM_LIMIT:
            raise ScenarioError(f'a team has {len(team)} players, more than the 11 that GRF holds')
        if team[0].role != PlayerRole.e_PlayerRole_GK:
            raise ScenarioError(f'the first player of the {side} team is not a goalkeeper, which hangs GRF once '
                                'the match is in open play')
        teams.append(tuple(team))
    values = {k: v for k, v in config._values.items() if k not in _SET_BY_ENVIRONMENT}
    reverse = values.pop('reverse_team_processing')
    if values['deterministic'] and reverse:
        raise ScenarioError('a deterministic scenario that turns reverse_team_processing on')
    if not values['deterministic']:
        values['game_engine_random_seed'] = 42  # each episode's drawn seed replaces it
    return Description(values=values, ball=tuple(config.ball_position[:2]), left=teams[0], right=teams[1])


# Episode numbers each scenario is recorded for: the first few, as GRF plays them, and pairs of
# both parities far apart, which catch a scenario that keys on more than the parity.
_PROBE_EPISODES = tuple(range(1, 9)) + tuple(n + p for n in (96, 1000, 65534, 2 ** 24, 2 ** 30) for p in (0, 1))


def describe(scenario, episodes=_PROBE_EPISODES):
    """The (even, odd) descriptions of a scenario file or `build_scenario` function. Every
    episode number of one parity must describe the same scenario, and both parities must have the
    same team sizes (one batch keeps one agent layout)."""
    build = load_scenario(scenario) if isinstance(scenario, (str, os.PathLike)) else scenario
    seen = {}
    for episode in episodes:
        found = _record(build, episode)
        first = seen.setdefault(episode % 2, (found, episode))
        if first[0] != found:
            raise ScenarioError(f'the scenario differs between episodes {first[1]} and {episode}, which have the '
                                'same parity; a bundle holds one template for each parity only')
    if set(seen) != {0, 1}:
        raise ScenarioError('expected episode numbers of both parities')
    even, odd = seen[0][0], seen[1][0]
    if (len(even.left), len(even.right)) != (len(odd.left), len(odd.right)):
        raise ScenarioError('the team sizes change with the parity of the episode')
    return even, odd


# ---- scenario files ---------------------------------------------------------------------------------

# A scenario file starts with `from . import *` for the role and team names; it is loaded as a
# module of this synthetic package, which provides them.
_PACKAGE_NAME = 'cuju_amd._scenario_files'


def _scenario_package():
    package = sys.modules.get(_PACKAGE_NAME)
    if package is None:
        package = types.ModuleType(_PACKAGE_NAME)
        package.__path__ = []
        names = {role.name: role for role in PlayerRole}
        names['Team'] = Team
        package.__dict__.update(names)
        package.__all__ = sorted(names)
        sys.modules[_PACKAGE_NAME] = package
    return package


def load_scenario(path):
    """Imports a scenario file and returns its `build_scenario`; errors the file raises pass."""
    _scenario_package()
    stem = os.path.splitext(os.path.basename(path))[0]
    spec = importlib.util.spec_from_file_location(f'{_PACKAGE_NAME}.{stem}', path)
    if spec is None or spec.loader is None:
        raise ScenarioError(f'cannot load the scenario file {path}')
    module = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = module
    try:
        spec.loader.exec_module(module)
    finally:
        sys.modules.pop(spec.name, None)
    build = getattr(module, 'build_scenario', None)
    if not callable(build):
        raise ScenarioError(f'expected a build_scenario function in {path}')
    return build


# ---- the library's builder ----------------------------------------------------------------------------

def c_description(description: Description, keep: list):
    """`struct cuju_scenario_description` of a description; `keep` holds its player arrays alive."""
    teams = []
    for team in (description.left, description.right):
        players = (_library.ScenarioPlayer * len(team))(*(_library.ScenarioPlayer(*p) for p in team))
        keep.append(players)
        teams.append(players)
    v = description.values
    flags = {name: int(v[name]) for name in ('use_magnet', 'offsides', 'deterministic', 'end_episode_on_score',
                                             'end_episode_on_possession_change', 'end_episode_on_out_of_play',
                                             'control_all_players')}
    return _library.ScenarioDescription(
        version=1, ball_x=description.ball[0], ball_y=description.ball[1],
        left_team=teams[0], left_size=len(description.left), right_team=teams[1], right_size=len(description.right),
        real_time=0,  # the environment's configuration sets it; the simulation never reads it
        left_team_difficulty=v['left_team_difficulty'], right_team_difficulty=v['right_team_difficulty'],
        game_duration=v['game_duration'], second_half=v['second_half'],
        game_engine_random_seed=v['game_engine_random_seed'], **flags)


# A player keeps 512 s of per-second position history, so a match lasts at most 51,199 ticks.
_LONGEST_TICKS = 512 * 100 - 1
_DEFAULT_TICKS_PER_STEP = 10  # GRF's physics_steps_per_frame


def _warn_if_too_long(descriptions):
    steps = max(d.values['game_duration'] for d in descriptions)
    if steps * _DEFAULT_TICKS_PER_STEP <= _LONGEST_TICKS:
        return
    ticks = _LONGEST_TICKS // steps
    advice = f'physics_steps_per_frame={ticks} or fewer plays it' if ticks else 'no batch plays it'
    warnings.warn(f'the scenario lasts {steps} steps, and a batch holds at most {_LONGEST_TICKS // _DEFAULT_TICKS_PER_STEP} '
                  f'steps of {_DEFAULT_TICKS_PER_STEP} ticks, since it keeps 512 seconds of position history for each '
                  f'player; {advice}', stacklevel=3)


def build_bundle(scenario, out, name=None, device='cpu', library=None, animations=None):
    """Writes the agentless bundle of a scenario file (or `build_scenario` function) to `out` and
    returns `out`. `name` defaults to the file's or function's module name. The library builds on
    the host whatever `device` names, so every device gives the same bytes."""
    del device
    even, odd = describe(scenario)
    _warn_if_too_long((even, odd))
    if name is None:
        if isinstance(scenario, (str, os.PathLike)):
            name = os.path.splitext(os.path.basename(scenario))[0]
        else:
            name = getattr(scenario, '__module__', 'scenario').rsplit('.', 1)[-1]
    lib = _library.load(library)
    keep = []
    pair = (c_description(even, keep), c_description(odd, keep))
    status = lib.cuju_scenario_build_bundle(
        ctypes.byref(pair[0]), ctypes.byref(pair[1]), name.encode(),
        os.fsencode(animations or os.path.join(_library.DATA, 'animations.bin')), os.fsencode(out))
    if status != 0:
        raise from_library(lib.cuju_last_error().decode())
    return out


# ---- the bundle cache -----------------------------------------------------------------------------------

# The cache is on when this names a directory, or is 1 for the default one.
_CACHE_VARIABLE = 'CUJU_BUNDLE_CACHE'
_CACHE_TAG = b'cuju_amd scenario bundle, cache format 2'


def cache_directory():
    """The bundle cache directory, or None while `CUJU_BUNDLE_CACHE` is unset, empty or 0."""
    value = os.environ.get(_CACHE_VARIABLE, '')
    if value in ('', '0'):
        return None
    return _default_cache_directory() if value == '1' else value


def _default_cache_directory():
    base = os.environ.get('XDG_CACHE_HOME') or os.path.join(os.path.expanduser('~'), '.cache')
    return os.path.join(base, 'cuju_amd', 'bundles')


def _file_sha256(path):
    h = hashlib.sha256()
    with open(path, 'rb') as f:
        for chunk in iter(lambda: f.read(1 << 20), b''):
            h.update(chunk)
    return h.digest()


def cached_bundle(scenario, directory=None, device='cpu', library=None, animations=None):
    """The bundle of a scenario file in the cache directory, built at the first request only. Its
    name carries a digest of everything the bytes depend on: the file, its name, the animation
    tables, the library and this module."""
    directory = directory or cache_directory() or _default_cache_directory()
    stem = os.path.splitext(os.path.basename(scenario))[0]
    key = hashlib.sha256(_CACHE_TAG)
    for part in (_file_sha256(scenario), stem.encode(),
                 _file_sha256(animations or os.path.join(_library.DATA, 'animations.bin')),
                 _file_sha256(os.path.abspath(library or _library.PRODUCT)), _file_sha256(os.path.abspath(__file__))):
        key.update(hashlib.sha256(part).digest())
    path = os.path.join(directory, f'{stem}-{key.hexdigest()[:32]}.cjb')
    if os.path.isfile(path):
        return path
    os.makedirs(directory, exist_ok=True)
    # Each builder writes a file of its own; the rename installs one whole bundle.
    handle, partial = tempfile.mkstemp(prefix=f'.{stem}-', suffix='.building', dir=directory)
    os.close(handle)
    try:
        build_bundle(scenario, partial, name=stem, device=device, library=library, animations=animations)
        os.replace(partial, path)
    finally:
        if os.path.exists(partial):
            os.remove(partial)
    return path

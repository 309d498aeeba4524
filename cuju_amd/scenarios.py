"""GRF scenario files to asset bundles, without GRF (python/cuju/scenarios.py).

A GRF scenario file defines `build_scenario(builder)`. `build_bundle` runs it with a stand-in for
GRF's builder for episodes of both parities and hands the two descriptions to the library's
`cuju_scenario_build_bundle`, which writes the agentless (`l0_r0`) bundle a batch loads:

    from cuju_amd import scenarios
    scenarios.build_bundle('my_drill.py', 'my_drill_l0_r0.cjb')

`BatchEnvironment` also takes the path of a scenario file in place of a bundle and builds it at
creation (into `CUJU_BUNDLE_CACHE` when that is set). A scenario that GRF refuses, or that one
bundle cannot hold, raises `ScenarioError`.
"""

from __future__ import annotations

import ctypes
import enum
import hashlib
import importlib.util
import os
import random
import sys
import tempfile
import types
import warnings

from . import library as _library
from .errors import ConfigurationError, from_library

__all__ = ['Builder', 'PlayerRole', 'ScenarioConfig', 'ScenarioError', 'Team', 'build_bundle', 'cache_directory',
           'cached_bundle', 'describe', 'load_scenario']

# GRF: creating an environment builds episode 1 twice and plays episode 2 first. Pairs of far
# episode numbers also catch a scenario that keys on more than the parity.
EPISODES = tuple(range(1, 9)) + tuple(10 ** k + parity for k in range(2, 10) for parity in (0, 1))
_TEAM_LIMIT = 11  # GRF: 11 formation slots and 11 persons a team


class PlayerRole(enum.IntEnum):
    """GRF's `e_PlayerRole`."""
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
    """GRF's `e_Team`."""
    e_Left = 0
    e_Right = 1


class ScenarioError(ConfigurationError):
    """A scenario that GRF refuses or that a bundle cannot hold. It is a `ValueError`."""


# GRF hands scenario values to C++ through boost.python, which converts as these do.
def _number(name, value):
    if not isinstance(value, (int, float)):  # bool is an int
        raise ScenarioError(f'expected a number for {name}, found {value!r}')
    return float(value)


def _integer(name, value, low=-2 ** 31, high=2 ** 31 - 1):
    if not isinstance(value, int):
        raise ScenarioError(f'expected an integer for {name}, found {value!r}')
    if not low <= value <= high:
        raise ScenarioError(f'expected {name} from {low} to {high}, found {value}')
    return int(value)


def _unsigned(name, value):
    return _integer(name, value, 0, 2 ** 32 - 1)


def _flag(name, value):
    if value is not None and not isinstance(value, int):
        raise ScenarioError(f'expected True or False for {name}, found {value!r}')
    return bool(value)


# GRF's `ScenarioConfig` fields a scenario may set, with their defaults (`main.hpp`).
DEFAULTS = {
    'use_magnet': (True, _flag), 'offsides': (True, _flag), 'real_time': (False, _flag),
    'left_team_difficulty': (1.0, _number), 'right_team_difficulty': (0.6, _number),
    'deterministic': (False, _flag), 'end_episode_on_score': (False, _flag),
    'end_episode_on_possession_change': (False, _flag), 'end_episode_on_out_of_play': (False, _flag),
    'game_duration': (3000, _integer), 'second_half': (999999999, _integer),
    'control_all_players': (False, _flag), 'game_engine_random_seed': (42, _unsigned),
    'reverse_team_processing': (False, _flag), 'left_agents': (1, _integer), 'right_agents': (0, _integer),
}
# The environment's configuration replaces these after `build_scenario`.
_OVERRIDDEN = ('left_agents', 'right_agents', 'real_time')
# GRF computes these at their first read and keeps them; a scenario may only read them.
_COMPUTED = ('dynamic_player_selection', 'controllable_left_players', 'controllable_right_players')


class _Player:
    """One `AddPlayer` call, as `libgame.FormationEntry` holds it."""

    def __init__(self, x, y, role, lazy, controllable):
        if not isinstance(role, PlayerRole):
            raise ScenarioError(f'expected a role such as e_PlayerRole_GK, found {role!r}')
        self.entry = (_number('x', x), _number('y', y), int(role), _flag('lazy', lazy),
                      _flag('controllable', controllable))

    @property
    def role(self):
        return self.entry[2]

    @property
    def controllable(self):
        return self.entry[4]


class ScenarioConfig:
    """What `builder.config()` returns: GRF's fields, with an unknown name kept and ignored as a
    boost.python instance keeps it (with a warning, since it changes nothing)."""

    def __init__(self):
        object.__setattr__(self, '_values', {k: v for k, (v, _) in DEFAULTS.items()})
        object.__setattr__(self, 'left_team', [])
        object.__setattr__(self, 'right_team', [])
        object.__setattr__(self, 'ball_position', [0.0, 0.0, 0.0])
        object.__setattr__(self, '_computed_read', False)

    def __getattr__(self, name):
        values = object.__getattribute__(self, '_values')
        if name in values:
            return values[name]
        if name in _COMPUTED:
            return self._computed(name)
        raise AttributeError(name)

    def __setattr__(self, name, value):
        if name in _COMPUTED:
            raise AttributeError(f"can't set attribute {name}")
        if name in DEFAULTS:
            self._values[name] = DEFAULTS[name][1](name, value)
        elif name in ('left_team', 'right_team', 'ball_position'):
            raise ScenarioError(f'set {name} through AddPlayer or SetBallPosition')
        else:
            warnings.warn(f'the scenario sets {name!r}, which GRF does not know and ignores', stacklevel=2)
            object.__setattr__(self, name, value)

    def _computed(self, name):
        object.__setattr__(self, '_computed_read', True)
        left = sum(p.controllable for p in self.left_team)
        right = sum(p.controllable for p in self.right_team)
        if name == 'controllable_left_players':
            return left
        if name == 'controllable_right_players':
            return right
        wanted_left, wanted_right = self._values['left_agents'], self._values['right_agents']
        return not ((left == wanted_left or wanted_left == 0) and (right == wanted_right or wanted_right == 0))


class Builder:
    """The `builder` a scenario's `build_scenario` receives, as GRF's `Scenario` behaves."""

    def __init__(self, episode_number):
        self._config = ScenarioConfig()
        self._team = Team.e_Left
        self._episode = episode_number

    def config(self):
        return self._config

    def ScenarioConfig(self):
        return self._config

    def SetTeam(self, team):
        self._team = team

    def AddPlayer(self, x, y, role, lazy=False, controllable=True):
        player = _Player(x, y, role, lazy, controllable)
        (self._config.left_team if self._team == Team.e_Left else self._config.right_team).append(player)

    def SetBallPosition(self, ball_x, ball_y):
        self._config.ball_position[0] = _number('ball_x', ball_x)
        self._config.ball_position[1] = _number('ball_y', ball_y)

    def EpisodeNumber(self):
        return self._episode


# Scenario files do `from . import *` for the role and team names; this package provides them.
_PACKAGE = 'cuju_amd._scenario_files'


def _package():
    package = sys.modules.get(_PACKAGE)
    if package is None:
        package = types.ModuleType(_PACKAGE)
        package.__path__ = []
        for role in PlayerRole:
            setattr(package, role.name, role)
        package.Team = Team
        package.__all__ = [role.name for role in PlayerRole] + ['Team']
        sys.modules[_PACKAGE] = package
    return package


def load_scenario(path):
    """Imports a scenario file and returns its `build_scenario`. Errors the file raises pass."""
    _package()
    name = os.path.splitext(os.path.basename(path))[0]
    spec = importlib.util.spec_from_file_location(f'{_PACKAGE}.{name}', path)
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


def _numpy_generator_state():
    numpy = sys.modules.get('numpy')
    if numpy is None:
        return None
    state = numpy.random.get_state()
    return state[0], state[1].tobytes(), state[2], state[3], state[4]


def _describe_one(build_scenario, episode):
    """The description `build_scenario` gives for one episode number."""
    before = random.getstate(), _numpy_generator_state()
    builder = Builder(episode)
    build_scenario(builder)
    if random.getstate() != before[0]:
        raise ScenarioError('the scenario draws from the random module of Python; GRF draws the seed of every '
                            'episode from that generator right after the scenario, so a bundle cannot hold it')
    if _numpy_generator_state() != before[1]:
        raise ScenarioError('the scenario draws from the global random generator of NumPy')
    config = builder.config()
    if config._computed_read:
        raise ScenarioError('the scenario reads controllable_left_players, controllable_right_players or '
                            'dynamic_player_selection, which GRF computes once at that read, before it sets the '
                            'agents, and keeps for the match, so a bundle cannot hold it')
    for side, team in (('left', config.left_team), ('right', config.right_team)):
        if not team:
            # GRF: `Scenario._FakePlayersForEmptyTeam` gives an empty team a lazy goalkeeper.
            team.append(_Player(-1.0, 0.42, PlayerRole.e_PlayerRole_GK, True, True))
        if len(team) > _TEAM_LIMIT:
            raise ScenarioError(f'a team has {len(team)} players, more than the 11 that GRF holds')
        if team[0].role != PlayerRole.e_PlayerRole_GK:
            raise ScenarioError(f'the first player of the {side} team is not a goalkeeper, which hangs GRF once '
                                'the match is in open play')
    values = {k: v for k, v in config._values.items() if k not in _OVERRIDDEN}
    if values['deterministic']:
        if values['reverse_team_processing']:
            raise ScenarioError('a deterministic scenario that turns reverse_team_processing on')
    else:
        values['game_engine_random_seed'] = 42  # GRF: each episode's seed replaces it
    del values['reverse_team_processing']
    return {'values': values, 'ball': tuple(config.ball_position[:2]),
            'left': [p.entry for p in config.left_team], 'right': [p.entry for p in config.right_team]}


def describe(scenario, episodes=EPISODES):
    """The (even, odd) descriptions of a scenario file or `build_scenario` function. Episode numbers
    of one parity must describe the same scenario, and both parities the same team sizes."""
    build = load_scenario(scenario) if isinstance(scenario, (str, os.PathLike)) else scenario
    first = {}
    for episode in episodes:
        description = _describe_one(build, episode)
        seen, seen_episode = first.setdefault(episode % 2, (description, episode))
        if seen != description:
            raise ScenarioError(f'the scenario differs between episodes {seen_episode} and {episode}, which have the '
                                'same parity; a bundle holds one template for each parity only')
    if set(first) != {0, 1}:
        raise ScenarioError('expected episode numbers of both parities')
    even, odd = first[0][0], first[1][0]
    if len(even['left']) != len(odd['left']) or len(even['right']) != len(odd['right']):
        raise ScenarioError('the team sizes change with the parity of the episode')
    return even, odd


def _as_struct(description, keep):
    teams = []
    for side in ('left', 'right'):
        players = (_library.ScenarioPlayer * len(description[side]))(
            *[_library.ScenarioPlayer(*entry) for entry in description[side]])
        keep.append(players)
        teams.append(players)
    v = description['values']
    return _library.ScenarioDescription(
        version=1, ball_x=description['ball'][0], ball_y=description['ball'][1],
        left_team=teams[0], left_size=len(description['left']), right_team=teams[1],
        right_size=len(description['right']), use_magnet=v['use_magnet'], offsides=v['offsides'],
        real_time=False,  # set by the environment's configuration; the simulation never reads it
        left_team_difficulty=v['left_team_difficulty'], right_team_difficulty=v['right_team_difficulty'],
        deterministic=v['deterministic'], end_episode_on_score=v['end_episode_on_score'],
        end_episode_on_possession_change=v['end_episode_on_possession_change'],
        end_episode_on_out_of_play=v['end_episode_on_out_of_play'], game_duration=v['game_duration'],
        second_half=v['second_half'], control_all_players=v['control_all_players'],
        game_engine_random_seed=v['game_engine_random_seed'])


# A player keeps 512 s of per-second position history, so a match lasts at most 51,199 ticks.
_LONGEST_TICKS = 512 * 100 - 1
_DEFAULT_TICKS = 10  # GRF's default physics_steps_per_frame


def _warn_if_too_long(descriptions):
    duration = max(d['values']['game_duration'] for d in descriptions)
    if duration * _DEFAULT_TICKS <= _LONGEST_TICKS:
        return
    ticks = _LONGEST_TICKS // duration
    advice = f'physics_steps_per_frame={ticks} or fewer plays it' if ticks else 'no batch plays it'
    warnings.warn(f'the scenario lasts {duration} steps, and a batch holds at most {_LONGEST_TICKS // _DEFAULT_TICKS} '
                  f'steps of {_DEFAULT_TICKS} ticks, since it keeps 512 seconds of position history for each '
                  f'player; {advice}', stacklevel=3)


def build_bundle(scenario, out, name=None, device='cpu', library=None, animations=None):
    """Writes the agentless bundle of a scenario file (or `build_scenario` function) to `out` and
    returns `out`. `name` defaults to the file's or module's name. The library builds on the host
    whatever `device` names, so every device gives the same bytes."""
    del device
    even, odd = describe(scenario)
    _warn_if_too_long([even, odd])
    if name is None:
        if isinstance(scenario, (str, os.PathLike)):
            name = os.path.splitext(os.path.basename(scenario))[0]
        else:
            name = getattr(scenario, '__module__', 'scenario').rsplit('.', 1)[-1]
    lib = _library.load(library)
    keep = []
    pair = [_as_struct(even, keep), _as_struct(odd, keep)]
    status = lib.cuju_scenario_build_bundle(
        ctypes.byref(pair[0]), ctypes.byref(pair[1]), name.encode(),
        os.fsencode(animations or os.path.join(_library.DATA, 'animations.bin')), os.fsencode(out))
    if status != 0:
        raise from_library(lib.cuju_last_error().decode())
    return out


# The cache is on when this names a directory, or is 1 for the default one.
_CACHE_VARIABLE = 'CUJU_BUNDLE_CACHE'
_CACHE_FORMAT = b'cuju_amd bundle cache 1'


def cache_directory():
    """The bundle cache directory, or None while `CUJU_BUNDLE_CACHE` is unset, empty or 0."""
    value = os.environ.get(_CACHE_VARIABLE, '')
    if value in ('', '0'):
        return None
    return _default_cache_directory() if value == '1' else value


def _default_cache_directory():
    base = os.environ.get('XDG_CACHE_HOME') or os.path.join(os.path.expanduser('~'), '.cache')
    return os.path.join(base, 'cuju_amd', 'bundles')


def _digest(path):
    h = hashlib.sha256()
    with open(path, 'rb') as f:
        for chunk in iter(lambda: f.read(1 << 20), b''):
            h.update(chunk)
    return h.hexdigest()


def cached_bundle(scenario, directory=None, device='cpu', library=None, animations=None):
    """The bundle of a scenario file in a cache directory, built on the first request only. The key
    covers the file's bytes, its name, the animation tables, the library and this module."""
    directory = directory or cache_directory() or _default_cache_directory()
    name = os.path.splitext(os.path.basename(scenario))[0]
    with open(scenario, 'rb') as f:
        source = f.read()
    key = hashlib.sha256()
    for part in (_CACHE_FORMAT, source, name.encode(),
                 _digest(animations or os.path.join(_library.DATA, 'animations.bin')).encode(),
                 _digest(os.path.abspath(library or _library.PRODUCT)).encode(),
                 _digest(os.path.abspath(__file__)).encode()):
        key.update(len(part).to_bytes(8, 'little') + part)
    path = os.path.join(directory, f'{name}-{key.hexdigest()[:40]}.cjb')
    if os.path.isfile(path):
        return path
    os.makedirs(directory, exist_ok=True)
    # Concurrent builders each write a file of their own; the rename installs one whole bundle.
    descriptor, partial = tempfile.mkstemp(prefix=f'.{name}-', suffix='.partial', dir=directory)
    os.close(descriptor)
    try:
        build_bundle(scenario, partial, name=name, device=device, library=library, animations=animations)
        os.replace(partial, path)
    finally:
        if os.path.exists(partial):
            os.remove(partial)
    return path

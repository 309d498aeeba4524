"""The scenario builder: GRF scenario files to agentless asset bundles (python/cuju/scenarios.py,
include/cuju/assets/scenario_builder.h).

* Every shipped bundle is rebuilt byte for byte from the description its own template stores:
  the shipped bundles are the reference builder's output for GRF's scenario files
  (tests/test_grf_config.py:103-109 checks three of them).
* Random descriptions build the same bytes as the reference library's `cuju_scenario_build_bundle`.
* Scenario files written for these tests go through `describe` and build what the reference
  builds from the same descriptions, and a built drill plays as the reference plays it.
* The refusals GRF's semantics force: a first player who is not a goalkeeper, more than 11 players,
  draws from `random`, reads of the computed fields, sizes that change with the parity.
"""

import ctypes
import glob
import os
import random as pyrandom

import numpy as np
import pytest

from conftest import DATA, PRODUCT, ROOT, digest_actions, play
from oracle import ref

SCENARIOS = os.path.join(ROOT, 'tests', 'golden', 'scenarios')
SHIPPED = sorted(glob.glob(os.path.join(DATA, 'assets', '*_l0_r0.cjb')))
ANIMATIONS = os.path.join(DATA, 'animations.bin')


def library_with_builder(path):
    from cuju_amd import library
    lib = ctypes.CDLL(path)
    lib.cuju_last_error.restype = ctypes.c_char_p
    lib.cuju_scenario_build_bundle.argtypes = [ctypes.POINTER(library.ScenarioDescription)] * 2 + [ctypes.c_char_p] * 3
    return lib


def build_with(path, pair, name, out):
    lib = library_with_builder(path)
    status = lib.cuju_scenario_build_bundle(ctypes.byref(pair[0]), ctypes.byref(pair[1]), name.encode(),
                                            ANIMATIONS.encode(), str(out).encode())
    return status, (lib.cuju_last_error().decode() if status else open(out, 'rb').read())


@pytest.mark.parametrize('path', SHIPPED, ids=[os.path.basename(p)[:-len('_l0_r0.cjb')] for p in SHIPPED])
def test_shipped_bundles_rebuild_byte_for_byte(path, host_library, tmp_path):
    from cuju_amd import library
    host = ctypes.CDLL(host_library)
    pair, keep = [], []
    for parity in (0, 1):
        left, right = (library.ScenarioPlayer * 11)(), (library.ScenarioPlayer * 11)()
        description = library.ScenarioDescription()
        keep += [left, right]
        assert host.cuju_debug_bundle_description(path.encode(), parity, ctypes.byref(description), left, right) == 0
        pair.append(description)
    name = os.path.basename(path)[:-len('_l0_r0.cjb')]
    status, built = build_with(PRODUCT, pair, name, tmp_path / 'built.cjb')
    assert status == 0, built
    with open(path, 'rb') as f:
        assert built == f.read()


def random_description(rng, size_left, size_right, keep):
    """A valid description: goalkeeper first, positions on the pitch, flags and duration drawn."""
    from cuju_amd import library
    teams = []
    for size in (size_left, size_right):
        players = (library.ScenarioPlayer * size)()
        for i in range(size):
            players[i] = library.ScenarioPlayer(rng.uniform(-1, 1), rng.uniform(-0.42, 0.42),
                                                0 if i == 0 else rng.randrange(1, 10), rng.random() < 0.2,
                                                rng.random() < 0.8)
        keep.append(players)
        teams.append(players)
    return library.ScenarioDescription(
        version=1, ball_x=rng.uniform(-1, 1), ball_y=rng.uniform(-0.42, 0.42), left_team=teams[0],
        left_size=size_left, right_team=teams[1], right_size=size_right, use_magnet=rng.random() < 0.8,
        offsides=rng.random() < 0.5, real_time=0, left_team_difficulty=rng.random(),
        right_team_difficulty=rng.random(), deterministic=rng.random() < 0.3,
        end_episode_on_score=rng.random() < 0.5, end_episode_on_possession_change=rng.random() < 0.3,
        end_episode_on_out_of_play=rng.random() < 0.3, game_duration=rng.randrange(50, 3001),
        second_half=rng.choice([999999999, rng.randrange(20, 1500)]), control_all_players=rng.random() < 0.2,
        game_engine_random_seed=rng.randrange(0, 2 ** 32))


@pytest.mark.parametrize('seed', range(12))
def test_random_descriptions_build_as_the_reference(seed, reference_library, tmp_path):
    rng = pyrandom.Random(seed)
    keep = []
    size_left, size_right = rng.randrange(1, 12), rng.randrange(1, 12)
    pair = [random_description(rng, size_left, size_right, keep) for _ in range(2)]
    mine = build_with(PRODUCT, pair, f'random_{seed}', tmp_path / 'mine.cjb')
    theirs = build_with(reference_library, pair, f'random_{seed}', tmp_path / 'theirs.cjb')
    assert mine[0] == theirs[0], (mine[1] if mine[0] else theirs[1])
    assert mine[1] == theirs[1]


@pytest.mark.parametrize('name', ['drill_3_vs_1_with_keeper', 'keeper_duel_deterministic'])
def test_scenario_files_build_as_the_reference(name, reference_library, tmp_path):
    from cuju_amd import scenarios
    source = os.path.join(SCENARIOS, name + '.py')
    out = scenarios.build_bundle(source, str(tmp_path / 'mine.cjb'))
    even, odd = scenarios.describe(source)
    keep = []
    pair = [scenarios.c_description(even, keep), scenarios.c_description(odd, keep)]
    status, theirs = build_with(reference_library, pair, name, tmp_path / 'theirs.cjb')
    assert status == 0, theirs
    with open(out, 'rb') as f:
        assert f.read() == theirs


def test_describe_follows_the_builder_semantics():
    from cuju_amd import scenarios
    even, odd = scenarios.describe(os.path.join(SCENARIOS, 'drill_3_vs_1_with_keeper.py'))
    assert even.ball == (0.55, 0.12) and odd.ball == (0.55, -0.12)
    assert [p.role for p in even.left] == [0, 9, 6, 7]
    # Not deterministic: every episode's seed replaces the scenario's.
    assert even.values['game_engine_random_seed'] == 42
    duel, _ = scenarios.describe(os.path.join(SCENARIOS, 'keeper_duel_deterministic.py'))
    assert duel.values['game_engine_random_seed'] == 1234
    assert duel.left[0].controllable is False and duel.right[1].lazy is True

    def empty_right(builder):
        builder.AddPlayer(-1.0, 0.0, scenarios.PlayerRole.e_PlayerRole_GK)
    # GRF gives an empty team a lazy goalkeeper.
    even, _ = scenarios.describe(empty_right)
    assert even.right == ((-1.0, 0.42, 0, True, True),)


def _refused(build, match):
    from cuju_amd import scenarios
    with pytest.raises(scenarios.ScenarioError, match=match):
        scenarios.describe(build)


def test_describe_refuses_what_a_bundle_cannot_hold():
    from cuju_amd.scenarios import PlayerRole
    gk, cf = PlayerRole.e_PlayerRole_GK, PlayerRole.e_PlayerRole_CF

    def forward_first(builder):
        builder.AddPlayer(0.0, 0.0, cf)
    _refused(forward_first, 'not a goalkeeper')

    def twelve(builder):
        builder.AddPlayer(-1.0, 0.0, gk)
        for i in range(11):
            builder.AddPlayer(0.0, 0.01 * i, cf)
    _refused(twelve, 'more than the 11')

    def draws(builder):
        builder.AddPlayer(-1.0, 0.0, gk)
        pyrandom.random()
    _refused(draws, 'random module')

    def reads_computed(builder):
        builder.AddPlayer(-1.0, 0.0, gk)
        _ = builder.config().controllable_left_players
    _refused(reads_computed, 'computes once')

    def grows(builder):
        builder.AddPlayer(-1.0, 0.0, gk)
        if builder.EpisodeNumber() % 2:
            builder.AddPlayer(0.0, 0.0, cf)
    _refused(grows, 'team sizes change')

    def drifts(builder):
        builder.AddPlayer(-1.0, 0.0, gk)
        builder.SetBallPosition(0.1 if builder.EpisodeNumber() < 1000 else 0.2, 0.0)
    _refused(drifts, 'differs between episodes')

    def bad_role(builder):
        builder.AddPlayer(-1.0, 0.0, 0)
    _refused(bad_role, 'expected a role')


def test_builder_refuses_invalid_descriptions(tmp_path):
    """The C ABI refuses what GRF cannot run, with the message in cuju_last_error."""
    from cuju_amd import library
    keep = []
    rng = pyrandom.Random(3)
    pair = [random_description(rng, 2, 2, keep) for _ in range(2)]
    pair[1].version = 2
    status, message = build_with(PRODUCT, pair, 'x', tmp_path / 'x.cjb')
    assert status == -1 and 'version' in message
    pair = [random_description(rng, 2, 2, keep), random_description(rng, 3, 2, keep)]
    status, message = build_with(PRODUCT, pair, 'x', tmp_path / 'x.cjb')
    assert status == -1 and 'parity' in message
    pair = [random_description(rng, 2, 2, keep) for _ in range(2)]
    for d in pair:
        d.left_team[0].role = 5
    status, message = build_with(PRODUCT, pair, 'x', tmp_path / 'x.cjb')
    assert status == -1 and 'goalkeeper' in message
    del library


def test_built_drill_plays_as_the_reference(reference_library, host_library, tmp_path):
    """A built drill, played by this engine (host build) and by the reference from the same bundle."""
    from cuju_amd import scenarios
    bundle = scenarios.build_bundle(os.path.join(SCENARIOS, 'drill_3_vs_1_with_keeper.py'),
                                    str(tmp_path / 'drill_l0_r0.cjb'))
    options = dict(environment_count=6, seed=5, threads=2, agent_counts=[(3, 0)])
    digests = []
    for path in (host_library, reference_library):
        batch = ref.ReferenceBatch(bundle, library_path=path, **options)
        try:
            digests.append(play(batch, 120, 6))
        finally:
            batch.close()
    assert digests[0] == digests[1]


def test_bundle_cache_builds_once(tmp_path, monkeypatch):
    from cuju_amd import scenarios
    monkeypatch.setenv('CUJU_BUNDLE_CACHE', str(tmp_path / 'cache'))
    source = os.path.join(SCENARIOS, 'keeper_duel_deterministic.py')
    first = scenarios.cached_bundle(source)
    stamp = os.stat(first).st_mtime_ns
    assert scenarios.cached_bundle(source) == first and os.stat(first).st_mtime_ns == stamp
    assert os.path.dirname(first) == str(tmp_path / 'cache')
    direct = scenarios.build_bundle(source, str(tmp_path / 'direct.cjb'))
    with open(first, 'rb') as a, open(direct, 'rb') as b:
        assert a.read() == b.read()

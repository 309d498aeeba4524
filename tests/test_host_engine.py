"""The engine's host build (the same sources as the gfx950 kernels, compiled for the CPU) against
the shipped digests and, tick by tick, against the reference library on the same seeds and
actions. The product never loads this build; it locates divergences on the CPU."""

import ctypes
import json
import os
import random

import numpy as np
import pytest

import libm_cases
from conftest import ROOT, digest_actions, play, short_cases
from oracle import ref
from oracle.ref import ReferenceBatch


@pytest.mark.parametrize('name,case', short_cases(), ids=[n for n, _ in short_cases()])
def test_host_engine_reproduces_shipped_digest(name, case, digests, host_library):
    batch = ref.ReferenceBatch(case['assets'], environment_count=digests['environments'], seed=7,
                               threads=4, library_path=host_library, **dict(case['options']))
    try:
        assert play(batch, digests['steps'], digests['environments']) == case['digest']
    finally:
        batch.close()


@pytest.mark.parametrize('assets,steps', [('11_vs_11_hard_stochastic_l11_r0', 60),
                                          ('5_vs_5_l4_r4', 80),
                                          ('academy_counterattack_hard_l4_r0', 80)])
def test_host_engine_matches_reference_every_tick(assets, steps, reference_library, host_library):
    """One tick per step, so every tick's full state is compared, not just the step's end."""
    options = dict(environment_count=2, seed=11, physics_steps_per_frame=1, threads=2)
    mine = ref.ReferenceBatch(assets, library_path=host_library, **options)
    theirs = ref.ReferenceBatch(assets, library_path=reference_library, **options)
    try:
        assert np.array_equal(mine.reset().view(np.uint32), theirs.reset().view(np.uint32))
        for step in range(steps):
            actions = digest_actions(step, 2, mine.agents, mine.action_count)
            a = [x.copy() for x in mine.step(actions)]
            b = [x.copy() for x in theirs.step(actions)]
            for x, y in zip(a, b):
                assert x.tobytes() == y.tobytes(), f'outputs differ at tick {step}'
            for e in range(2):
                assert mine.raw_state(e) == theirs.raw_state(e), f'state of env {e} differs at tick {step}'
    finally:
        mine.close()
        theirs.close()


def test_masked_reset_and_explicit_seeds(reference_library, host_library):
    options = dict(environment_count=4, seed=3, threads=2)
    mine = ref.ReferenceBatch('academy_3_vs_1_with_keeper_l1_r0', library_path=host_library, **options)
    theirs = ref.ReferenceBatch('academy_3_vs_1_with_keeper_l1_r0', library_path=reference_library, **options)
    try:
        for batch in (mine, theirs):
            batch.reset()
        for step in range(30):
            actions = digest_actions(step, 4, mine.agents, mine.action_count)
            assert mine.step(actions)[0].tobytes() == theirs.step(actions)[0].tobytes()
            if step % 10 == 9:
                mask = np.array([1, 0, step % 20 == 9, 1], dtype=np.uint8)
                seeds = np.array([-1, 5, 123456789, 4294967295], dtype=np.int64)
                assert mine.reset(seeds=seeds, mask=mask).tobytes() == theirs.reset(seeds=seeds, mask=mask).tobytes()
        for e in range(4):
            assert mine.get_state(e) == theirs.get_state(e)
    finally:
        mine.close()
        theirs.close()


def test_episode_seeds_follow_cpython_random(host_library):
    """GRF draws each episode seed with CPython's `random.randint(0, 2000000000)` after
    `random.seed(seed * 2**32 + index)`: Python's own generator is the oracle."""
    lib = ctypes.CDLL(host_library)
    lib.cuju_debug_episode_seeds.argtypes = [ctypes.c_ulonglong, ctypes.c_uint, ctypes.c_int, ctypes.c_void_p]
    for seed, index in [(0, 0), (0, 1), (7, 3), (2**32 - 1, 2**32 - 1), (123456789012, 77), (2**63, 5)]:
        out = np.zeros(8, dtype=np.uint32)
        lib.cuju_debug_episode_seeds(seed, index, 8, out.ctypes.data)
        rng = random.Random(seed * 2**32 + index)
        assert out.tolist() == [rng.randint(0, 2000000000) for _ in range(8)]


def test_world_generator_is_mt19937(host_library):
    """The world's generator against numpy's MT19937 under Knuth's seeding (std::mt19937's and
    Boost's seed; Boost's extra normalization touches only bits no draw reads), over 2,000 words
    (three state renewals), and its uniform floats against that word stream: each is the word
    over 2**32 in float, scaled to [low, high), drawn again when it rounds up to `high`."""
    lib = ctypes.CDLL(host_library)
    lib.cuju_debug_world_rng.argtypes = [ctypes.c_uint, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                         ctypes.c_void_p, ctypes.c_void_p]
    last, unused = np.zeros(10000, dtype=np.uint32), np.zeros(10000, dtype=np.float32)
    lib.cuju_debug_world_rng(5489, 10000, 0.0, 1.0, last.ctypes.data, unused.ctypes.data)
    assert int(last[-1]) == 4123659995  # the C++ standard's check of std::mt19937 (seed 5489)
    count = 2000
    for seed, low, high in [(5489, 0.0, 1.0), (0, -3.0, 5.5), (2**32 - 1, 1.0, 4.0), (1, 0.0, 1e-30)]:
        words = np.zeros(count, dtype=np.uint32)
        uniforms = np.zeros(count, dtype=np.float32)
        lib.cuju_debug_world_rng(seed, count, low, high, words.ctypes.data, uniforms.ctypes.data)
        bits = np.random.MT19937()
        bits._legacy_seeding(seed)
        stream = bits.random_raw(3 * count).astype(np.uint32)
        assert words.tolist() == stream[:count].tolist()
        lo, hi = np.float32(low), np.float32(high)
        expected, k = [], 0
        while len(expected) < count:
            r = np.float32(np.float32(stream[k]) / np.float32(2.0**32)) * np.float32(hi - lo) + lo
            k += 1
            if r < hi:
                expected.append(np.float32(r))
        assert uniforms.tobytes() == np.array(expected, dtype=np.float32).tobytes()


@pytest.mark.parametrize('assets', ['11_vs_11_hard_stochastic_l11_r0', 'academy_corner_l1_r0'])
def test_set_state_continues_as_the_reference(assets, reference_library, host_library):
    """States of a played batch load into another batch (environments shuffled) in the reference
    and in the engine; both then agree byte for byte on the outputs and on every later state
    (reference `cuju_environment_set_state`, src/environment_api.h:390-404)."""
    environments, played, after = 3, 25, 12
    source = ReferenceBatch(assets, environment_count=environments, seed=7, library_path=reference_library)
    source.reset()
    for step in range(played):
        source.step(digest_actions(step, environments, source.agents, source.action_count))
    states = [source.raw_state(i) for i in range(environments)]
    source.close()
    targets = [ReferenceBatch(assets, environment_count=environments, seed=11, library_path=path)
               for path in (reference_library, host_library)]
    for batch in targets:
        batch.reset()
        for index in range(environments):
            match, episode = states[(index + 1) % environments]
            batch.set_raw_state(index, match, episode)
    reference, engine = targets
    assert np.array_equal(reference.observation(), engine.observation())
    for index in range(environments):
        assert engine.raw_state(index) == reference.raw_state(index)
        assert engine.raw_state(index)[0] == states[(index + 1) % environments][0]
    for step in range(after):
        actions = digest_actions(step + 3, environments, reference.agents, reference.action_count)
        for a, b in zip(reference.step(actions), engine.step(actions)):
            assert np.array_equal(a, b)
    for index in range(environments):
        assert engine.get_state(index) == reference.get_state(index)
    for batch in targets:
        batch.close()


def test_set_state_refuses_another_scenario(reference_library, host_library):
    source = ReferenceBatch('academy_corner_l1_r0', environment_count=1, seed=7, library_path=host_library)
    source.reset()
    match, episode = source.raw_state(0)
    source.close()
    target = ReferenceBatch('academy_empty_goal_l1_r0', environment_count=1, seed=7, library_path=host_library)
    target.reset()
    with pytest.raises(RuntimeError, match='scenario'):
        target.set_raw_state(0, match, episode)
    with pytest.raises(RuntimeError, match='do not load'):
        target.set_raw_state(0, b'\x00' * 16, episode)
    target.close()


def test_time_walk_matches_the_direct_estimate(host_library):
    """The time-to-target estimate along the precomputed walk, and the possession scan's shortcut
    for targets the walk cannot reach, equal GRF's direct loop (ai_time.h:102-409) on random
    players, movements, targets and time limits, near and far. Each player takes eight targets in
    a row, as a possession scan does, and a third of the targets sit within a metre of the
    shortcut's bound."""
    lib = ctypes.CDLL(host_library)
    rng = np.random.default_rng(5)
    players, per = 25_000, 8
    n = players * per
    pos = np.column_stack([rng.uniform(-55, 55, players), rng.uniform(-36, 36, players), rng.choice([0.0, 0.1], players)])
    speed = rng.choice([0.0, 1.0, 1.8, 1.80001, 3.0, 6.0, 9.0], players) * rng.uniform(0.5, 1.5, players)
    angle = rng.uniform(-np.pi, np.pi, players)
    mov = np.column_stack([speed * np.cos(angle), speed * np.sin(angle), rng.choice([0.0, 0.3], players)])
    velocity = rng.uniform(5, 9.5, players)
    precise = rng.integers(0, 2, players)
    pos, mov, velocity, precise = (np.repeat(x, per, axis=0) for x in (pos, mov, velocity, precise))
    # The shortcut's bound: 0.36 |movement| + 0.9 + 0.35 (0.94 maximum velocity), from the start.
    bound = np.linalg.norm(mov[:, :2], axis=1) * 0.36 + 0.9 + 0.35 * 0.94 * velocity
    reach = rng.choice([0.5, 3.0, 10.0, 20.0, 40.0, 60.0], n) * rng.uniform(0, 1, n)
    near = rng.uniform(size=n) < 1 / 3
    reach[near] = bound[near] + rng.uniform(-0.5, 0.5, near.sum())
    turn = rng.uniform(-np.pi, np.pi, n)
    target = np.column_stack([pos[:, 0] + reach * np.cos(turn), pos[:, 1] + reach * np.sin(turn), np.zeros(n)])
    limit = np.where(rng.uniform(size=n) < 0.3, -1.0, rng.integers(0, 3000, n).astype(float))
    limit[rng.uniform(size=n) < 0.1] = rng.choice([680.0, 689.0, 690.0, 695.0, 699.0, 700.0])
    cases = np.column_stack([pos, mov, target, velocity, precise, limit]).astype(np.float32)
    out = np.zeros((n, 6), dtype=np.uint32)
    lib.cuju_debug_time_needed(ctypes.c_void_p(cases.ctypes.data), n, ctypes.c_void_p(out.ctypes.data))
    assert np.array_equal(out[:, :2], out[:, 2:4])
    assert np.array_equal(out[:, :2], out[:, 4:])
    walked = np.linalg.norm(mov[:, :2], axis=1) > 2.0
    assert walked.sum() > n // 3


def test_device_time_bias_rounds_as_the_division():
    """The device computes GRF's acceleration bias (10 k) / 700 as a reciprocal product with one
    fused correction (engine/ball.h, TimeNeededBias); for every step index the walks use (k < 200)
    that rounds exactly as the float division."""
    from fractions import Fraction

    def fma(a, b, c):
        exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
        near = np.float32(float(exact))
        best = near
        for d in (np.nextafter(near, np.float32(-np.inf)), near, np.nextafter(near, np.float32(np.inf))):
            e, b0 = abs(Fraction(float(d)) - exact), abs(Fraction(float(best)) - exact)
            if e < b0 or (e == b0 and int(np.float32(d).view(np.int32)) % 2 == 0):
                best = d
        return np.float32(best)

    r = np.float32(1) / np.float32(700)
    for k in range(200):
        x = np.float32(10 * k)
        q = x * r
        assert fma(fma(-q, np.float32(700), x), r, q) == x / np.float32(700), k


LIBM_GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'libm.json')
LIBM_PORTS = os.path.join(ROOT, 'oracle', '_ref', 'liblibm_ports.so')


def _libm_golden():
    with open(LIBM_GOLDEN) as f:
        return json.load(f)


def _host_libm(host_library):
    lib = ctypes.CDLL(host_library)
    lib.cuju_debug_libm_range.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_longlong, ctypes.c_void_p]
    lib.cuju_debug_libm.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_longlong]
    lib.cuju_debug_libm_double.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.c_longlong]
    return lib


@pytest.mark.parametrize('name', sorted(libm_cases.UNARY_FLOAT))
def test_engine_unary_float_math_is_the_reference_port_on_every_input(name, host_library):
    """sinf, cosf, atanf, acosf and asinf of the engine give the reference ports' bits
    (include/cuju/libm/sincosf.h:61-212, inverse_trigonometric_float.h:32-272, asinf.h:40-95) on all
    2**32 inputs: the checksum over every output equals the one the ports wrote
    (tests/golden/make_libm.py)."""
    lib = _host_libm(host_library)
    which = libm_cases.UNARY_FLOAT[name]
    digest = libm_cases.exhaustive_digest(
        lambda first, out: lib.cuju_debug_libm_range(which, first, len(out), out.ctypes.data))
    assert digest == _libm_golden()['exhaustive'][name]


def _compare_with_ports(name, got, want):
    kind = np.uint32 if got.dtype == np.float32 else np.uint64
    a = np.frombuffer(libm_cases.canonical(got), dtype=kind)
    b = np.frombuffer(libm_cases.canonical(want), dtype=kind)
    differ = np.flatnonzero(a != b)
    assert differ.size == 0, f'{name}: {differ.size} outputs differ from the reference port, the first at sample {differ[0]}'


@pytest.mark.parametrize('name', sorted(libm_cases.SAMPLED_FLOAT))
def test_engine_float_math_is_the_reference_port_on_samples(name, host_library):
    """powf (include/cuju/libm/powf.h:93-198), atan2f and sincosf on special values, every pair of
    exponents, random bit patterns and the step's ranges: the checksum equals the ports', and
    output for output equals them where the port library is built."""
    lib = _host_libm(host_library)
    which = libm_cases.SAMPLED_FLOAT[name]
    x, y = libm_cases.float_pairs(name)
    out = np.empty_like(x)
    lib.cuju_debug_libm(which, x.ctypes.data, y.ctypes.data, out.ctypes.data, len(x))
    if os.path.isfile(LIBM_PORTS):
        ports = ctypes.CDLL(LIBM_PORTS)
        ports.oracle_libm_float.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_longlong]
        want = np.empty_like(x)
        ports.oracle_libm_float(which, x.ctypes.data, y.ctypes.data, want.ctypes.data, len(x))
        _compare_with_ports(name, out, want)
    assert libm_cases.sample_digest(out) == _libm_golden()['sampled_float'][name]


@pytest.mark.parametrize('name', sorted(libm_cases.SAMPLED_DOUBLE))
def test_engine_double_math_is_the_reference_port_on_samples(name, host_library):
    """Double sin, cos (include/cuju/libm/sin_double.h:30-266), pow (pow.h:447-651), acos
    (acos_double.h:29-143) and sincos on special values, every exponent, random bit patterns, large
    reduction arguments and the step's ranges, as the ports compute them."""
    lib = _host_libm(host_library)
    which = libm_cases.SAMPLED_DOUBLE[name]
    x, y = libm_cases.double_pairs(name)
    out = np.empty_like(x)
    lib.cuju_debug_libm_double(which, x.ctypes.data, y.ctypes.data, out.ctypes.data, len(x))
    if os.path.isfile(LIBM_PORTS):
        ports = ctypes.CDLL(LIBM_PORTS)
        ports.oracle_libm_double.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_longlong]
        want = np.empty_like(x)
        ports.oracle_libm_double(which, x.ctypes.data, y.ctypes.data, want.ctypes.data, len(x))
        _compare_with_ports(name, out, want)
    assert libm_cases.sample_digest(out) == _libm_golden()['sampled_double'][name]


def test_libm_checks_catch_a_one_bit_change():
    """The checksums see a change of the last bit of one output of one block, and NaN payloads
    and signs do not count."""
    def fill(first, out, flip=None):
        out[:] = np.arange(first, first + len(out), dtype=np.uint64).astype(np.uint32).view(np.float32)
        if flip is not None and first <= flip < first + len(out):
            out.view(np.uint32)[flip - first] ^= 1
    base = libm_cases.exhaustive_digest(fill, threads=8)
    assert base != libm_cases.exhaustive_digest(lambda f, o: fill(f, o, flip=0x3F800000), threads=8)
    nan_a = np.array([np.nan, 1.0], dtype=np.float32)
    nan_b = nan_a.copy()
    nan_b.view(np.uint32)[0] = 0xFFC00001
    assert libm_cases.sample_digest(nan_a) == libm_cases.sample_digest(nan_b)


def _same(a, b):
    """Byte equality of two observations, arrays or raw dictionaries of arrays."""
    if isinstance(a, dict):
        return sorted(a) == sorted(b) and all(_same(a[k], b[k]) for k in a)
    return np.ascontiguousarray(a).tobytes() == np.ascontiguousarray(b).tobytes()


@pytest.mark.parametrize('representation,stacked,with_raw', [('extracted', False, True), ('extracted', True, False),
                                                             ('raw', False, False)])
def test_host_engine_smm_and_raw_match_reference(representation, stacked, with_raw, reference_library, host_library):
    """The SMM (one frame and a stack of four) and the raw arrays, with the final observations of
    episodes that end, against the reference library on short academy episodes and a 5-a-side game
    in one batch (observation_encoding.h:119-148, batch_core.h:52-210)."""
    options = dict(environment_count=6, seed=5, threads=2, representation=representation, stacked=stacked,
                   with_raw=with_raw, assignment=[0, 1, 0, 1, 0, 1])
    assets = ['academy_empty_goal_close_l1_r0', '5_vs_5_l4_r4']
    mine = ref.ReferenceBatch(assets, library_path=host_library, **options)
    theirs = ref.ReferenceBatch(assets, library_path=reference_library, **options)
    try:
        assert _same(mine.reset(), theirs.reset())
        ended = 0
        for step in range(70):
            actions = digest_actions(step, 6, mine.agents, mine.action_count)
            a, b = mine.step(actions), theirs.step(actions)
            for x, y, what in zip(a, b, ('observation', 'reward', 'done')):
                assert _same(x, y), f'{what} at step {step}'
            if b[2].any():
                ended += 1
                assert _same(mine.final_observation(), theirs.final_observation()), f'final at step {step}'
                if with_raw:
                    assert _same(mine.raw(final=True), theirs.raw(final=True)), f'final raw at step {step}'
            if with_raw:
                assert _same(mine.raw(), theirs.raw()), f'raw at step {step}'
        assert ended > 0
    finally:
        mine.close()
        theirs.close()


def test_every_action_of_the_full_set_plays_as_the_reference(reference_library, host_library):
    """Random actions over all 33 of the `full` set (presses, releases, the built-in AI, keeper
    rush, pressure and switch) on agents of both teams, several per team, with the raw arrays
    (which hold each agent's sticky actions) and the states at the end, against the reference
    library (environment.h:14-330)."""
    options = dict(environment_count=4, seed=11, threads=2, action_set='full', with_raw=True,
                   assignment=[0, 1, 0, 1])
    assets = ['11_vs_11_kaggle_l3_r2', '5_vs_5_l2_r3']
    mine = ref.ReferenceBatch(assets, library_path=host_library, **options)
    theirs = ref.ReferenceBatch(assets, library_path=reference_library, **options)
    rng = np.random.default_rng(33)
    try:
        assert mine.action_count == 33
        assert _same(mine.reset(), theirs.reset())
        for step in range(160):
            actions = rng.integers(0, 33, size=(4, mine.agents)).astype(np.int32)
            a, b = mine.step(actions), theirs.step(actions)
            for x, y, what in zip(a, b, ('observation', 'reward', 'done')):
                assert _same(x, y), f'{what} at step {step}'
            assert _same(mine.raw(), theirs.raw()), f'raw at step {step}'
        for e in range(4):
            assert mine.get_state(e) == theirs.get_state(e), f'state of environment {e}'
    finally:
        mine.close()
        theirs.close()


@pytest.mark.parametrize('ticks_per_step', [10, 5])
def test_a_step_ticks_until_play(ticks_per_step, host_library):
    """GRF's environment step runs whole steps of ticks until play is on (environment.h:539-556):
    every environment step runs a positive multiple of the ticks per step, and a stoppage makes
    some run many more. The host build counts the ticks of each environment step."""
    batch = ref.ReferenceBatch('11_vs_11_hard_stochastic_l11_r0', environment_count=96, seed=0, threads=4,
                               library_path=host_library, physics_steps_per_frame=ticks_per_step)
    lib = ref.library(host_library)
    lib.cuju_debug_step_ticks.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    ticks = np.zeros(96, dtype=np.int64)
    seen = []
    try:
        batch.reset()
        for step in range(40):
            batch.step(digest_actions(step, 96, batch.agents, batch.action_count))
            assert lib.cuju_debug_step_ticks(batch._handle, ticks.ctypes.data) == 96
            seen.append(ticks.copy())
    finally:
        batch.close()
    seen = np.array(seen)
    assert (seen >= ticks_per_step).all() and (seen % ticks_per_step == 0).all()
    assert (seen > ticks_per_step).any()


def test_difficulty_override_plays_as_the_reference(reference_library, host_library):
    """Per-environment difficulties (negative keeps the scenario's) change the AI identically."""
    difficulty = np.array([[-1.0, 0.25], [0.75, -1.0], [0.1, 0.9]], dtype=np.float32)
    digests = []
    for path in (host_library, reference_library):
        batch = ref.ReferenceBatch('11_vs_11_stochastic_l1_r0', environment_count=3, seed=8, threads=2,
                                   library_path=path, difficulty=difficulty)
        try:
            digests.append(play(batch, 60, 3))
        finally:
            batch.close()
    assert digests[0] == digests[1]


def test_episode_values_and_scenario_names_match_the_reference(reference_library, host_library):
    """`cuju_environment_episode` and `cuju_environment_scenario`, after episodes have ended."""
    import ctypes
    assets = ['academy_empty_goal_close_l1_r0', '5_vs_5_l2_r1']
    options = dict(environment_count=4, seed=3, threads=2, assignment=[0, 1, 0, 1], episode_number=5,
                   difficulty=np.array([[-1.0, 0.5]] * 4, dtype=np.float32))
    results = []
    for path in (host_library, reference_library):
        batch = ref.ReferenceBatch(assets, library_path=path, **options)
        lib = batch._lib
        lib.cuju_environment_episode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        lib.cuju_environment_scenario.restype = ctypes.c_char_p
        lib.cuju_environment_scenario.argtypes = [ctypes.c_void_p, ctypes.c_int]
        try:
            batch.reset()
            seen = []
            for step in range(90):
                batch.step(digest_actions(step, 4, batch.agents, batch.action_count))
                if step % 30 == 29:
                    for e in range(4):
                        values = np.zeros(17, dtype=np.int64)
                        difficulty = np.zeros(4, dtype=np.float32)
                        assert lib.cuju_environment_episode(batch._handle, e, values.ctypes.data, difficulty.ctypes.data) == 0
                        seen.append((values.tolist(), difficulty.tolist()))
            names = [lib.cuju_environment_scenario(batch._handle, k) for k in range(3)]
            results.append((seen, names))
        finally:
            batch.close()
    assert results[0] == results[1]
    assert results[0][1] == [b'academy_empty_goal_close', b'5_vs_5', None]
    assert any(values[2] > 1 for values, _ in results[0][0])  # some environment has reset since


@pytest.mark.parametrize('representation', ['extracted', 'simple115v2'])
def test_set_stack_continues_as_the_reference(representation, reference_library, host_library):
    """A stack set from outside (`cuju_environment_set_stack`), an SMM one included, whose marks the
    library rebuilds so the next steps erase exactly them, continues as the reference continues."""
    import ctypes
    name = b'smm' if representation == 'extracted' else b'simple115'
    outputs = []
    for path in (host_library, reference_library):
        batch = ref.ReferenceBatch('5_vs_5_l2_r1', environment_count=2, seed=6, threads=2, library_path=path,
                                   representation=representation, stacked=True)
        lib = batch._lib
        lib.cuju_environment_set_stack.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p,
                                                   ctypes.c_ulonglong]
        try:
            batch.reset()
            seen = []
            for step in range(12):
                batch.step(digest_actions(step, 2, batch.agents, batch.action_count))
            # Environment 1 takes environment 0's match and a stack of env 0's frames, oldest last.
            match, episode = batch.raw_state(0)
            batch.set_raw_state(1, match, episode)
            frames = np.ascontiguousarray(batch.observation()[0])
            width = frames.shape[-1] // 4
            reordered = np.concatenate([frames[..., width * f:width * (f + 1)] for f in (3, 1, 2, 0)], axis=-1)
            stack = np.ascontiguousarray(reordered).tobytes()
            assert lib.cuju_environment_set_stack(batch._handle, 1, name, stack, len(stack)) == 0
            seen.append(np.ascontiguousarray(batch.observation()).tobytes())
            for step in range(12, 24):
                out = batch.step(digest_actions(step, 2, batch.agents, batch.action_count))
                seen.append(b''.join(np.ascontiguousarray(x).tobytes() for x in out))
            outputs.append(seen)
        finally:
            batch.close()
    assert outputs[0] == outputs[1]


def test_set_stack_refuses_what_no_minimap_holds(host_library):
    import ctypes
    batch = ref.ReferenceBatch('5_vs_5_l1_r0', environment_count=1, seed=6, threads=1, library_path=host_library,
                               representation='extracted', stacked=True)
    lib = batch._lib
    lib.cuju_environment_set_stack.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.c_void_p,
                                               ctypes.c_ulonglong]
    try:
        batch.reset()
        frames = np.ascontiguousarray(batch.observation()[0]).copy()
        frames.reshape(-1)[5] = 7
        stack = frames.tobytes()
        assert lib.cuju_environment_set_stack(batch._handle, 0, b'smm', stack, len(stack)) == -1
        assert b'minimap' in lib.cuju_last_error()
        assert lib.cuju_environment_set_stack(batch._handle, 0, b'smm', stack, len(stack) - 1) == -1
        assert b'bytes' in lib.cuju_last_error()
    finally:
        batch.close()


def test_smm_of_other_dimensions_matches_the_reference(reference_library, host_library):
    """GRF's `channel_dimensions` sets the SMM's size; marks fall into the smaller or larger grid as
    the reference puts them."""
    digests = []
    for path in (host_library, reference_library):
        batch = ref.ReferenceBatch('5_vs_5_l2_r1', environment_count=3, seed=4, threads=2, library_path=path,
                                   representation='extracted', stacked=True, channel_dimensions=(37, 21))
        try:
            digests.append(play(batch, 60, 3))
        finally:
            batch.close()
    assert digests[0] == digests[1]

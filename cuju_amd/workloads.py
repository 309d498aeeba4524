"""The five benchmark workloads of the batched step, and the counter hash that feeds them.

Every input a workload consumes (actions, reset masks, reset seeds, the bundle of each environment)
is a pure function of (seed, step, global environment index, column), where the global index is
`first_index + i`. So a batch that holds any slice of a workload's environments consumes exactly
the inputs those environments get in the full batch, the reference CPU library and the device
consume identical inputs, and a sample of environments can be replayed anywhere. The hash is
SplitMix64's finalizer (Steele, Lea and Flood, "Fast splittable pseudorandom number generators",
OOPSLA 2014) over a linear combination of the four counters; a draw is its top 31 bits.

Workloads (the reference's episode semantics are `include/cuju/batch/batch_core.h:601-649`):

1. `5_vs_5_l4_r0`, 64 environments, `simple115` (4 agents, the keeper under the built-in AI).
2. `11_vs_11_stochastic_l1_r0`, 4,096 environments (opponent difficulty 0.6).
3. `11_vs_11_hard_stochastic_l11_r0`, 16,384 environments, 11 agents (difficulty 0.95): the
   headline throughput workload.
4. `11_vs_11_stochastic_l11_r11`, 8,192 environments, both sides controlled, 4-frame stacked
   observations; every 512 steps a drawn 10% of the environments restart with drawn seeds.
5. 32,768 environments in one mixed batch: half finishing drills (1-3 controlled attackers
   against 0-2 defenders and a keeper under the built-in AI, the ball 20-35 m from goal,
   400-step episodes), a quarter `5_vs_5_l4_r0`, a quarter `11_vs_11_stochastic_l1_r0`.
"""

from __future__ import annotations

import dataclasses
import os

import numpy as np

ACTIONS = 19
_MASK64 = (1 << 64) - 1
# Weights of (seed, step, index, column) and the offset of the combination.
_WEIGHTS = (0x9E3779B97F4A7C15, 0xD1B54A32D192ED03, 0xAEF17502108EF2D9, 0xF58E2B3A4C5D6E71)
_OFFSET = 0x632BE59BD9B4E019
_MIX = (0xBF58476D1CE4E5B9, 0x94D049BB133111EB)


def _mix_int(x: int) -> int:
    x ^= x >> 30
    x = (x * _MIX[0]) & _MASK64
    x ^= x >> 27
    x = (x * _MIX[1]) & _MASK64
    return x ^ (x >> 31)


def draw_scalar(seed: int, step: int, index: int, column: int) -> int:
    """One 31-bit draw, with Python integers (the definition the array forms must equal)."""
    x = (_OFFSET + seed * _WEIGHTS[0] + step * _WEIGHTS[1] + index * _WEIGHTS[2] + column * _WEIGHTS[3]) & _MASK64
    return _mix_int(x) >> 33


def draw(seed: int, step: int, indices, columns: int) -> np.ndarray:
    """Draws `[len(indices)][columns]` as int64 in [0, 2**31), with numpy."""
    i = np.asarray(indices, dtype=np.uint64)[:, None]
    c = np.arange(columns, dtype=np.uint64)[None, :]
    with np.errstate(over='ignore'):
        base = np.uint64((_OFFSET + (seed & _MASK64) * _WEIGHTS[0] + (step & _MASK64) * _WEIGHTS[1]) & _MASK64)
        x = base + i * np.uint64(_WEIGHTS[2]) + c * np.uint64(_WEIGHTS[3])
        x ^= x >> np.uint64(30)
        x *= np.uint64(_MIX[0])
        x ^= x >> np.uint64(27)
        x *= np.uint64(_MIX[1])
        x ^= x >> np.uint64(31)
    return (x >> np.uint64(33)).astype(np.int64)


def _signed(value: int) -> int:
    value &= _MASK64
    return value - (1 << 64) if value >> 63 else value


def draw_torch(torch, seed: int, step: int, first_index: int, count: int, columns: int, device):
    """`draw` for indices first_index .. first_index + count - 1, computed on `device` with int64
    arithmetic (which wraps as uint64 does); right shifts are made logical by masking."""
    i = torch.arange(count, device=device, dtype=torch.int64)[:, None] + first_index
    c = torch.arange(columns, device=device, dtype=torch.int64)[None, :]
    base = _signed(_OFFSET + (seed & _MASK64) * _WEIGHTS[0] + (step & _MASK64) * _WEIGHTS[1])
    x = i * _signed(_WEIGHTS[2]) + c * _signed(_WEIGHTS[3]) + base

    def shr(v, k):
        return (v >> k) & ((1 << (64 - k)) - 1)

    x = x ^ shr(x, 30)
    x = x * _signed(_MIX[0])
    x = x ^ shr(x, 27)
    x = x * _signed(_MIX[1])
    x = x ^ shr(x, 31)
    return shr(x, 33)


def actions(seed, step, first_index, count, agents, action_count=ACTIONS):
    """The actions of environments first_index .. first_index + count - 1 at `step`, int32."""
    return (draw(seed, step, np.arange(first_index, first_index + count), agents) % action_count).astype(np.int32)


def actions_torch(torch, seed, step, first_index, count, agents, device, action_count=ACTIONS):
    return (draw_torch(torch, seed, step, first_index, count, agents, device) % action_count).to(torch.int32)


def masked_reset(seed, step, first_index, count, percent):
    """The mask (uint8) and int64 seeds in [0, 2**32) of a masked reset drawn at `step`."""
    d = draw(seed + 1, step, np.arange(first_index, first_index + count), 3)
    mask = (d[:, 0] % 100 < percent).astype(np.uint8)
    seeds = (d[:, 1] << 1) ^ (d[:, 2] & 1)
    return mask, (seeds & 0xFFFFFFFF).astype(np.int64)


# ---- finishing drills -------------------------------------------------------------------------------

# Field x of GRF's coordinates for a ball `metres` from the opponent's goal line:
# x_env = (55 - d) / 54.4 (include/cuju/simulation/environment.h:355-359).
def ball_x(metres: float) -> float:
    return (55.0 - metres) / 54.4


DRILL_ATTACKERS = (1, 2, 3)
DRILL_DEFENDERS = (0, 1, 2)
DRILL_DISTANCES = (20.0, 25.0, 30.0, 35.0)
DRILL_STEPS = 400


@dataclasses.dataclass(frozen=True)
class Drill:
    attackers: int
    defenders: int
    metres: float

    @property
    def name(self) -> str:
        return f'drill_{self.attackers}v{self.defenders}_k_{int(self.metres * 10)}dm'

    def build_scenario(self, builder):
        """A GRF scenario function: the left keeper (outside the agents' control) and the
        attackers, one on the ball; the right keeper and defenders between the ball and the goal.
        The drill's side switches with the episode parity."""
        from .scenarios import PlayerRole, Team
        config = builder.config()
        config.game_duration = DRILL_STEPS
        config.deterministic = False
        config.offsides = False
        config.end_episode_on_score = True
        config.end_episode_on_out_of_play = True
        config.end_episode_on_possession_change = True
        side = 1.0 if builder.EpisodeNumber() % 2 == 0 else -1.0
        x = ball_x(self.metres)
        y = 0.1 * side
        builder.SetBallPosition(x, y)
        builder.SetTeam(Team.e_Left)
        builder.AddPlayer(-1.0, 0.0, PlayerRole.e_PlayerRole_GK, controllable=False)
        spots = [(x - 0.02, y, PlayerRole.e_PlayerRole_CF), (x - 0.1, y - 0.22 * side, PlayerRole.e_PlayerRole_LM),
                 (x - 0.14, y + 0.24 * side, PlayerRole.e_PlayerRole_RM)]
        for px, py, role in spots[:self.attackers]:
            builder.AddPlayer(px, py, role)
        builder.SetTeam(Team.e_Right)
        builder.AddPlayer(-1.0, 0.0, PlayerRole.e_PlayerRole_GK)
        # The right team's own frame mirrors both axes.
        guards = [(-(x + 0.12), -(y + 0.04 * side), PlayerRole.e_PlayerRole_CB),
                  (-(x + 0.2), -(y - 0.15 * side), PlayerRole.e_PlayerRole_CB)]
        for px, py, role in guards[:self.defenders]:
            builder.AddPlayer(px, py, role)


DRILLS = tuple(Drill(a, d, m) for a in DRILL_ATTACKERS for d in DRILL_DEFENDERS for m in DRILL_DISTANCES)


def drill_bundles(directory: str, library=None) -> list:
    """Builds the bundle of every drill and returns their paths, `<drill>_l0_r0.cjb` in a
    subdirectory of `directory` named by a digest of what the bytes depend on: the builder's
    library (`library`, by default this package's), the animation tables and the drill
    definitions of this module. A bundle is built once per digest and installed by rename, so a
    reader never finds a partial file or one from another builder."""
    import hashlib
    import tempfile
    from . import library as _library
    from . import scenarios
    key = hashlib.sha256(b'cuju_amd drill bundles 1')
    for path in (os.path.abspath(library or _library.PRODUCT), os.path.join(_library.DATA, 'animations.bin'),
                 os.path.abspath(__file__)):
        with open(path, 'rb') as f:
            key.update(hashlib.sha256(f.read()).digest())
    folder = os.path.join(directory, key.hexdigest()[:24])
    os.makedirs(folder, exist_ok=True)
    paths = []
    for drill in DRILLS:
        out = os.path.join(folder, drill.name + '_l0_r0.cjb')
        if not os.path.isfile(out):
            handle, partial = tempfile.mkstemp(prefix=f'.{drill.name}-', suffix='.building', dir=folder)
            os.close(handle)
            try:
                scenarios.build_bundle(drill.build_scenario, partial, name=drill.name, library=library)
                os.replace(partial, out)
            finally:
                if os.path.exists(partial):
                    os.remove(partial)
        paths.append(out)
    return paths


# ---- the five workloads -----------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class Workload:
    number: int
    environments: int
    assets: tuple  # names or, for workload 5, kinds resolved by `batch_assets`
    agents: int
    options: dict
    reset_every: int = 0
    reset_percent: int = 0
    description: str = ''

    @property
    def stacked(self) -> bool:
        return bool(self.options.get('stacked'))

    def assignment(self, first_index: int, count: int):
        """The bundle of each environment (workload 5 only): drills for global indices 0 and 1
        modulo 4, the drill drawn from the index; then 5-a-side, then 11-a-side."""
        if self.number != 5:
            return None
        g = np.arange(first_index, first_index + count)
        pick = draw(self.number, 0, g, 1)[:, 0] % len(DRILLS)
        kind = g % 4
        return np.where(kind < 2, pick, np.where(kind == 2, len(DRILLS), len(DRILLS) + 1)).astype(np.int32)

    def batch_assets(self, drill_paths=None):
        """Assets and agent counts for a batch: names, or bundle paths with (left, right) counts."""
        if self.number != 5:
            return list(self.assets), None
        if drill_paths is None:
            raise ValueError('workload 5 needs the drill bundles (drill_bundles)')
        data = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'data', 'assets')
        paths = list(drill_paths) + [os.path.join(data, '5_vs_5_l0_r0.cjb'),
                                     os.path.join(data, '11_vs_11_stochastic_l0_r0.cjb')]
        counts = [(d.attackers, 0) for d in DRILLS] + [(4, 0), (1, 0)]
        return paths, counts

    def batch_options(self, first_index: int, count: int, drill_paths=None) -> dict:
        assets, counts = self.batch_assets(drill_paths)
        options = dict(self.options)
        options['first_index'] = first_index
        options['environment_count'] = count
        if counts is not None:
            options['agent_counts'] = counts
            options['assignment'] = self.assignment(first_index, count)
        return dict(assets=assets, **options)


WORKLOADS = {
    1: Workload(1, 64, ('5_vs_5_l4_r0',), 4, {'representation': 'simple115'},
                description='5_vs_5_l4_r0: 64 environments x 4 agents, simple115, auto reset'),
    2: Workload(2, 4096, ('11_vs_11_stochastic_l1_r0',), 1, {},
                description='11_vs_11_stochastic_l1_r0: 4096 environments x 1 agent, simple115v2, auto reset'),
    3: Workload(3, 16384, ('11_vs_11_hard_stochastic_l11_r0',), 11, {},
                description='11_vs_11_hard_stochastic_l11_r0: 16384 environments x 11 agents, simple115v2, '
                            '3000-step episodes, auto reset'),
    4: Workload(4, 8192, ('11_vs_11_stochastic_l11_r11',), 22, {'stacked': True}, reset_every=512, reset_percent=10,
                description='11_vs_11_stochastic_l11_r11: 8192 environments x 22 agents, 4-frame stacked simple115v2, '
                            '10% masked resets with drawn seeds every 512 steps'),
    5: Workload(5, 32768, ('drills', '5_vs_5_l4_r0', '11_vs_11_stochastic_l1_r0'), 4, {},
                description='mixed: 32768 environments, half drills (1-3 attackers v 0-2 defenders + keeper, '
                            '20-35 m, 400-step episodes), a quarter 5_vs_5_l4_r0, a quarter 11_vs_11_stochastic_l1_r0'),
}

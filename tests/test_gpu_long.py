"""Long horizons on the MI355X, in one loop so that every batch runs at once, each on a stream of
its own:

* the reference's five long digests (python/cuju/data/digests.json `long_cases`): full 3,010-step
  matches and 1,500-2,000-step drill runs with raw, SMM and checkpoint outputs, 4 environments each
  (the reference's tests/test_long.py:59-69);
* long episodes of each of the five benchmark workloads at the geometry the workload's full batch
  gets, as the benchmark runs it, against per-environment digests of the reference CPU library
  (`tests/golden/episodes.json`, written by `tests/golden/make_episodes.py`): the end of the
  workload's index range (`first_index`) in four full wavefronts, 8 environments of 8 lanes each
  for the 16,384-environment workload, 16 of 4 lanes for the 32,768-environment mixed batch, 4 of
  16 for the 8,192 self-play batch, 2 of 32 for 4,096, and 1 of 64 for the 64 environments of
  workload 1, whose start range (8 environments) plays too. `CUJU_AMD_LONG_RANGES=all` adds the
  start range of every workload, one environment to a wavefront.

Horizons: 5,000 steps for the 16,384-environment workload (the headline), 3,000 for the others;
`CUJU_AMD_EPISODE_STEPS` sets one horizon for all (10,000 is the last golden checkpoint).

The long digests put one environment in a wavefront (`lockstep.one_match_per_wavefront`): a step
of a small batch then takes the time of one match. HIP spreads the streams over the process's
hardware queues (4 by default), and the batches that share a queue run one after another, so a
lockstep step costs about a quarter of the sum of the batches' own step times; the batches are
made in order of falling cost, so that the costly ones land on different queues.
`CUJU_AMD_LONG_PARTS` (default `digests,1,2,3,4,5`) names the parts to play, so a 10,000-step run
can be split over several processes.
"""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

import episodes
import lockstep
from conftest import PRODUCT, ROOT, load_digests
from cuju_amd import workloads

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(ROOT, 'tests', 'golden', 'episodes.json')


def host(x):
    return x.detach().cpu().numpy()


# Horizon of each workload's episodes unless CUJU_AMD_EPISODE_STEPS sets one for all.
HORIZONS = {3: 5000}
DEFAULT_HORIZON = 3000
# A lockstep step's cost of a batch, by environments per wavefront (ms, measured alone on an MI355X):
# the order in which batches take streams.
COST = {1: 20, 2: 30, 4: 41, 8: 60, 16: 77}


class DeviceSide:
    """A `cuju_amd.BatchEnvironment` of one workload range on its own stream, `matches`
    environments to a wavefront."""

    def __init__(self, workload, first_index, count, drill_paths, matches):
        import cuju_amd
        options = workload.batch_options(first_index, count, drill_paths)
        assets = options.pop('assets')
        with lockstep.matches_per_wavefront(matches):
            self.batch = cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0',
                                                   seed=episodes.seed_of(workload), **options)
        got, lanes = self.batch.geometry
        assert got == matches, f'asked for {matches} environments per wavefront, the batch has {got}'
        self.geometry = f'{got} x {lanes} lanes'
        self.stream = torch.cuda.Stream()
        self.stacked = workload.stacked

    def reset(self):
        with torch.cuda.stream(self.stream):
            obs = self.batch.reset()
        self.stream.synchronize()
        return host(obs)

    def reset_masked(self, mask, seeds):
        with torch.cuda.stream(self.stream):
            obs = self.batch.reset(seeds=seeds, mask=torch.as_tensor(mask.astype(bool)))
        self.stream.synchronize()
        return host(obs)

    def launch(self, actions):
        with torch.cuda.stream(self.stream):
            self.out = self.batch.step(torch.as_tensor(actions, device='cuda:0'))

    def collect(self):
        self.stream.synchronize()
        obs, reward, done, info = self.out
        done = host(done).astype(np.uint8)
        final = host(info['final_observation']) if done.any() else None
        return host(obs), host(reward), done, final

    def state(self, index):
        state = self.batch.get_state(index, stacked=self.stacked)
        return episodes.engine_bytes(state) if self.stacked else state

    def close(self):
        self.batch.close()


def test_long_horizons_match_the_reference(tmp_path, capsys):
    with open(GOLDEN) as f:
        golden = json.load(f)
    forced = os.environ.get('CUJU_AMD_EPISODE_STEPS')
    drill_paths = workloads.drill_bundles(str(tmp_path / 'drills'))
    built = {os.path.basename(p): hashlib.sha256(open(p, 'rb').read()).hexdigest() for p in drill_paths}
    assert built == golden['drill_bundles'], 'the drill bundles differ from the reference builder\'s'

    parts = os.environ.get('CUJU_AMD_LONG_PARTS', 'digests,' + ','.join(map(str, sorted(workloads.WORKLOADS))))
    parts = {p.strip() for p in parts.split(',') if p.strip()}
    unknown = parts - {'digests'} - {str(n) for n in workloads.WORKLOADS}
    assert not unknown, f'CUJU_AMD_LONG_PARTS names no part {sorted(unknown)}'
    every_range = os.environ.get('CUJU_AMD_LONG_RANGES', 'production') == 'all'
    report = lockstep.uncaptured(capsys)
    digests = load_digests()
    planned = []
    for number in sorted(n for n in workloads.WORKLOADS if str(n) in parts):
        w = workloads.WORKLOADS[number]
        horizon = int(forced) if forced else HORIZONS.get(number, DEFAULT_HORIZON)
        checkpoints = [c for c in golden['checkpoints'] if c <= horizon]
        assert checkpoints, f'no golden checkpoint at or below {horizon} steps'
        for first, count, matches in episodes.sample_ranges(w):
            if every_range or matches == episodes.PRODUCTION_MATCHES[number]:
                planned.append((COST[matches], w, first, count, matches, checkpoints))
    runs = []
    try:
        for _, w, first, count, matches, checkpoints in sorted(planned, key=lambda p: -p[0]):
            side = DeviceSide(w, first, count, drill_paths, matches)
            run = episodes.EpisodeRun(w, first, count, side, checkpoints=checkpoints)
            report(f'{run.name}: {side.geometry}, to step {max(checkpoints)}')
            runs.append(run)
        if 'digests' in parts:
            with lockstep.one_match_per_wavefront():
                for name, case in sorted(digests['long_cases'].items()):
                    runs.append(lockstep.DigestRun(name, case, digests['environments'], digests['seed'],
                                                   case['steps']))
        lockstep.play(runs, label='long horizons', report=report)
        failed = [r.name for r in runs if isinstance(r, lockstep.DigestRun) and r.hexdigest() != r.case['digest']]
        for r in runs:
            if isinstance(r, episodes.EpisodeRun):
                expected = golden['workloads'][str(r.workload.number)][str(r.first_index)]
                for checkpoint in r.checkpoints:
                    for i, (got, want) in enumerate(zip(r.digests[checkpoint], expected[str(checkpoint)], strict=True)):
                        if got != want:
                            failed.append(f'{r.name}: environment {r.first_index + i} at step {checkpoint}')
                report(f'{r.name}: {r.count} environments checked at steps {list(r.checkpoints)}')
        assert not failed, f'digests that differ from the reference: {failed}'
    finally:
        for r in runs:
            (r.side if isinstance(r, episodes.EpisodeRun) else r).close()

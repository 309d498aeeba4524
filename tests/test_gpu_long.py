"""Long horizons on the MI355X, every batch on a stream of its own, each stream at its own pace:

* the reference's five long digests (python/cuju/data/digests.json `long_cases`): full 3,010-step
  matches and 1,500-2,000-step drill runs with raw, SMM and checkpoint outputs, 4 environments each,
  one environment of 16 lanes to a wavefront (the reference's tests/test_long.py:59-69);
* 10,000 steps of each of the five benchmark workloads at the geometry the workload's full batch
  gets, as the benchmark runs it (8 environments of 8 lanes to a wavefront for the
  16,384-environment headline, 16 of 4 for the 32,768-environment mixed batch, 4 of 16 for the
  8,192 self-play batch, 2 of 32 for 4,096, 1 of 64 for 64): one batch of four blocks, one
  wavefront each, that play global steps 0-3,000, 2,500-5,500, 5,000-8,000 and 7,000-10,000 of
  the same environments (`segments.py`), against the reference CPU library playing the same
  batch, and block 0 against the committed goldens at step 3,000 (`tests/golden/episodes.json`,
  written by `tests/golden/make_episodes.py`).

HIP spreads the streams over the process's hardware queues (4 by default); batches that share a
queue run one after another. `CUJU_AMD_LONG_PARTS` (default `digests,1,2,3,4,5`) names the parts
to play.
"""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

import episodes
import lockstep
from conftest import PRODUCT, REFERENCE, ROOT, load_digests
from cuju_amd import workloads

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(ROOT, 'tests', 'golden', 'episodes.json')


def host(x):
    return x.detach().cpu().numpy()


# Seconds the four-block batch of each workload takes for its 3,000 steps alone on an MI355X.
BLOCK_SECONDS = {1: 54, 2: 90, 3: 222, 4: 123, 5: 231}


def test_long_horizons_match_the_reference(tmp_path, capsys):
    import concurrent.futures
    import segments
    with open(GOLDEN) as f:
        golden = json.load(f)
    drill_paths = workloads.drill_bundles(str(tmp_path / 'drills'))
    built = {os.path.basename(p): hashlib.sha256(open(p, 'rb').read()).hexdigest() for p in drill_paths}
    assert built == golden['drill_bundles'], 'the drill bundles differ from the reference builder\'s'

    parts = os.environ.get('CUJU_AMD_LONG_PARTS', 'digests,' + ','.join(map(str, sorted(workloads.WORKLOADS))))
    parts = {p.strip() for p in parts.split(',') if p.strip()}
    unknown = parts - {'digests'} - {str(n) for n in workloads.WORKLOADS}
    assert not unknown, f'CUJU_AMD_LONG_PARTS names no part {sorted(unknown)}'
    report = lockstep.uncaptured(capsys)
    numbers = sorted(n for n in workloads.WORKLOADS if str(n) in parts)
    # The reference plays block 0's environments to the blocks' starting steps, all workloads at once.
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, len(numbers))) as pool:
        states = dict(zip(numbers, pool.map(
            lambda n: segments.starting_states(workloads.WORKLOADS[n], drill_paths, REFERENCE), numbers)))
    report(f'reference states at steps {list(segments.STARTS[1:])} for workloads {numbers}')
    oracle_pool = concurrent.futures.ThreadPoolExecutor(max_workers=max(1, len(numbers)))
    expected = {n: oracle_pool.submit(segments.play_oracle, segments.BlockRun(
        workloads.WORKLOADS[n], segments.OracleBlocks(workloads.WORKLOADS[n], drill_paths, REFERENCE), states[n]))
        for n in numbers}
    # Streams on distinct hardware queues (HIP gives the process four; some may be taken), each a
    # lane that plays its batches one after another; the batches go to the least loaded lane by
    # their cost, the seconds their steps take alone on an MI355X.
    streams = lockstep.concurrent_streams(4, candidates=24)
    report(f'{len(streams)} streams run side by side')
    items = []
    for n in numbers:
        w = workloads.WORKLOADS[n]
        items.append((BLOCK_SECONDS[n], ('blocks', n)))
    digests = load_digests()
    if 'digests' in parts:
        for name, case in sorted(digests['long_cases'].items()):
            items.append((case['steps'] * 0.020, ('digest', name)))
    lanes = [[] for _ in streams]
    load = [0.0] * len(streams)
    runs = []
    try:
        for cost, (kind, key) in sorted(items, key=lambda item: -item[0]):
            lane = min(range(len(streams)), key=lambda i: load[i])
            load[lane] += cost
            if kind == 'blocks':
                w = workloads.WORKLOADS[key]
                side = segments.DeviceBlocks(w, drill_paths, PRODUCT, episodes.PRODUCTION_MATCHES[key], streams[lane])
                matches, lanes_per_match = side.geometry
                assert matches == episodes.PRODUCTION_MATCHES[key], (key, side.geometry)
                run = segments.BlockRun(w, side, states[key])
                report(f'lane {lane}: {run.name}: {matches} x {lanes_per_match} lanes, {run.count} environments, '
                       f'{segments.SEGMENT} steps')
            else:
                case = digests['long_cases'][key]
                with lockstep.one_match_per_wavefront():
                    run = lockstep.DigestRun(key, case, digests['environments'], digests['seed'], case['steps'], streams[lane])
                report(f'lane {lane}: long digest {key}, {case["steps"]} steps')
            lanes[lane].append(run)
            runs.append(run)
        lockstep.play_lanes(lanes, label='long horizons', report=report)
        failed = [r.name for r in runs if isinstance(r, lockstep.DigestRun) and r.hexdigest() != r.case['digest']]
        for r in runs:
            if not isinstance(r, segments.BlockRun):
                continue
            n = r.workload.number
            want = expected[n].result()
            for i, (got, ref_digest) in enumerate(zip(r.digests, want, strict=True)):
                if got != ref_digest:
                    failed.append(f'{r.name}: block {i // r.m} environment {i % r.m} against the reference')
            first = segments.first_index(r.workload)
            goldens = golden['workloads'][str(n)][str(first)]['3000'][:r.m]
            for i in range(r.m):
                if want[i] != goldens[i]:
                    failed.append(f'{r.name}: the reference\'s block 0 environment {i} against the goldens')
            report(f'{r.name}: {r.count} environments checked, global steps 0-10,000')
        assert not failed, f'digests that differ from the reference: {failed}'
    finally:
        oracle_pool.shutdown(wait=True)
        for r in runs:
            r.side.close() if isinstance(r, segments.BlockRun) else r.close()

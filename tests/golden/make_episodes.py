"""Writes `episodes.json`: per-environment digests of the five benchmark workloads over long
episodes, played on the reference CPU library built into `oracle/_ref/` (see `tests/episodes.py`
for the sample and the digest). It runs in the build container, where the reference sources are:

    python tests/golden/make_episodes.py

Workload 5's drill bundles are built by the reference library's own scenario builder; their
SHA-256 goes into the file, so a device run can check that this package's builder made the same
bundles.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import json
import os
import sys
import tempfile
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

OUT = os.path.join(HERE, 'episodes.json')


# Environments of one job: a sampled range splits into jobs of at most this many, since each
# environment's digest depends on its global index alone, not on the batch it plays in.
JOB = 8


def _play(number, first_index, count, drill_paths):
    from cuju_amd import workloads
    import episodes
    workload = workloads.WORKLOADS[number]
    side = episodes.OracleSide(workload, first_index, count, drill_paths, threads=1)
    run = episodes.EpisodeRun(workload, first_index, count, side)
    start = time.time()
    run.start()
    while not run.done:
        run.launch()
        run.collect()
    side.close()
    return number, first_index, run.digests, time.time() - start


def main():
    from cuju_amd import workloads
    from oracle import ref
    import episodes
    directory = tempfile.mkdtemp(prefix='drills_')
    drill_paths = workloads.drill_bundles(directory, library=ref.LIBRARY)
    bundles = {os.path.basename(p): hashlib.sha256(open(p, 'rb').read()).hexdigest() for p in drill_paths}
    ranges = [(n, first, count) for n in sorted(workloads.WORKLOADS)
              for first, count, _ in episodes.sample_ranges(workloads.WORKLOADS[n])]
    jobs = [(n, first + k, min(JOB, count - k)) for n, first, count in ranges for k in range(0, count, JOB)]
    result = {'checkpoints': list(episodes.CHECKPOINTS), 'drill_bundles': bundles, 'workloads': {}}
    found = {}
    with concurrent.futures.ProcessPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
        futures = [pool.submit(_play, n, first, count, drill_paths) for n, first, count in jobs]
        for f in concurrent.futures.as_completed(futures):
            number, first, digests, seconds = f.result()
            print(f'workload {number} from {first}: {seconds:.0f} s', flush=True)
            found[number, first] = digests
    # Each range's digests, its jobs' in index order.
    for n, first, count in ranges:
        entry = result['workloads'].setdefault(str(n), {})
        parts = [found[n, first + k] for k in range(0, count, JOB)]
        entry[str(first)] = {str(c): [d for part in parts for d in part[c]] for c in episodes.CHECKPOINTS}
    with open(OUT, 'w') as f:
        json.dump(result, f, indent=1, sort_keys=True)
        f.write('\n')
    print(f'wrote {OUT}')


if __name__ == '__main__':
    main()

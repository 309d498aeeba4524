"""Plays many small device batches at once: each on a stream of its own, all stepped in lockstep
from the host, so that their kernels run side by side on the GPU. A step of a small batch takes
about as long as the step of one match, so the batches cost together what one costs alone.

A run has `start()`, `launch()` (enqueue one step), `collect()` (wait for it and absorb its
outputs) and `done`. `one_match_per_wavefront()` makes the batches created inside it put a single
environment in each wavefront: a wavefront then follows one match's control flow, and a step of a
small batch takes the least time. The environments of a wavefront are independent, so the
geometry changes no result; the tests that run the library's geometries (up to 32 environments in
a wavefront) cover the code where matches of a wavefront wait for each other.
"""

from __future__ import annotations

import contextlib
import hashlib
import os
import time

import numpy as np
import torch

from conftest import PRODUCT, digest_actions


@contextlib.contextmanager
def matches_per_wavefront(matches, lanes=None):
    """Batches created inside put `matches` environments in each wavefront, of `lanes` lanes each
    (by default the library's choice for that many)."""
    settings = {'CUJU_AMD_MATCHES': str(matches), 'CUJU_AMD_LANES': None if lanes is None else str(lanes)}
    before = {name: os.environ.get(name) for name in settings}
    for name, value in settings.items():
        if value is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = value
    try:
        yield
    finally:
        for name, value in before.items():
            if value is None:
                os.environ.pop(name, None)
            else:
                os.environ[name] = value


def one_match_per_wavefront():
    """One environment of 16 lanes in each wavefront."""
    return matches_per_wavefront(1, 16)


def uncaptured(capsys):
    """A report function that prints to the terminal whatever pytest captures."""
    def report(line):
        with capsys.disabled():
            print(line, flush=True)
    return report


def raw_bytes(x):
    if isinstance(x, dict):
        return b''.join(raw_bytes(x[name]) for name in sorted(x))
    return np.ascontiguousarray(x.detach().cpu().numpy()).tobytes()


class DigestRun:
    """A digest case of the reference's self-check (tests/conftest.py:69-98 of the reference):
    SHA-256 over the reset observation, every step's observation, reward and done, then every
    environment's state."""

    def __init__(self, name, case, environments, seed, steps, stream=None):
        import cuju_amd
        self.name, self.case, self.environments, self.steps = name, case, environments, steps
        self.batch = cuju_amd.BatchEnvironment(case['assets'], library=PRODUCT, device='cuda:0',
                                               environment_count=environments, seed=seed, **dict(case['options']))
        self.stream = stream or torch.cuda.Stream()
        self.step = 0

    def start(self):
        with torch.cuda.stream(self.stream):
            first = self.batch.reset()
        self.stream.synchronize()
        self.digest = hashlib.sha256(raw_bytes(first))

    def launch(self):
        with torch.cuda.stream(self.stream):
            actions = torch.as_tensor(digest_actions(self.step, self.environments, self.batch.agents,
                                                     self.batch.action_count), device='cuda:0')
            self.out = self.batch.step(actions)

    def collect(self):
        self.stream.synchronize()
        for x in self.out[:3]:
            self.digest.update(raw_bytes(x))
        self.step += 1
        if self.done and self.batch.stack == 1:
            for index in range(self.environments):
                self.digest.update(self.batch.get_state(index))

    def ready(self):
        return self.stream.query()

    @property
    def done(self):
        return self.step >= self.steps

    def hexdigest(self):
        return self.digest.hexdigest()

    def close(self):
        self.batch.close()


def play(runs, label='lockstep', every=250, report=print):
    """Starts every run, then steps the live ones together until all are done. Every `every`
    steps `report` gets a progress line: a test passes one that writes past pytest's capture, so
    that a long run keeps printing."""
    for r in runs:
        r.start()
    begin = time.time()
    step = 0
    while True:
        live = [r for r in runs if not r.done]
        if not live:
            return
        for r in live:
            r.launch()
        for r in live:
            r.collect()
        step += 1
        if every and step % every == 0:
            report(f'{label}: step {step}, {len(live)} batches running, {time.time() - begin:.0f} s')


def concurrent_streams(k, candidates=16, spin=4_000_000):
    """Up to `k` streams whose kernels run side by side: HIP spreads streams over a few hardware
    queues, and the kernels of streams that share one run one after another. Each candidate joins
    the chosen ones if a spin kernel on it and on every chosen stream together takes about as long
    as one alone."""
    def together(streams):
        torch.cuda.synchronize()
        start = time.perf_counter()
        for st in streams:
            with torch.cuda.stream(st):
                torch.cuda._sleep(spin)
        torch.cuda.synchronize()
        return time.perf_counter() - start
    pool = [torch.cuda.Stream() for _ in range(candidates)]
    together(pool[:1])
    alone = min(together(pool[:1]) for _ in range(3))
    chosen = [pool[0]]
    for st in pool[1:]:
        if len(chosen) == k:
            break
        if together(chosen + [st]) < 1.5 * alone:
            chosen.append(st)
    return chosen


def play_lanes(lanes, label='lanes', every_s=30.0, report=print):
    """Plays lanes of runs: each lane is a list of runs that play one after another on the lane's
    stream, every lane at its own pace (one step of each lane in flight; a lane whose step has
    finished is collected and launched again at once). A run has start(), launch(), ready(),
    collect(), done and step."""
    cursors = [0] * len(lanes)
    active = []
    for i, lane in enumerate(lanes):
        if lane:
            lane[0].start()
            active.append(i)
    for i in active:
        lanes[i][0].launch()
    begin = last = time.time()
    while active:
        progressed = False
        for i in list(active):
            run = lanes[i][cursors[i]]
            if not run.ready():
                continue
            run.collect()
            progressed = True
            if run.done:
                cursors[i] += 1
                if cursors[i] == len(lanes[i]):
                    active.remove(i)
                    continue
                run = lanes[i][cursors[i]]
                run.start()
            run.launch()
        if not progressed:
            time.sleep(0.0005)
        if every_s and time.time() - last >= every_s:
            last = time.time()
            state = '; '.join(f'lane {i}: {lanes[i][cursors[i]].name} step {lanes[i][cursors[i]].step}' for i in active)
            report(f'{label}: {last - begin:.0f} s; {state}')

"""Throughput of the step engine on one MI355X, for the five benchmark workloads.

The workloads are those of `cuju_amd.workloads`:

1. `5_vs_5_l4_r0`, 64 environments x 4 agents, `simple115`;
2. `11_vs_11_stochastic_l1_r0`, 4,096 environments x 1 agent;
3. `11_vs_11_hard_stochastic_l11_r0`, 16,384 environments x 11 agents (the right team is the
   built-in AI at difficulty 0.95): the headline, whose figures are the line's top-level ones;
4. `11_vs_11_stochastic_l11_r11`, 8,192 environments x 22 agents, 4-frame stacked, with masked
   resets of a drawn 10% every 512 steps;
5. 32,768 environments of drills, 5-a-side and 11-a-side in one mixed batch.

Method (the reference's, `examples/benchmark.py:21-53`, `docs/performance.md:22-29`): every batch is
created and reset, and plays `--warmup` untimed steps; then `--steps` timed steps of each workload
run in `--rounds` interleaved rounds, each round playing its share of the steps of workload 1,
then 2, ..., then 5. A workload's value is its environments times its timed steps over the wall
time of those steps (each round's steps bracketed by device synchronizations); `rounds` gives the
rate of each round with the median and spread. A step is one `BatchEnvironment.step` of every
environment of the batch. Actions are uniform integers in [0, 19) from the workloads' counter hash
of (seed, step, environment, agent), computed on the device before the timed steps; workload 4's
masked resets run inside the timed steps when they fall in them. The reference discards its first
100 steps, as the default `--warmup` does; the steps right after a reset are cheaper than open
play, so a line with fewer says so.

For each workload the line also gives the step kernel's launch durations (HIP events on the stream
the kernel runs on), its roofline (the algorithmic HBM bytes of a launch over its mean duration,
against 8 TB/s) with the HBM traffic rocprofv3 measured for the same window where one was
profiled, and the reference's own CPU thread pool on this host's cores, timed over the same
steps, rounds and inputs on a sample of the workload's environments.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# The reference world's size (sizeof(cuju::simulation::World), 11 players a side), read and written
# once per environment step: the per-unit figure of the roofline, independent of this engine's own
# layout (its World is 373,536 B).
WORLD_BYTES = 373_552
STEADY_WARMUP = 100
HEADLINE = 3
# Environments of a workload that the CPU baseline plays (all of them below this).
CPU_SAMPLE = 2048

# HBM bytes one step launch moves, read + written, from rocprofv3 FETCH_SIZE and WRITE_SIZE passes
# (each scaled by what the counter reads for a 1 GiB device copy), keyed by (workload,
# environments, warm-up steps, timed steps, rounds): the window of launches the profile averaged.
MEASURED_TRAFFIC = {
    (1, 64, 5, 20, 3): (75848861, 'profiles/step_kernel_5v5_64_driver_window.md'),
    (2, 4096, 5, 20, 3): (65277143487, 'profiles/step_kernel_11v11_4096_driver_window.md'),
    (3, 16384, 5, 20, 3): (191055945597, 'profiles/step_kernel_11v11_hard_16384_driver_window.md'),
    (4, 8192, 5, 20, 3): (109599148534, 'profiles/step_kernel_11v11_selfplay_stacked_8192_driver_window.md'),
    (5, 32768, 5, 20, 3): (185300503006, 'profiles/step_kernel_mixed_32768_driver_window.md'),
    (1, 64, 100, 30, 3): (77848709, 'profiles/step_kernel_5v5_64.md'),
    (2, 4096, 100, 30, 3): (65060719838, 'profiles/step_kernel_11v11_4096.md'),
    (3, 16384, 100, 30, 3): (193424500413, 'profiles/step_kernel_11v11_hard_16384.md'),
    (4, 8192, 100, 30, 3): (110546197410, 'profiles/step_kernel_11v11_selfplay_stacked_8192.md'),
    (5, 32768, 100, 30, 3): (192416493757, 'profiles/step_kernel_mixed_32768.md'),
}


def algorithmic_bytes(workload, agents_present, agent_axis):
    """The compulsory HBM bytes of one environment step: the world read and written once, the
    actions read, the observation written (the stacked frames shifted: 3 of 4 read back), the
    reward, done and score written."""
    stack = 4 if workload.stacked else 1
    io = agents_present * (4 + 460 * stack) + (345 * agents_present * 4 if stack == 4 else 0) + 4 * agent_axis + 5
    return 2 * WORLD_BYTES + io


def metric_name(workload, environments):
    """The headline metric's name for workload 3 at its full size; otherwise one naming the run."""
    if workload.number == HEADLINE and environments == workload.environments:
        return 'env steps/sec on 1 MI355X (11v11, 16384 envs) + bit-exact digest match'
    return f'env steps/sec on 1 MI355X (workload {workload.number}, {environments} envs) + bit-exact digest match'


def cpu_model():
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def round_sizes(steps, rounds):
    """The timed steps of each round: `steps` split as evenly as `rounds` allows."""
    rounds = max(1, min(rounds, steps))
    return [steps // rounds + (1 if r < steps % rounds else 0) for r in range(rounds)]


def summary(environments, walls, sizes):
    rates = [environments * n / w for n, w in zip(sizes, walls)]
    median = statistics.median(rates)
    return {'env_steps_per_s': rates, 'median': median, 'spread': (max(rates) - min(rates)) / median}


class DeviceRun:
    """One workload's batch on the device: reset, warm-up, then timed rounds."""

    def __init__(self, torch, workload, environments, seed, drill_paths, device):
        import numpy as np
        import cuju_amd
        self.torch, self.workload, self.environments, self.seed, self.device = torch, workload, environments, seed, device
        options = workload.batch_options(0, environments, drill_paths)
        assets = options.pop('assets')
        self.env = cuju_amd.BatchEnvironment(assets, device=device, seed=seed, **options)
        self.agents = self.env.agents
        present = (self.env.left_agents + self.env.right_agents).numpy().astype(np.float64)
        self.bytes_per_step = float(np.mean([algorithmic_bytes(workload, a, self.agents) for a in present]))
        self.matches, self.lanes = self.env.geometry
        torch.cuda.synchronize()
        start = time.perf_counter()
        self.env.reset()
        self.env.synchronize()
        self.reset_seconds = time.perf_counter() - start
        self.step = 0
        self.launch_ms, self.walls = [], []

    def _masked_reset(self):
        from cuju_amd import workloads
        w = self.workload
        if w.reset_every and self.step % w.reset_every == 0:
            mask, seeds = workloads.masked_reset(self.seed, self.step, 0, self.environments, w.reset_percent)
            self.env.reset(seeds=seeds, mask=self.torch.as_tensor(mask.astype(bool)))

    def _actions(self, step):
        from cuju_amd import workloads
        return workloads.actions_torch(self.torch, self.seed, step, 0, self.environments, self.agents, self.device)

    def warm_up(self, steps):
        for k in range(steps):
            self.env.step(self._actions(self.step))
            self.step += 1
            self._masked_reset()
            if k % 25 == 24:
                self.env.synchronize()
        self.env.synchronize()

    def timed(self, steps):
        torch = self.torch
        actions = [self._actions(self.step + k) for k in range(steps)]
        stream = torch.cuda.current_stream(self.device)
        begin = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        end = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        torch.cuda.synchronize()
        wall = time.perf_counter()
        for k in range(steps):
            begin[k].record(stream)
            self.env.step(actions[k])
            end[k].record(stream)
            self.step += 1
            self._masked_reset()
        self.env.synchronize()
        torch.cuda.synchronize()
        self.walls.append(time.perf_counter() - wall)
        self.launch_ms += [b.elapsed_time(e) for b, e in zip(begin, end)]

    def close(self):
        self.env.close()


class CpuRun:
    """The reference CPU library (its own thread pool, every core it may use) on the first
    environments of a workload, fed the same inputs as the device."""

    def __init__(self, workload, environments, seed, drill_paths):
        from oracle import ref
        options = workload.batch_options(0, environments, drill_paths)
        assets = options.pop('assets')
        self.workload, self.environments, self.seed = workload, environments, seed
        self.batch = ref.ReferenceBatch(assets, seed=seed, threads=0, **options)
        self.batch.reset()
        self.agents = self.batch.agents
        self.step = 0
        self.walls = []

    def _advance(self, actions):
        from cuju_amd import workloads
        w = self.workload
        self.batch.step(actions)
        self.step += 1
        if w.reset_every and self.step % w.reset_every == 0:
            mask, seeds = workloads.masked_reset(self.seed, self.step, 0, self.environments, w.reset_percent)
            self.batch.reset(seeds=seeds, mask=mask)

    def _actions(self, step):
        from cuju_amd import workloads
        return workloads.actions(self.seed, step, 0, self.environments, self.agents)

    def warm_up(self, steps):
        for _ in range(steps):
            self._advance(self._actions(self.step))

    def timed(self, steps):
        inputs = [self._actions(self.step + k) for k in range(steps)]
        start = time.perf_counter()
        for k in range(steps):
            self._advance(inputs[k])
        self.walls.append(time.perf_counter() - start)

    def close(self):
        self.batch.close()


def cpu_baselines(numbers, args, drill_paths, report):
    """The CPU thread pool over the device's window: the same warm-up, the same timed steps in the
    same interleaved rounds, each workload on its first `CPU_SAMPLE` environments."""
    from cuju_amd import workloads
    from oracle import ref
    if not os.path.isfile(ref.LIBRARY):
        return {}
    sizes = round_sizes(args.steps, args.rounds)
    runs = {}
    try:
        for n in numbers:
            w = workloads.WORKLOADS[n]
            runs[n] = CpuRun(w, min(w.environments, args.cpu_environments), args.seed, drill_paths)
            runs[n].warm_up(args.warmup)
            report(f'CPU workload {n}: {runs[n].environments} environments warmed up')
        for size in sizes:
            for n in numbers:
                runs[n].timed(size)
        out = {}
        for n, r in runs.items():
            rounds = summary(r.environments, r.walls, sizes)
            out[n] = {'value': r.environments * sum(sizes) / sum(r.walls), 'unit': 'env_steps/s',
                      'cores': r.batch.threads, 'kind': 'reference', 'cpu': cpu_model(), 'rounds': rounds,
                      'sample': f'environments 0-{r.environments - 1} of workload {n}: after a reset and {args.warmup} '
                                f'warm-up steps, {sum(sizes)} timed steps in {len(sizes)} interleaved rounds, the '
                                f'same steps and counter-hash actions as the device'}
        return out
    finally:
        for r in runs.values():
            r.close()


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument('--gpus', type=int, default=1)
    parser.add_argument('--steps', type=int, default=30, help='timed steps of each workload, over all rounds')
    parser.add_argument('--warmup', type=int, default=STEADY_WARMUP)
    parser.add_argument('--rounds', type=int, default=3)
    parser.add_argument('--configs', default='1,2,3,4,5', help='the workloads to run, in round order')
    parser.add_argument('--config', type=int, default=None, choices=[1, 2, 3, 4, 5],
                        help='run this workload alone (its line is then the top-level one)')
    parser.add_argument('--environments', type=int, default=None, help='with --config: default the workload\'s')
    parser.add_argument('--seed', type=int, default=0)
    parser.add_argument('--cpu-environments', type=int, default=CPU_SAMPLE)
    parser.add_argument('--no-cpu', action='store_true')
    parser.add_argument('--matches', type=int, default=None, help='environments per workgroup (one wavefront)')
    parser.add_argument('--copy-probe', action='store_true',
                        help='also run a 1 GiB device-to-device copy, the calibration of HBM byte counters')
    args = parser.parse_args()
    if args.matches is not None:
        os.environ['CUJU_AMD_MATCHES'] = str(args.matches)
    if args.gpus != 1:
        print(f'bench.py measures one GPU: every GPU box here has one, and the engine has no multi-GPU path '
              f'(environments shard by first_index with no exchange); asked for --gpus {args.gpus}.', file=sys.stderr)
        sys.exit(2)
    numbers = [args.config] if args.config else [int(n) for n in args.configs.split(',') if n.strip()]
    if args.environments and len(numbers) != 1:
        parser.error('--environments needs --config')
    headline = HEADLINE if HEADLINE in numbers else numbers[0]

    def report(text):
        print(f'[bench] {text}', file=sys.stderr, flush=True)

    import torch
    from cuju_amd import workloads

    device = torch.device('cuda', 0)
    torch.cuda.set_device(device)
    drill_paths = None
    if 5 in numbers:
        drill_paths = workloads.drill_bundles(os.path.join(tempfile.gettempdir(), 'cuju_amd_drills'))
    runs = {}
    for n in numbers:
        w = workloads.WORKLOADS[n]
        report(f'workload {n}: creating {args.environments or w.environments} environments')
        runs[n] = DeviceRun(torch, w, args.environments or w.environments, args.seed, drill_paths, device)
        runs[n].warm_up(args.warmup)
        report(f'workload {n}: {runs[n].matches} x {runs[n].lanes} lanes per wavefront, {args.warmup} warm-up steps '
               f'done')
    sizes = round_sizes(args.steps, args.rounds)
    for r, size in enumerate(sizes):
        for n in numbers:
            runs[n].timed(size)
        report(f'round {r + 1} of {len(sizes)}: ' +
               ', '.join(f'{n}: {runs[n].walls[-1] / size * 1000:.1f} ms' for n in numbers))
    for run in runs.values():
        run.close()
    if args.copy_probe:
        source = torch.empty(1 << 28, dtype=torch.float32, device=device).fill_(1.0)
        target = torch.empty_like(source)
        torch.cuda.synchronize()
        target.copy_(source)
        torch.cuda.synchronize()
        report('copy probe: 1 GiB read, 1 GiB written')

    baselines = {}
    if not args.no_cpu:
        report('timing the reference CPU thread pool')
        baselines = cpu_baselines(numbers, args, drill_paths, report)

    steps = sum(sizes)
    results = {}
    for n, run in runs.items():
        w = run.workload
        mean_launch_s = statistics.fmean(run.launch_ms) / 1000.0
        achieved = run.bytes_per_step * run.environments / mean_launch_s / 1e9
        traffic = MEASURED_TRAFFIC.get((n, run.environments, args.warmup, steps, len(sizes)))
        cpu = baselines.get(n)
        value = run.environments * steps / sum(run.walls)
        results[n] = {
            'workload': w.description, 'number': n, 'environments': run.environments, 'agents': run.agents,
            'geometry': {'environments_per_wavefront': run.matches, 'lanes_per_environment': run.lanes},
            'value': value, 'unit': 'env_steps/s', 'ms_per_step': sum(run.walls) / steps * 1000.0,
            'reset_seconds': run.reset_seconds,
            'launch_ms': {'mean': mean_launch_s * 1000.0, 'median': statistics.median(run.launch_ms),
                          'min': min(run.launch_ms), 'max': max(run.launch_ms)},
            'rounds': summary(run.environments, run.walls, sizes),
            'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                         'frac': achieved / HBM_PEAK_GBS, 'bytes_per_env_step': run.bytes_per_step,
                         'traffic': traffic[0] if traffic else None,
                         'traffic_window': (f'warm-up {args.warmup}, timed {steps} in {len(sizes)} rounds: {traffic[1]}'
                                            if traffic else 'not profiled for this window')},
            'cpu_baseline': cpu,
            'vs_cpu': value / cpu['value'] if cpu else None,
        }
    top = results[headline]
    w = runs[headline].workload
    line = {
        'metric': metric_name(w, top['environments']),
        'value': top['value'],
        'unit': 'env_steps/s',
        'n_gpus': 1,
        'steps': steps,
        'warmup': args.warmup,
        'ms_per_step': top['ms_per_step'],
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic: counter-hash uniform actions in [0, 19) on the shipped bundles (workload 5: drills built '
                'by the scenario builder)',
        'config': {'workload': w.description, 'number': headline, 'environments': top['environments'],
                   'agents': top['agents'], 'geometry': top['geometry'], 'reset_seconds': top['reset_seconds'],
                   'steady_state': args.warmup >= STEADY_WARMUP, 'rounds': len(sizes),
                   'interleaved_with': [n for n in numbers if n != headline]},
        'launch_ms': top['launch_ms'],
        'rounds': top['rounds'],
        'roofline': top['roofline'],
        'cpu_baseline': top['cpu_baseline'],
        'configs': {str(n): r for n, r in results.items()},
    }
    if args.warmup < STEADY_WARMUP:
        line['config']['note'] = (f'{args.warmup} warm-up steps: the timed steps include early ones, which are '
                                  f'cheaper than open play; the reference discards {STEADY_WARMUP}')
    print(json.dumps(line))


if __name__ == '__main__':
    main()

"""Throughput of the step engine on one MI355X.

The default workload is the headline configuration (workload 3 of `cuju_amd.workloads`): 16,384
environments of `11_vs_11_hard_stochastic` with all 11 left players under agents (the right team
is the built-in AI at difficulty 0.95), 3,000-step episodes, `simple115v2` observations
[16384, 11, 115] and automatic resets. `--config N` runs workload N instead (1: 5-a-side, 64
environments; 2: 11-a-side with one agent, 4,096; 4: self-play stacked with masked resets, 8,192;
5: the mixed batch of drills, 5-a-side and 11-a-side, 32,768).

A step is one `BatchEnvironment.step` of every environment. Actions are uniform integers in
[0, 19) from the workloads' counter hash of (seed, step, environment, agent), computed on the
device before the timed steps; workload 4's masked resets (every 512 steps, 10% of the
environments, drawn seeds) run inside the timed loop when they fall in it. `--warmup` steps run
untimed after the reset; the reference's own benchmark discards 100, and the first steps after a
reset are cheaper than open play, so a line with fewer says so. The value is environment steps
per second over the timed steps (wall clock, inputs resident in HBM).

Beside it the line reports the per-launch step-kernel durations (HIP events on the stream the
kernel runs on; median and spread over three rounds of the timed steps), the roofline of the step
kernel (algorithmic HBM bytes per launch over its mean duration, against 8 TB/s) with the HBM
traffic rocprofv3 measured for the same window where one was profiled, and the reference's own
CPU thread pool on this host's cores, timed on a bounded sample of the same workload.
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
# layout (its World is 373,440 B).
WORLD_BYTES = 373_552
STEADY_WARMUP = 100

# HBM bytes one step launch moves, read + written, from rocprofv3 FETCH_SIZE and WRITE_SIZE passes
# (each scaled by what the counter reads for a 1 GiB device copy), keyed by (workload,
# environments, warm-up steps, timed steps): the window of launches the profile averaged.
MEASURED_TRAFFIC = {
    (1, 64, 100, 30): (32_089_784 + 21_041_280, 'profiles/step_kernel_5v5_64.md'),
    (2, 4096, 100, 30): (30_384_280_765 + 19_816_283_962, 'profiles/step_kernel_11v11_4096.md'),
    (3, 16384, 100, 30): (166_511_157_054 + 57_339_453_066, 'profiles/step_kernel_11v11_hard_16384.md'),
    (3, 16384, 5, 20): (163_100_588_575 + 57_903_079_374, 'profiles/step_kernel_11v11_hard_16384_driver_window.md'),
    (4, 8192, 100, 30): (83_858_483_976 + 43_813_706_133, 'profiles/step_kernel_11v11_selfplay_stacked_8192.md'),
    (5, 32768, 100, 30): (173_930_563_037 + 56_983_406_873, 'profiles/step_kernel_mixed_32768.md'),
}


def algorithmic_bytes(workload, agents_present, agent_axis):
    """The compulsory HBM bytes of one environment step: the world read and written once, the
    actions read, the observation written (the stacked frames shifted: 3 of 4 read back), the
    reward, done and score written."""
    stack = 4 if workload.stacked else 1
    io = agents_present * (4 + 460 * stack) + (345 * agents_present * 4 if stack == 4 else 0) + 4 * agent_axis + 5
    return 2 * WORLD_BYTES + io


def cpu_model():
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_baseline(workload, environments, steps, warmup, seed, drill_paths):
    """The reference CPU library (its own thread pool, every core it may use) on a sample of the
    workload's environments, timed after the same warm-up as the device, on the same inputs."""
    from cuju_amd import workloads
    from oracle import ref
    if not os.path.isfile(ref.LIBRARY):
        return None
    options = workload.batch_options(0, environments, drill_paths)
    assets = options.pop('assets')
    batch = ref.ReferenceBatch(assets, seed=seed, threads=0, **options)
    batch.reset()
    agents = batch.agents
    for step in range(warmup):
        batch.step(workloads.actions(seed, step, 0, environments, agents))
    inputs = [workloads.actions(seed, warmup + k, 0, environments, agents) for k in range(steps)]
    start = time.perf_counter()
    for k in range(steps):
        batch.step(inputs[k])
    seconds = time.perf_counter() - start
    threads = batch.threads
    batch.close()
    return {'value': environments * steps / seconds, 'unit': 'env_steps/s', 'cores': threads, 'kind': 'reference',
            'cpu': cpu_model(),
            'sample': f'environments 0-{environments - 1} of workload {workload.number}, {steps} timed steps after a '
                      f'reset and {warmup} warm-up steps, the same counter-hash actions as the device'}


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument('--gpus', type=int, default=1)
    parser.add_argument('--steps', type=int, default=30)
    parser.add_argument('--warmup', type=int, default=STEADY_WARMUP)
    parser.add_argument('--config', type=int, default=3, choices=[1, 2, 3, 4, 5])
    parser.add_argument('--environments', type=int, default=None, help='default: the workload\'s')
    parser.add_argument('--seed', type=int, default=0)
    parser.add_argument('--cpu-environments', type=int, default=None)
    parser.add_argument('--cpu-steps', type=int, default=None)
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

    import numpy as np
    import torch
    import cuju_amd
    from cuju_amd import workloads

    workload = workloads.WORKLOADS[args.config]
    environments = args.environments or workload.environments
    device = torch.device('cuda', 0)
    torch.cuda.set_device(device)
    drill_paths = None
    if workload.number == 5:
        drill_paths = workloads.drill_bundles(os.path.join(tempfile.gettempdir(), 'cuju_amd_drills'))
    options = workload.batch_options(0, environments, drill_paths)
    assets = options.pop('assets')
    print(f'[bench] creating {environments} environments of workload {workload.number}', file=sys.stderr, flush=True)
    env = cuju_amd.BatchEnvironment(assets, device=device, seed=args.seed, **options)
    agents = env.agents
    present = (env.left_agents + env.right_agents).numpy().astype(np.float64)
    bytes_per_step = float(np.mean([algorithmic_bytes(workload, a, agents) for a in present]))
    torch.cuda.synchronize()
    start = time.perf_counter()
    env.reset()
    env.synchronize()
    reset_seconds = time.perf_counter() - start
    print(f'[bench] reset took {reset_seconds:.2f} s', file=sys.stderr, flush=True)

    def masked_reset(step):
        if workload.reset_every and (step + 1) % workload.reset_every == 0:
            mask, seeds = workloads.masked_reset(args.seed, step + 1, 0, environments, workload.reset_percent)
            env.reset(seeds=seeds, mask=torch.as_tensor(mask.astype(bool)))

    step = 0
    for k in range(args.warmup):
        env.step(workloads.actions_torch(torch, args.seed, step, 0, environments, agents, device))
        masked_reset(step)
        step += 1
        if k % 25 == 24:
            env.synchronize()
            print(f'[bench] {k + 1} warm-up steps', file=sys.stderr, flush=True)
    env.synchronize()
    print(f'[bench] {args.warmup} warm-up steps done', file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream(device)
    actions = [workloads.actions_torch(torch, args.seed, step + k, 0, environments, agents, device)
               for k in range(args.steps)]
    begin = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter()
    for k in range(args.steps):
        begin[k].record(stream)
        env.step(actions[k])
        end[k].record(stream)
        masked_reset(step + k)
    env.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall
    launch_ms = [b.elapsed_time(e) for b, e in zip(begin, end)]
    mean_launch_s = sum(launch_ms) / len(launch_ms) / 1000.0
    rounds = [chunk for chunk in np.array_split(np.array(launch_ms), min(3, args.steps)) if len(chunk)]
    round_rates = [environments * len(chunk) / (chunk.sum() / 1000.0) for chunk in rounds]
    value = environments * args.steps / wall
    achieved = bytes_per_step * environments / mean_launch_s / 1e9
    print(f'[bench] {args.steps} steps in {wall:.2f} s, mean step kernel {mean_launch_s * 1000:.1f} ms', file=sys.stderr,
          flush=True)
    env.close()
    if args.copy_probe:
        source = torch.empty(1 << 28, dtype=torch.float32, device=device).fill_(1.0)
        target = torch.empty_like(source)
        torch.cuda.synchronize()
        target.copy_(source)
        torch.cuda.synchronize()
        print('[bench] copy probe: 1 GiB read, 1 GiB written', file=sys.stderr, flush=True)

    baseline = None
    if not args.no_cpu:
        print('[bench] timing the reference CPU thread pool', file=sys.stderr, flush=True)
        cpu_environments = args.cpu_environments or min(environments, 2048)
        cpu_steps = args.cpu_steps or (60 if workload.number != 1 else 600)
        baseline = cpu_baseline(workload, cpu_environments, cpu_steps, args.warmup, args.seed, drill_paths)

    traffic = MEASURED_TRAFFIC.get((workload.number, environments, args.warmup, args.steps))
    line = {
        'metric': 'env steps/sec on 1 MI355X (11v11, 16384 envs) + bit-exact digest match',
        'value': value,
        'unit': 'env_steps/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': wall / args.steps * 1000.0,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic: counter-hash uniform actions in [0, 19) on the shipped bundles (workload 5: drills built '
                'by the scenario builder)',
        'config': {'workload': workload.description, 'number': workload.number, 'environments': environments,
                   'agents': agents, 'reset_seconds': reset_seconds,
                   'steady_state': args.warmup >= STEADY_WARMUP},
        'launch_ms': {'mean': mean_launch_s * 1000.0, 'median': statistics.median(launch_ms), 'min': min(launch_ms),
                      'max': max(launch_ms)},
        'rounds': {'env_steps_per_s': round_rates, 'median': statistics.median(round_rates),
                   'spread': (max(round_rates) - min(round_rates)) / statistics.median(round_rates)},
        'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': achieved / HBM_PEAK_GBS, 'bytes_per_env_step': bytes_per_step,
                     'traffic': traffic[0] if traffic else None,
                     'traffic_window': (f'warm-up {args.warmup}, timed {args.steps}: {traffic[1]}' if traffic
                                        else 'not profiled for this window')},
        'cpu_baseline': baseline,
    }
    if args.warmup < STEADY_WARMUP:
        line['config']['note'] = (f'{args.warmup} warm-up steps: the timed steps include early ones, which are '
                                  f'cheaper than open play; the reference discards {STEADY_WARMUP}')
    print(json.dumps(line))


if __name__ == '__main__':
    main()

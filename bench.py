"""Throughput of the step engine on one MI355X.

The workload is the headline configuration: 16,384 environments of `11_vs_11_hard_stochastic`
with all 11 left players under agents (the right team is the built-in AI at difficulty 0.95),
3,000-step episodes, `simple115v2` observations [16384, 11, 115] and automatic resets. A step is
one `BatchEnvironment.step` of every environment. Actions are uniform integers in [0, 19) from a
counter-based hash of (seed, step, environment, agent), computed on the device inside the timed
loop (a few microseconds). As the reference's benchmark does, the first 100 steps after the reset
are discarded: early steps are cheaper (few stoppages, short histories). The value is environment
steps per second over the timed steps, with the inputs resident in HBM.

Beside it the line reports the roofline of the step kernel (algorithmic HBM bytes per launch over
its measured duration, against 8 TB/s) and the reference's own CPU thread pool on this host's
cores, timed on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

ASSETS = '11_vs_11_hard_stochastic_l11_r0'
ENVIRONMENTS = 16384
AGENTS = 11
ACTIONS = 19
HBM_PEAK_GBS = 8000.0
# Algorithmic bytes of one environment step: the world read and written once (2 x 373,552 B)
# plus the compulsory I/O of this configuration (actions, observations, reward, done, score).
BYTES_PER_ENV_STEP = 752_257
# HBM bytes one step launch moves at 16,384 environments, read + written, from rocprofv3
# FETCH_SIZE and WRITE_SIZE passes scaled by a 1 GiB copy (profiles/step_kernel_11v11_hard_16384.md).
MEASURED_TRAFFIC = {16384: 144_371_218_771 + 53_184_601_872}


def counter_actions(torch, seed, step, environments, agents, device):
    """SplitMix64 of (seed, step, environment, agent), reduced to [0, 19)."""
    env = torch.arange(environments, device=device, dtype=torch.int64)[:, None]
    agent = torch.arange(agents, device=device, dtype=torch.int64)[None, :]
    x = (seed * 0x9E3779B9 + step * 0x632BE5AB + env * 0x85EBCA77 + agent * 0xC2B2AE3D) & 0x7FFFFFFFFFFFFFFF
    x = (x ^ (x >> 30)) * 0x3F58476D1CE4E5B9 & 0x7FFFFFFFFFFFFFFF
    x = (x ^ (x >> 27)) * 0x14AF1C8B9A4A5E1D & 0x7FFFFFFFFFFFFFFF
    x = x ^ (x >> 31)
    return (x % ACTIONS).to(torch.int32)


def cpu_baseline(environments, steps, warmup, seed):
    """The reference CPU library (its own thread pool, every core it may use) on a sample, timed
    after the same warm-up as the device."""
    from oracle import ref
    import numpy as np
    if not os.path.isfile(ref.LIBRARY):
        return None
    batch = ref.ReferenceBatch(ASSETS, environment_count=environments, seed=seed, threads=0)
    batch.reset()
    rng = np.random.default_rng(seed)
    for _ in range(warmup):
        batch.step(rng.integers(0, ACTIONS, size=(environments, AGENTS), dtype=np.int32))
    actions = [rng.integers(0, ACTIONS, size=(environments, AGENTS), dtype=np.int32) for _ in range(steps)]
    start = time.perf_counter()
    for step in range(steps):
        batch.step(actions[step])
    seconds = time.perf_counter() - start
    threads = batch.threads
    batch.close()
    return {'value': environments * steps / seconds, 'unit': 'env_steps/s', 'cores': threads, 'kind': 'reference',
            'sample': f'{environments} environments of {ASSETS}, {steps} timed steps after a reset and {warmup} '
                      f'warm-up steps, uniform random actions'}


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument('--gpus', type=int, default=1)
    parser.add_argument('--steps', type=int, default=30)
    parser.add_argument('--warmup', type=int, default=100)
    parser.add_argument('--environments', type=int, default=ENVIRONMENTS)
    parser.add_argument('--seed', type=int, default=0)
    parser.add_argument('--cpu-environments', type=int, default=2048)
    parser.add_argument('--cpu-steps', type=int, default=60)
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

    import torch
    import cuju_amd

    device = torch.device('cuda', 0)
    torch.cuda.set_device(device)
    print(f'[bench] creating {args.environments} environments of {ASSETS}', file=sys.stderr, flush=True)
    env = cuju_amd.BatchEnvironment(ASSETS, environment_count=args.environments, seed=args.seed, device=device)
    torch.cuda.synchronize()
    start = time.perf_counter()
    env.reset()
    env.synchronize()
    reset_seconds = time.perf_counter() - start
    print(f'[bench] reset took {reset_seconds:.2f} s', file=sys.stderr, flush=True)
    step = 0
    for k in range(args.warmup):
        env.step(counter_actions(torch, args.seed, step, args.environments, AGENTS, device))
        step += 1
        if k % 25 == 24:
            env.synchronize()
            print(f'[bench] {k + 1} warm-up steps', file=sys.stderr, flush=True)
    env.synchronize()
    print(f'[bench] {args.warmup} warm-up steps done', file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream(device)
    actions = [counter_actions(torch, args.seed, step + k, args.environments, AGENTS, device) for k in range(args.steps)]
    begin = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter()
    for k in range(args.steps):
        begin[k].record(stream)
        env.step(actions[k])
        end[k].record(stream)
    env.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall
    launch_ms = [b.elapsed_time(e) for b, e in zip(begin, end)]
    mean_launch_s = sum(launch_ms) / len(launch_ms) / 1000.0
    value = args.environments * args.steps / wall
    achieved = BYTES_PER_ENV_STEP * args.environments / mean_launch_s / 1e9
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
        baseline = cpu_baseline(args.cpu_environments, args.cpu_steps, args.warmup, args.seed)

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
        'data': 'synthetic: counter-hash uniform actions in [0, 19) on the shipped 11_vs_11_hard_stochastic bundle',
        'config': {'workload': f'{ASSETS}: {args.environments} environments x {AGENTS} agents, simple115v2, '
                               f'3000-step episodes, auto reset', 'environments': args.environments,
                   'agents': AGENTS, 'reset_seconds': reset_seconds},
        'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': achieved / HBM_PEAK_GBS, 'traffic': MEASURED_TRAFFIC.get(args.environments)},
        'cpu_baseline': baseline,
    }
    print(json.dumps(line))


if __name__ == '__main__':
    main()

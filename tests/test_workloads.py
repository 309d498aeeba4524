"""The workloads' inputs: the counter hash gives the same draws as Python integers, numpy and torch
(so the host, the oracle and the device consume identical inputs), a slice of a workload gets the
inputs of the same environments in the full batch, and workload 5's drill family and assignment;
and the bench's algorithmic bytes of each workload."""

import numpy as np
import torch

from cuju_amd import workloads


def test_draws_agree_between_python_numpy_and_torch():
    seed, step, first, count, columns = 1003, 4097, 16376, 8, 11
    a = workloads.draw(seed, step, np.arange(first, first + count), columns)
    b = workloads.draw_torch(torch, seed, step, first, count, columns, 'cpu').numpy()
    c = np.array([[workloads.draw_scalar(seed, step, first + i, j) for j in range(columns)] for i in range(count)])
    assert a.dtype == np.int64 and (a >= 0).all() and (a < 2 ** 31).all()
    assert np.array_equal(a, b) and np.array_equal(a, c)
    t = workloads.actions_torch(torch, seed, step, first, count, columns, 'cpu').numpy()
    assert np.array_equal(t, workloads.actions(seed, step, first, count, columns))


def test_actions_are_uniform_and_slices_agree():
    full = workloads.actions(3, 12, 0, 4096, 11)
    assert full.min() == 0 and full.max() == 18
    counts = np.bincount(full.reshape(-1), minlength=19)
    assert counts.min() > 0.9 * full.size / 19 and counts.max() < 1.1 * full.size / 19
    assert np.array_equal(workloads.actions(3, 12, 1000, 24, 11), full[1000:1024])


def test_masked_resets_draw_a_tenth_with_seeds_in_range():
    mask, seeds = workloads.masked_reset(4, 512, 0, 8192, 10)
    assert 0.08 < mask.mean() < 0.12
    assert seeds.min() >= 0 and seeds.max() <= 0xFFFFFFFF
    m2, s2 = workloads.masked_reset(4, 512, 100, 50, 10)
    assert np.array_equal(m2, mask[100:150]) and np.array_equal(s2, seeds[100:150])


def test_drill_family_and_the_mixed_assignment():
    assert len(workloads.DRILLS) == 36
    distances = sorted({d.metres for d in workloads.DRILLS})
    assert distances[0] == 20 and distances[-1] == 35
    assert 0.36 < workloads.ball_x(35) < workloads.ball_x(20) < 0.65
    w = workloads.WORKLOADS[5]
    assignment = w.assignment(0, 32768)
    drills = len(workloads.DRILLS)
    assert (assignment < drills).mean() == 0.5
    assert (assignment == drills).mean() == 0.25 and (assignment == drills + 1).mean() == 0.25
    assert len(set(assignment[assignment < drills].tolist())) == drills
    assert np.array_equal(w.assignment(32760, 8), assignment[32760:])


def test_the_bench_counts_the_algorithmic_bytes_of_each_workload():
    """B_step = 2 x 373,552 (the reference world read and written) + the compulsory I/O of the
    workload's agents: 748,981 B for workload 1, 747,577 for 2, 752,257 for 3, 818,125 for 4."""
    import bench
    expected = {1: (4, 4, 748_981), 2: (1, 1, 747_577), 3: (11, 11, 752_257), 4: (22, 22, 818_125)}
    for number, (present, axis, total) in expected.items():
        assert bench.algorithmic_bytes(workloads.WORKLOADS[number], present, axis) == total, number


def test_the_bench_splits_its_timed_steps_into_rounds():
    import bench
    assert bench.round_sizes(20, 3) == [7, 7, 6]
    assert bench.round_sizes(30, 3) == [10, 10, 10]
    assert bench.round_sizes(2, 3) == [1, 1]
    s = bench.summary(100, [1.0, 2.0, 0.5], [10, 10, 10])
    assert s['env_steps_per_s'] == [1000.0, 500.0, 2000.0] and s['median'] == 1000.0 and s['spread'] == 1.5


def test_the_bench_refuses_more_than_one_gpu():
    import subprocess
    import sys
    import bench
    done = subprocess.run([sys.executable, bench.__file__, '--gpus', '2'], capture_output=True, text=True)
    assert done.returncode == 2 and 'one GPU' in done.stderr


def test_the_cpu_baseline_times_the_device_window_in_interleaved_rounds(reference_library):
    """The reference pool plays each workload's sample over the same warm-up and rounds."""
    import argparse
    import bench
    args = argparse.Namespace(steps=3, rounds=2, warmup=2, seed=0, cpu_environments=4)
    out = bench.cpu_baselines([1, 3], args, None, lambda text: None)
    assert sorted(out) == [1, 3]
    for n, line in out.items():
        assert line['kind'] == 'reference' and line['cores'] >= 1 and line['value'] > 0
        assert len(line['rounds']['env_steps_per_s']) == 2
        assert 'environments 0-3' in line['sample'] and '3 timed steps in 2 interleaved rounds' in line['sample']

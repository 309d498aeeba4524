"""`cuju_environment_step_no_alloc`, the step for callers that cannot allocate: through the C ABI it
gives, call for call, the outputs of `cuju_environment_step` on a twin batch, with two batches of
different sizes calling it in turn (each call reuses the static scratch array the previous call
left), and it refuses a batch larger than its array."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import PRODUCT
from cuju_amd import workloads

pytestmark = pytest.mark.gpu


def host(x):
    return x.detach().cpu().numpy()


def twins(assets, count, seed):
    import cuju_amd
    made = [cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', environment_count=count, seed=seed)
            for _ in range(2)]
    for b in made:
        b.reset()
    return made


def test_no_alloc_step_equals_the_step_on_batches_of_two_sizes():
    from cuju_amd import library
    lib = library.load(PRODUCT)
    large = twins('5_vs_5_l4_r4', 40, 5)
    small = twins('11_vs_11_stochastic_l2_r1', 12, 6)
    try:
        stream = torch.cuda.current_stream().cuda_stream
        for step in range(30):
            for (fixed, ordinary), seed in ((large, 5), (small, 6)):
                actions = torch.as_tensor(workloads.actions(seed, step, 0, fixed.environment_count, fixed.agents),
                                          device='cuda:0')
                assert lib.cuju_environment_step_no_alloc(fixed._handle(), actions.data_ptr(), stream) == 0, \
                    lib.cuju_last_error().decode()
                expected = ordinary.step(actions)
                torch.cuda.synchronize()
                for name, got, want in zip(('observation', 'reward', 'done'),
                                           (fixed._observation, fixed._reward, fixed._done), expected[:3]):
                    assert host(got).tobytes() == host(want).astype(host(got).dtype).tobytes(), \
                        f'{name} of the {fixed.environment_count}-environment batch at step {step}'
                assert host(fixed._final).tobytes() == host(expected[3]['final_observation']).tobytes()
        for fixed, ordinary in (large, small):
            for i in range(fixed.environment_count):
                assert fixed.get_state(i) == ordinary.get_state(i), f'state {i}'
    finally:
        for b in large + small:
            b.close()


def test_no_alloc_step_refuses_a_batch_beyond_its_array():
    import cuju_amd
    from cuju_amd import library
    lib = library.load(PRODUCT)
    batch = cuju_amd.BatchEnvironment('academy_empty_goal_close', library=PRODUCT, device='cuda:0',
                                      environment_count=65)
    try:
        batch.reset()
        actions = torch.zeros((65, 1), dtype=torch.int32, device='cuda:0')
        status = lib.cuju_environment_step_no_alloc(batch._handle(), actions.data_ptr(),
                                                     torch.cuda.current_stream().cuda_stream)
        assert status == -1
        assert 'at most 64 environments' in lib.cuju_last_error().decode()
    finally:
        batch.close()

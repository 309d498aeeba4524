"""`torch.compile` traces a step whole, through the `cuju_amd::advance` operator, and gives the
outputs of an eager step (tests/test_compile.py of the reference); the async step, the torch
allocator (and closing a batch whose step still runs on a side stream), and the memory estimate."""

import pytest
import torch

from conftest import PRODUCT, digest_actions

pytestmark = pytest.mark.gpu
STEPS = 40


def outputs_bytes(observation, reward, done, information):
    tensors = (observation, reward, done, information['final_observation'], information['score_reward'])
    return b''.join(t.detach().cpu().numpy().tobytes() for t in tensors)


def step(batch, actions):
    return batch.step(actions)


def reset_done(batch):
    batch.reset_done()


def play(step, reset_done, **options):
    import cuju_amd
    batch = cuju_amd.BatchEnvironment('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=3, **options)
    try:
        batch.reset()
        found = []
        for index in range(STEPS):
            actions = torch.as_tensor(digest_actions(index, 3, batch.agents, batch.action_count), device='cuda:0')
            found.append(outputs_bytes(*step(batch, actions)))
            if not options.get('auto_reset', True):
                reset_done(batch)
        return found
    finally:
        batch.close()


@pytest.mark.parametrize('auto_reset', [True, False])
def test_a_compiled_step_equals_an_eager_one(auto_reset):
    torch._dynamo.reset()
    compiled = (torch.compile(step, fullgraph=True, backend='aot_eager'),
                torch.compile(reset_done, fullgraph=True, backend='aot_eager'))
    options = {'auto_reset': auto_reset, 'seed': 11}
    assert play(*compiled, **options) == play(step, reset_done, **options)


def test_a_squeezed_batch_compiles():
    import cuju_amd
    torch._dynamo.reset()

    def run(step):
        batch = cuju_amd.BatchEnvironment('academy_empty_goal_close', library=PRODUCT, device='cuda:0',
                                          environment_count=2, squeeze=True)
        try:
            batch.reset()
            return [outputs_bytes(*step(batch, torch.full((2,), index % 19, device='cuda:0'))) for index in range(10)]
        finally:
            batch.close()

    assert run(torch.compile(step, fullgraph=True, backend='aot_eager')) == run(step)


def test_step_async_then_wait_equals_step():
    import cuju_amd
    found = []
    for use_async in (False, True):
        batch = cuju_amd.BatchEnvironment('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=3, seed=2)
        try:
            batch.reset()
            seen = []
            for index in range(20):
                actions = torch.as_tensor(digest_actions(index, 3, batch.agents, batch.action_count), device='cuda:0')
                if use_async:
                    batch.step_async(actions)
                    seen.append(outputs_bytes(*batch.step_wait()))
                else:
                    seen.append(outputs_bytes(*batch.step(actions)))
            found.append(seen)
        finally:
            batch.close()
    assert found[0] == found[1]


def test_torch_allocator_and_debug_give_the_same_steps():
    """`allocator='torch'` takes the batch's memory from PyTorch's caching allocator (it shows in
    torch's statistics and returns at close), and a `debug` batch waits at every call; both step
    as the default batch does."""
    import cuju_amd
    found = []
    for options in ({}, {'allocator': 'torch'}, {'debug': True, 'threads': 4, 'pin_memory': True}):
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        batch = cuju_amd.BatchEnvironment('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=3, seed=2,
                                          **options)
        try:
            if options.get('allocator') == 'torch':
                assert torch.cuda.memory_allocated() - before >= 3 * 370_000
            batch.reset()
            seen = []
            for index in range(20):
                actions = torch.as_tensor(digest_actions(index, 3, batch.agents, batch.action_count), device='cuda:0')
                seen.append(outputs_bytes(*batch.step(actions)))
            found.append(seen)
        finally:
            batch.close()
        torch.cuda.synchronize()
        # Only the last actions tensor may remain; the batch's memory went back.
        assert torch.cuda.memory_allocated() - before < 1 << 20
    assert found[0] == found[1] == found[2]
    with pytest.raises(ValueError, match='allocator'):
        cuju_amd.BatchEnvironment('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=1, allocator='numa')


def test_memory_estimate_is_what_the_batch_reports():
    import cuju_amd
    estimate = cuju_amd.memory_estimate('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=8)
    batch = cuju_amd.BatchEnvironment('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=8)
    try:
        assert estimate == batch.memory_bytes > 8 * 373_552
        assert estimate.local_memory_bytes == 0
    finally:
        batch.close()


def test_closing_waits_for_a_step_on_a_side_stream():
    """A batch on the torch allocator hands its blocks back at close(): the steps launched on a side
    stream have ended by then, so no block returns to the pool while a kernel still writes it."""
    import cuju_amd
    batch = cuju_amd.BatchEnvironment('11_vs_11_hard_stochastic_l11_r0', library=PRODUCT, device='cuda:0',
                                      environment_count=64, allocator='torch', seed=0)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        batch.reset()
        actions = torch.zeros((64, batch.agents), dtype=torch.int32, device='cuda:0')
        for _ in range(3):
            batch.step(actions)
    batch.close()
    assert side.query()


def test_memory_estimate_of_a_batch_larger_than_the_device_allocates_nothing():
    """The estimate sizes a batch without allocating it, so a batch that cannot fit still gets its
    size."""
    import cuju_amd
    torch.cuda.synchronize()
    free_before, total = torch.cuda.mem_get_info()
    count = int(total // 480_000) + 1024
    estimate = cuju_amd.memory_estimate('5_vs_5_l4_r4', library=PRODUCT, device='cuda:0', environment_count=count)
    free_after, _ = torch.cuda.mem_get_info()
    assert estimate > total
    assert free_after == free_before

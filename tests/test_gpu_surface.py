"""The batch's calling surface on the MI355X, each case against the reference CPU library given the
same inputs:

* a batch made with `first_index` plays exactly the matching environments of a larger batch
  (the reference's tests/test_first_index.py:31-35, src/environment_api.h:56-58,78-80);
* a HIP graph that captures a step, and one that captures a masked reset with a device mask and
  no seeds, replay as eager calls do (tests/test_masked_reset.py:36-94, docs/backends.md:85-126);
* `torch.compile` steps and `step_async`/`step_wait` (tests/test_compile.py:52-104);
* stacked states: `set_state(stacked=True)` loads the engine bytes and GRF's frame stack, and the
  batch continues as the reference does after `cuju_environment_set_state` and
  `cuju_environment_set_stack` (src/environment_api.h:392-419);
* `cuju_environment_episode` after episodes have ended (src/environment_api.h:470-516).
"""

import ctypes

import numpy as np
import pytest
import torch

from conftest import PRODUCT
from cuju_amd import workloads
from oracle import ref

pytestmark = pytest.mark.gpu


def host(x):
    return x.detach().cpu().numpy()


def gpu_batch(assets, **options):
    import cuju_amd
    return cuju_amd.BatchEnvironment(assets, library=PRODUCT, device='cuda:0', **options)


def same_outputs(mine, theirs, what):
    for x, y, name in zip(mine[:3], theirs, ('observation', 'reward', 'done')):
        assert host(x).astype(y.dtype).tobytes() == np.ascontiguousarray(y).tobytes(), f'{name} {what}'


def test_first_index_slice_equals_the_sub_batch(reference_library):
    """Environments 20-31 of a 32-environment batch and a 12-environment batch from index 20 draw
    the same episode seeds and, given the same actions, play the same steps and states."""
    assets, seed, steps = '11_vs_11_stochastic_l2_r0', 3, 60
    whole = gpu_batch(assets, environment_count=32, seed=seed)
    part = gpu_batch(assets, environment_count=12, seed=seed, first_index=20)
    theirs = ref.ReferenceBatch(assets, environment_count=12, seed=seed, first_index=20, threads=0,
                                library_path=reference_library)
    try:
        a, b = host(whole.reset()), host(part.reset())
        assert a[20:].tobytes() == b.tobytes()
        assert b.tobytes() == theirs.reset().tobytes()
        for step in range(steps):
            actions = workloads.actions(seed, step, 0, 32, 2)
            x = whole.step(torch.as_tensor(actions, device='cuda:0'))
            y = part.step(torch.as_tensor(actions[20:], device='cuda:0'))
            for u, v in zip(x[:3], y[:3]):
                assert host(u)[20:].tobytes() == host(v).tobytes(), f'step {step}'
            same_outputs(y, theirs.step(actions[20:]), f'at step {step}')
        for i in range(12):
            assert whole.get_state(20 + i) == part.get_state(i) == theirs.get_state(i), f'state {i}'
    finally:
        whole.close()
        part.close()
        theirs.close()


def test_graph_captured_step_and_masked_reset_replay_as_eager(reference_library):
    """One graph holds a step on device actions, another a masked reset whose device mask comes
    from the done flags (no seeds, so the reset draws them). Each replay reads the actions and mask
    copied into the captured tensors, with eager work and synchronizations between replays, and its
    outputs equal an eager batch's and the reference's."""
    assets, environments, seed = 'academy_counterattack_easy_l2_r0', 16, 4
    captured = gpu_batch(assets, environment_count=environments, seed=seed, auto_reset=False)
    eager = gpu_batch(assets, environment_count=environments, seed=seed, auto_reset=False)
    theirs = ref.ReferenceBatch(assets, environment_count=environments, seed=seed, threads=0, auto_reset=False,
                                library_path=reference_library)
    stream = torch.cuda.Stream()
    try:
        assert host(captured.reset()).tobytes() == host(eager.reset()).tobytes() == theirs.reset().tobytes()
        static_actions = torch.zeros((environments, 2), dtype=torch.int32, device='cuda:0')
        static_mask = torch.zeros(environments, dtype=torch.bool, device='cuda:0')
        # The first eager step on a side stream, as torch's capture recipe warms up.
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            warm = workloads.actions(seed, 0, 0, environments, 2)
            static_actions.copy_(torch.as_tensor(warm))
            same_outputs(captured.step(static_actions), theirs.step(warm), 'at the warm-up step')
        torch.cuda.current_stream().wait_stream(stream)
        eager.step(torch.as_tensor(warm, device='cuda:0'))
        step_graph, reset_graph = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(step_graph):
            outputs = captured.step(static_actions)
        with torch.cuda.graph(reset_graph):
            captured.reset(mask=static_mask)
        ended = 0
        for step in range(1, 90):
            actions = workloads.actions(seed, step, 0, environments, 2)
            static_actions.copy_(torch.as_tensor(actions))
            step_graph.replay()
            expected = eager.step(torch.as_tensor(actions, device='cuda:0'))
            torch.cuda.synchronize()
            for u, v in zip(outputs[:3], expected[:3]):
                assert host(u).tobytes() == host(v).tobytes(), f'replay of step {step}'
            done = theirs.step(actions)
            same_outputs(outputs, done, f'at replayed step {step}')
            if done[2].any():
                ended += 1
                static_mask.copy_(torch.as_tensor(done[2].astype(bool)))
                reset_graph.replay()
                eager.reset(mask=torch.as_tensor(done[2].astype(bool), device='cuda:0'))
                obs = theirs.reset(mask=done[2])
                torch.cuda.synchronize()
                assert host(captured.observation()).tobytes() == host(eager.observation()).tobytes() == obs.tobytes()
        assert ended > 0, 'no episode ended, so the captured reset never replayed'
        for i in range(environments):
            assert captured.get_state(i) == theirs.get_state(i), f'state {i}'
    finally:
        captured.close()
        eager.close()
        theirs.close()


def _step(batch, actions):
    return batch.step(actions)


def test_compiled_and_async_steps_match_the_reference(reference_library):
    """A `torch.compile`d step (through the `cuju_amd::step` operator) and `step_async` then
    `step_wait` give the reference's outputs, auto resets included."""
    assets, environments, seed = '5_vs_5_l4_r4', 6, 8
    torch._dynamo.reset()
    compiled = torch.compile(_step, fullgraph=True, backend='aot_eager')
    a = gpu_batch(assets, environment_count=environments, seed=seed)
    b = gpu_batch(assets, environment_count=environments, seed=seed)
    theirs = ref.ReferenceBatch(assets, environment_count=environments, seed=seed, threads=0,
                                library_path=reference_library)
    try:
        a.reset()
        b.reset()
        theirs.reset()
        for step in range(60):
            actions = workloads.actions(seed, step, 0, environments, 8)
            expected = theirs.step(actions)
            x = compiled(a, torch.as_tensor(actions, device='cuda:0'))
            b.step_async(torch.as_tensor(actions, device='cuda:0'))
            y = b.step_wait()
            same_outputs(x, expected, f'of the compiled step {step}')
            same_outputs(y, expected, f'of the async step {step}')
            if expected[2].any():
                final = theirs.final_observation().tobytes()
                assert host(x[3]['final_observation']).tobytes() == final == host(y[3]['final_observation']).tobytes()
    finally:
        a.close()
        b.close()
        theirs.close()


def test_stacked_states_continue_as_the_reference(reference_library):
    """Stacked states of one device batch load into another batch, shuffled across environments;
    the reference loads the same engine bytes and frames through its C ABI. Both then play on
    identically, and the episode values agree."""
    assets, environments = '11_vs_11_stochastic_l2_r1', 4
    options = dict(environment_count=environments, stacked=True, rewards='scoring,checkpoints')
    source = gpu_batch(assets, seed=21, **options)
    mine = gpu_batch(assets, seed=22, **options)
    theirs = ref.ReferenceBatch(assets, seed=22, threads=0, library_path=reference_library, **options)
    try:
        source.reset()
        for step in range(45):
            source.step(torch.as_tensor(workloads.actions(21, step, 0, environments, 3), device='cuda:0'))
        states = [source.get_state(i, stacked=True) for i in range(environments)]
        frames = host(source.observation())
        mine.reset()
        theirs.reset()
        for i in range(environments):
            j = (i + 1) % environments
            mine.set_state(i, states[j], stacked=True)
            (length,) = np.frombuffer(states[j][:4], dtype='<i4')
            # The episode words of the state: `get_state` of the source, read back through the C ABI.
            words = (ctypes.c_int * (3 + 22))()
            size = ctypes.c_ulonglong()
            source._lib.cuju_environment_get_state(source._handle(), j, ctypes.byref(size), words)
            theirs.set_raw_state(i, states[j][4 + length:], list(words))
            theirs.set_stack(i, 'simple115', frames[j])
        assert host(mine.observation()).tobytes() == theirs.observation().tobytes()
        for i in range(environments):
            assert mine.get_state(i, stacked=True) == states[(i + 1) % environments]
        for step in range(40):
            actions = workloads.actions(22, step, 0, environments, 3)
            same_outputs(mine.step(torch.as_tensor(actions, device='cuda:0')), theirs.step(actions), f'at step {step}')
        values = np.zeros(17, dtype=np.int64)
        difficulty = np.zeros(4, dtype=np.float32)
        for i in range(environments):
            assert mine._lib.cuju_environment_episode(mine._handle(), i, values.ctypes.data, difficulty.ctypes.data) == 0
            want_values, want_difficulty = theirs.episode(i)
            assert values.tolist() == want_values.tolist(), f'episode values of environment {i}'
            assert difficulty.tobytes() == want_difficulty.tobytes()
    finally:
        source.close()
        mine.close()
        theirs.close()


def test_episode_values_after_episodes_end(reference_library):
    """`cuju_environment_episode` on a mixed batch whose short episodes end and reset: seeds,
    resets so far, bundles, steps, designated players and difficulties equal the reference's."""
    assets = ['academy_empty_goal_close_l1_r0', 'academy_3_vs_1_with_keeper_l3_r0']
    options = dict(environment_count=8, seed=13, assignment=[0, 1] * 4)
    mine = gpu_batch(assets, **options)
    theirs = ref.ReferenceBatch(assets, threads=0, library_path=reference_library, **options)
    try:
        mine.reset()
        theirs.reset()
        ends = 0
        for step in range(150):
            actions = workloads.actions(13, step, 0, 8, 3)
            mine.step(torch.as_tensor(actions, device='cuda:0'))
            ends += int(theirs.step(actions)[2].sum())
        assert ends > 0
        values = np.zeros(17, dtype=np.int64)
        difficulty = np.zeros(4, dtype=np.float32)
        for i in range(8):
            assert mine._lib.cuju_environment_episode(mine._handle(), i, values.ctypes.data, difficulty.ctypes.data) == 0
            want_values, want_difficulty = theirs.episode(i)
            assert values.tolist() == want_values.tolist(), f'episode values of environment {i}'
            assert difficulty.tobytes() == want_difficulty.tobytes()
    finally:
        mine.close()
        theirs.close()

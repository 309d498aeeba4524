"""The block procedure of the ten-thousand-step GPU check (`segments.py`), on the CPU: the
engine's host build plays a batch whose blocks start from the reference's mid-match states
(`cuju_environment_set_state`, with the observation stack of a stacked batch) and must reach the
reference's digests, masked resets and episode ends included. Short blocks keep it to seconds."""

import pytest

import segments
from conftest import HOST
from cuju_amd import workloads

STARTS = (0, 200, 400, 520)
SEGMENT = 300


@pytest.mark.parametrize('number', [1, 4])
def test_blocks_from_reference_states_play_as_the_reference(number, reference_library):
    w = workloads.WORKLOADS[number]
    states = segments.starting_states(w, None, reference_library, starts=STARTS)
    assert sorted(states) == list(STARTS[1:])
    digests = {}
    for name, library in (('reference', reference_library), ('host', HOST)):
        run = segments.BlockRun(w, segments.OracleBlocks(w, None, library, blocks=len(STARTS)), states, STARTS, SEGMENT)
        digests[name] = segments.play_oracle(run)
    assert len(digests['host']) == len(STARTS) * segments.episodes.PRODUCTION_MATCHES[number]
    assert digests['host'] == digests['reference']
    # The blocks differ from one another: each plays its own stretch of the match.
    m = segments.episodes.PRODUCTION_MATCHES[number]
    assert len({digests['host'][b * m] for b in range(len(STARTS))}) == len(STARTS)


def test_the_inputs_of_each_block_are_those_of_its_global_steps():
    w = workloads.WORKLOADS[4]
    inputs = segments.Inputs(w, 4, STARTS)
    f, seed = segments.first_index(w), segments.episodes.seed_of(w)
    a = inputs.actions(7)
    for b, s in enumerate(STARTS):
        assert (a[b * 4:(b + 1) * 4] == workloads.actions(seed, s + 7, f, 4, w.agents)).all()
    # Global step 512 ends block 2's local step 111 (400 + 111 + 1): only block 2 resets then.
    mask, seeds, due = inputs.masked_reset(111)
    assert due.tolist() == [False] * 8 + [True] * 4 + [False] * 4
    want_mask, want_seeds = workloads.masked_reset(seed, 512, f, 4, w.reset_percent)
    assert (mask[8:12] == want_mask).all() and (seeds[8:12] == want_seeds).all() and not mask[:8].any()
    assert inputs.masked_reset(110) is None

"""The reference's long digests on the MI355X: full 3,010-step matches and long drill runs with the
raw, SMM and checkpoint outputs (python/cuju/data/digests.json `long_cases`). A step of four
environments costs about as much as a full batch, so the five cases play at once, each batch on a
stream of its own. Opt-in, as the reference's tests/test_long.py is: CUJU_AMD_LONG=1."""

import hashlib
import os

import numpy as np
import pytest
import torch

from conftest import PRODUCT, digest_actions, load_digests

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get('CUJU_AMD_LONG') != '1', reason='long digests run with CUJU_AMD_LONG=1')]


def raw_bytes(x):
    if isinstance(x, dict):
        return b''.join(raw_bytes(x[name]) for name in sorted(x))
    return np.ascontiguousarray(x.detach().cpu().numpy()).tobytes()


def test_gpu_reproduces_long_digests():
    import cuju_amd
    digests = load_digests()
    environments = digests['environments']
    cases = sorted(digests['long_cases'].items())
    runs = []
    for name, case in cases:
        batch = cuju_amd.BatchEnvironment(case['assets'], library=PRODUCT, device='cuda:0', environment_count=environments,
                                          seed=digests['seed'], **dict(case['options']))
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            first = batch.reset()
        stream.synchronize()
        digest = hashlib.sha256(raw_bytes(first))
        runs.append(dict(name=name, case=case, batch=batch, stream=stream, digest=digest))
    try:
        longest = max(case['steps'] for _, case in cases)
        for step in range(longest):
            live = [r for r in runs if step < r['case']['steps']]
            for r in live:
                with torch.cuda.stream(r['stream']):
                    actions = torch.as_tensor(digest_actions(step, environments, r['batch'].agents,
                                                             r['batch'].action_count), device='cuda:0')
                    r['out'] = r['batch'].step(actions)
            for r in live:
                r['stream'].synchronize()
                for x in r['out'][:3]:
                    r['digest'].update(raw_bytes(x))
            if step % 250 == 249:
                print(f'long digests: step {step + 1} of {longest}', flush=True)
        for r in runs:
            if r['batch'].stack == 1:
                for index in range(environments):
                    r['digest'].update(r['batch'].get_state(index))
        failed = [r['name'] for r in runs if r['digest'].hexdigest() != r['case']['digest']]
        assert not failed, f'long digests that differ: {failed}'
    finally:
        for r in runs:
            r['batch'].close()

"""The package-level helpers of the reference's `cuju` (python/cuju/__init__.py:34-62) that this
package mirrors: the shipped bundles and their scenarios (python/cuju/_batch/assets.py:16-36), and
the default library path (python/cuju/_batch/library.py:82-95). CPU only."""

import os

import pytest
import torch

import cuju_amd
from cuju_amd import library
from cuju_amd.errors import ChoiceError


def test_bundled_assets_are_the_checksummed_bundles():
    listed = set()
    with open(os.path.join(library.DATA, 'SHA256SUMS')) as sums:
        for line in sums:
            name = line.split()[-1]
            if name.startswith('assets/') and name.endswith('.cjb'):
                listed.add(name[len('assets/'):-len('.cjb')])
    bundles = cuju_amd.bundled_assets()
    assert bundles == sorted(bundles) and set(bundles) == listed and '11_vs_11_hard_stochastic_l0_r0' in bundles
    for name in bundles:
        path, counts = cuju_amd.resolve_assets(name)
        assert os.path.isfile(path) and counts == (-1, -1)


def test_bundled_scenarios_name_each_bundle_once():
    scenarios = cuju_amd.bundled_scenarios()
    assert scenarios == sorted(set(scenarios))
    assert {name.rsplit('_l', 1)[0] for name in cuju_amd.bundled_assets()} == set(scenarios)
    # Any agent counts of a shipped scenario resolve to its bundle.
    path, counts = cuju_amd.resolve_assets('5_vs_5_l2_r3')
    assert path.endswith('5_vs_5_l0_r0.cjb') and counts == (2, 3)


def test_library_path_names_the_hip_library():
    for device in (None, 'cuda', 'cuda:3', 'auto', torch.device('cuda', 1)):
        assert cuju_amd.library_path(device) == library.PRODUCT
    with pytest.raises(ChoiceError):
        cuju_amd.library_path('cpu')
    assert isinstance(cuju_amd.__version__, str) and cuju_amd.__version__


def test_digest_hashes_tensors_dictionaries_sequences_and_bytes():
    import hashlib

    import numpy as np

    from conftest import digest_actions
    from cuju_amd.digests import digest_actions as package_actions

    a = torch.arange(6, dtype=torch.int32).reshape(2, 3).t()
    b = torch.tensor([1.5, -0.0], dtype=torch.float32)
    value = cuju_amd.Digest()
    value.update(a)
    value.update({'z': b, 'a': a})
    value.update([b'xy', (b, a)])
    fork = value.copy()
    fork.update(b'more')
    expected = hashlib.sha256()
    for part in (a, a, b, b'xy', b, a):
        expected.update(part if isinstance(part, bytes) else part.contiguous().numpy().tobytes())
    assert value.hexdigest() == expected.hexdigest() != fork.hexdigest()
    with pytest.raises(TypeError):
        value.update(3)
    for step in (0, 1, 57):
        assert np.array_equal(package_actions(step, 5, 3, 19).numpy(), digest_actions(step, 5, 3, 19))


def test_a_batch_refuses_to_be_pickled():
    import pickle
    batch = object.__new__(cuju_amd.BatchEnvironment)
    with pytest.raises(TypeError):
        pickle.dumps(batch)

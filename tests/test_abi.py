"""The C ABI: the product library exports every entry point that include/cuju_amd.h declares, and
the package declares the same list. No call runs here: without a GPU only loading is checked."""

import ctypes
import os
import re

import pytest

from conftest import PRODUCT, ROOT


def declared():
    with open(os.path.join(ROOT, 'include', 'cuju_amd.h')) as f:
        text = f.read()
    return sorted(set(re.findall(r'\b(cuju_[a-z_]+)\s*\(', text)))


def test_header_declares_the_reference_entry_points():
    names = declared()
    for required in ['cuju_last_error', 'cuju_backend', 'cuju_environment_create', 'cuju_environment_destroy',
                     'cuju_environment_reset', 'cuju_environment_reset_masked', 'cuju_environment_step',
                     'cuju_environment_get_state', 'cuju_environment_buffer']:
        assert required in names


def test_product_library_exports_every_declared_symbol():
    if not os.path.isfile(PRODUCT):
        pytest.fail('the HIP library is not built: run `python -m cuju_amd.build`')
    lib = ctypes.CDLL(PRODUCT)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing
    lib.cuju_backend.restype = ctypes.c_char_p
    assert lib.cuju_backend() == b'cuda'


def test_package_binds_the_declared_symbols():
    from cuju_amd import library
    assert sorted(n for n, _, _ in library.SIGNATURES) == declared()


def test_package_fails_loudly_without_the_library(tmp_path):
    from cuju_amd import library, MissingFileError
    with pytest.raises(MissingFileError):
        library.load(str(tmp_path / 'absent.so'))


def _error_cases(path):
    """(status, message) of each failing call of the C ABI, in order, through the library at `path`."""
    import numpy as np
    from oracle import ref
    lib = ref.library(path)
    out = []

    def configuration(**changes):
        assets = (ctypes.c_char_p * 1)(ref.resolve_asset('academy_empty_goal_close_l1_r0')[0].encode())
        counts = (ctypes.c_int * 2)(1, 0)
        fields = dict(version=2, assets=assets, asset_count=1, animations=os.path.join(ref.DATA, 'animations.bin').encode(),
                      environment_count=2, seed=3, action_set=0, observation=2, ticks_per_step=10, smm_width=96,
                      smm_height=72, stack=1, agent_counts=ctypes.addressof(counts))
        fields.update(changes)
        return ctypes.byref(ref.Configuration(**fields)), (assets, counts)

    for changes in (dict(version=3), dict(environment_count=0), dict(allocate=1)):
        cfg, _keep = configuration(**changes)
        handle = lib.cuju_environment_create(cfg)
        out.append((handle is None, lib.cuju_last_error() if handle is None else b''))
        if handle is not None:
            lib.cuju_environment_destroy(handle)
    cfg, _keep = configuration()
    handle = lib.cuju_environment_create(cfg)
    assert handle, lib.cuju_last_error()
    try:
        assert lib.cuju_environment_reset(handle, None, None, None) == 0
        for bad in (19, -20):
            actions = np.full(2, bad, dtype=np.int32)
            out.append((lib.cuju_environment_step(handle, actions.ctypes.data, 0, None, 0), lib.cuju_last_error()))
        size = ctypes.c_ulonglong()
        episode = (ctypes.c_int * 25)()
        for index in (2, -1):
            pointer = lib.cuju_environment_get_state(handle, index, ctypes.byref(size), episode)
            out.append((pointer is None, lib.cuju_last_error()))
        out.append((lib.cuju_environment_buffer(handle, b'no_such_buffer') is None, lib.cuju_last_error()))
        out.append((lib.cuju_environment_set_state(handle, 0, None, 0, episode), lib.cuju_last_error()))
        out.append((lib.cuju_environment_set_state(handle, 0, b'\0' * 16, 16, episode), lib.cuju_last_error()))
    finally:
        lib.cuju_environment_destroy(handle)
    return out


def test_error_convention_matches_the_reference(reference_library, host_library):
    """The status and message of each failing call, through the engine's host build (the same C ABI
    code as the product) and the reference library (src/environment_api.h): refused
    configurations (null and a message), actions outside [-n, n) (-2, before any environment
    steps), environments out of range. Where this library says more than the reference, the
    status still agrees: an unknown buffer is null (with a message here, none there), and bytes
    that hold no state are -1 with the reference's message as a prefix (the reference adds the
    field where the bytes stop). A configuration with `allocate` and no `release` is refused here
    (a batch could not give its memory back); the reference takes it."""
    mine, theirs = _error_cases(host_library), _error_cases(reference_library)
    assert mine[2] == (True, b'expected both allocate and release, or neither')
    assert theirs[2][0] is False
    del mine[2], theirs[2]
    statuses = [status for status, _ in mine]
    assert statuses == [status for status, _ in theirs]
    assert statuses == [True, True, -2, -2, True, True, True, -1, -1]
    for (_, a), (_, b) in list(zip(mine, theirs))[:6]:
        assert a == b
    assert mine[6][1] == b'no buffer named no_such_buffer'
    assert mine[8][1] == b'expected the bytes of a state, found bytes that do not load'
    assert theirs[8][1].startswith(mine[8][1])

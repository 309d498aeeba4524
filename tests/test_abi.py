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

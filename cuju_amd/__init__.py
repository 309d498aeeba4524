"""A batched Google Research Football step engine for the AMD Instinct MI355X (gfx950).

`BatchEnvironment` steps many matches in one HIP launch and is bit-identical to the reference
CPU engine for the same seeds and actions. The native library is built in-tree by
`python -m cuju_amd.build`.
"""

from .environment import (BatchEnvironment, bundled_assets, bundled_scenarios, episode_pickle, memory_estimate,
                          resolve_assets)
from .digests import Digest, digest
from .library import library_path
from .errors import (ActionRangeError, ArgumentError, ChoiceError, ClosedError, ConfigurationError,
                     DeviceError, EnvironmentIndexError, Error, LibraryError, MissingFileError,
                     StateError, UndefinedPathError)

__version__ = '0.2.0'

__all__ = ['BatchEnvironment', 'Digest', 'bundled_assets', 'bundled_scenarios', 'digest', 'episode_pickle', 'library_path',
           'memory_estimate', 'resolve_assets', '__version__', 'Error', 'ConfigurationError',
           'ChoiceError', 'ArgumentError', 'ActionRangeError', 'EnvironmentIndexError', 'StateError',
           'ClosedError', 'DeviceError', 'UndefinedPathError', 'LibraryError', 'MissingFileError']

"""A batched Google Research Football step engine for the AMD Instinct MI355X (gfx950).

`BatchEnvironment` steps many matches in one HIP launch and is bit-identical to the reference
CPU engine for the same seeds and actions. The native library is built in-tree by
`python -m cuju_amd.build`.
"""

from .environment import BatchEnvironment, episode_pickle, memory_estimate, resolve_assets
from .errors import (ActionRangeError, ArgumentError, ChoiceError, ClosedError, ConfigurationError,
                     DeviceError, EnvironmentIndexError, Error, LibraryError, MissingFileError,
                     StateError, UndefinedPathError)

__all__ = ['BatchEnvironment', 'episode_pickle', 'memory_estimate', 'resolve_assets', 'Error', 'ConfigurationError',
           'ChoiceError', 'ArgumentError', 'ActionRangeError', 'EnvironmentIndexError', 'StateError',
           'ClosedError', 'DeviceError', 'UndefinedPathError', 'LibraryError', 'MissingFileError']

"""The exception classes of the batch, as the reference names them (python/cuju/errors.py:29-92)."""


class Error(Exception):
    """Base class of the errors of this package."""


class ConfigurationError(Error, ValueError):
    """A batch configuration that the library refuses."""


class ChoiceError(ConfigurationError, KeyError):
    """An option outside its choices."""


class ArgumentError(Error, ValueError):
    """An argument of a call outside its domain."""


class ActionRangeError(Error, IndexError):
    """An action index outside [-action_count, action_count)."""


class EnvironmentIndexError(Error, IndexError, RuntimeError):
    """An environment index outside the batch."""


class StateError(Error, ValueError, RuntimeError):
    """Bytes that are not a state of the environment."""


class ClosedError(Error, RuntimeError):
    """A call on a closed batch."""


class DeviceError(Error, RuntimeError):
    """A failure of the HIP device."""


class UndefinedPathError(Error, RuntimeError):
    """An environment reached a path that GRF leaves undefined."""


class LibraryError(Error, RuntimeError):
    """Any other failure of the library."""


class MissingFileError(Error, FileNotFoundError):
    """A bundle, the animation tables or the library is missing."""


def from_library(message: str) -> Error:
    """The exception for a failure message of the library (python/cuju/errors.py:84-92)."""
    if 'reached a path that GRF leaves undefined' in message or 'reached a state that no match reaches' in message:
        return UndefinedPathError(message)
    if message.startswith('hip') or 'launch' in message:
        return DeviceError(message)
    return LibraryError(message)

"""Error types of the reference crate (src/error.rs:9-49), raised from C ABI statuses."""


class Mamba3Error(Exception):
    """Base of every failure that is not a programming bug."""


class ConfigError(Mamba3Error):
    """Error::Config -- a configuration is internally inconsistent."""


class ShapeError(Mamba3Error):
    """Error::Shape -- shapes that cannot be reconciled."""


class RankError(ShapeError):
    """Error::Rank -- a tensor holds an unexpected rank."""

    def __init__(self, expected, got, shape):
        super().__init__(f"expected rank {expected}, got {got} (shape {list(shape)})")
        self.expected, self.got, self.shape = expected, got, list(shape)


class UnsupportedError(Mamba3Error):
    """Error::Unsupported -- recognised but not implemented for this path."""


class DeviceError(Mamba3Error):
    """A HIP runtime call failed (no reference counterpart)."""


class ArgumentError(Mamba3Error, ValueError):
    """A required buffer is missing or malformed (no reference counterpart)."""


class StateDictError(Mamba3Error):
    """Error::StateDict -- a checkpoint / state dict does not fit the model."""


class IoError(Mamba3Error, OSError):
    """Error::Io -- a checkpoint file could not be read or written."""


class JsonError(Mamba3Error, ValueError):
    """Error::Json -- a checkpoint file is not the expected JSON."""

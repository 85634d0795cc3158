"""mamba3 -- MI355X (gfx950) implementation of the Mamba-3 SSD scan and decode step.

Mirrors the reference crate's `ssm` module and inference cache
(BectorVoom/mamba-trainer: src/ssm/{config,scan}.rs, src/infer/mod.rs) over the
C ABI of libmamba3_hip.so (include/mamba3_ssm.h).
"""
from . import _lib
from .error import (ArgumentError, ConfigError, DeviceError, Mamba3Error, RankError, ShapeError,
                    UnsupportedError)
from .infer import StateCache
from .ssm import (Discretization, ScanInputs, ScanOutput, SsmConfig, SsmMode, SsmState,
                  StateDynamics, mamba3_scan, mamba3_step, mamba3_step_, shift_left, ssd_chunked)


def library_path() -> str:
    return _lib.LIB_PATH


def launch_count() -> int:
    """Kernel launches issued by the library (the reference's launch counter)."""
    return int(_lib.lib().m3_launch_count())


def selftest_mfma() -> int:
    """Run the on-device MFMA lane-layout check; 0 means the layouts hold."""
    import ctypes
    r = ctypes.c_int32(-1)
    _lib.check(_lib.lib().m3_selftest_mfma(ctypes.byref(r)))
    return int(r.value)

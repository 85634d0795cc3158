"""ctypes binding of libmamba3_hip.so (include/mamba3_ssm.h).

Loading fails loudly when the library is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

from .error import (ArgumentError, ConfigError, DeviceError, IoError, JsonError, Mamba3Error,
                    RankError, ShapeError, StateDictError, UnsupportedError)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmamba3_hip.so")

M3_OK, M3_ERR_CONFIG, M3_ERR_SHAPE, M3_ERR_RANK = 0, 1, 2, 3
M3_ERR_UNSUPPORTED, M3_ERR_HIP, M3_ERR_ARGUMENT = 4, 5, 6
M3_ERR_STATE_DICT, M3_ERR_IO, M3_ERR_JSON = 7, 8, 9
M3_F32, M3_BF16, M3_F16 = 0, 1, 2

_Z = C.c_size_t
_P = C.c_void_p
_FP = C.POINTER(C.c_float)


class SsmConfigC(C.Structure):
    _fields_ = [
        ("d_model", _Z), ("n_heads", _Z), ("head_dim", _Z), ("d_state", _Z), ("n_groups", _Z),
        ("discretization", C.c_int32), ("dynamics", C.c_int32),
        ("rank", _Z), ("chunk_size", _Z), ("conv_kernel", _Z),
        ("bc_norm", C.c_int32), ("bc_bias", C.c_int32), ("post_gate_norm", C.c_int32),
        ("skip_connection", C.c_int32),
        ("dt_min", C.c_float), ("dt_max", C.c_float), ("dt_init_floor", C.c_float),
        ("a_init_min", C.c_float), ("a_init_max", C.c_float),
        ("bias", C.c_int32),
    ]


class SsmStateC(C.Structure):
    _fields_ = [("h", _P), ("last_u", _P), ("angle", _P)]


class SsmStateFactoredC(C.Structure):
    """m3_ssm_state_factored."""
    _fields_ = [("h", _P), ("x_prev", _P), ("b_prev", _P), ("angle", _P)]


class ScanInputsC(C.Structure):
    _fields_ = [
        ("batch", _Z), ("seq", _Z), ("heads", _Z), ("head_dim", _Z), ("d_state", _Z),
        ("rank", _Z), ("dtype", C.c_int32),
        ("x", _P), ("b", _P), ("c", _P), ("dt", _P), ("a_log", _P), ("lambda_", _P),
        ("theta", _P), ("d_skip", _P), ("state", C.POINTER(SsmStateC)),
        ("chunk_size", _Z), ("want_state", C.c_int32),
        ("workspace", _P), ("workspace_bytes", _Z),
    ]


class ScanGradsC(C.Structure):
    """m3_scan_grads (include/mamba3_ssm.h)."""
    _fields_ = [(n, _P) for n in ("dy", "dh", "dangle", "dx", "db", "dc", "ddt", "dlambda",
                                  "da_log", "dtheta", "dd_skip", "dh0", "dlast_u0", "dangle0",
                                  "dlast_u")]


class ScanOutputC(C.Structure):
    _fields_ = [("y", _P), ("state", SsmStateC)]


class SsdArgsC(C.Structure):
    _fields_ = [
        ("batch", _Z), ("seq", _Z), ("heads", _Z), ("head_dim", _Z), ("d_state", _Z),
        ("dtype", C.c_int32),
        ("x", _P), ("b", _P), ("c", _P), ("a", _P), ("g", _P), ("w", _P),
        ("initial_state", _P), ("chunk_size", _Z), ("want_state", C.c_int32),
    ]


class StepInputsC(C.Structure):
    _fields_ = [
        ("batch", _Z), ("heads", _Z), ("head_dim", _Z), ("d_state", _Z), ("rank", _Z),
        ("dtype", C.c_int32),
        ("x", _P), ("b", _P), ("c", _P), ("dt", _P), ("lambda_", _P), ("a_log", _P),
        ("theta", _P), ("d_skip", _P),
    ]


# Every exported symbol of include/mamba3_ssm.h with its ctypes signature.
class MixerDimsC(C.Structure):
    """m3_mixer_dims (mamba3_mixer.h)."""
    _fields_ = [("tokens", _Z), ("heads", _Z), ("head_dim", _Z), ("d_state", _Z), ("rank", _Z),
                ("groups", _Z), ("discretization", C.c_int32), ("dynamics", C.c_int32),
                ("norm_eps", C.c_float)]


class Conv1dC(C.Structure):
    """m3_conv1d (mamba3_mixer.h)."""
    _fields_ = [("kernel_size", _Z), ("seq_len", _Z), ("weight", _P), ("bias", _P),
                ("history", _P), ("new_history", _P)]


SIGNATURES = {
    "m3_config_default": (C.c_int, [C.POINTER(SsmConfigC)]),
    "m3_config_validate": (C.c_int, [C.POINTER(SsmConfigC)]),
    "m3_config_d_inner": (_Z, [C.POINTER(SsmConfigC)]),
    "m3_config_bc_width": (_Z, [C.POINTER(SsmConfigC)]),
    "m3_config_theta_width": (_Z, [C.POINTER(SsmConfigC)]),
    "m3_config_lambda_width": (_Z, [C.POINTER(SsmConfigC)]),
    "m3_config_in_proj_width": (_Z, [C.POINTER(SsmConfigC)]),
    "m3_discretization_fixed_lambda": (C.c_float, [C.c_int32]),
    "m3_scan": (C.c_int, [C.POINTER(ScanInputsC), C.POINTER(ScanOutputC), _P]),
    "m3_scan_gated": (C.c_int, [C.POINTER(ScanInputsC), C.POINTER(ScanOutputC), _P, _Z, _Z, _P]),
    "m3_scan_workspace_bytes": (_Z, [C.POINTER(ScanInputsC)]),
    "m3_scan_no_alloc": (C.c_int, [C.POINTER(ScanInputsC), C.POINTER(ScanOutputC), _P]),
    "m3_scan_backward": (C.c_int, [C.POINTER(ScanInputsC), C.POINTER(ScanGradsC), _P]),
    "m3_scan_backward_workspace_bytes": (_Z, [C.POINTER(ScanInputsC)]),
    "m3_ssd_chunked": (C.c_int, [C.POINTER(SsdArgsC), _P, _P, _P]),
    "m3_step": (C.c_int, [C.POINTER(StepInputsC), C.POINTER(SsmStateC), _P, _P]),
    "m3_step_factored": (C.c_int, [C.POINTER(StepInputsC), C.POINTER(SsmStateFactoredC), _P, _P]),
    "m3_state_unfactor": (C.c_int, [_Z, _Z, _Z, _Z, _Z, C.c_int32, _P, _P, _P, _P, _P]),
    "m3_step_layers": (C.c_int, [_Z, C.POINTER(StepInputsC), C.POINTER(SsmStateC),
                                 C.POINTER(SsmStateFactoredC), C.POINTER(_P), _P]),
    "m3_status_string": (C.c_char_p, [C.c_int]),
    "m3_last_error": (C.c_char_p, []),
    "m3_launch_count": (C.c_uint64, []),
    "m3_debug_scan_options": (C.c_int, [C.c_int32, C.c_int32, C.c_int32]),
    "m3_selftest_mfma": (C.c_int, [C.POINTER(C.c_int32)]),
    # mamba3_mixer.h
    "m3_rms_norm": (C.c_int, [_Z, _Z, _P, _Z, _P, C.c_float, _P, _Z, _P]),
    "m3_quantize_int8_columns": (C.c_int, [_Z, _Z, _P, _P, _P, _P]),
    "m3_linear_workspace_bytes": (_Z, []),
    "m3_linear": (C.c_int, [_Z, _Z, _Z, _P, _P, _P, _P, _P, _P, _Z, _P]),
    "m3_linear_nt": (C.c_int, [_Z, _Z, _Z, _P, _P, _P, _P, _P, _P, _Z, _P]),
    "m3_mixer_in_proj_width": (_Z, [C.POINTER(MixerDimsC)]),
    "m3_mixer_prologue": (C.c_int, [C.POINTER(MixerDimsC)] + [_P] * 12),
    "m3_mixer_prologue_conv": (C.c_int, [C.POINTER(MixerDimsC), C.POINTER(Conv1dC)] + [_P] * 12),
    "m3_mixer_gate": (C.c_int, [_Z, _Z, _P, _P, _Z, _P, C.c_float, _P, _P]),
    "m3_embedding_lookup": (C.c_int, [_Z, _Z, _P, _Z, _P, _P, _P]),
    "m3_mixer_step": (C.c_int, [C.POINTER(MixerDimsC)] + [_P] * 7 +
                      [C.POINTER(SsmStateC), C.POINTER(SsmStateFactoredC), _P, _P]),
    "m3_mixer_step_conv": (C.c_int, [C.POINTER(MixerDimsC), C.POINTER(Conv1dC)] + [_P] * 8 +
                           [C.c_float, C.POINTER(SsmStateC), C.POINTER(SsmStateFactoredC), _P, _P]),
    # mamba3_checkpoint.h
    "m3_checkpoint_load": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "m3_state_dict_load": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "m3_state_dict_free": (None, [_P]),
    "m3_state_dict_len": (_Z, [_P]),
    "m3_state_dict_entry": (C.c_int, [_P, _Z, C.POINTER(C.c_char_p), C.POINTER(_Z),
                                      C.POINTER(C.POINTER(_Z)), C.POINTER(_FP), C.POINTER(_Z)]),
    "m3_state_dict_find": (C.c_int64, [_P, C.c_char_p]),
    "m3_checkpoint_step": (C.c_uint64, [_P]),
    "m3_checkpoint_metadata": (C.c_char_p, [_P]),
    "m3_state_dict_save": (C.c_int, [C.c_char_p, C.c_int32, C.c_uint64, C.c_char_p, _Z,
                                     C.POINTER(C.c_char_p), C.POINTER(_Z),
                                     C.POINTER(C.POINTER(_Z)), C.POINTER(_FP), C.POINTER(_Z)]),
}

_lib = None


def lib():
    """Load libmamba3_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python mamba-trainer_amd/build_lib.py` "
                "(or __graft_entry__.build()); there is no fallback implementation")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


_ERRORS = {
    M3_ERR_CONFIG: ConfigError,
    M3_ERR_SHAPE: ShapeError,
    M3_ERR_RANK: ShapeError,
    M3_ERR_UNSUPPORTED: UnsupportedError,
    M3_ERR_HIP: DeviceError,
    M3_ERR_ARGUMENT: ArgumentError,
    M3_ERR_STATE_DICT: StateDictError,
    M3_ERR_IO: IoError,
    M3_ERR_JSON: JsonError,
}


def check(status: int):
    if status == M3_OK:
        return
    msg = lib().m3_last_error().decode(errors="replace")
    raise _ERRORS.get(status, Mamba3Error)(msg)

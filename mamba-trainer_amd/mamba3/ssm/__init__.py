"""The Mamba-3 SSM: configuration, the chunked scan and the decode step (src/ssm/mod.rs)."""
from .config import Discretization, SsmConfig, SsmConfigBuilder, SsmMode, StateDynamics
from .scan import (ScanGrads, ScanInputs, ScanOutput, SsmState, SsmStateFactored, mamba3_scan,
                   mamba3_scan_backward, mamba3_scan_gated, mamba3_step, mamba3_step_, mamba3_step_factored_,
                   shift_left, ssd_chunked)

__all__ = [
    "Discretization", "SsmConfig", "SsmConfigBuilder", "SsmMode", "StateDynamics",
    "ScanGrads", "ScanInputs", "ScanOutput", "SsmState", "SsmStateFactored", "mamba3_scan",
    "mamba3_scan_backward", "mamba3_scan_gated", "mamba3_step", "mamba3_step_", "mamba3_step_factored_",
    "shift_left", "ssd_chunked",
]

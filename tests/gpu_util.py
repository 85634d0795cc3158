"""Helpers for the GPU parity tests: numpy <-> device tensors, one-call runners
for the HIP path (through the mamba3 package, i.e. the C ABI) and for the
oracle on the same inputs."""
from __future__ import annotations

import numpy as np
import torch

import oracle

DEV = "cuda:0"


def dev(a, dtype=torch.float32):
    if a is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(dtype)


def host(t):
    if t is None:
        return None
    return t.detach().float().cpu().numpy()


def run_scan(inp, dtype=torch.float32, chunk=64, want_state=True, theta=True, skip=None,
             state=None, chunk_parallel=True):
    """inp: dict from cases.baseline_inputs (x, b, c, dt, a_log, lam, theta, h0, ...)."""
    from mamba3.ssm import ScanInputs, SsmState, mamba3_scan
    si = ScanInputs(dev(inp["x"], dtype), dev(inp["b"], dtype), dev(inp["c"], dtype),
                    dev(inp["dt"]), dev(inp["a_log"]), dev(inp["lam"]))
    if theta and inp.get("theta") is not None:
        si = si.with_theta(dev(inp["theta"], dtype))
    if skip is not None:
        si = si.with_skip(dev(skip))
    if state is not None:
        si = si.with_state(SsmState(dev(state[0]), dev(state[1]),
                                    dev(state[2]) if state[2] is not None else None))
    si = si.with_chunk_size(chunk).with_state_output(want_state).with_chunk_parallel(chunk_parallel)
    out = mamba3_scan(si)
    torch.cuda.synchronize()
    st = out.state
    return (host(out.y), host(st.h) if st else None, host(st.last_u) if st else None,
            host(st.angle) if st else None)


def oracle_scan(inp, theta=True, skip=None, state=None):
    s = state or (None, None, None)
    return oracle.scan_recurrence_f64(inp["x"], inp["b"], inp["c"], inp["dt"], inp["a_log"],
                                      inp["lam"], inp.get("theta") if theta else None, skip,
                                      s[0], s[1], s[2] if theta else None)

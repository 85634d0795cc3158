"""The CPU oracle is pinned before anything is compared with it.

Every check in oracle_checks.py must pass on the oracle as built, and every
planted mistake (a dropped term, a wrong sign or index, a transposed operand)
must make at least one check fail.  CPU only.
"""
import numpy as np
import pytest

import oracle
import oracle_checks


@pytest.mark.parametrize("name,fn,tol", oracle_checks.CHECKS, ids=[c[0] for c in oracle_checks.CHECKS])
def test_oracle_check(name, fn, tol):
    err = fn()
    assert err <= tol, f"{name}: worst error {err} > {tol}"


def test_noise_is_the_reference_lcg():
    """tests/ssm.rs:26-34, recomputed here with Python integers."""
    mask = (1 << 64) - 1
    s = (1 * 6364136223846793005 + 1) & mask
    want = []
    for _ in range(64):
        s = (s * 6364136223846793005 + 1442695040888963407) & mask
        want.append(np.float32(np.float32(s >> 33) / np.float32(1 << 31)) - np.float32(1.0))
    got = oracle.noise(64, 1)
    assert np.array_equal(got, np.array(want, np.float32))
    assert got.min() >= -1.0 and got.max() < 1.0


@pytest.mark.parametrize("fault", sorted(oracle.FAULTS))
def test_planted_mistakes_are_caught(fault):
    with oracle.fault(fault):
        results = oracle_checks.run_all()
    failed = [k for k, (ok, _) in results.items() if not ok]
    assert failed, f"planted mistake '{fault}' passed every oracle check"
    # and with the fault removed, everything passes again
    assert all(ok for ok, _ in oracle_checks.run_all().values())

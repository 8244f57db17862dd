"""The device-built rotary tables (nanochat_amd.rotary, fp64 on the GPU as model/modeling.py:169-176 builds them)
against the oracle's (numpy fp64, pinned to the closed form in test_oracle.py), over 131072 positions (the longest
contexts the decode tests run) at both RoPE bases the build uses."""

import numpy as np
import pytest

from nanochat_amd.rotary import rotary_tables
from oracle import golden as G

pytestmark = pytest.mark.gpu

N = 131072


def near_midpoint(v64: np.ndarray, slack: np.ndarray) -> np.ndarray:
    """Where an fp64 value lies within `slack` of the midpoint between its two fp32 neighbours: there, an fp64
    evaluation error of that size may round either way."""
    f = v64.astype(np.float32)
    other = np.nextafter(f, np.where(v64 >= f, np.float32(np.inf), np.float32(-np.inf)))
    mid = (f.astype(np.float64) + other.astype(np.float64)) / 2
    return np.abs(v64 - mid) <= slack


@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_rotary_tables_match_the_oracle(gpu, theta):
    """Bit-equal everywhere except where the fp64 value sits so close to an fp32 rounding midpoint that one fp64 ulp
    of the angle (t * 2^-52 radians, from the device's pow) can flip the rounding; there, the device value is within
    one fp32 ulp plus that slack of the fp64 value. The exempt entries are a tiny fraction."""
    cos, sin = rotary_tables(N, theta, gpu)
    want_cos, want_sin = G.rotary_tables(N, theta)
    exponent = np.arange(0, 128, 2, dtype=np.float64) / 128
    angles = np.outer(np.arange(N, dtype=np.float64), float(theta) ** -exponent)
    slack = 4 * np.abs(angles) * 2.0 ** -52 + 4 * 2.0 ** -53
    for got, want, v64 in ((cos, want_cos, np.cos(angles)), (sin, want_sin, np.sin(angles))):
        got = got.cpu().numpy()
        assert got.shape == (N, 64) and got.dtype == np.float32
        exempt = near_midpoint(v64, slack)
        differ = got.view(np.uint32) != want.view(np.uint32)
        assert not (differ & ~exempt).any(), np.argwhere(differ & ~exempt)[:5]
        # where they differ, the device value is still a rounding of a value within the slack of the fp64 one
        ulp = np.spacing(np.abs(v64).astype(np.float32)).astype(np.float64)
        assert (np.abs(got.astype(np.float64) - v64) <= ulp + slack)[differ].all()
        assert exempt.mean() < 1e-3, exempt.mean()
        print(f"theta {theta:g}: {int(differ.sum())} of {got.size} entries differ, {int(exempt.sum())} exempt",
              flush=True)

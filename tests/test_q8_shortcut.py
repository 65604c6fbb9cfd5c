"""CPU: the q8 code shortcut of the device quantizers (mc_core.h q8_code_fast /
q8_code_exact) against the IEEE division it replaces.

The kernels compute roundf(v / d) for d = fl(amax / 127) as rint(v * rcp(d)), where
rcp is the hardware reciprocal (v_rcp_f32, within 1 ulp of 1/d), and fall back to
the division only where the product lies within 2^-14 of a half-integer, or where
d is zero, subnormal or not finite.  The argument is an error bound
(|v * rcp(d) - fl(v/d)| < 2^-15 for |v/d| <= 127 (1 + 2^-24)); this checks it in
IEEE float32 with the reciprocal taken as fl(1/d) and as its neighbours one ulp
below and above (every value a 1-ulp reciprocal can return), on random blocks
across the exponent range and on the adversarial values: exact half-integer
multiples of d and their neighbours.  The GPU parity tests check the kernels
themselves, bit for bit, against the oracle's division."""
import numpy as np

f32 = np.float32


def roundf(x):
    """C roundf (half away from zero) of float32 values, exact in float64."""
    x = x.astype(np.float64)
    return np.where(x >= 0, np.floor(x + 0.5), -np.floor(-x + 0.5))


def shortcut(v, amax, ulp=0):
    """ulp: the reciprocal's error in ulps of fl(1/d) (-1, 0 or +1)."""
    d = (amax / f32(127)).astype(f32)
    dok = (d >= f32(2.0 ** -126)) & (d <= np.finfo(f32).max)
    inv = (f32(1) / np.where(dok, d, f32(1))).astype(f32)
    if ulp:
        inv = np.nextafter(inv, np.full_like(inv, np.inf if ulp > 0 else -np.inf)).astype(f32)
    with np.errstate(invalid="ignore"):                  # inf * 0 in a degenerate block
        y = (v * np.where(dok, inv, f32(0))[:, None]).astype(f32)
    r = np.rint(y)
    slow = (~dok[:, None]) | (np.abs((y - r).astype(f32)) >= f32(0.5 - 2.0 ** -14))
    return r, slow, d


def exact(v, d):
    with np.errstate(all="ignore"):
        return roundf((v / np.where(d != 0, d, f32(1))[:, None]).astype(f32))


def test_shortcut_equals_division_off_the_slow_path():
    rng = np.random.default_rng(11)
    n_slow = n = 0
    for kind in ("random", "half", "next_to_half"):
        for _ in range(8):
            scale = (f32(10.0) ** rng.uniform(-37, 37, 4096).astype(f32)).astype(f32)
            v = (rng.standard_normal((4096, 32)).astype(f32) * scale[:, None]).astype(f32)
            if kind != "random":
                d0 = (np.abs(v).max(1) / f32(127)).astype(f32)
                k = rng.integers(-127, 127, v.shape).astype(f32) + f32(0.5)
                v = (k * d0[:, None]).astype(f32)
                if kind == "next_to_half":
                    v = np.nextafter(v, np.where(rng.random(v.shape) < 0.5, -np.inf, np.inf).astype(f32)).astype(f32)
                v = np.clip(v, -127 * d0[:, None], 127 * d0[:, None]).astype(f32)
            amax = np.abs(v).max(1).astype(f32)
            for ulp in (0, -1, 1):
                r, slow, d = shortcut(v, amax, ulp)
                want = exact(v, d)
                fast = ~slow & (amax[:, None] != 0)
                assert np.array_equal(r[fast], want[fast]), (kind, ulp)
                n_slow += int(slow.sum())
                n += v.size
    # the division is the rare path (half-integer cases and tiny blocks force it here)
    assert n_slow < n // 4


def test_degenerate_blocks_take_the_division():
    v = np.array([[0.0] * 32, [1e-40] + [0.0] * 31, [np.inf] + [1.0] * 31], f32)
    amax = np.abs(v).max(1).astype(f32)
    _, slow, _ = shortcut(v, amax)
    assert slow.all()

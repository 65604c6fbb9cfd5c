"""CPU: the oracle's SSM_CONV (kernels/ssm-conv.cu:5-57) pinned by closed forms, an
independent fp64 correlation, F16 tap rounding and linearity; the C entry point's
argument checks (host-only paths, no device call)."""
import ctypes as C

import numpy as np
import pytest


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


@pytest.mark.parametrize("nc", [3, 4, 5, 9, 15])
def test_impulse_gives_the_taps(O, nc):
    n_s, nr, n_t = 2, 5, 20
    w = _rand((nr, nc), 1)
    p = 11                                            # one unit input at column p of every row
    x = np.zeros((n_s, nr, nc - 1 + n_t), np.float32)
    x[:, :, p] = 1.0
    y = O.ssm_conv(x, w)
    for t in range(n_t):
        j = p - t                                     # the tap that meets column p at token t
        want = w[:, j] if 0 <= j < nc else np.zeros(nr, np.float32)
        assert np.array_equal(y[0, t], want) and np.array_equal(y[1, t], want)


def test_constant_input_sums_the_taps(O):
    nc, nr, n_t = 4, 7, 9
    w = _rand((nr, nc), 2)
    x = np.full((1, nr, nc - 1 + n_t), 0.5, np.float32)
    y = O.ssm_conv(x, w)
    np.testing.assert_allclose(y[0], np.broadcast_to(0.5 * w.astype(np.float64).sum(1), (n_t, nr)), rtol=1e-6,
                               atol=1e-7)


@pytest.mark.parametrize("silu", [False, True])
def test_matches_fp64_correlation(O, silu):
    nc, n_s, nr, n_t = 4, 3, 33, 50
    x = _rand((n_s, nr, nc - 1 + n_t), 3)
    w = _rand((nr, nc), 4, 0.5)
    b = _rand((nr,), 5) if silu else None
    y = O.ssm_conv(x, w, bias=b, silu=silu)
    ref = np.empty((n_s, n_t, nr))
    for s in range(n_s):
        for r in range(nr):
            ref[s, :, r] = np.correlate(x[s, r].astype(np.float64), w[r].astype(np.float64), mode="valid")
    if silu:
        ref = ref + b.astype(np.float64)
        ref = ref / (1.0 + np.exp(-ref))
    assert O.rel_l2(y, ref) < 1e-6


def test_f16_taps_are_the_rounded_f32_taps(O):
    nc, nr, n_t = 5, 16, 12
    x = _rand((2, nr, nc - 1 + n_t), 6)
    w16 = _rand((nr, nc), 7).astype(np.float16)
    assert np.array_equal(O.ssm_conv(x, w16), O.ssm_conv(x, w16.astype(np.float32)))


def test_linear_in_x(O):
    nc, nr, n_t = 9, 8, 30
    x1, x2 = _rand((1, nr, nc - 1 + n_t), 8), _rand((1, nr, nc - 1 + n_t), 9)
    w = _rand((nr, nc), 10)
    lhs = O.ssm_conv(2.0 * x1 + x2, w).astype(np.float64)
    rhs = 2.0 * O.ssm_conv(x1, w).astype(np.float64) + O.ssm_conv(x2, w)
    assert O.rel_l2(lhs, rhs) < 1e-6


def test_entry_point_argument_checks(mc):
    lib = mc.lib()
    x = np.zeros((1, 4, 8), np.float32)
    w = np.zeros((4, 4), np.float32)
    d = np.zeros((1, 5, 4), np.float32)
    b = np.zeros(4, np.float32)

    def call(nc=4, wtype=0, bias=None, silu=0, x_nb0=4, dst_nb0=4, w_nb1=16, x_nb1=32):
        return lib.ggml_hip_ssm_conv_f32(x.ctypes.data, x_nb0, x_nb1, 128, w.ctypes.data, wtype, w_nb1,
                                         None if bias is None else bias.ctypes.data, silu, d.ctypes.data, dst_nb0, 16,
                                         80, nc, 4, 5, 1, None)
    assert call(nc=6) != 0 and b"kernel sizes" in lib.ggml_hip_moe_last_error()
    assert call(wtype=2) != 0 and b"F32 or F16" in lib.ggml_hip_moe_last_error()
    assert call(bias=b, silu=0) != 0 and b"SiLU" in lib.ggml_hip_moe_last_error()
    assert call(x_nb0=8) != 0
    assert call(dst_nb0=8) != 0
    assert call(w_nb1=12) != 0                        # fewer than nc taps per row
    assert call(x_nb1=28) != 0                        # rows shorter than nc - 1 + n_t

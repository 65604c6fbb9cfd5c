"""GPU: SSM_CONV with F32/F16 taps (ggml_hip_ssm_conv_f32, the replacement of
kernels/ssm-conv.cu) against the CPU oracle on the same inputs, through the C ABI.
Without SiLU the sums are the same fused multiply-adds in the same order: bit-exact.
With SiLU the device expf differs from the host's by a few ulp: rel-L2 <= 1e-6."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_SILU = 1e-6


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CASES = [  # nc, n_s, nr, n_t, f16, silu, bias
    (4, 1, 256, 1, True, True, True),        # decode step
    (4, 2, 200, 100, True, True, True),      # ragged channel tile
    (3, 3, 128, 513, False, False, False),   # ragged token tile
    (5, 1, 192, 64, True, False, False),
    (9, 2, 64, 33, False, True, False),
    (15, 1, 320, 130, True, True, True),
]


@pytest.mark.parametrize("nc,n_s,nr,n_t,f16,silu,bias", CASES)
def test_ssm_conv_matches_oracle(torch_gpu, mc, O, nc, n_s, nr, n_t, f16, silu, bias):
    torch = torch_gpu
    _note(f"ssm_conv nc={nc} n_s={n_s} nr={nr} n_t={n_t} f16={f16} silu={silu} bias={bias}")
    rng = np.random.default_rng(nc * 1000 + n_t)
    x = rng.standard_normal((n_s, nr, nc - 1 + n_t)).astype(np.float32)
    w = (rng.standard_normal((nr, nc)) * 0.5).astype(np.float16 if f16 else np.float32)
    b = rng.standard_normal(nr).astype(np.float32) if bias else None
    want = O.ssm_conv(x, w, bias=b, silu=silu)
    got = mc.ssm_conv(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(),
                      bias=None if b is None else torch.from_numpy(b).cuda(), silu=silu)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    if silu:
        err = O.rel_l2(got, want)
        _note(f"  rel_l2={err:.3e}")
        assert err <= TOL_SILU
    else:
        assert np.array_equal(got, want)


def test_ssm_conv_strided_rows(torch_gpu, mc, O):
    """conv_x rows padded past nc - 1 + n_t and dst rows wider than nr (views)."""
    torch = torch_gpu
    nc, n_s, nr, n_t = 4, 2, 96, 70
    _note("ssm_conv strided views")
    rng = np.random.default_rng(77)
    xb = rng.standard_normal((n_s, nr, nc - 1 + n_t + 5)).astype(np.float32)
    w = rng.standard_normal((nr, nc)).astype(np.float16)
    x = torch.from_numpy(xb).cuda()[:, :, :nc - 1 + n_t]
    out_big = torch.full((n_s, n_t, nr + 32), -7.0, dtype=torch.float32, device="cuda")
    mc.ssm_conv(x, torch.from_numpy(w).cuda(), out=out_big[:, :, :nr], n_t=n_t)
    torch.cuda.synchronize()
    got = out_big.cpu().numpy()
    assert np.array_equal(got[:, :, :nr], O.ssm_conv(xb[:, :, :nc - 1 + n_t], w))
    assert np.all(got[:, :, nr:] == -7.0)

"""CPU: the two GLU ops the reference's epilogue calls but does not define
(kernels/moe-cache.cu:271-275), pinned against model definitions this
environment holds (the transformers package), not against a restatement of the
oracle's own formula:

  SWIGLU_OAI    gpt-oss experts' gate (GptOssExperts._apply_gate: alpha 1.702,
                limit 7; gate clamped above, up clamped both sides,
                (up + 1) * gate * sigmoid(alpha * gate)), the model ggml's
                swiglu_oai op and its default alpha / limit were made for;
  SWIGLU_CLAMP  DeepSeek-V4's clamped SwiGLU MLP (DeepseekV4MLP.forward:
                silu(min(gate, limit)) * clamp(up, -limit, limit)).

The oracle's or_glu (oracle/mc_oracle.c) must agree with them elementwise; the
GPU epilogue is held to or_glu by the GEMV parity tests.  A plausible slip
(limit applied to the wrong operand, a missing +1, alpha dropped, the clamp
one-sided) moves the sampled values far beyond the tolerance.
"""
import types

import numpy as np
import pytest

torch = pytest.importorskip("torch")

TOL = 2e-6      # fp32 expf / sigmoid of two libraries: a few ulp


def _samples(seed, n=4096):
    rng = np.random.default_rng(seed)
    g = np.concatenate([rng.normal(0, 4, n), rng.uniform(-20, 20, n // 4),
                        [0.0, -0.0, 7.0, -7.0, 6.999, 7.001, 50.0, -50.0]]).astype(np.float32)
    u = np.concatenate([rng.normal(0, 4, n), rng.uniform(-20, 20, n // 4),
                        [7.0, -7.0, 0.0, 1.0, -1.0, 7.5, -7.5, 3.0]]).astype(np.float32)
    return g, u


def _close(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return np.all(np.abs(got - want) <= TOL * np.maximum(1.0, np.abs(want)))


def test_swiglu_oai_matches_gpt_oss(O):
    mod = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    g, u = _samples(1)
    ns = types.SimpleNamespace(alpha=1.702, limit=7.0)
    gate_up = torch.from_numpy(np.stack([g, u], axis=-1).reshape(-1))      # gate at even, up at odd positions
    want = mod.GptOssExperts._apply_gate(ns, gate_up[None]).numpy()[0]
    got = np.array([O.glu(O.GLU_SWIGLU_OAI, float(a), float(b), 0.0) for a, b in zip(g, u)], np.float32)
    assert _close(got, want)
    # the op ignores glu_limit: the constants are fixed (ggml's default alpha / limit)
    got2 = np.array([O.glu(O.GLU_SWIGLU_OAI, float(a), float(b), 3.0) for a, b in zip(g, u)], np.float32)
    assert np.array_equal(got, got2)


@pytest.mark.parametrize("limit", [7.0, 2.5, 10.0])
def test_swiglu_clamp_matches_deepseek_v4(O, limit):
    mod = pytest.importorskip("transformers.models.deepseek_v4.modeling_deepseek_v4")
    g, u = _samples(2)
    G, U = torch.from_numpy(g), torch.from_numpy(u)
    ns = types.SimpleNamespace(gate_proj=lambda x: G, up_proj=lambda x: U, down_proj=lambda h: h,
                               act_fn=torch.nn.functional.silu, limit=limit)
    want = mod.DeepseekV4MLP.forward(ns, None).numpy()
    got = np.array([O.glu(O.GLU_SWIGLU_CLAMP, float(a), float(b), limit) for a, b in zip(g, u)], np.float32)
    assert _close(got, want)


def test_oai_and_clamp_are_distinguished(O):
    """The two ops differ where the model definitions differ (the +1 and alpha), so neither check can
    pass with the other op's formula."""
    for a, b in ((1.0, 0.5), (-2.0, 3.0), (6.0, -1.0)):
        assert abs(O.glu(O.GLU_SWIGLU_OAI, a, b, 7.0) - O.glu(O.GLU_SWIGLU_CLAMP, a, b, 7.0)) > 1e-2

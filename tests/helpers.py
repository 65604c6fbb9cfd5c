"""Seeded synthetic MUL_MAT_ID problems shared by the parity tests."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

# relative L2 bounds used by the parity tests
TOL_CPU = 1e-3      # GPU (CPU-compatible activations) vs ggml-CPU MUL_MAT_ID restatement
TOL_SAME = 1e-5     # GPU vs the oracle on the very same activation bytes (fp32 summation order only)
TOL_Q8_1_VS_CPU = 1.2e-2   # K-quant weights, q8_1 activations (the reference's format) vs ggml-CPU's q8_K
                           # (measured 7.9e-3 .. 8.2e-3 for Q2_K..Q6_K at K = 4096)


def weights(wtype, n_experts, R, K, seed, std=0.02):
    x = O.fill_normal(seed, n_experts * R * K, 0.0, std).reshape(n_experts * R, K)
    return O.quantize_weights_fast(wtype, x).reshape(n_experts, R, -1)


def activations(n_rows, K, seed):
    return O.fill_normal(seed, n_rows * K, 0.0, 1.0).reshape(n_rows, K)


def routing(n_tok, n_used, n_experts, seed):
    return O.topk_uniform(seed, n_experts, n_used, n_tok)


def special_rows(K):
    """Activation rows exercising quantizer edge cases: zeros, exact ties, huge/tiny, sign flips."""
    rows = []
    z = np.zeros(K, np.float32)
    rows.append(z)
    t = np.zeros(K, np.float32)
    t[::2] = 127.0 / 2 * 0.01          # q = 63.5 -> ties at .5
    t[1::2] = -127.0 * 0.01
    rows.append(t)
    big = np.full(K, -3.0e4, np.float32)
    big[5::7] = 1.0e-30
    rows.append(big)
    r = np.arange(K, dtype=np.float32) % 33 - 16.0
    rows.append(r * 0.125)
    one = np.zeros(K, np.float32)
    one[K // 3] = -2.5
    rows.append(one)
    return np.stack(rows)

"""CPU: pins the oracle's MUL_MAT_ID (ggml-CPU restatement and the fused-op
variant) against a numpy fp64 evaluation on dequantized operands."""
import numpy as np
import pytest

from oracle import oracle as O


def _deq_experts(t, w, K):
    n, R, _ = w.shape
    return O.dequantize(t, w.reshape(n * R, -1), K).reshape(n, R, K).astype(np.float64)


@pytest.mark.parametrize("t", O.WEIGHT_TYPES)
def test_cpu_mul_mat_id_brute_force(t):
    K, R, n_as, n_tok, n_used = 512, 20, 6, 3, 4
    w = O.quantize_weights(t, O.fill_normal(10 + t, n_as * R * K, 0, 0.02).reshape(-1, K)).reshape(n_as, R, -1)
    x = O.fill_normal(20 + t, n_tok * K).reshape(n_tok, K)
    ids = O.topk_uniform(30 + t, n_as, n_used, n_tok)
    got = O.cpu_mul_mat_id_f32(wtype=t, K=K, R=R, n_as=n_as, src0=w, src1=x, ids=ids, nthreads=3)
    wd = _deq_experts(t, w, K)
    act_t = O.lib().or_act_type(t, O.ACT_CPU)
    for tok in range(n_tok):
        aq = O.quantize_act(t, O.ACT_CPU, x[tok])
        ad = O.dequantize(act_t, aq, K)[0].astype(np.float64)
        for c in range(n_used):
            want = wd[ids[tok, c]] @ ad
            assert np.allclose(got[tok, c], want, rtol=1e-5, atol=1e-6 * np.abs(want).max()), (t, tok, c)
    # the oracle's threading does not change the result
    assert np.array_equal(got, O.cpu_mul_mat_id_f32(wtype=t, K=K, R=R, n_as=n_as, src0=w, src1=x, ids=ids, nthreads=1))


def test_cpu_mul_mat_id_repeated_expert_and_broadcast_rows():
    """Two tokens picking the same expert, and src1 with one row per slot (down-projection shape)."""
    t, K, R, n_as = O.Q4_K, 256, 8, 4
    w = O.quantize_weights(t, O.fill_normal(5, n_as * R * K, 0, 0.02).reshape(-1, K)).reshape(n_as, R, -1)
    ids = np.array([[2, 0], [2, 3]], np.int32)
    x = O.fill_normal(6, 2 * 2 * K).reshape(2, 2, K)             # [tok, slot, K]
    got = O.cpu_mul_mat_id_f32(wtype=t, K=K, R=R, n_as=n_as, src0=w, src1=x, ids=ids, nthreads=2)
    wd = _deq_experts(t, w, K)
    for tok in range(2):
        for c in range(2):
            ad = O.dequantize(O.Q8_K, O.quantize_act(t, O.ACT_CPU, x[tok, c]), K)[0].astype(np.float64)
            assert np.allclose(got[tok, c], wd[ids[tok, c]] @ ad, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("glu_op", [O.GLU_SWIGLU, O.GLU_GEGLU, O.GLU_REGLU])
def test_fused_mul_mat_id_post_ops(glu_op):
    """scale -> bias -> GLU(gate, up) and the shared expert, against numpy on the same activation bytes."""
    t, st, K, R, n_as, n_tok, n_used = O.Q2_K, O.Q4_K, 512, 12, 5, 2, 3
    up = O.quantize_weights(t, O.fill_normal(40, n_as * R * K, 0, 0.02).reshape(-1, K)).reshape(n_as, R, -1)
    gate = O.quantize_weights(t, O.fill_normal(41, n_as * R * K, 0, 0.02).reshape(-1, K)).reshape(n_as, R, -1)
    shu = O.quantize_weights(st, O.fill_normal(42, R * K, 0, 0.02).reshape(-1, K))
    shg = O.quantize_weights(st, O.fill_normal(43, R * K, 0, 0.02).reshape(-1, K))
    x = O.fill_normal(44, n_tok * K).reshape(n_tok, K)
    ids = O.topk_uniform(45, n_as, n_used, n_tok)
    rng = np.random.default_rng(46)
    xb, gb = rng.standard_normal((n_as, R)).astype(np.float32) * 0.1, rng.standard_normal((n_as, R)).astype(np.float32) * 0.1
    xs, gs = rng.uniform(0.5, 1.5, n_as).astype(np.float32), rng.uniform(0.5, 1.5, n_as).astype(np.float32)
    act = np.stack([O.quantize_q8_1(r) for r in x]).reshape(n_tok, 1, -1)
    dst, sh = O.mul_mat_id(wtype=t, K=K, R=R, n_as=n_as, src0=up, gate=gate, ids=ids, act=act, act_kind=O.ACT_Q8_1,
                           x_bias=xb, gate_bias=gb, x_scale=xs, gate_scale=gs, glu_op=glu_op, sh_type=st, sh_up=shu,
                           sh_gate=shg)
    ud, gd = _deq_experts(t, up, K), _deq_experts(t, gate, K)
    sud, sgd = O.dequantize(st, shu, K).astype(np.float64), O.dequantize(st, shg, K).astype(np.float64)
    sig = lambda z: 1 / (1 + np.exp(-z))
    f = {O.GLU_SWIGLU: lambda g, u: u * g * sig(g),
         O.GLU_GEGLU: lambda g, u: u * 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * g * (1 + 0.044715 * g * g))),
         O.GLU_REGLU: lambda g, u: u * np.maximum(g, 0)}[glu_op]
    for tok in range(n_tok):
        ad = O.dequantize(O.Q8_1, act[tok, 0], K)[0].astype(np.float64)
        for c in range(n_used):
            e = ids[tok, c]
            u = (ud[e] @ ad) * xs[e] + xb[e]
            g = (gd[e] @ ad) * gs[e] + gb[e]
            assert np.allclose(dst[tok, c], f(g, u), rtol=2e-5, atol=2e-6)
        assert np.allclose(sh[tok], f(sgd @ ad, sud @ ad), rtol=2e-5, atol=2e-6)


def test_combine_against_numpy():
    rng = np.random.default_rng(7)
    o = rng.standard_normal((2, 5, 1024)).astype(np.float32)
    w = rng.uniform(0, 1, (2, 5)).astype(np.float32)
    sh = rng.standard_normal((2, 1024)).astype(np.float32)
    res = rng.standard_normal((2, 1024)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, 1024).astype(np.float32)
    x, y = O.combine_q8_1(o, w, shared=sh, residual=res)
    want = res.astype(np.float64) + sh + (w[:, :, None].astype(np.float64) * o).sum(1)
    assert np.allclose(x, want, rtol=1e-6, atol=1e-5)
    x2, yn = O.combine_q8_1(o, w, shared=sh, residual=res, rms_norm=True, eps=1e-6)
    x3, ynw = O.combine_q8_1(o, w, shared=sh, residual=res, rms_norm=True, norm_weight=nw, eps=1e-6)
    assert np.array_equal(x, x2) and np.array_equal(x, x3)
    for t in range(2):
        assert np.array_equal(y[t], O.quantize_q8_1(x[t]))
        ss = float((x[t].astype(np.float64) ** 2).sum())
        assert abs(O.rms_sum(x[t]) - ss) <= 1e-5 * ss
        s64 = 1.0 / np.sqrt(ss / 1024 + 1e-6)
        # the normalized rows: rms 1 (times the weight), within the q8_1 resolution
        for q, ref in ((yn[t], x[t] * s64), (ynw[t], x[t] * s64 * nw)):
            deq = O.dequantize(O.Q8_1, q, 1024)[0]
            assert O.rel_l2(deq, ref) < 0.01
        # exactly q8_1 of (x * s) * weight with s from the canonical sum
        s32 = np.float32(1.0) / np.sqrt(np.float32(O.rms_sum(x[t]) / np.float32(1024) + np.float32(1e-6)))
        assert np.array_equal(ynw[t], O.quantize_q8_1((x[t] * s32) * nw))
    # the fixed summation order: chunk sums of 256 values added in order
    xt = x[0]
    chunks = [O.rms_sum(xt[256 * j:256 * j + 256]) for j in range(4)]
    total = np.float32(0)
    for c in chunks:
        total = np.float32(total + np.float32(c))
    assert O.rms_sum(xt) == total


@pytest.mark.parametrize("wtype", [2, 10, 12])
def test_avx2_vec_dot_bit_identical_to_scalar(O, wtype):
    """The AVX2 Q2_K / Q4_K x q8_K dots (the CPU baseline's) equal the scalar restatement bit for bit: same
    per-super-block integers, same fp32 combination order.  Random blocks (every code and scale value),
    extreme activations (+-127 everywhere) and a zero row."""
    rng = np.random.default_rng(wtype)
    K = 4096
    rb = O.row_bytes(wtype, K)
    for trial in range(40):
        w = rng.integers(0, 256, rb, dtype=np.uint8)
        # finite fp16 block scales
        bb = O.block_bytes(wtype)
        for off in ((80, 82) if wtype == 10 else (0, 2) if wtype == 12 else (0,)):
            for b in range(K // O.block_elems(wtype)):
                h = np.array([rng.uniform(-0.05, 0.05)], np.float16).view(np.uint8)
                w[b * bb + off:b * bb + off + 2] = h
        if trial == 0:
            x = np.full(K, 3.0, np.float32)
        elif trial == 1:
            x = np.zeros(K, np.float32)
        else:
            x = rng.standard_normal(K).astype(np.float32) * (10.0 ** rng.uniform(-3, 3))
        a = O.quantize_q8_K(x) if wtype != 2 else O.quantize_q8_0(x)
        O.set_simd(False)
        ref = O.vec_dot_cpu(wtype, K, w, a)
        O.set_simd(True)
        got = O.vec_dot_cpu(wtype, K, w, a)
        assert np.float32(got).view(np.uint32) == np.float32(ref).view(np.uint32), (trial, got, ref)
        assert np.float32(ref).view(np.uint32) == np.float32(O.vec_dot(wtype, O.ACT_CPU, K, w, a)).view(np.uint32)


def test_cpu_mul_mat_id_simd_equals_scalar(O):
    import helpers as H
    for wtype in (2, 10, 12):
        w = H.weights(wtype, 8, 64, 2048, seed=5 + wtype)
        x = H.activations(3, 2048, seed=6)
        ids = H.routing(3, 4, 8, seed=7)
        O.set_simd(False)
        ref = O.cpu_mul_mat_id_f32(wtype=wtype, K=2048, R=64, n_as=8, src0=w, src1=x, ids=ids)
        O.set_simd(True)
        got = O.cpu_mul_mat_id_f32(wtype=wtype, K=2048, R=64, n_as=8, src0=w, src1=x, ids=ids)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))

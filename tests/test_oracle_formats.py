"""CPU: pins the oracle's block formats, activation quantizers and dot products.

Every check here uses something other than the oracle's own formula:
  * numpy's float16/float32 arithmetic as an independent evaluator;
  * single-element known-answer blocks built from the ggml layout stated in the
    inverse direction (byte/bit -> element index), so a transposed index or a
    swapped nibble in the oracle's element -> byte mapping fails;
  * quantize -> dequantize round trips through the independently written
    synthetic quantizer, with error bounds fixed by each format's bit width;
  * the integer-sum dots against fp64 dot products of dequantized values.
"""
import numpy as np
import pytest

from oracle import oracle as O

TYPES = O.WEIGHT_TYPES
BYTES = {O.Q4_0: 18, O.Q5_0: 22, O.Q8_0: 34, O.Q2_K: 84, O.Q3_K: 110, O.Q4_K: 144, O.Q5_K: 176, O.Q6_K: 210,
         O.Q8_1: 36, O.Q8_K: 292}


def f16(v):
    return int(np.array([v], np.float16).view(np.uint16)[0])


# ---------------------------------------------------------------- fp16
def test_fp16_to_fp32_exhaustive():
    L = O.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_fp16_to_fp32(int(v)) for v in h], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)])) and np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_fp32_to_fp16_matches_numpy_rne():
    L = O.lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 5.960464477539063e-08, 2.98e-08, 2.99e-08,
                  6.1035156e-05, 6.1e-05, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], np.float32)])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([L.or_fp32_to_fp16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_block_sizes():
    for t, b in BYTES.items():
        assert O.block_bytes(t) == b
    assert O.row_bytes(O.Q2_K, 4096) * 768 == 1_032_192          # cfg2 expert matrix
    assert O.row_bytes(O.Q4_K, 4096) * 768 == 1_769_472
    assert O.row_bytes(O.Q4_0, 2048) * 1024 == 1_179_648          # cfg1 expert matrix


# ---------------------------------------------------------------- activation quantizers
def _roundf(v32):
    """C roundf (half away from zero) evaluated in float64 on float32 inputs (exact)."""
    v = v32.astype(np.float64)
    t = np.trunc(v)
    return t + np.sign(v) * (np.abs(v - t) >= 0.5)


def _q8_1_numpy(x):
    x = x.astype(np.float32).reshape(-1, 32)
    out = []
    for b in x:
        amax = np.float32(np.max(np.abs(b)))
        d = np.float32(amax / np.float32(127.0))
        q = np.zeros(32, np.int8) if amax == 0 else _roundf((b / d).astype(np.float32)).astype(np.int8)
        s = b.copy()
        for off in (16, 8, 4, 2, 1):
            s = (s + s[np.arange(32) ^ off]).astype(np.float32)
        out.append(np.concatenate([np.array([d, s[0]], np.float16).view(np.uint8), q.view(np.uint8)]))
    return np.concatenate(out)


def test_q8_1_against_numpy_and_closed_forms():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32),
                        np.zeros(32, np.float32),                             # all-zero block: d = s = 0, q = 0
                        np.full(32, 0.635, np.float32),                      # constant block: q = 127 everywhere
                        (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5)])
    got = O.quantize_q8_1(x)
    assert np.array_equal(got, _q8_1_numpy(x))
    blk = got.reshape(-1, 36)
    z = blk[128]
    assert np.all(z == 0)
    c = blk[129]
    assert np.all(c[4:].view(np.int8) == 127)
    r = blk[130]
    q = r[4:].view(np.int8)
    assert q[0] == -127 and q[31] == round(15 * 127 / 16)   # +-amax -> +-127, 7.5*127/8 = 119.06 -> 119


def test_q8_0_against_numpy():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(2048).astype(np.float32), np.zeros(32, np.float32)])
    got = O.quantize_q8_0(x).reshape(-1, 34)
    for b, xb in zip(got, x.reshape(-1, 32)):
        amax = np.float32(np.max(np.abs(xb)))
        d = np.float32(amax / np.float32(127.0))
        idv = np.float32(1.0) / d if d else np.float32(0.0)
        q = _roundf((xb * idv).astype(np.float32)).astype(np.int8)
        assert b[:2].view(np.float16)[0] == np.float16(d)
        assert np.array_equal(b[2:].view(np.int8), q)


def test_q8_K_against_numpy():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(1024).astype(np.float32), np.zeros(256, np.float32)])
    x[300] = -7.0                                       # largest |x| negative -> positive iscale
    got = O.quantize_q8_K(x).reshape(-1, 292)
    for b, xb in zip(got, x.reshape(-1, 256)):
        d = b[:4].view(np.float32)[0]
        qs = b[4:260].view(np.int8)
        bs = b[260:].view(np.int16)
        if not np.any(xb):
            assert d == 0 and np.all(qs == 0)
            continue
        i = int(np.argmax(np.abs(xb)))                  # first index of the largest |x|
        iscale = np.float32(-127.0) / xb[i]
        want = np.minimum(127, np.rint((iscale * xb).astype(np.float32))).astype(np.int8)   # rint: half to even
        assert np.array_equal(qs, want)
        assert d == np.float32(1.0) / iscale
        assert np.array_equal(bs, qs.reshape(16, 16).astype(np.int32).sum(1))


# ---------------------------------------------------------------- single-element known answers
# Layout facts in the byte -> element direction (ggml block definitions).
def _kat_blocks(t):
    """Yields (block bytes, expected dequantized 32/256 values) with exactly one non-trivial element."""
    rng = np.random.default_rng(10 + t)
    if t == O.Q4_0:          # d | qs[16]: qs[j] low nibble = element j, high nibble = element j+16; value (q-8)*d
        for j in rng.choice(16, 4, replace=False):
            for hi in (0, 1):
                b = np.zeros(18, np.uint8)
                b[0:2] = np.array([0.5], np.float16).view(np.uint8)
                b[2:] = 0x88
                b[2 + j] = (0x8 | (0x3 << 4)) if hi else (0x3 | (0x8 << 4))
                y = np.zeros(32, np.float32)
                y[j + 16 * hi] = (3 - 8) * 0.5
                yield b, y
    elif t == O.Q5_0:        # d | qh[4] (bit j -> 5th bit of element j) | qs[16]; value (q-16)*d
        for j in rng.choice(32, 4, replace=False):
            b = np.zeros(22, np.uint8)
            b[0:2] = np.array([0.25], np.float16).view(np.uint8)
            qh = 0xFFFFFFFF & ~(1 << j)          # every element 16 except element j -> 0 + nibble
            b[2:6] = np.array([qh], np.uint32).view(np.uint8)
            b[6:] = 0x00
            y = np.zeros(32, np.float32)
            y[j] = (0 - 16) * 0.25
            yield b, y
    elif t == O.Q8_0:
        b = np.zeros(34, np.uint8)
        b[0:2] = np.array([2.0], np.float16).view(np.uint8)
        b[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
        yield b, (np.arange(32) - 16).astype(np.float32) * 2
    elif t == O.Q2_K:        # scales[16] | qs[64] | d | dmin; qs byte b, bit pair p -> element 128(b//32) + 32p + b%32
        for (byte, p) in [(0, 0), (5, 1), (31, 3), (32, 0), (47, 2), (63, 3)]:
            el = 128 * (byte // 32) + 32 * p + byte % 32
            b = np.zeros(84, np.uint8)
            b[80:82] = np.array([1.0], np.float16).view(np.uint8)
            b[82:84] = np.array([0.5], np.float16).view(np.uint8)
            s = el // 16
            b[s] = 0x3 | (0x2 << 4)                 # scale 3, min 2 for that element's sub-block only
            b[16 + byte] = 0x3 << (2 * p)
            y = np.zeros(256, np.float32)
            y[16 * s:16 * s + 16] = -0.5 * 2
            y[el] = 1.0 * 3 * 3 - 0.5 * 2
            yield b, y
    elif t == O.Q3_K:        # hmask[32] | qs[64] | scales[12] | d; hmask byte l bit k -> element 128(k//4) + 32(k%4) + l
        for (l, k) in [(0, 0), (7, 3), (31, 4), (16, 7)]:
            el = 128 * (k // 4) + 32 * (k % 4) + l
            b = np.zeros(110, np.uint8)
            b[108:110] = np.array([0.5], np.float16).view(np.uint8)
            b[:32] = 0xFF                               # every high bit set: code = low2
            b[l] &= ~(1 << k) & 0xFF                    # clear it for element el: code = low2 - 4
            # scale of sub-block s (6 bit, -32): low 4 bits in byte s (s < 8, low nibble) or s-8 (high nibble),
            # high 2 bits in byte 8 + s%4 at bit 2*(s//4); store 33 (=> +1) everywhere
            sc = np.zeros(12, np.uint8)
            for s in range(16):
                v = 33
                if s < 8: sc[s] |= v & 0xF
                else: sc[s - 8] |= (v & 0xF) << 4
                sc[8 + s % 4] |= ((v >> 4) & 3) << (2 * (s // 4))
            b[96:108] = sc
            y = np.zeros(256, np.float32)
            y[el] = 0.5 * 1 * (0 - 4)
            yield b, y
    elif t in (O.Q4_K, O.Q5_K):   # d | dmin | scales[12] | (qh[32]) | qs[128]; qs byte b: low nibble ->
        # element 64(b//32) + b%32, high nibble -> element 64(b//32) + 32 + b%32; qh byte l bit g -> element 32g + l
        q5 = t == O.Q5_K
        for (byte, hi) in [(0, 0), (9, 1), (63, 0), (100, 1), (127, 1)]:
            el = 64 * (byte // 32) + 32 * hi + byte % 32
            g = el // 32
            n = 176 if q5 else 144
            b = np.zeros(n, np.uint8)
            b[0:2] = np.array([1.0], np.float16).view(np.uint8)
            b[2:4] = np.array([0.25], np.float16).view(np.uint8)
            sc = np.zeros(12, np.uint8)     # 6-bit scale 5 and min 3 for sub-block g (layout of get_scale_min_k4)
            if g < 4:
                sc[g], sc[g + 4] = 5, 3
            else:
                sc[g + 4] = 5 | (3 << 4)
            b[4:16] = sc
            qs_off = 48 if q5 else 16
            b[qs_off + byte] = (0x7 << 4) if hi else 0x7
            val = 7
            if q5:
                b[16 + el % 32] |= 1 << g
                val += 16
            y = np.zeros(256, np.float32)
            y[32 * g:32 * g + 32] = -0.25 * 3
            y[el] = 1.0 * 5 * val - 0.25 * 3
            yield b, y
    elif t == O.Q6_K:        # ql[128] | qh[64] | scales[16] | d; ql byte b: low nibble -> element 128(b//64) + b%64,
        # high -> element 128(b//64) + 64 + b%64; qh byte c, bit pair p -> element 128(c//32) + 32p + c%32
        for el in [0, 37, 100, 127, 128, 200, 255]:
            n, r = el // 128, el % 128
            b = np.zeros(210, np.uint8)
            b[208:210] = np.array([0.5], np.float16).view(np.uint8)
            b[:128] = 0x00
            b[128:192] = 0xAA                        # high 2 bits = 2 everywhere -> code 32 -> value 0
            b[192:208] = np.int8(-3).view(np.uint8)  # every scale -3
            qb = 64 * n + r % 64
            if r < 64: b[qb] = 0x5
            else: b[qb] = 0x5 << 4
            c = 32 * n + r % 32
            p = r // 32
            b[128 + c] = (int(b[128 + c]) & ~(3 << (2 * p)) & 0xFF) | (1 << (2 * p))   # high bits 1 for element el
            y = np.zeros(256, np.float32)
            y[el] = 0.5 * -3 * ((5 | (1 << 4)) - 32)
            yield b, y


@pytest.mark.parametrize("t", TYPES)
def test_single_element_known_answers(t):
    n = 0
    for b, want in _kat_blocks(t):
        got = O.dequantize(t, b, len(want))[0]
        assert np.array_equal(got, want), (O.TYPE_NAMES[t], np.nonzero(got - want))
        n += 1
    assert n > 0


# ---------------------------------------------------------------- round trips and dot identities
ROUNDTRIP_BOUND = {O.Q8_0: 0.01, O.Q6_K: 0.03, O.Q5_0: 0.06, O.Q5_K: 0.06, O.Q4_0: 0.12, O.Q4_K: 0.12,
                   O.Q3_K: 0.25, O.Q2_K: 0.45}


@pytest.mark.parametrize("t", TYPES)
def test_quantize_dequantize_round_trip(t):
    x = O.fill_normal(100 + t, 8 * 1024, 0.0, 0.02).reshape(8, 1024)
    q = O.quantize_weights(t, x)
    assert q.shape[1] == O.row_bytes(t, 1024)
    err = O.rel_l2(O.dequantize(t, q, 1024), x)
    assert err < ROUNDTRIP_BOUND[t], err
    # a coarser format never beats a finer one on the same data by much (ordering sanity)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("kind", [O.ACT_CPU, O.ACT_Q8_1])
def test_vec_dot_equals_fp64_dot_of_dequantized(t, kind):
    K = 1024
    w = O.quantize_weights(t, O.fill_normal(200 + t, 4 * K, 0.0, 0.02).reshape(4, K))
    wd = O.dequantize(t, w, K).astype(np.float64)
    for s in range(3):
        a = O.fill_normal(300 + s, K)
        aq = O.quantize_act(t, kind, a)
        ad = O.dequantize(O.lib().or_act_type(t, kind), aq, K)[0].astype(np.float64)
        for r in range(4):
            got = O.vec_dot(t, kind, K, w[r], aq)
            want = float(wd[r] @ ad)
            assert abs(got - want) <= 2e-6 * np.abs(wd[r] * ad).sum(), (O.TYPE_NAMES[t], kind, got, want)


@pytest.mark.parametrize("t", TYPES)
def test_block_isums_brute_force(t):
    """Integer partial sums equal brute-force sums of (code * q8) recovered from the dequantizer."""
    be = O.block_elems(t)
    w = O.quantize_weights(t, O.fill_normal(400 + t, be, 0.0, 0.02).reshape(1, be))[0]
    rng = np.random.default_rng(t)
    q8 = rng.integers(-127, 128, be).astype(np.int8)
    got = O.block_isums(t, w, q8)
    deq = O.dequantize(t, w, be)[0].astype(np.float64)
    # the isums recombine to the exact dot with the dequantized block
    if t in (O.Q4_0, O.Q5_0, O.Q8_0):
        d = np.float64(w[:2].view(np.float16)[0])
        assert abs(got[0] * d - deq @ q8) <= 1e-9 * max(1.0, abs(deq @ q8))
    else:
        rec = O.vec_dot(t, O.ACT_Q8_1, be, w, np.concatenate(
            [np.concatenate([np.array([1.0, 0.0], np.float16).view(np.uint8), q8[32 * g:32 * g + 32].view(np.uint8)])
             for g in range(8)]))
        assert abs(rec - deq @ q8) <= 1e-5 * max(1.0, np.abs(deq * q8).sum())


# ---------------------------------------------------------------- GLU against independent evaluators
def test_glu_ops_against_numpy():
    from scipy.special import erf
    g = np.linspace(-9, 9, 181).astype(np.float32)
    u = np.linspace(-8, 6, 181).astype(np.float32)[::-1].copy()
    sig = lambda z: 1.0 / (1.0 + np.exp(-z))
    G, U = g.astype(np.float64), u.astype(np.float64)
    want = {
        O.GLU_REGLU: U * np.maximum(G, 0),
        O.GLU_GEGLU: U * 0.5 * G * (1 + np.tanh(np.sqrt(2 / np.pi) * G * (1 + 0.044715 * G * G))),
        O.GLU_SWIGLU: U * G * sig(G),
        O.GLU_SWIGLU_OAI: np.minimum(G, 7) * sig(1.702 * np.minimum(G, 7)) * (1 + np.clip(U, -7, 7)),
        O.GLU_GEGLU_ERF: U * 0.5 * G * (1 + erf(G / np.sqrt(2))),
        O.GLU_GEGLU_QUICK: U * G * sig(1.702 * G),
        O.GLU_SWIGLU_CLAMP: np.minimum(G, 2.5) * sig(np.minimum(G, 2.5)) * np.clip(U, -2.5, 2.5),
    }
    for op, w in want.items():
        got = np.array([O.glu(op, float(a), float(b), 2.5) for a, b in zip(g, u)])
        assert np.allclose(got, w, rtol=2e-5, atol=1e-5), op

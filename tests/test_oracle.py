"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against the reference's own known-answer
tests (cited file:line), against closed forms / exact integer arithmetic /
f64 brute force, and against bitwise identities that a dropped term, wrong
index or transposed operand would break.  CPU only.
"""
import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import synth


# ------------------------------------------------------------------ generator
def test_splitmix64_published_vector(orc):
    # SplitMix64 (Steele, Lea, Flood 2014) from seed 0: first outputs.
    assert orc.splitmix64_stream(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_generator_numpy_matches_c(orc):
    for seed in (0, 1001, 2002, 3003):
        np.testing.assert_array_equal(synth.splitmix64(seed, 64),
                                      np.array(orc.splitmix64_stream(seed, 64), dtype=np.uint64))
        a = synth.normal(seed, 10001, 0.0, 0.02)
        b = orc.fill_normal(seed, 10001, 0.0, 0.02)
        # libm vs numpy transcendental functions may differ in the last f64
        # ulp; after rounding to f32 the values agree to within one f32 ulp.
        assert np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-30)) < 2.5e-7


def test_generator_moments():
    z = synth.normal(12345, 1_000_000).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    assert abs(np.mean(z ** 3)) < 2e-2 and abs(np.mean(z ** 4) - 3.0) < 5e-2


# ------------------------------------------------------------------ fp32 GEMM
def test_kats_matmul(orc):
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert orc.matmul(a, b).tolist() == [[58, 64], [139, 154]]         # ops.zig:969-1005
    w_t = a.T.copy()
    assert orc.matmul(np.ones((1, 3), np.float32), w_t).tolist() == [[6, 15]]  # ops.zig:937-967
    i2 = np.eye(2, dtype=np.float32)
    assert orc.matmul(np.array([[1, 2], [3, 4]], np.float32), i2).tolist() == [[1, 2], [3, 4]]  # :1023-1046
    x = np.array([[1, 2, 3]], np.float32)
    w = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    assert orc.matmul(x, w).tolist() == [[22, 28]]                       # main.zig:141-148


def test_kat_matvec(orc):
    # ops.zig:1048-1076
    y = orc.matvec(np.array([[1, 2, 3], [4, 5, 6]], np.float32), np.array([1, 2, 3], np.float32))
    assert y.tolist() == [14.0, 32.0]


def test_kat_bias(orc):
    # addBiasInPlace ops.zig:2629-2654 (ones + [0.1, 0.2, 0.3]), via a
    # product that yields exact ones.
    a = np.ones((2, 1), np.float32)
    b = np.ones((1, 3), np.float32)
    got = orc.matmul_bias(a, b, np.array([0.1, 0.2, 0.3], np.float32))
    np.testing.assert_allclose(got, [[1.1, 1.2, 1.3], [1.1, 1.2, 1.3]], atol=1e-3)


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (4, 24, 9), (5, 25, 10), (8, 49, 33), (13, 50, 64),
                                   (64, 96, 128), (7, 8, 1), (4, 23, 16)])
def test_blocked_equals_naive_bitwise(orc, m, n, k):
    # Every branch of the register-blocked fallback (4x24, 4x8, scalar
    # columns, leftover rows) must perform the same per-element sum.
    a = synth.normal_matrix(1, m, k)
    b = synth.normal_matrix(2, k, n)
    ref = orc.matmul_naive(a, b)
    np.testing.assert_array_equal(orc.matmul(a, b), ref)
    np.testing.assert_array_equal(orc.matmul_mt(a, b, 3), ref)


def test_naive_is_ascending_k_f32(orc):
    # Restate one element in pure Python f32 arithmetic (ascending k,
    # separate multiply and add rounding).
    a = synth.normal_matrix(3, 2, 37)
    b = synth.normal_matrix(4, 37, 3)
    got = orc.matmul_naive(a, b)
    for i in range(2):
        for j in range(3):
            acc = np.float32(0.0)
            for kk in range(37):
                acc = np.float32(acc + np.float32(a[i, kk] * b[kk, j]))
            assert got[i, j] == acc


def test_exact_integer_products(orc):
    rng = np.random.default_rng(0)
    a = rng.integers(-20, 21, size=(33, 70))
    b = rng.integers(-20, 21, size=(70, 45))
    np.testing.assert_array_equal(orc.matmul(a.astype(np.float32), b.astype(np.float32)),
                                  (a @ b).astype(np.float32))


def test_f64_brute_force_and_planted_mistakes(orc):
    a = synth.normal_matrix(5, 24, 48)
    b = synth.normal_matrix(6, 48, 24)
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    got = orc.matmul(a, b)
    # f32 ascending sums: error bounded by ~K * eps * sum|a||b|
    bound = 48 * 2 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(got - ref64) <= bound)
    assert rel_err(got, ref64) < 1e-5
    np.testing.assert_allclose(orc.matmul_f64(a, b), ref64, rtol=1e-12, atol=1e-12)
    # The same check rejects plausible mistakes.
    sq_a, sq_b = synth.normal_matrix(15, 32, 32), synth.normal_matrix(16, 32, 32)
    sq_ref = sq_a.astype(np.float64) @ sq_b.astype(np.float64)
    assert rel_err(orc.matmul(sq_a, sq_b), sq_ref) < 1e-5
    assert rel_err(orc.matmul(sq_a, np.ascontiguousarray(sq_b.T)), sq_ref) > 1e-2  # transposed operand
    assert rel_err(orc.matmul(a[:, :-1], b[:-1]), ref64) > 1e-3               # dropped k term
    assert rel_err(-got, ref64) > 1.0                                          # sign


def test_bias_is_separate_rounded_add(orc):
    a = synth.normal_matrix(7, 9, 31)
    b = synth.normal_matrix(8, 31, 26)
    bias = synth.normal(9, 26)
    np.testing.assert_array_equal(orc.matmul_bias(a, b, bias), orc.matmul(a, b) + bias[None, :])


def test_sgemm_alpha_beta_closed_form(orc):
    a = synth.normal_matrix(10, 6, 10)
    b = synth.normal_matrix(11, 10, 7)
    c = synth.normal_matrix(12, 6, 7)
    t = orc.matmul(a, b)
    np.testing.assert_array_equal(orc.sgemm(a, b, c, 1.0, 0.0), t)
    np.testing.assert_array_equal(orc.sgemm(a, b, c, 2.0, 0.5), np.float32(2.0) * t + np.float32(0.5) * c)
    nan = np.full((6, 7), np.nan, np.float32)
    assert np.isfinite(orc.sgemm(a, b, nan, 1.0, 0.0)).all()


# ------------------------------------------------------------------ quantizers
def test_q8_kats(orc):
    # zero tensor -> scale 1, zeros (quantization.zig:1022-1038)
    q, s = orc.quantize_q8(np.zeros(10, np.float32))
    assert s == 1.0 and not q.any()
    # extremes (quantization.zig:1120-1144)
    q, s = orc.quantize_q8(np.array([100, -100, 0, 50, -50], np.float32))
    assert q[:3].tolist() == [127, -127, 0]
    assert abs(s - 100 / 127) < 1e-4
    # roundtrip within 1% of max (quantization.zig:963-997)
    t = np.array([2.5, -1.0, 0.5, -2.0, 0.0, 1.5], np.float32)
    q, s = orc.quantize_q8(t)
    assert np.all(np.abs(orc.dequantize_q8(q, s) - t) <= 2.5 * 0.01)


def test_round_half_away_from_zero(orc):
    # Zig @round: ties away from zero.  max = 127 makes inv exactly 1.
    t = np.array([127, 0.5, -0.5, 1.5, 2.5, -2.5], np.float32)
    q, s = orc.quantize_q8(t)
    assert s == 1.0
    assert q.tolist() == [127, 1, -1, 2, 3, -3]   # np.round would give 0, -0, 2, 2, -2
    t4 = np.array([7, 0.5, -0.5, 2.5, -3.5, 6.5], np.float32)
    p, s4 = orc.quantize_q4(t4)
    assert s4 == 1.0
    assert [orc.q4_get(p, i) for i in range(6)] == [7, 1, -1, 3, -4, 7]


def test_q8_invariants(orc):
    w = synth.normal(2002, 100_000, 0.0, 0.02)
    q, s = orc.quantize_q8(w)
    mx = np.max(np.abs(w))
    assert np.float32(s) == np.float32(mx) / np.float32(127.0)
    assert np.max(np.abs(q.astype(int))) == 127
    assert q[np.argmax(np.abs(w))] == np.sign(w[np.argmax(np.abs(w))]) * 127
    err = np.abs(orc.dequantize_q8(q, s).astype(np.float64) - w)
    assert np.all(err <= s / 2 * (1 + 1e-5) + 1e-12)


def test_q4_packing_kat(orc):
    # quantization.zig:1185-1214: values [-7,-3,0,3,7,-1,1,-2] in 4 bytes,
    # low nibble = even index, two's complement nibbles.
    p = np.zeros(4, np.uint8)
    vals = [-7, -3, 0, 3, 7, -1, 1, -2]
    for i, v in enumerate(vals):
        orc.q4_set(p, i, v)
    assert [orc.q4_get(p, i) for i in range(8)] == vals
    assert p.tolist() == [0xD9, 0x30, 0xF7, 0xE1]
    # a stored 0x8 nibble reads back as -8; set() clamps to [-7, 7]
    assert orc.q4_get(np.array([0x88], np.uint8), 0) == -8
    orc.q4_set(p, 0, -100)
    assert orc.q4_get(p, 0) == -7


def test_q4_kats(orc):
    p, s = orc.quantize_q4(np.zeros(10, np.float32))       # quantization.zig:1239-1255
    assert s == 1.0 and not p.any() and p.size == 5
    p, s = orc.quantize_q4(np.array([100, -100, 0, 50, -50], np.float32))  # :1337-1360
    assert [orc.q4_get(p, i) for i in range(3)] == [7, -7, 0]
    assert abs(s - 100 / 7) < 1e-4
    t = np.array([2.5, -1.0, 0.5, -2.0, 0.0, 1.5], np.float32)  # :1150-1183
    p, s = orc.quantize_q4(t)
    assert np.all(np.abs(orc.dequantize_q4(p, 6, s) - t) <= 2.5 * 0.15)
    p, _ = orc.quantize_q4(np.ones(7, np.float32))          # odd count: ceil(n/2) bytes
    assert p.size == 4 and p[-1] >> 4 == 0


def test_q8k_kats(orc):
    # quantization.zig:1366-1405 (100 elements over 4 blocks)
    i = np.arange(100)
    t = (np.sin(np.float32(0.1) * i.astype(np.float32)) * ((i // 32 + 1) * 10)).astype(np.float32)
    q, sc = orc.quantize_q8k(t)
    assert sc.size == 4
    back = orc.dequantize_q8k(q, sc)
    assert np.all(np.abs(back - t) <= np.abs(t) * 0.02 + 0.1)
    for b in range(4):
        blk = t[b * 32:(b + 1) * 32]
        assert np.float32(sc[b]) == np.float32(np.max(np.abs(blk))) / np.float32(127.0)
    # outliers (quantization.zig:1407-1453): block scales beat one scale
    t = np.empty(64, np.float32)
    t[:32] = 0.1 + np.sin(np.arange(32, dtype=np.float32) * np.float32(0.1)) * 0.05
    t[32] = 100.0
    t[33:] = 1.0 + np.cos(np.arange(33, 64, dtype=np.float32) * np.float32(0.1)) * 0.5
    q8, s8 = orc.quantize_q8(t)
    qk, sk = orc.quantize_q8k(t)
    e8 = np.sum(np.abs(t[:32] - orc.dequantize_q8(q8, s8)[:32]))
    ek = np.sum(np.abs(t[:32] - orc.dequantize_q8k(qk, sk)[:32]))
    assert ek <= e8
    # all-zero block -> scale 1, q = 0
    z = np.zeros(40, np.float32)
    z[35] = 1.0
    qz_, sz = orc.quantize_q8k(z)
    assert sz[0] == 1.0 and not qz_[:32].any()


# ---------------------------------------------------------- quantized matmuls
def test_q_matmuls_equal_f32_on_dequantized(orc):
    # The scalar loops (quantization.zig:158-203, 477-525, 778-824) are
    # c += a * (f32(q) * s) in ascending k: bitwise the fp32 fallback on the
    # dequantized weight.
    a = synth.normal_matrix(21, 6, 40)
    w = synth.normal_matrix(22, 40, 48, 0.02)
    q, s = orc.quantize_q8(w)
    np.testing.assert_array_equal(orc.matmul_q8(a, q, s), orc.matmul_naive(a, orc.dequantize_q8(q, s)))
    np.testing.assert_array_equal(orc.matmul_q8_mt(a, q, s, 3), orc.matmul_q8(a, q, s))
    qk, sk = orc.quantize_q8k(w)
    np.testing.assert_array_equal(orc.matmul_q8k(a, qk, sk), orc.matmul_naive(a, orc.dequantize_q8k(qk, sk)))
    p, s4 = orc.quantize_q4(w)
    deq4 = orc.dequantize_q4(p, 40 * 48, s4).reshape(40, 48)
    np.testing.assert_array_equal(orc.matmul_q4(a, p, 40, 48, s4), orc.matmul_naive(a, deq4))
    np.testing.assert_array_equal(orc.matmul_q4_mt(a, p, 40, 48, s4, 2), orc.matmul_q4(a, p, 40, 48, s4))


def test_q_matmul_accuracy_kats(orc):
    # quantization.zig:1040-1083 (Q8, 5% + 0.1) and 1257-1300 (Q4, 15% + 0.5)
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    ref = orc.matmul(a, b)
    q, s = orc.quantize_q8(b)
    assert np.all(np.abs(orc.matmul_q8(a, q, s) - ref) <= np.abs(ref) * 0.05 + 0.1)
    p, s4 = orc.quantize_q4(b)
    assert np.all(np.abs(orc.matmul_q4(a, p, 3, 2, s4) - ref) <= np.abs(ref) * 0.15 + 0.5)
    # Q8_K 2x64 . 64x32 with sin/cos data, 5% + 0.1 (quantization.zig:1455-1492)
    a = np.sin(np.arange(128, dtype=np.float32) * np.float32(0.1)).reshape(2, 64)
    b = np.cos(np.arange(2048, dtype=np.float32) * np.float32(0.1)).reshape(64, 32)
    ref = orc.matmul(a, b)
    qk, sk = orc.quantize_q8k(b)
    assert np.all(np.abs(orc.matmul_q8k(a, qk, sk) - ref) <= np.abs(ref) * 0.05 + 0.1)


def _rel_rmse(orig, got):
    # computeErrorMetrics (quantization.zig:1533-1568): rmse / mean|orig|
    d = np.abs(orig.astype(np.float32) - got.astype(np.float32)).astype(np.float64)
    return np.sqrt(np.mean(d * d)) / np.mean(np.abs(orig.astype(np.float64)))


def test_large_matrix_accuracy_kats(orc):
    # quantization.zig:1570-1618 (Q8_0, 16x768 . 768x768, rel < 5%)
    a = (np.sin(np.arange(16 * 768, dtype=np.float32) * np.float32(0.01)) * 2).reshape(16, 768).astype(np.float32)
    b = (np.cos(np.arange(768 * 768, dtype=np.float32) * np.float32(0.01)) * 2).reshape(768, 768).astype(np.float32)
    ref = orc.matmul(a, b)
    q, s = orc.quantize_q8(b)
    assert _rel_rmse(ref, orc.matmul_q8(a, q, s)) < 0.05
    # :1620-1668 (Q4_0, 4x64 . 64x32, max error < 0.1)
    a = (np.sin(np.arange(256, dtype=np.float32) * np.float32(0.1)) * 0.5).reshape(4, 64).astype(np.float32)
    b = (np.cos(np.arange(2048, dtype=np.float32) * np.float32(0.1)) * 0.5).reshape(64, 32).astype(np.float32)
    ref = orc.matmul(a, b)
    p, s4 = orc.quantize_q4(b)
    assert np.max(np.abs(ref - orc.matmul_q4(a, p, 64, 32, s4))) < 0.1
    # :1670-1719 (Q8_K, 16x512 . 512x512 with per-block ranges, rel < 5%)
    a = (np.sin(np.arange(16 * 512, dtype=np.float32) * np.float32(0.01)) * 2).reshape(16, 512).astype(np.float32)
    i = np.arange(512 * 512)
    b = (np.cos(i.astype(np.float32) * np.float32(0.01)) * (1.0 + (i // 32 % 10) * 0.5)).astype(np.float32)
    b = b.reshape(512, 512)
    ref = orc.matmul(a, b)
    qk, sk = orc.quantize_q8k(b)
    assert _rel_rmse(ref, orc.matmul_q8k(a, qk, sk)) < 0.05


def test_roundtrip_realistic_distribution(orc):
    # quantization.zig:1796-1851
    i = np.arange(10000, dtype=np.float32)
    t = (np.sin(i * np.float32(0.1)) * np.cos(i * np.float32(0.03)) * 0.1).astype(np.float32)
    q, s = orc.quantize_q8(t)
    assert _rel_rmse(t, orc.dequantize_q8(q, s)) < 0.01
    qk, sk = orc.quantize_q8k(t)
    assert _rel_rmse(t, orc.dequantize_q8k(qk, sk)) < 0.01
    p, s4 = orc.quantize_q4(t)
    assert _rel_rmse(t, orc.dequantize_q4(p, t.size, s4)) < 0.15


# ---------------------------------------------------------------- activations
def test_erf_as_within_published_bound(orc):
    # Abramowitz & Stegun 7.1.26 is published with |error| <= 1.5e-7; in f32
    # the five-term sum (terms up to 1.4 with alternating signs) and the
    # final 1 - poly * exp(-x^2) add a few ulps of 1 (worst near x = 0.02).
    # A wrong coefficient or a dropped term breaks this by orders of
    # magnitude.
    import math
    xs = np.linspace(-6.0, 6.0, 24001).astype(np.float32)
    worst = max(abs(orc.erf_as(float(x)) - math.erf(float(x))) for x in xs)
    assert worst <= 1.5e-7 + 3.5e-7, worst
    assert orc.erf_as(0.0) == 0.0
    for x in (0.1, 0.5, 1.3, 2.7, 5.0):
        assert orc.erf_as(-x) == -orc.erf_as(x)
    assert orc.erf_as(10.0) == 1.0 and orc.erf_as(-10.0) == -1.0


def test_gelu_exact_closed_form(orc):
    # x/2 (1 + erf(x/sqrt 2)) with the erf error above; GELU(x) - GELU(-x) = x.
    import math
    x = synth.normal(501, 4099, 0.0, 2.0)
    got = orc.gelu_exact(x).astype(np.float64)
    ref = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in x.astype(np.float64)])
    assert np.all(np.abs(got - ref) <= 0.5 * np.abs(x) * 4e-7 + 1e-7)
    neg = orc.gelu_exact(-x).astype(np.float64)
    assert np.all(np.abs((got - neg) - x) <= 1e-6 * np.abs(x) + 1e-7)
    assert orc.gelu_exact(np.zeros(9, np.float32)).tolist() == [0.0] * 9


def test_gelu_tanh_reference_kat(orc):
    # src/core/ops.zig:2456-2480 (five elements: the scalar tail only).
    got = orc.gelu_tanh(np.array([-2.0, -1.0, 0.0, 1.0, 2.0], np.float32))
    for g, want, tol in zip(got, [-0.0454, -0.1588, 0.0, 0.8412, 1.9545], [0.01, 0.01, 0.001, 0.01, 0.01]):
        assert abs(g - want) <= tol


def test_gelu_tanh_tail_is_exact_tanh(orc):
    # Elements from n - n % 8 on use tanh itself (ops.zig:1972-1978).
    import math
    x = synth.normal(502, 8 * 5 + 7, 0.0, 2.0)
    got = orc.gelu_tanh(x).astype(np.float64)
    c = math.sqrt(2.0 / math.pi)
    ref = np.array([0.5 * v * (1.0 + math.tanh(c * (v + 0.044715 * v ** 3))) for v in x.astype(np.float64)])
    tail = slice(40, 47)
    assert np.all(np.abs(got[tail] - ref[tail]) <= 1e-6 * (np.abs(ref[tail]) + 1e-3))
    # The vector part is the rational form: within its ~2e-2 of the exact
    # curve but visibly different from it somewhere on this sample.
    body = slice(0, 40)
    d = np.abs(got[body] - ref[body])
    assert np.all(d <= 0.03 * np.abs(x[body]).astype(np.float64) + 1e-6) and d.max() > 1e-4


def test_gelu_tanh_vector_form_properties(orc):
    # The 8-wide loop's tanh is x(27 + x^2) / (27 + 9 x^2), clamped to
    # [-1, 1] (ops.zig:1980-1997): odd (so GELU(x) - GELU(-x) = x), slope 1
    # at 0, and it reaches 1 exactly where x(27 + x^2) = 27 + 9 x^2, i.e.
    # (x - 3)^3 = 0: for inner = sqrt(2/pi)(x + 0.044715 x^3) >= 3 the
    # output is exactly x, below it strictly less.
    x = np.array([0.5, 1.0, 2.0, 2.3, 2.6, 3.0, 4.0, 6.0], np.float32)
    g = orc.gelu_tanh(x)
    gn = orc.gelu_tanh(-x)
    assert np.all(np.abs((g.astype(np.float64) - gn) - x) <= 1e-6 * x)
    inner = 0.7978845608 * (x.astype(np.float64) + 0.044715 * x.astype(np.float64) ** 3)
    sat = inner >= 3.0 + 1e-5
    below = inner <= 3.0 - 1e-3
    assert sat.any() and below.any()
    assert np.all(g[sat] == x[sat]) and np.all(g[below] < x[below])
    eps = np.float32(1e-3)
    small = orc.gelu_tanh(np.full(8, eps, np.float32))[0]
    slope = (float(small) - float(eps) / 2) / (float(eps) ** 2 / 2)  # = sqrt(2/pi) * tanh'(0)
    assert abs(slope - 0.7978845608) < 5e-3
    # The rational form differs from the KAT's exact-tanh values at x = 2
    # by more than the KAT tolerance: the split is observable.
    g8 = orc.gelu_tanh(np.array([2.0] * 8 + [2.0], np.float32))
    assert abs(g8[0] - 1.9545) > 0.01 and abs(g8[8] - 1.9545) <= 0.01


# ---------------------------------------------------------------- F16 weights
def test_f16_widening_exhaustive(orc):
    # Every binary16 pattern widens exactly as numpy's IEEE conversion.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.from_f16(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_narrowing_round_to_nearest_even(orc):
    # numpy's f32 -> f16 cast is IEEE round to nearest even: ties, subnormal
    # ties, the 65504 / 65520 overflow edge, signed zeros, infinities.
    edge = np.array([0.0, -0.0, 1.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.0, 65520.0, 1e6,
                     -65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25,
                     np.inf, -np.inf, 5.96e-8, 6.1e-5], dtype=np.float32)
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2 ** 32, size=400000, dtype=np.uint64).astype(np.uint32)
    rand = bits.view(np.float32)
    rand = rand[~np.isnan(rand)]
    scaled = (rng.standard_normal(200000) * np.exp2(rng.integers(-30, 18, size=200000))).astype(np.float32)
    for v in (edge, rand, scaled):
        got = orc.to_f16(v)
        with np.errstate(over="ignore"):
            ref = v.astype(np.float16).view(np.uint16)
        assert np.array_equal(got, ref)
    nan = orc.to_f16(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)[0])


def test_matmul_f16_equals_widened_f32(orc):
    rng = np.random.default_rng(12)
    for (m, n, k) in [(1, 7, 5), (5, 33, 17), (9, 64, 40)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        h = orc.to_f16(rng.standard_normal((k, n)).astype(np.float32) * 0.1)
        np.testing.assert_array_equal(orc.matmul_f16(a, h), orc.matmul_naive(a, orc.from_f16(h)))


# ------------------------------------------------ per-column quantization
def test_quantize_cols_definition(orc):
    # Per-column = the pinned per-tensor quantizer on each column; the packed
    # int4 layout round-trips; a zero column gets scale 1 and q = 0; the
    # product equals the f32 matmul of the dequantized weight (the
    # reference's dequantize-then-accumulate) bitwise.
    rng = np.random.default_rng(31)
    w = (rng.standard_normal((37, 11)) * np.exp(rng.standard_normal(11))[None, :]).astype(np.float32)
    w[:, 3] = 0.0
    q, s = orc.quantize_q8_cols(w)
    for j in range(11):
        qj, sj = orc.quantize_q8(np.ascontiguousarray(w[:, j]))
        np.testing.assert_array_equal(q[:, j], qj.reshape(-1))
        assert s[j] == np.float32(sj)
    assert s[3] == 1.0 and not q[:, 3].any()
    p, s4 = orc.quantize_q4_cols(w)
    vals = orc._unpack_q4(p, w.size).reshape(37, 11)
    for j in range(11):
        pj, sj = orc.quantize_q4(np.ascontiguousarray(w[:, j]))
        np.testing.assert_array_equal(vals[:, j], orc._unpack_q4(pj, 37))
        assert s4[j] == np.float32(sj)
    np.testing.assert_array_equal(orc._pack_q4(vals), p)
    a = rng.standard_normal((5, 37)).astype(np.float32)
    deq = orc.dequantize_cols(17, q, s, 37, 11)
    np.testing.assert_array_equal(orc.matmul_cols(a, 17, q, s, 37, 11), orc.matmul_naive(a, deq))
    ref = np.zeros((5, 11), np.float32)
    for i in range(5):
        for kk in range(37):
            ref[i] += a[i, kk] * (q[kk].astype(np.float32) * s)
    np.testing.assert_array_equal(orc.matmul_cols(a, 17, q, s, 37, 11), ref)
    # Columns that share one max reduce to the per-tensor formats: same bytes,
    # same scale in every column, and the per-tensor matmuls' result.
    w2 = np.clip(w, -0.9, 0.9)
    w2[0, :] = 1.0
    w2[1, ::2] = -1.0
    q8, s8 = orc.quantize_q8_cols(w2)
    qt, st = orc.quantize_q8(w2)
    np.testing.assert_array_equal(q8.reshape(-1), qt.reshape(-1))
    assert (s8 == np.float32(st)).all()
    np.testing.assert_array_equal(orc.matmul_cols(a, 17, q8, s8, 37, 11), orc.matmul_q8(a, qt.reshape(37, 11), st))
    p4, s4b = orc.quantize_q4_cols(w2)
    pt, st4 = orc.quantize_q4(w2)
    np.testing.assert_array_equal(p4, pt.reshape(-1))
    assert (s4b == np.float32(st4)).all()
    np.testing.assert_array_equal(orc.matmul_cols(a, 18, p4, s4b, 37, 11), orc.matmul_q4(a, pt, 37, 11, st4))

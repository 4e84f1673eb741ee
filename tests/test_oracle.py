"""Pins the CPU oracle (oracle/nn_oracle.c) against what the reference fixes.

Known-answer tests are the reference's own inline constants; everything else is checked
against an independent computation (numpy int64 / float64, closed forms, invariants),
never by retyping the oracle's loop. Reference citations are file:line in
neuralnet-cpp-dev/neuralnet.cpp v1.18.0.
"""
import math
import os

import numpy as np
import pytest

from conftest import normal, uniform

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- trit_pack layout

def test_trit_layout_kat(orc):
    # src/ternary_gemm_test.cpp:79-89: tau = 1 -> threshold 0.5, codes = trit + 2, LSB first
    w = np.array([1.0, -1.0, 0.0, 0.4, -0.4, 1.0, -1.0, 0.0,
                  0.9, -0.9, 0.1, -0.1, 0.6, -0.6, 0.0, 0.0], np.float32)
    expect = [3, 1, 2, 2, 2, 3, 1, 2, 3, 1, 2, 2, 3, 1, 2, 2]
    word = orc.trit_pack(w[None, :], np.array([1.0], np.float32))[0, 0]
    assert [(int(word) >> (2 * j)) & 3 for j in range(16)] == expect


def test_trit_tail_is_code2(orc):
    # src/ternary_gemm_test.cpp:91-99: K=5 -> positions 5..15 hold code 2 (trit 0), not code 0
    w = np.array([1.0, -1.0, 0.0, 0.4, -0.4], np.float32)
    wq = orc.trit_pack(w[None, :], np.array([1.0], np.float32))
    assert orc.trits_of(wq, 16)[0].tolist() == [1, -1, 0, 0, 0] + [0] * 11
    assert int(wq[0, 0]) >> 10 == (0xAAAAAAAA >> 10)


def test_words_per_row_constants(orc):
    # src/ternary_gemm_test.cpp:74-77, :102-104
    L = orc.lib()
    assert (L.orc_trit_words_per_row(16), L.orc_trit_words_per_row(17), L.orc_trit_words_per_row(1)) == (1, 2, 1)
    assert L.orc_trit_words_per_row(512) * 4 == 128  # 0.25 B / weight
    assert (L.orc_i8_words_per_row(7), L.orc_i8_words_per_row(4), L.orc_i8_words_per_row(1)) == (2, 1, 1)


def test_trit_pack_matches_threshold_rule(orc):
    # ternary_gemm_test.cpp:224-251 (engine pack == host pack_row) with the double-precision
    # threshold of t1_58_test.cpp:238-252 as the independent rule
    W = uniform((33, 70), 7)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    wq = orc.trit_pack(W, tau)
    t = orc.trits_of(wq, 70)
    w64, h = W.astype(np.float64), 0.5 * tau.astype(np.float64)[:, None]
    expect = np.where(w64 > h, 1, np.where(w64 < -h, -1, 0))
    assert np.array_equal(t, expect)


# ---------------------------------------------------------------- absmean tau (KAT)

KRAW_W = np.array([[1.0, 0.3, -0.3, 0.3], [0.4, -0.4, 0.1, -0.1], [0.7, 0.6, 0.5, 0.1]], np.float32)
KX = np.array([[1.0, -2.0], [0.5, 1.0], [-1.0, 0.25], [2.0, -0.5]], np.float32)


def test_tau_kat(orc):
    # src/t1_58_test.cpp:207-217, :291: tau = {0.475, 0.25, 0.475} to 1e-6
    tau = orc.row_absmean(KRAW_W)
    assert np.all(np.abs(tau.astype(np.float64) - [0.475, 0.25, 0.475]) < 1e-6)
    # trits of t1_58_test.cpp:322-326: row0 keeps the 0.3s (absmean), row1 zeroes the 0.1s
    t = orc.trits_of(orc.trit_pack(KRAW_W, tau), 4)
    assert t.tolist() == [[1, 1, -1, 1], [1, -1, 0, 0], [1, 1, 1, 0]]


def test_tau_close_to_float64(orc):
    W = normal((64, 6912), 11, 0.0, 0.02)
    tau = orc.row_absmean(W)
    ref = np.abs(W.astype(np.float64)).mean(axis=1)
    assert np.max(np.abs(tau - ref) / ref) < 1e-6


def test_zero_fraction_gaussian_absmean(orc):
    # sanity invariant: per-tensor absmean on N(0, 0.02) leaves P(|z| <= 0.5*sqrt(2/pi)) zeros
    W = normal((1024, 1024), 0xB17A0001, 0.0, 0.02)
    tau = np.full(1024, np.abs(W.astype(np.float64)).mean(), np.float32)
    t = orc.trits_of(orc.trit_pack(W, tau), 1024)
    expect = math.erf(0.5 * math.sqrt(2 / math.pi) / math.sqrt(2))
    assert abs(float((t == 0).mean()) - expect) < 0.005
    assert abs(expect - 0.310) < 0.001


# ---------------------------------------------------------------- int8 quantization

def test_quantize_special_cases(orc):
    # docs/internal/21-quantized-weights.md:973-975; src/int8_act_test.cpp:86-137
    q = orc.quantize_one
    assert q(1.0, 0.0) == 0                       # s == 0 -> 0
    assert q(float("nan"), 1.0) == 0              # NaN -> 0
    assert q(2.5, 1.0) == 3 and q(-2.5, 1.0) == -3  # round half away from zero
    assert q(0.5, 1.0) == 1 and q(-0.5, 1.0) == -1
    assert q(0.49999997, 1.0) == 0
    assert q(1000.0, 1.0) == 127 and q(-1000.0, 1.0) == -127  # clamp to +-127 (never -128)
    assert q(float("inf"), 1.0) == 127 and q(float("-inf"), 1.0) == -127
    assert q(1.0, float("inf")) == 0


def test_quantize_layout_and_values(orc):
    # src/int8_act_test.cpp:86-137: M=5, N=7 (tail word), a zero column and a NaN
    xm = uniform((5, 7), 11)
    s = np.abs(xm).max(axis=0)
    xm[:, 0] = 0.0
    xm[1, 1] = np.nan
    out = orc.quantize_i8(xm, s, True)
    assert out.shape == (5, 2)
    b = out.view(np.uint8).reshape(5, 8)
    assert np.all(b[:, 7] == 0)                  # tail byte
    q = orc.container_to_int8(out, 7).astype(np.int64)
    assert np.all(q[:, 0] == 0) and q[1, 1] == 0
    v = xm.astype(np.float64) / s.astype(np.float64)
    ok = ~np.isnan(v)
    # q is the integer nearest to x/s (s = absmax -> |x/s| <= 1 -> q in {-1, 0, 1})
    assert np.all(np.abs(q[ok] - v[ok]) <= 0.5 + 1e-6)
    assert set(np.unique(q)) <= {-1, 0, 1}


def test_quantize_row_scale_and_clamp(orc):
    x = uniform((9, 13), 3, -300.0, 300.0)
    sc = np.full(9, 1.3, np.float32)
    q = orc.container_to_int8(orc.quantize_i8(x, sc, False), 13).astype(np.int64)
    v = np.clip(x.astype(np.float64) / 1.3, -127, 127)
    assert np.all(np.abs(q - v) <= 0.5 + 1e-6)
    assert q.min() >= -127 and q.max() <= 127


def test_act_scale_multiplies_reciprocal(orc):
    # compute_layer_bitlinear.hpp:443-447: s = max|x| * fl(1/127), a multiply, not a divide
    X = normal((300, 9), 5)
    s = orc.act_scale(X)
    mx = np.abs(X).max(axis=0)
    assert np.array_equal(s, (mx * np.float32(1.0 / 127.0)).astype(np.float32))


def test_unpack_roundtrip(orc):
    # src/int8_act_test.cpp:140-168
    x = uniform((3, 6), 23)
    s = np.maximum(0.3, np.abs(x[0]) + 0.1).astype(np.float32)
    packed = orc.quantize_i8(x, s, True)
    u = orc.unpack_i8(packed, 6)
    assert np.array_equal(u, orc.container_to_int8(packed, 6).astype(np.float32))
    assert np.all(np.abs(u) <= 127)


# ---------------------------------------------------------------- matmul_q_i8

def _case(orc, N, K, M, seed):
    """int8_act_test.cpp:171-205 inputs: uniform W, tau = per-row absmean (double), X, s = absmax."""
    W = uniform((N, K), seed)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    X = uniform((K, M), seed + 1)
    s = np.abs(X).max(axis=0).astype(np.float32)
    wq = orc.trit_pack(W, tau)
    xq = orc.quantize_i8(X, s, True)
    return wq, tau, xq, s


@pytest.mark.parametrize("N,K,M,seed", [(130, 17, 6, 31), (512, 256, 8, 41), (65, 33, 1, 3),
                                        (9, 100, 3, 5)])
def test_matmul_q_i8_bruteforce(orc, N, K, M, seed):
    wq, tau, xq, s = _case(orc, N, K, M, seed)
    acc = orc.matmul_q_i8_acc(wq, xq, K, M)
    t = orc.trits_of(wq, K).astype(np.int64)
    q = orc.container_to_int8(xq, M).astype(np.int64)
    assert np.array_equal(acc.astype(np.int64), t @ q)
    Y = orc.matmul_q_i8(wq, tau, xq, s, K, M)
    # src/int8_act_test.cpp:233: (tau_m * s_n) * float(acc), numpy float32 ops are IEEE
    ts = tau[:, None] * s[None, :]
    assert np.array_equal(Y, ts * (t @ q).astype(np.float32))
    # the epilogue order matters: tau * (s * acc) differs somewhere on this data
    alt = tau[:, None] * (s[None, :] * acc.astype(np.float32))
    if N * M > 500:
        assert not np.array_equal(Y, alt)


@pytest.mark.parametrize("N,K,M", [(130, 17, 6), (512, 256, 8), (1024, 1024, 8), (100, 6912, 3)])
def test_rowblock_bit_identical(orc, N, K, M):
    wq, tau, xq, s = _case(orc, N, K, M, 77)
    assert np.array_equal(orc.matmul_q_i8_rowblock(wq, tau, xq, s, K, M),
                          orc.matmul_q_i8(wq, tau, xq, s, K, M))


def test_bias_add(orc):
    Y = normal((5, 3), 1)
    b = normal((5,), 2)
    assert np.array_equal(orc.add_row_broadcast(Y, b), Y + b[:, None])


# ---------------------------------------------------------------- RMSNorm

def test_rmsnorm_close_to_float64(orc):
    X = normal((2560, 33), 9)
    g = normal((2560,), 10, 1.0, 0.1)
    out = orc.rmsnorm(X, g, 1e-6)
    x64 = X.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=0) + 1e-6) * g.astype(np.float64)[:, None]
    assert np.max(np.abs(out - ref) / np.maximum(np.abs(ref), 1e-3)) < 2e-6


# ---------------------------------------------------------------- LayerNorm

def _layernorm64(X, g, b, eps):
    x64 = X.astype(np.float64)
    d = x64 - x64.mean(axis=0)
    return d / np.sqrt((d ** 2).mean(axis=0) + eps) * g.astype(np.float64)[:, None] + b.astype(np.float64)[:, None]


@pytest.mark.parametrize("F,M,loc,eps", [(2560, 33, 0.0, 1e-5), (6912, 5, 4.0, 1e-5), (300, 17, -2.5, 1e-6),
                                         (4, 9, 1.0, 1e-2)])
def test_layernorm_close_to_float64(orc, F, M, loc, eps):
    """The mean is subtracted (loc != 0), the variance is the biased one (a 1/(F-1) variance is
    2e-4 off at F=2560), eps sits inside the square root (F=4, eps=1e-2 moves every value), and
    beta is added after the gain."""
    X = normal((F, M), F + M, loc, 1.0)
    g = normal((F,), 10, 1.0, 0.1)
    b = normal((F,), 11, 0.0, 0.5)
    out = orc.layernorm(X, g, b, eps)
    ref = _layernorm64(X, g, b, eps)
    # fp32 sums of F values around a mean of |loc| leave ~1e-6 absolute in d = x - mean
    assert np.max(np.abs(out - ref) - 1e-5 * np.abs(ref)) < 5e-6


def test_layernorm_exact_cases(orc):
    """A constant token (every deviation 0) and F = 1 give beta exactly, whatever gamma and eps."""
    F, M = 257, 4
    X = normal((F, M), 5)
    X[:, 1] = 3.25
    X[:, 3] = -1e30
    g = normal((F,), 6, 1.0, 0.1)
    b = normal((F,), 7)
    out = orc.layernorm(X, g, b, 1e-5)
    assert np.array_equal(out[:, 1], b) and np.array_equal(out[:, 3], b)
    X1 = normal((1, 6), 8)
    g1, b1 = np.array([2.0], np.float32), np.array([-0.75], np.float32)
    assert np.array_equal(orc.layernorm(X1, g1, b1, 1e-5), np.full((1, 6), -0.75, np.float32))


def test_layernorm_unit_gain_standardizes(orc):
    """gamma = 1, beta = 0: every token has mean ~0 and variance ~1 / (1 + eps / var)."""
    X = normal((1024, 8), 9, 2.0, 3.0)
    out = orc.layernorm(X, np.ones(1024, np.float32), np.zeros(1024, np.float32), 1e-5)
    o64 = out.astype(np.float64)
    assert np.max(np.abs(o64.mean(axis=0))) < 1e-6
    var = X.astype(np.float64).var(axis=0)
    assert np.allclose(o64.var(axis=0), var / (var + 1e-5), rtol=0, atol=1e-5)


def test_rmsnorm_quant_is_the_sequence(orc):
    X = normal((700, 21), 12)
    g = np.ones(700, np.float32)
    xq, s = orc.rmsnorm_quant_i8(X, g, 1e-6)
    n = orc.rmsnorm(X, g, 1e-6)
    s2 = orc.act_scale(n)
    assert np.array_equal(s, s2)
    assert np.array_equal(xq, orc.quantize_i8(n, s2, True))


# ---------------------------------------------------------------- MI355X tile layout

@pytest.mark.parametrize("N,K", [(1, 1), (16, 256), (17, 257), (33, 40), (130, 17), (64, 1000)])
def test_repack_roundtrip(orc, N, K):
    rng = np.random.default_rng(N * 1000 + K)
    wq = rng.integers(0, 2 ** 32, size=(N, (K + 15) // 16), dtype=np.uint64).astype(np.uint32)
    rp = orc.repack(wq, K)
    assert rp.size == ((N + 15) // 16 * 16) * ((K + 255) // 256 * 256) // 16
    assert np.array_equal(orc.unrepack(rp, N, K), wq)


def test_repack_layout_feeds_the_mfma_mapping(orc):
    """Decode the tiles the way the kernel's MFMAs consume them (numpy, vectorized) and
    check the resulting code matrix and a product against the reference container."""
    N, K = 40, 600
    W = normal((N, K), 4)
    tau = np.abs(W).mean(axis=1).astype(np.float32)
    wq = orc.trit_pack(W, tau)
    rp = orc.repack(wq, K)
    RT, KT = (N + 15) // 16, (K + 255) // 256
    t = rp.reshape(RT, KT, 4, 16, 4)  # [rt][kt][g][r][q]
    codes = np.zeros((RT * 16, KT * 256), np.int64)
    for j in range(4):
        for b in range(4):
            c = (t >> np.uint32(8 * b + 2 * j)) & np.uint32(3)  # [rt][kt][g][r][q]
            # k = 256kt + 64j + 16g + 4q + b ; row = 16rt + r
            for g in range(4):
                for q in range(4):
                    cols = np.arange(KT) * 256 + 64 * j + 16 * g + 4 * q + b
                    codes[:, cols] = c[:, :, g, :, q].transpose(0, 2, 1).reshape(RT * 16, KT)
    trit = orc.trits_of(wq, K).astype(np.int64)
    assert np.array_equal(codes[:N, :K] - 2, trit)
    assert np.all(codes[N:, :] == 2) and np.all(codes[:, ((K + 15) // 16) * 16:] == 2)
    x = np.random.default_rng(1).integers(-127, 128, size=(KT * 256,))
    x[K:] = 0
    assert np.array_equal(codes[:N] @ x - 2 * x.sum(), trit @ x[:K])


# ---------------------------------------------------------------- golden fixtures

def test_golden_fixtures(orc):
    path = os.path.join(GOLDEN, "matmul_q_i8.npz")
    with np.load(path, allow_pickle=False) as z:
        names = sorted({k.split("__")[0] for k in z.files})
        assert len(names) >= 3
        for name in names:
            g = {k.split("__")[1]: z[k] for k in z.files if k.startswith(name + "__")}
            N, K, M = (int(v) for v in g["shape"])
            if "W" in g:
                assert np.array_equal(orc.trit_pack(g["W"], g["tau"]), g["wq"]), name
            assert np.array_equal(orc.quantize_i8(g["X"], g["s"], True), g["xq"]), name
            assert np.array_equal(orc.matmul_q_i8_acc(g["wq"], g["xq"], K, M), g["acc"]), name
            assert np.array_equal(orc.matmul_q_i8(g["wq"], g["tau"], g["xq"], g["s"], K, M), g["Y"]), name


# ------------------------------------------------------------------ float-activation GEMM (a10)

def _ref_patterns(rows, K, N):
    """The reference test's generators: W = 0.13*((r*7 + c*3) % 11) - 0.6,
    X = 0.21*((k + 2n) % 9) - 0.8, tau = per-row absmean (src/ternary_gemm_test.cpp:187-210)."""
    r = np.arange(rows)[:, None]
    c = np.arange(K)[None, :]
    W = (np.float32(0.13) * ((r * 7 + c * 3) % 11).astype(np.float32) - np.float32(0.6)).astype(np.float32)
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    X = (np.float32(0.21) * ((k + 2 * n) % 9).astype(np.float32) - np.float32(0.8)).astype(np.float32)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    return W, X, tau


@pytest.mark.parametrize("rows,K,N", [(7, 40, 3), (65, 17, 65), (9, 100, 3), (256, 40, 1)])
def test_matmul_q_against_float64(orc, rows, K, N):
    W, X, tau = _ref_patterns(rows, K, N)
    wq = orc.trit_pack(W, tau)
    trits = orc.trits_of(wq, K).astype(np.float64)
    ref = (tau.astype(np.float64)[:, None] * trits) @ X.astype(np.float64)
    got = orc.matmul_q(wq, tau, X, K)
    assert np.max(np.abs(got - ref)) <= 1e-6 * max(1.0, np.max(np.abs(ref)))


@pytest.mark.parametrize("K,M,N", [(40, 7, 3), (17, 65, 65), (33, 129, 7), (100, 9, 1)])
def test_matmul_q_t_against_float64(orc, K, M, N):
    # A stored (K, M): tau per stored row k, as the reference's transA form
    A, _, tau = _ref_patterns(K, M, 1)
    B = normal((K, N), K * 3 + N, 0.0, 1.0)
    Aq = orc.trit_pack(A, tau)
    trits = orc.trits_of(Aq, M).astype(np.float64)          # (K, M)
    ref = (tau.astype(np.float64)[:, None] * trits).T @ B.astype(np.float64)
    got = orc.matmul_q_t(Aq, tau, B, M)
    assert got.shape == (M, N)
    assert np.max(np.abs(got - ref)) <= 1e-6 * max(1.0, np.max(np.abs(ref)))


def test_matmul_q_identity_gives_scaled_trits(orc):
    """Closed form: B = I makes Y the dequantized weights tau[n] * trit(n, k) exactly."""
    N, K = 19, 37
    W = normal((N, K), 11, 0.0, 0.02)
    tau = orc.row_absmean(W)
    wq = orc.trit_pack(W, tau)
    got = orc.matmul_q(wq, tau, np.eye(K, dtype=np.float32), K)
    assert np.array_equal(got, (tau[:, None] * orc.trits_of(wq, K)).astype(np.float32))
    # and the transposed form on the same container reads it column-wise
    got_t = orc.matmul_q_t(wq, tau, np.eye(N, dtype=np.float32), K)
    assert np.array_equal(got_t, (tau[:, None] * orc.trits_of(wq, K)).astype(np.float32).T)


# ---------------------------------------------------------------- gated activations, FFN block

def _ulp_dist(a32: np.ndarray, ref64: np.ndarray) -> np.ndarray:
    """Distance in fp32 ulps between a32 and the float32 rounding of ref64 (finite values)."""
    r32 = ref64.astype(np.float32)
    ia = a32.view(np.int32).astype(np.int64)
    ib = r32.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-2**31) - ia, ia)
    ib = np.where(ib < 0, np.int64(-2**31) - ib, ib)
    return np.abs(ia - ib)


def test_exp_within_2ulp_of_float64(orc):
    x = np.linspace(-87.0, 88.72, 2_000_003, dtype=np.float32)
    x = np.concatenate([x, uniform((200_000,), 5, -1.0, 1.0), uniform((50_000,), 6, -1e-4, 1e-4)])
    e = orc.exp(x)
    ref = np.exp(x.astype(np.float64))
    assert _ulp_dist(e, ref).max() <= 2
    # exact points and the documented edges
    assert orc.exp(np.float32([0.0]))[0] == 1.0
    assert orc.exp(np.float32([-0.0]))[0] == 1.0
    assert np.isinf(orc.exp(np.float32([88.73, 100.0, 1e30, np.inf]))).all()
    assert (orc.exp(np.float32([-87.01, -100.0, -1e30, -np.inf])) == 0.0).all()
    assert np.isnan(orc.exp(np.float32([np.nan])))[0]
    # e^88.72 is still finite (FLT_MAX = e^88.7228...)
    assert np.isfinite(orc.exp(np.float32([88.72])))[0]


def test_swiglu_close_to_float64(orc):
    F, M = 300, 7
    Y1 = normal((2 * F, M), 21, 0.0, 4.0)
    h = orc.glu(Y1, orc.ACT_SWIGLU)
    g = Y1[:F].astype(np.float64)
    u = Y1[F:].astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    assert np.max(np.abs(h - ref) / np.maximum(np.abs(ref), 1e-30)) < 4e-7


def test_glu_special_cases(orc):
    one = lambda g, u, a: orc.lib().orc_glu_one(g, u, a)
    # SwiGLU: silu(0) = 0, silu(g) -> g for large g, -> -0 for very negative g
    assert one(0.0, 5.0, 0) == 0.0
    assert one(200.0, 1.5, 0) == 300.0
    assert one(-200.0, 1.0, 0) == 0.0
    assert math.isnan(one(float("nan"), 1.0, 0))
    assert math.isnan(one(float("-inf"), 1.0, 0))  # -inf * sigma(-inf) = -inf * 0
    # ReLU^2-GLU: (max(g,0))^2 * u, NaN gate -> 0 (the select), exact on representable values
    assert one(3.0, 2.0, 1) == 18.0
    assert one(-3.0, 2.0, 1) == 0.0
    assert one(float("nan"), 2.0, 1) == 0.0
    g = normal((1000,), 22, 0.0, 3.0)
    u = normal((1000,), 23, 0.0, 3.0)
    Y1 = np.concatenate([g[None, :], u[None, :]])
    r = np.maximum(g.astype(np.float64), 0.0)
    ref = r * r * u.astype(np.float64)
    out = orc.glu(Y1, orc.ACT_RELU2)[0]
    assert np.max(np.abs(out - ref) / np.maximum(np.abs(ref), 1e-30)) < 2.5e-7


def test_glu_interleave_rows(orc):
    F = 12
    src = orc.glu_src_rows(F)
    assert len(src) == 32
    assert list(src[:16]) == list(range(0, 8)) + list(range(12, 20))
    assert list(src[16:]) == [8, 9, 10, 11, -1, -1, -1, -1, 20, 21, 22, 23, -1, -1, -1, -1]
    K = 40
    W = normal((2 * F, K), 24)
    tau = orc.row_absmean(W)
    wq = orc.trit_pack(W, tau)
    b = normal((2 * F,), 25)
    wo, to, bo = orc.glu_interleave(wq, tau, b, F, K)
    for r, s in enumerate(src):
        if s < 0:
            assert (orc.trits_of(wo[r:r + 1], K) == 0).all() and to[r] == 0 and bo[r] == 0
        else:
            assert np.array_equal(wo[r], wq[s]) and to[r] == tau[s] and bo[r] == b[s]


@pytest.mark.parametrize("act", [0, 1])
def test_ffn_block_is_the_composition(orc, act):
    d, F, M = 96, 40, 5
    X = normal((d, M), 31)
    gamma = normal((d,), 32, 1.0, 0.1)
    W1 = normal((2 * F, d), 33, 0.0, 0.02)
    W2 = normal((d, F), 34, 0.0, 0.02)
    t1, t2 = orc.row_absmean(W1), orc.row_absmean(W2)
    wq1, wq2 = orc.trit_pack(W1, t1), orc.trit_pack(W2, t2)
    b1, b2 = normal((2 * F,), 35, 0.0, 0.1), normal((d,), 36, 0.0, 0.1)
    Y, h = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, b1, wq2, t2, b2, act)

    def bitlinear(x, wq, tau, b, K):
        s = orc.act_scale(x)
        q = orc.container_to_int8(orc.quantize_i8(x, s, True), x.shape[1]).astype(np.int64)
        acc = orc.trits_of(wq, K).astype(np.int64) @ q
        return (tau[:, None] * s[None, :]) * acc.astype(np.float32) + b[:, None]

    x1 = orc.rmsnorm(X, gamma, 1e-6)
    y1 = bitlinear(x1, wq1, t1, b1, d)
    h_ref = orc.glu(y1, act)
    assert np.array_equal(h, h_ref)
    assert np.array_equal(Y, bitlinear(h_ref, wq2, t2, b2, F))
    # no norm: gamma None feeds X straight to fc1's quantizer
    Y0, _ = orc.ffn_glu_i8(X, None, 0.0, F, wq1, t1, b1, wq2, t2, b2, act)
    assert np.array_equal(Y0, bitlinear(orc.glu(bitlinear(X, wq1, t1, b1, d), act), wq2, t2, b2, F))
    # SubLN: an RMSNorm of the gated output (eps 1e-5, the RMSNorm default) before fc2
    gs = normal((F,), 37, 1.0, 0.1)
    Ys, hs = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, b1, wq2, t2, b2, act, gamma_sub=gs, eps_sub=1e-5)
    assert np.array_equal(hs, h_ref)
    assert np.array_equal(Ys, bitlinear(orc.rmsnorm(h_ref, gs, 1e-5), wq2, t2, b2, F))
    assert not np.array_equal(Ys, Y)


def test_model_file_fixtures_reproducible(tmp_path):
    """The committed .nnmodel fixtures are exactly what tests/golden/make_nnmodel.py writes,
    and their v8 tails verify with hashlib's sha256."""
    import hashlib
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    subprocess.run([sys.executable, os.path.join(GOLDEN, "make_nnmodel.py"), str(tmp_path)], check=True,
                   cwd=os.path.dirname(here), capture_output=True)
    names = sorted(p.name for p in tmp_path.iterdir())
    assert len(names) == 6
    for n in names:
        with open(os.path.join(GOLDEN, n), "rb") as f:
            committed = f.read()
        assert (tmp_path / n).read_bytes() == committed, n
        if n != "nnmodel_v7.nnmodel":
            body, digest, tail = committed[:-37], committed[-37:-5], committed[-5:]
            assert tail == b"NNEND"
            assert (hashlib.sha256(body).digest() == digest) == (n != "nnmodel_corrupt.nnmodel"), n

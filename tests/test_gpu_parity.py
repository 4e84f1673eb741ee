"""GPU parity: every libnn-hip.so entry point of the BitLinear W1.58A8 path against the CPU
oracle on the same seeded inputs, bit for bit (integer containers, int32 accumulators and
the fp32 epilogue, whose order the kernels keep). Large shapes are checked on sampled rows
(the oracle runs on the same rows) plus size-independent properties. The float-activation
GEMM (matmul_q / matmul_q_t), whose accumulation order the reference leaves open, is checked
against the oracle's float64 evaluation within the reference's own tolerances.

Reference tests mirrored: src/int8_act_test.cpp [1]-[3], src/ternary_gemm_test.cpp [1]-[4]
and [6], src/t1_58_test.cpp [5].
"""
import numpy as np
import pytest

from conftest import normal, uniform

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def say(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------ trit_pack / tau

@pytest.mark.parametrize("N,K", [(7, 40), (130, 17), (3, 4), (1024, 1024), (2560, 6912), (33, 1)])
def test_trit_pack_and_tau(ctx, orc, N, K):
    say(f"trit_pack/row_absmean N={N} K={K}")
    W = normal((N, K), 1000 + N + K, 0.0, 0.02)
    W[0, :min(K, 3)] = 0.0
    tau_g = host(ctx.row_absmean(dev(W)))
    tau_o = orc.row_absmean(W)
    assert np.array_equal(tau_g, tau_o)
    wq_g = host(ctx.trit_pack(dev(W), dev(tau_o)), np.uint32)
    assert np.array_equal(wq_g, orc.trit_pack(W, tau_o))


def test_tau_kat_on_gpu(ctx, orc):
    # src/t1_58_test.cpp:207-217: tau = {0.475, 0.25, 0.475}
    W = np.array([[1.0, 0.3, -0.3, 0.3], [0.4, -0.4, 0.1, -0.1], [0.7, 0.6, 0.5, 0.1]], np.float32)
    tau = host(ctx.row_absmean(dev(W)))
    assert np.all(np.abs(tau.astype(np.float64) - [0.475, 0.25, 0.475]) < 1e-6)
    t = orc.trits_of(host(ctx.trit_pack(dev(W), dev(tau)), np.uint32), 4)
    assert t.tolist() == [[1, 1, -1, 1], [1, -1, 0, 0], [1, 1, 1, 0]]


def test_trit_pack_ties_and_nan(ctx, orc):
    tau = np.array([1.0, 2.0], np.float32)
    W = np.array([[0.5, -0.5, 0.50000006, -0.50000006, np.nan, np.inf, -np.inf, 0.0],
                  [1.0, -1.0, 1.0000001, -1.0000001, 0.0, -0.0, 3.0, -3.0]], np.float32)
    got = host(ctx.trit_pack(dev(W), dev(tau)), np.uint32)
    assert np.array_equal(got, orc.trit_pack(W, tau))


# ------------------------------------------------------------------ int8 quantization

def test_quantize_i8_kat(ctx, orc):
    # src/int8_act_test.cpp:86-137: 5x7, zero column (s == 0), one NaN
    xm = uniform((5, 7), 11)
    s = np.abs(xm).max(axis=0)
    xm[:, 0] = 0.0
    xm[1, 1] = np.nan
    s[0] = 0.0
    got = host(ctx.quantize_i8(dev(xm), dev(s), True), np.uint32)
    assert np.array_equal(got, orc.quantize_i8(xm, s, True))


@pytest.mark.parametrize("rows,cols,col_scale", [(256, 13, True), (1024, 8, True), (9, 33, False),
                                                 (2560, 1, True)])
def test_quantize_unpack(ctx, orc, rows, cols, col_scale):
    say(f"quantize/unpack {rows}x{cols} col_scale={col_scale}")
    x = normal((rows, cols), rows + cols, 0.0, 3.0)
    x.flat[::97] *= 40.0
    sc = orc.act_scale(x) if col_scale else (np.abs(x).max(axis=1) / 127.0).astype(np.float32)
    q = host(ctx.quantize_i8(dev(x), dev(sc), col_scale), np.uint32)
    assert np.array_equal(q, orc.quantize_i8(x, sc, col_scale))
    u = host(ctx.unpack_i8(dev(q), cols))
    assert np.array_equal(u, orc.unpack_i8(q, cols))


def test_col_reduce_max_abs_scale(ctx, orc):
    X = normal((777, 19), 5)
    X[3, 4] = np.nan
    a = ctx.abs(dev(X))
    m = host(ctx.col_reduce_max(a))
    assert np.array_equal(m, orc.col_absmax(X))
    s_seq = ctx.col_reduce_max(a)
    ctx.scale_inplace(s_seq, 1.0 / 127.0)
    s_fused = host(ctx.act_scale(dev(X)))
    assert np.array_equal(host(s_seq), orc.act_scale(X))
    assert np.array_equal(s_fused, orc.act_scale(X))


# ------------------------------------------------------------------ matmul_q_i8 (reference layout)

def make_case(orc, N, K, M, seed, gaussian=False, outliers=False):
    if gaussian:
        W = normal((N, K), seed, 0.0, 0.02)
        tau = np.full(N, np.abs(W.astype(np.float64)).mean(), np.float32)
        X = normal((K, M), seed + 1)
        if outliers:
            rng = np.random.default_rng(seed)
            idx = rng.choice(K * M, size=max(1, K * M // 1000), replace=False)
            X.flat[idx] *= 20.0
        s = orc.act_scale(X)
    else:
        W = uniform((N, K), seed)
        tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
        X = uniform((K, M), seed + 1)
        s = np.abs(X).max(axis=0).astype(np.float32)
    return W, tau, X, s, orc.trit_pack(W, tau), orc.quantize_i8(X, s, True)


@pytest.mark.parametrize("N,K,M,seed", [
    (130, 17, 6, 31),      # int8_act_test [3]: K, N not multiples, crosses the RB=64 row block
    (512, 256, 8, 41),     # int8_act_test [3] GPU: 2B4T order
    (1024, 1024, 8, 0xB17A0001),
    (65, 33, 1, 3), (9, 100, 3, 5), (256, 40, 1, 7),   # ternary_gemm_test [6] tails / N=1
    (64, 16, 16, 9), (64, 16, 17, 9),               # GEMV/GEMM boundary
    (192, 48, 320, 11), (130, 300, 130, 13),         # GEMM tails in both directions
])
def test_matmul_q_i8(ctx, orc, N, K, M, seed):
    say(f"matmul_q_i8 N={N} K={K} M={M}")
    gaussian = (seed == 0xB17A0001)
    _, tau, _, s, wq, xq = make_case(orc, N, K, M, seed, gaussian=gaussian)
    Y = host(ctx.matmul_q_i8(dev(wq), dev(tau), dev(xq), dev(s), K, M))
    assert np.array_equal(Y, orc.matmul_q_i8(wq, tau, xq, s, K, M))


def test_golden_fixtures_on_gpu(ctx):
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "matmul_q_i8.npz")
    with np.load(path, allow_pickle=False) as z:
        names = sorted({k.split("__")[0] for k in z.files})
        for name in names:
            g = {k.split("__")[1]: z[k] for k in z.files if k.startswith(name + "__")}
            N, K, M = (int(v) for v in g["shape"])
            say(f"golden {name}")
            xq = host(ctx.quantize_i8(dev(g["X"]), dev(g["s"]), True), np.uint32)
            assert np.array_equal(xq, g["xq"]), name
            Y = host(ctx.matmul_q_i8(dev(g["wq"]), dev(g["tau"]), dev(g["xq"]), dev(g["s"]), K, M))
            assert np.array_equal(Y, g["Y"]), name
            if "W" in g:
                assert np.array_equal(host(ctx.trit_pack(dev(g["W"]), dev(g["tau"])), np.uint32), g["wq"])


# ------------------------------------------------------------------ repacker

@pytest.mark.parametrize("N,K", [(1, 1), (17, 257), (130, 17), (2560, 2560), (640, 6912)])
def test_repack_roundtrip(ctx, orc, N, K):
    say(f"repack N={N} K={K}")
    rng = np.random.default_rng(N + K)
    wq = rng.integers(0, 2 ** 32, size=(N, (K + 15) // 16), dtype=np.uint64).astype(np.uint32)
    rp = ctx.repack(dev(wq), K)
    if N * K <= 640 * 6912:
        assert np.array_equal(host(rp, np.uint32), orc.repack(wq, K))
    assert np.array_equal(host(ctx.unrepack(rp, N, K), np.uint32), wq)


# ------------------------------------------------------------------ fused activation quant

@pytest.mark.parametrize("K,M", [(2560, 1), (6912, 16), (17, 5), (2560, 33), (4096, 300), (1024, 8)])
def test_act_quant_i8(ctx, orc, nnhip, K, M):
    say(f"act_quant K={K} M={M}")
    X = normal((K, M), K * 7 + M, 0.0, 1.0)
    X.flat[::1009] *= 20.0
    xi, s, rs, xq = ctx.act_quant_i8(dev(X), want_container=True)
    s_o = orc.act_scale(X)
    xq_o = orc.quantize_i8(X, s_o, True)
    assert np.array_equal(host(s), s_o)
    assert np.array_equal(host(xq, np.uint32), xq_o)
    q = orc.container_to_int8(xq_o, M).T  # (M, K)
    xi_h = host(xi)
    assert np.array_equal(xi_h[:, :K], q)
    assert np.all(xi_h[:, K:] == 0)
    assert np.array_equal(host(rs), q.astype(np.int64).sum(axis=1))
    # container -> xi conversion and back
    xi2, rs2 = ctx.act_from_container(dev(xq_o), K, M)
    assert np.array_equal(host(xi2), xi_h) and np.array_equal(host(rs2), host(rs))
    assert np.array_equal(host(ctx.act_to_container(xi, K, M), np.uint32), xq_o)


@pytest.mark.parametrize("F,M,eps", [(2560, 1, 1e-6), (2560, 16, 1e-5), (2560, 100, 1e-6),
                                     (6912, 64, 1e-6), (300, 3, 1e-6)])
def test_rmsnorm_quant(ctx, orc, F, M, eps):
    say(f"rmsnorm_quant F={F} M={M}")
    X = normal((F, M), F + M, 0.0, 1.0)
    g = normal((F,), 3, 1.0, 0.1)
    out = host(ctx.rmsnorm(dev(X), dev(g), eps))
    assert np.array_equal(out, orc.rmsnorm(X, g, eps))
    xi, s, rs, xq = ctx.rmsnorm_quant_i8(dev(X), dev(g), eps, want_container=True)
    xq_o, s_o = orc.rmsnorm_quant_i8(X, g, eps)
    assert np.array_equal(host(s), s_o)
    assert np.array_equal(host(xq, np.uint32), xq_o)
    assert np.array_equal(host(xi)[:, :F], orc.container_to_int8(xq_o, M).T)


@pytest.mark.parametrize("F,M,loc", [(2560, 33, 0.0), (6912, 64, 3.0), (1, 5, 0.0), (17, 1, -1.0), (300, 1000, 0.5),
                                     (13, 2048, 0.0), (2560, 31, 0.0)])
def test_layernorm(ctx, orc, F, M, loc):
    say(f"layernorm F={F} M={M}")
    X = normal((F, M), F + M, loc, 1.0)
    if M > 2:
        X[:, 2] = 0.625          # a constant token: beta exactly
    g = normal((F,), 3, 1.0, 0.1)
    b = normal((F,), 4, 0.0, 0.5)
    out = host(ctx.layernorm(dev(X), dev(g), dev(b), 1e-5))
    ref = orc.layernorm(X, g, b, 1e-5)
    assert np.array_equal(out, ref)
    if M > 2:
        assert np.array_equal(out[:, 2], b)


def test_layernorm_rejects_short_gain(ctx, nnhip):
    import torch
    X = torch.zeros((8, 3), device="cuda")
    with pytest.raises(nnhip.NNHipError):
        ctx.layernorm(X, torch.ones(7, device="cuda"), torch.zeros(8, device="cuda"))


def check_quant(ctx, orc, X, g=None, eps=1e-6):
    """act_quant_i8 (g None) or rmsnorm_quant_i8 on X (K, M) against the oracle, all outputs."""
    K, M = X.shape
    if g is None:
        xi, s, rs, xq = ctx.act_quant_i8(dev(X), want_container=True)
        s_o = orc.act_scale(X)
        xq_o = orc.quantize_i8(X, s_o, True)
    else:
        xi, s, rs, xq = ctx.rmsnorm_quant_i8(dev(X), dev(g), eps, want_container=True)
        xq_o, s_o = orc.rmsnorm_quant_i8(X, g, eps)
    assert np.array_equal(host(s), s_o)
    assert np.array_equal(host(xq, np.uint32), xq_o)
    q = orc.container_to_int8(xq_o, M).T
    xi_h = host(xi)
    assert np.array_equal(xi_h[:, :K], q)
    assert np.all(xi_h[:, K:] == 0)
    assert np.array_equal(host(rs), q.astype(np.int64).sum(axis=1))


# M > 64 runs the register-resident kernel (rounds of 512 rows; 8 tokens per 16-wave block when
# M % 4 == 0, M <= 8192 and K <= 5120, or K <= 7168 without RMSNorm, where each wave reads one
# contiguous band of rows; 4 tokens per 8-wave block otherwise; M % 4 != 0 takes the scalar-load
# path), M <= 64 the one-token kernel; K = 11264 is the largest instantiation of both, K = 11265
# the fallback. M = 2052 and 1028 leave a half-empty last group of 8 tokens; K = 5121 and 6912
# end inside a band.
@pytest.mark.parametrize("K,M", [(1, 36), (255, 37), (512, 40), (513, 128), (1000, 66), (2560, 2048),
                                 (4096, 2048), (2560, 2052), (5120, 1028), (5121, 1024), (512, 8196),
                                 (6912, 132), (11264, 40), (11265, 36)])
@pytest.mark.parametrize("norm", [False, True])
def test_token_kernel_shapes(ctx, orc, K, M, norm):
    say(f"token kernel K={K} M={M} norm={norm}")
    X = normal((K, M), K * 31 + M, 0.0, 1.0)
    X.flat[::977] *= 20.0
    g = normal((K,), K + 5, 1.0, 0.2) if norm else None
    check_quant(ctx, orc, X, g)


# M <= 64 runs the one-token-per-block kernel (one sum-of-squares part per thread, R rows of
# 512); K = 11265 is past its largest instantiation (the one-wave-per-token fallback).
@pytest.mark.parametrize("K,M", [(1, 1), (255, 7), (512, 32), (513, 3), (2560, 16), (6912, 16), (11264, 5),
                                 (11265, 2)])
@pytest.mark.parametrize("norm", [False, True])
def test_token_one_shapes(ctx, orc, K, M, norm):
    say(f"one-token kernel K={K} M={M} norm={norm}")
    X = normal((K, M), K * 13 + M, 0.0, 1.0)
    X.flat[::613] *= 20.0
    g = normal((K,), K + 9, 1.0, 0.2) if norm else None
    check_quant(ctx, orc, X, g)
    if norm:
        assert np.array_equal(host(ctx.rmsnorm(dev(X), dev(g), 1e-6)), orc.rmsnorm(X, g, 1e-6))


@pytest.mark.parametrize("norm", [False, True])
def test_token_one_special_values(ctx, orc, norm):
    """NaN, infinities and all-zero tokens at decode sizes (M = 8)."""
    say(f"one-token kernel special values norm={norm}")
    K, M = 2560, 8
    X = normal((K, M), 99, 0.0, 1.0)
    X[5, 0] = np.nan
    X[7, 1] = np.inf
    X[9, 2] = -np.inf
    X[:, 3] = 0.0
    X[:, 4] *= np.float32(1e-30)
    X[:, 5] *= np.float32(1e30)
    g = normal((K,), 4, 1.0, 0.2) if norm else None
    check_quant(ctx, orc, X, g)


def test_quant_near_ties(ctx, orc):
    """x / s on and within a few ulps of half-integers: the division-free path must hand these
    to the exact division. Each token holds one 127 (s = fl(127 * fl(1/127))) and values
    (n + 1/2) * (1 + d) with d in {0, +-2^-23, +-2^-20, +-2^-14}."""
    say("act_quant near ties")
    rng = np.random.default_rng(7)
    K, M = 1024, 64
    n = rng.integers(-126, 126, size=(K, M)).astype(np.float64)
    d = rng.choice([0.0, 2.0 ** -23, -2.0 ** -23, 2.0 ** -20, -2.0 ** -20, 2.0 ** -14, -2.0 ** -14], size=(K, M))
    X = ((n + 0.5) * (1.0 + d)).astype(np.float32)
    X[0, :] = 127.0
    X[1, ::3] = -127.0
    check_quant(ctx, orc, X)
    # and scaled so that s is far from 1
    check_quant(ctx, orc, (X * np.float32(0.0371)).astype(np.float32))
    # the same values at decode sizes (one-token kernel)
    check_quant(ctx, orc, np.ascontiguousarray(X[:, :16]))


@pytest.mark.parametrize("K,M", [(1024, 2048), (6912, 132), (2560, 100)])
def test_quant_near_ties_register_kernel(ctx, orc, K, M):
    """The same near-tie values through the register kernel (M > 64: 8 tokens per block at
    K = 1024, 4 per block at K = 6912, the scalar-load path at M = 100): a flagged round is
    recomputed by the exact division-free code, bit for bit the division's."""
    say(f"act_quant near ties, register kernel K={K} M={M}")
    rng = np.random.default_rng(K + M)
    n = rng.integers(-126, 126, size=(K, M)).astype(np.float64)
    d = rng.choice([0.0, 2.0 ** -23, -2.0 ** -23, 2.0 ** -17, -2.0 ** -17, 2.0 ** -15, -2.0 ** -15, 2.0 ** -14,
                    -2.0 ** -14], size=(K, M))
    X = ((n + 0.5) * (1.0 + d)).astype(np.float32)
    X[0, :] = 127.0
    X[1, ::3] = -127.0
    check_quant(ctx, orc, X)
    check_quant(ctx, orc, (X * np.float32(0.0371)).astype(np.float32))
    g = normal((K,), K + 1, 1.0, 0.2)
    check_quant(ctx, orc, X, g)


@pytest.mark.parametrize("K,M", [(2560, 2048), (6912, 132)])
@pytest.mark.parametrize("norm", [False, True])
def test_token_regs_special_values(ctx, orc, K, M, norm):
    """NaN, infinities, all-zero tokens, and tokens whose scale is below 2^-100 (prescaled exact
    path), subnormal (its reciprocal overflows) or made of subnormals, through the register
    kernel (M > 64)."""
    say(f"register kernel special values K={K} M={M} norm={norm}")
    X = normal((K, M), K + M, 0.0, 1.0)
    X[5, 0] = np.nan
    X[7, 1] = np.inf
    X[9, 2] = -np.inf
    X[:, 3] = 0.0
    X[:, 4] *= np.float32(1e-30)
    X[:, 5] *= np.float32(1e30)
    X[:, 6] *= np.float32(1e-37)
    X[:, 7] *= np.float32(1e-43)
    X[:, 8] = np.float32(1e-45)
    X[11, 9] = np.nan
    X[11, 10] = -np.inf
    X[12, 10] = np.inf
    g = normal((K,), 4, 1.0, 0.2) if norm else None
    check_quant(ctx, orc, X, g)


# ------------------------------------------------------------------ fast-path GEMV / GEMM

def fast_case(ctx, orc, N, K, M, seed, outliers=False):
    W, tau, X, s, wq, xq = make_case(orc, N, K, M, seed, gaussian=True, outliers=outliers)
    rp = ctx.repack(dev(wq), K)
    xi, s_d, rs = ctx.act_quant_i8(dev(X))
    assert np.array_equal(host(s_d), s)
    return tau, s, wq, xq, rp, xi, s_d, rs


@pytest.mark.parametrize("N,K,M", [(2560, 2560, 1), (6912, 2560, 1), (2560, 6912, 1),
                                   (2560, 2560, 16), (640, 2560, 16), (6912, 2560, 7)])
def test_decode_gemv_shapes(ctx, orc, N, K, M):
    say(f"gemv N={N} K={K} M={M}")
    tau, s, wq, xq, rp, xi, s_d, rs = fast_case(ctx, orc, N, K, M, N + K + M)
    b = normal((N,), 99)
    Y = host(ctx.ternary_matmul(rp, dev(tau), xi, s_d, rs, N, K, M, bias=dev(b)))
    ref = orc.add_row_broadcast(orc.matmul_q_i8_rowblock(wq, tau, xq, s, K, M), b)
    assert np.array_equal(Y, ref)


@pytest.mark.parametrize("N,K,M,bias", [
    (100, 1024, 3, True), (2561, 2560, 5, False), (17, 4096, 16, True), (2560, 6912, 16, True),
    (10000, 2560, 16, False), (1, 2560, 1, True), (33, 6900, 2, True), (640, 2560, 13, False),
    (20000, 2560, 2, True),   # more row tiles than the deep variant takes: the streaming GEMV
])
def test_decode_gemv_deep(ctx, orc, N, K, M, bias):
    """The deep single-problem GEMV (all k stages in flight, activations staged in LDS by DMA,
    up to 110 KB at K = 6912, M = 16) on its k-tile counts 4, 10, 16, 27 with row / token / k
    tails, bit for bit."""
    say(f"deep gemv N={N} K={K} M={M} bias={bias}")
    tau, s, wq, xq, rp, xi, s_d, rs = fast_case(ctx, orc, N, K, M, 3 * N + K + M)
    b = normal((N,), 98) if bias else None
    Y = host(ctx.ternary_matmul(rp, dev(tau), xi, s_d, rs, N, K, M, bias=dev(b) if bias else None))
    ref = orc.matmul_q_i8(wq, tau, xq, s, K, M)
    if bias:
        ref = orc.add_row_broadcast(ref, b)
    assert np.array_equal(Y, ref)


def c3_case(ctx, orc, N, K, M, seed):
    """Config 2 inputs at full size: W ~ N(0, 0.02) ternarized by per-tensor absmean on the GPU
    (trit_pack is checked bit for bit elsewhere; the oracle reads the same container), X ~ N(0, 1)
    with 0.1% of the elements at 20x, quantized per token by the GPU and by the oracle."""
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    W = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    tau_d = W.abs().double().mean().float().expand(N).contiguous()
    wq_d = ctx.trit_pack(W, tau_d)
    del W
    rp = ctx.repack(wq_d, K)
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((K, M), dtype=np.float32)
    idx = rng.choice(K * M, size=max(1, K * M // 1000), replace=False)
    X.flat[idx] *= np.float32(20.0)
    xi, s_d, rs = ctx.act_quant_i8(dev(X))
    s = orc.act_scale(X)
    assert np.array_equal(host(s_d), s)
    xq = orc.quantize_i8(X, s, True)
    return host(wq_d, np.uint32), host(tau_d), xq, s, rp, tau_d, xi, s_d, rs


@pytest.mark.parametrize("N,K,M", [(4096, 4096, 256), (11008, 4096, 256), (4096, 4096, 1024), (11008, 4096, 1024),
                                   (4096, 4096, 2048), (11008, 4096, 2048), (4096, 4096, 4096), (11008, 4096, 4096),
                                   (2560, 2560, 100)])
def test_prefill_gemm_shapes(ctx, orc, N, K, M):
    """BASELINE config 2 (K=4096, N in {4096, 11008}, M up to 4096; 0.1% activation outliers at 20x):
    every row of Y bit for bit against the oracle's CpuEngine restatement (row-block decode + dense
    f32 microkernel, exact because every partial sum is an integer below 2^24), the check of
    src/int8_act_test.cpp:171-238."""
    say(f"gemm N={N} K={K} M={M}")
    wq, tau, xq, s, rp, tau_d, xi, s_d, rs = c3_case(ctx, orc, N, K, M, 5 + M + N)
    Y = host(ctx.ternary_matmul(rp, tau_d, xi, s_d, rs, N, K, M))
    ref = orc.matmul_q_i8_rowblock(wq, tau, xq, s, K, M)
    bad = Y != ref
    assert not bad.any(), f"{int(bad.sum())} of {Y.size} outputs differ, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("N,K,M", [(11008, 4096, 4096), (4096, 4096, 2048)])
def test_prefill_gemm_unit_scales_sums(ctx, orc, N, K, M):
    """Size-independent exact identities with tau = 1 and s = 1 (then Y = float(acc) exactly, since
    |acc| <= 127 K < 2^24): for every token m, sum_n Y[n, m] = sum_k (sum_n trit[n, k]) q[k, m], and for
    every row n, sum_m Y[n, m] = sum_k trit[n, k] (sum_m q[k, m]), in int64 on the host. A dropped or
    repeated k tile, row tile or token block changes one of the two."""
    import torch
    say(f"gemm unit-scale sums N={N} K={K} M={M}")
    wq, _, xq, _, rp, _, xi, _, rs = c3_case(ctx, orc, N, K, M, 77 + M + N)
    ones_n = torch.ones(N, dtype=torch.float32, device="cuda")
    ones_m = torch.ones(M, dtype=torch.float32, device="cuda")
    Y = host(ctx.ternary_matmul(rp, ones_n, xi, ones_m, rs, N, K, M)).astype(np.float64)
    assert np.array_equal(Y, np.rint(Y))
    t = orc.trits_of(wq, K).astype(np.int64)                                    # (N, K)
    q = xq.view(np.int8).reshape(K, -1)[:, :M].astype(np.int64)                # (K, M)
    col = t.sum(axis=0) @ q                                                     # (M,)
    row = t @ q.sum(axis=1)                                                     # (N,)
    assert np.array_equal(Y.sum(axis=0).astype(np.int64), col)
    assert np.array_equal(Y.sum(axis=1).astype(np.int64), row)


@pytest.mark.parametrize("tile", [1, 2, 3])
@pytest.mark.parametrize("N,K,M", [(300, 520, 200), (130, 300, 130), (64, 256, 17), (1000, 2560, 96),
                                   (4096, 4096, 256), (30000, 520, 300), (11008, 1024, 1024),
                                   (4100, 768, 2056)])
def test_prefill_gemm_each_tile(ctx, orc, tile, N, K, M):
    """Every block tile of the prefill GEMM (256x128, 128x128, 64x64) forced on shapes with
    tails in N, M and K, with a bias: bit-exact against the oracle (every row below 2e10
    multiply-adds, sampled rows above). (30000, 520, 300), (11008, 1024, 1024) and (4100, 768, 2056)
    run several block rounds, with and without the XCD-aware block order, odd k-tile counts and
    edge blocks."""
    say(f"gemm tile={tile} N={N} K={K} M={M}")
    tau, s, wq, xq, rp, xi, s_d, rs = fast_case(ctx, orc, N, K, M, 17 + N + M, outliers=True)
    b = normal((N,), 98)
    ctx.set_gemm_tile(tile)
    try:
        Y = host(ctx.ternary_matmul(rp, dev(tau), xi, s_d, rs, N, K, M, bias=dev(b)))
    finally:
        ctx.set_gemm_tile(0)
    rows = np.arange(N) if N * M * K <= 2e10 else np.unique(np.concatenate([np.arange(0, N, 61), [N - 1]]))
    ref = orc.add_row_broadcast(orc.matmul_q_i8_rowblock(wq[rows], tau[rows], xq, s, K, M), b[rows])
    assert np.array_equal(Y[rows], ref)


@pytest.mark.parametrize("N,K,M", [(4608, 768, 2048), (11008, 1024, 1024), (2560, 520, 4096), (4615, 520, 2000)])
def test_prefill_gemm_split_rows(ctx, orc, N, K, M):
    """Shapes on which the automatic tile choice splits the rows on a 256-CU device: 256 x 128
    blocks over the rows that fill whole rounds (4096, 8192, 2048 and 4096 rows here), the rest in
    a second launch of 64 x 64 (the first) or 128 x 128 blocks; (4615, 520, 2000) ends both
    launches' last blocks inside the tile (rows and tokens). Every row against the oracle, with a
    bias; the same bits
    as the 256 x 128 tile over all rows; and the residual epilogue (the rows' residual moves
    with them) the same bits as add(res, ternary_matmul)."""
    say(f"gemm split N={N} K={K} M={M}")
    tau, s, wq, xq, rp, xi, s_d, rs = fast_case(ctx, orc, N, K, M, 23 + N + M, outliers=True)
    b = normal((N,), 99)
    Y = host(ctx.ternary_matmul(rp, dev(tau), xi, s_d, rs, N, K, M, bias=dev(b)))
    ref = orc.add_row_broadcast(orc.matmul_q_i8_rowblock(wq, tau, xq, s, K, M), b)
    assert np.array_equal(Y, ref)
    ctx.set_gemm_tile(1)
    try:
        Y1 = host(ctx.ternary_matmul(rp, dev(tau), xi, s_d, rs, N, K, M, bias=dev(b)))
    finally:
        ctx.set_gemm_tile(0)
    assert np.array_equal(Y1.view(np.uint32), Y.view(np.uint32))
    res = normal((N, M), 100)
    Yr = host(ctx.ternary_matmul_add(rp, dev(tau), xi, s_d, rs, N, K, M, dev(res), bias=dev(b)))
    Yr_ref = host(ctx.add(dev(res), dev(Y)))
    assert np.array_equal(Yr.view(np.uint32), Yr_ref.view(np.uint32))


def test_gemm_tile_setter_rejects(ctx, nnhip):
    with pytest.raises(nnhip.NNHipError):
        ctx.set_gemm_tile(4)
    with pytest.raises(nnhip.NNHipError):
        ctx.set_gemm_tile(-1)


def test_grouped_gemv_matches_single(ctx, orc):
    say("grouped gemv")
    import torch
    shapes = [(2560, 2560), (640, 2560), (6912, 2560), (2560, 6912), (100, 300)]
    probs, singles = [], []
    for i, (N, K) in enumerate(shapes):
        tau, s, wq, xq, rp, xi, s_d, rs = fast_case(ctx, orc, N, K, 1 + (i % 2) * 15, 50 + i)
        M = 1 + (i % 2) * 15
        y = torch.empty((N, M), dtype=torch.float32, device="cuda")
        probs.append(dict(rp=rp, tau=dev(tau), xi=xi, s=s_d, rowsum=rs, bias=None, y=y, N=N, K=K, M=M))
        singles.append(host(ctx.ternary_matmul(rp, probs[-1]["tau"], xi, s_d, rs, N, K, M)))
    h = ctx.group_create(probs)
    for _ in range(3):
        ctx.group_run(h)
    ctx.sync()
    for p, ref in zip(probs, singles):
        assert np.array_equal(host(p["y"]), ref)
    ctx.group_destroy(h)


STACK_SHAPES = [("q", 2560, 2560), ("k", 2560, 640), ("v", 2560, 640), ("o", 2560, 2560),
                ("gate", 2560, 6912), ("up", 2560, 6912), ("down", 6912, 2560)]   # (name, K, N)


def stack_group(ctx, orc, layers, M, seed, bias_layer=-1, shapes=None):
    """A reduced-depth copy of bench.py's headline group: `layers` x the seven BitNet-2B shapes,
    weights N(0, 0.02) ternarized by per-tensor absmean on the GPU (trit_pack is checked bit for
    bit elsewhere; the oracle below reads the same containers), one quantized activation block
    per K shared by every problem of that K. Returns the problems and their host operands."""
    import torch
    gen = torch.Generator(device="cuda")
    acts = {}
    shapes = STACK_SHAPES if shapes is None else shapes
    for K in sorted({K for (_, K, _) in shapes}):
        X = normal((K, M), seed + K)
        xi, s_d, rs = ctx.act_quant_i8(dev(X))
        s = orc.act_scale(X)
        assert np.array_equal(host(s_d), s)
        acts[K] = (xi, s_d, rs, orc.quantize_i8(X, s, True), s)
    probs, hosts = [], []
    for layer in range(layers):
        for idx, (name, K, N) in enumerate(shapes):
            gen.manual_seed(seed * 131 + layer * 16 + idx)
            W = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
            tau = W.abs().double().mean().float().expand(N).contiguous()
            wq = ctx.trit_pack(W, tau)
            rp = ctx.repack(wq, K)
            del W
            xi, s_d, rs, xq, s = acts[K]
            b = normal((N,), seed + 7 * layer + idx) if layer == bias_layer else None
            y = torch.full((N, M), float("nan"), dtype=torch.float32, device="cuda")
            probs.append(dict(rp=rp, tau=tau, xi=xi, s=s_d, rowsum=rs, bias=dev(b) if b is not None else None,
                              y=y, N=N, K=K, M=M))
            hosts.append((host(wq, np.uint32), host(tau), xq, s, b, name, layer))
    return probs, hosts


def check_stack_group(ctx, orc, probs, hosts, expect_lds):
    h = ctx.group_create(probs)
    try:
        info = ctx.group_info(h)
        assert info["lds"] == expect_lds, info
        for _ in range(3):   # repeated runs rewrite the same bits
            ctx.group_run(h)
        ctx.sync()
    finally:
        ctx.group_destroy(h)
    for p, (wq, tau, xq, s, b, name, layer) in zip(probs, hosts):
        ref = orc.matmul_q_i8_rowblock(wq, tau, xq, s, p["K"], p["M"])
        if b is not None:
            ref = orc.add_row_broadcast(ref, b)
        Y = host(p["y"])
        assert np.array_equal(Y, ref), f"layer {layer} {name}: {int(np.sum(Y != ref))} of {Y.size} differ"


def test_grouped_gemv_headline_group_lds(ctx, orc):
    """The benchmarked launch: bench.py's M=1 layer-stack group (here 3 layers x q/k/v/o/gate/up/down,
    activations shared per K, so they fit the LDS budget and the LDS variant runs), every output row
    of every problem bit for bit against the oracle's CpuEngine restatement; layer 1 carries a bias.
    Mirrors the int32 + epilogue check of src/int8_act_test.cpp:210-236."""
    say("grouped gemv: headline group (LDS variant), 3 layers x 7 shapes, M=1")
    probs, hosts = stack_group(ctx, orc, 3, 1, 0xA1, bias_layer=1)
    check_stack_group(ctx, orc, probs, hosts, expect_lds=True)


def test_grouped_gemv_m16_group_lds(ctx, orc):
    """bench.py's M=16 sweep group (2 layers x 7 shapes): its two activation blocks (40 KB at
    K=2560, 110 KB at K=6912) are staged together by 16-wave blocks (one per CU), token rows
    XOR-swizzled; every row of every problem bit for bit against the oracle."""
    say("grouped gemv: M=16 group (one LDS launch of 16-wave blocks), 2 layers x 7 shapes")
    probs, hosts = stack_group(ctx, orc, 2, 16, 0xA2, bias_layer=0)
    check_stack_group(ctx, orc, probs, hosts, expect_lds=True)


def test_grouped_gemv_split_lds_launches(ctx, orc):
    """Activation blocks over the 16-wave budget together (K=2560 and two K=6912 blocks at M=16:
    261 KB): a launch of 4-wave blocks for the 40 KB block and one of 16-wave blocks for each
    110 KB block, every problem against the oracle."""
    say("grouped gemv: three LDS launches (M=16)")
    p1, h1 = stack_group(ctx, orc, 1, 16, 0xA5, bias_layer=0)
    p2, h2 = stack_group(ctx, orc, 1, 16, 0xA6, shapes=[("down2", 6912, 1000)])
    check_stack_group(ctx, orc, p1 + p2, h1 + h2, expect_lds=True)


@pytest.mark.parametrize("M", [16, 9, 2])
def test_grouped_gemv_lds_swizzle_tokens(ctx, orc, M):
    """The LDS variant with M tokens (rows staged with the unit swizzle u ^ (t & 7)): the K=2560
    shapes of one layer share one activation block that fits the budget, every problem against
    the oracle."""
    say(f"grouped gemv: LDS variant at M={M}")
    probs, hosts = stack_group(ctx, orc, 1, M, 0xA3 + M, bias_layer=0)
    keep = [i for i, p in enumerate(probs) if p["K"] == 2560]
    check_stack_group(ctx, orc, [probs[i] for i in keep], [hosts[i] for i in keep], expect_lds=True)


def test_grouped_gemv_mixed_register(ctx, orc):
    """An activation block over the 16-wave LDS budget (K=10240 at M=16: 160 KB) runs the register
    variant in a launch of its own, beside an LDS launch for the K=2560 problems."""
    say("grouped gemv: LDS + register launches (K=2560 and K=10240, M=16)")
    shapes = [("a", 2560, 2560), ("b", 10240, 700), ("c", 2560, 640), ("d", 10240, 2560)]
    probs, hosts = stack_group(ctx, orc, 1, 16, 0xA4, bias_layer=0, shapes=shapes)
    check_stack_group(ctx, orc, probs, hosts, expect_lds="mixed")
    keep = [i for i, p in enumerate(probs) if p["K"] == 10240]
    check_stack_group(ctx, orc, [probs[i] for i in keep], [hosts[i] for i in keep], expect_lds=False)


def test_invalid_arguments_raise(ctx, nnhip):
    import torch
    rp = torch.zeros(64, dtype=torch.int32, device="cuda")
    x = torch.zeros((1, 256), dtype=torch.int8, device="cuda")
    f = torch.zeros(16, dtype=torch.float32, device="cuda")
    i = torch.zeros(16, dtype=torch.int32, device="cuda")
    with pytest.raises(nnhip.NNHipError):   # K = 0
        ctx.ternary_matmul(rp, f, x, f, i, 16, 0, 1)
    with pytest.raises(nnhip.NNHipError):   # K beyond the int32 accumulator bound
        ctx.ternary_matmul(rp, f, x, f, i, 16, 300000, 1)
    with pytest.raises(nnhip.NNHipError):   # misaligned xi
        bad = torch.zeros(300, dtype=torch.int8, device="cuda")[1:257].view(1, 256)
        ctx.ternary_matmul(rp, f, bad, f, i, 16, 256, 1)


# ------------------------------------------------------------------ float-activation GEMM (a10)

GEMM_SHAPES = [(64, 16, 64), (128, 32, 64), (64, 32, 128), (192, 48, 320), (65, 17, 65),
               (129, 33, 7), (256, 40, 1), (9, 100, 3), (130, 16, 130)]


def check_gemm_shape(ctx, orc, M, K, N, trans_a, f16):
    """src/ternary_gemm_test.cpp:435-526: A latent 0.17*((r*7 + c*3) % 13) - 0.9 stored (M, K)
    (or (K, M) for transA), tau per stored row absmean, B 0.21*((k + 2n) % 9) - 0.8; the
    f16 mode rounds B and the reference to f16. Tolerance 1e-4 / 4e-3 x max(1, max|ref|)."""
    import torch
    sr, al = (K, M) if trans_a else (M, K)
    r = np.arange(sr)[:, None]
    c = np.arange(al)[None, :]
    A = (np.float32(0.17) * ((r * 7 + c * 3) % 13).astype(np.float32) - np.float32(0.9)).astype(np.float32)
    tau = np.abs(A.astype(np.float64)).mean(axis=1).astype(np.float32)
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    B = (np.float32(0.21) * ((k + 2 * n) % 9).astype(np.float32) - np.float32(0.8)).astype(np.float32)
    if f16:
        B = B.astype(np.float16).astype(np.float32)
    packed = ctx.trit_pack(dev(A), dev(tau))
    assert np.array_equal(host(packed, np.uint32), orc.trit_pack(A, tau))
    Bd = dev(B).to(torch.float16) if f16 else dev(B)
    if trans_a:
        got = ctx.matmul_q_t(packed, dev(tau), Bd, M, out_f16=f16)
        ref = orc.matmul_q_t(host(packed, np.uint32), tau, B, M)
    else:
        got = ctx.matmul_q(packed, dev(tau), Bd, K, out_f16=f16)
        ref = orc.matmul_q(host(packed, np.uint32), tau, B, K)
    if f16:
        ref = ref.astype(np.float16).astype(np.float32)
    g = got.float().cpu().numpy()
    assert g.shape == (M, N)
    scale = max(1.0, float(np.max(np.abs(ref))))
    err = float(np.max(np.abs(g.astype(np.float64) - ref.astype(np.float64))))
    assert err <= (4e-3 if f16 else 1e-4) * scale, (M, K, N, trans_a, f16, err)


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
@pytest.mark.parametrize("trans_a", [False, True])
@pytest.mark.parametrize("f16", [False, True])
def test_matmul_q_shapes(ctx, orc, M, K, N, trans_a, f16):
    say(f"matmul_q M={M} K={K} N={N} transA={trans_a} f16={f16}")
    check_gemm_shape(ctx, orc, M, K, N, trans_a, f16)


@pytest.mark.parametrize("M,K,N", [(2048, 2560, 64), (2560, 2048, 64)])
@pytest.mark.parametrize("trans_a", [False, True])
def test_matmul_q_large(ctx, orc, M, K, N, trans_a):
    say(f"matmul_q large M={M} K={K} N={N} transA={trans_a}")
    check_gemm_shape(ctx, orc, M, K, N, trans_a, False)


def test_matmul_q_decode_gaussian(ctx, orc):
    """The decode shape of the default BitLinear branch: N(0, 0.02) weights with per-tensor
    absmean, one f32 token."""
    N, K = 2560, 6912
    W = normal((N, K), 21, 0.0, 0.02)
    tau = np.full(N, np.abs(W.astype(np.float64)).mean(), np.float32)
    X = normal((K, 1), 22, 0.0, 1.0)
    wq = ctx.trit_pack(dev(W), dev(tau))
    got = host(ctx.matmul_q(wq, dev(tau), dev(X), K))
    ref = orc.matmul_q(host(wq, np.uint32), tau, X, K)
    assert np.max(np.abs(got - ref)) <= 1e-4 * max(1.0, np.max(np.abs(ref)))


@pytest.mark.parametrize("nbytes", [4, 12, 16, 20, 4096, 1000004, (64 << 20) + 12])
def test_stream_xor(ctx, nbytes):
    """nnhip_stream_xor: out ^= xor of all words (any word count, the 16-byte body and the
    tail); a second call cancels the first."""
    import torch
    print(f"stream_xor bytes={nbytes}", flush=True)
    words = np.random.default_rng(nbytes).integers(0, 2 ** 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src = dev(words)
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx.stream_xor(src, out)
    got = int(out.cpu().numpy().view(np.uint32)[0])
    assert got == int(np.bitwise_xor.reduce(words))
    ctx.stream_xor(src, out)
    assert int(out.cpu().numpy().view(np.uint32)[0]) == 0

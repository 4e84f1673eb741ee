"""GPU parity of the float-activation product on the MFMA path (nnhip_ternary_matmul_f): f32 /
f16 activations split into four int8 digits of a per-token 31-bit fixed point, ternary x int8
products, int64 combine. Checked against the oracle's float64 evaluation of
(tau o trit) . B (src/ternary_gemm_test.cpp:141-170): within 2e-6 x max(1, max|ref|) (f32 out;
the reference itself allows 1e-4) and, for f16 outputs, within the reference's 4e-3; NaN and
infinity patterns exactly.

Reference: ComputeEngine::matmul_q on the BitLinear f32 branch
(include/neuralnet.cpp/compute_layer_bitlinear.hpp:459-466).
"""
import numpy as np
import pytest

from conftest import normal, uniform

pytestmark = pytest.mark.gpu

TOL = 2e-6


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t):
    return t.float().cpu().numpy()


def say(msg):
    print(msg, flush=True)


def case(ctx, orc, N, K, W=None, seed=0):
    if W is None:
        W = normal((N, K), seed, 0.0, 0.02)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    wq = orc.trit_pack(W, tau)
    rp = ctx.repack(dev(wq), K)
    return wq, tau, rp


def check(got, ref, tol):
    scale = max(1.0, float(np.nanmax(np.abs(np.where(np.isfinite(ref), ref, 0)))))
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN pattern differs"
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], ref[inf]), "infinities differ"
    fin = np.isfinite(ref)
    err = float(np.max(np.abs(got[fin].astype(np.float64) - ref[fin].astype(np.float64)))) if fin.any() else 0.0
    assert err <= tol * scale, err


@pytest.mark.parametrize("N,K,M", [(2560, 6912, 1), (2560, 2560, 4), (6912, 2560, 16), (640, 2560, 7),
                                   (100, 520, 3), (65, 17, 65), (300, 1000, 40), (2560, 4096, 2)])
def test_matmul_f_gaussian(ctx, orc, N, K, M):
    say(f"ternary_matmul_f N={N} K={K} M={M}")
    wq, tau, rp = case(ctx, orc, N, K, seed=N + K + M)
    X = normal((K, M), 7 + M)
    X[:, ::3] *= 37.0  # tokens of different magnitudes
    got = host(ctx.ternary_matmul_f(rp, dev(tau), dev(X), N, K))
    check(got, orc.matmul_q(wq, tau, X, K), TOL)


def test_matmul_f_reference_pattern(ctx, orc):
    """src/ternary_gemm_test.cpp:435-526 patterns (the int8 digits see exact 0.21 * j - 0.8 values)."""
    M, K, N = 192, 48, 320    # rows, reduction, tokens
    r = np.arange(M)[:, None]
    c = np.arange(K)[None, :]
    A = (np.float32(0.17) * ((r * 7 + c * 3) % 13).astype(np.float32) - np.float32(0.9)).astype(np.float32)
    wq, tau, rp = case(ctx, orc, M, K, W=A)
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    B = (np.float32(0.21) * ((k + 2 * n) % 9).astype(np.float32) - np.float32(0.8)).astype(np.float32)
    got = host(ctx.ternary_matmul_f(rp, dev(tau), dev(B), M, K))
    check(got, orc.matmul_q(wq, tau, B, K), TOL)


@pytest.mark.parametrize("b16,y16", [(True, False), (False, True), (True, True)])
def test_matmul_f_half(ctx, orc, b16, y16):
    import torch
    N, K, M = 1000, 2560, 5
    say(f"ternary_matmul_f f16 in={b16} out={y16}")
    wq, tau, rp = case(ctx, orc, N, K, seed=3)
    X = normal((K, M), 4)
    if b16:
        X = X.astype(np.float16).astype(np.float32)
    Xd = dev(X).to(torch.float16) if b16 else dev(X)
    got = host(ctx.ternary_matmul_f(rp, dev(tau), Xd, N, K, out_f16=y16))
    ref = orc.matmul_q(wq, tau, X, K)
    if y16:
        ref = ref.astype(np.float16).astype(np.float32)
    check(got, ref, 4e-3 if y16 else TOL)


def test_matmul_f_special_values(ctx, orc):
    """NaN and infinities give the IEEE result of the reference's per-term products; zero,
    subnormal-only and very wide tokens stay within tolerance."""
    N, K, M = 300, 1000, 8
    say("ternary_matmul_f special values")
    W = normal((N, K), 5, 0.0, 0.02)
    W[:, 10] = 0.0          # trit 0 at k = 10 for every row
    W[::2, 20] = 1.0        # +1 at k = 20 for even rows
    W[1::2, 20] = -1.0      # -1 for odd rows
    wq, tau, rp = case(ctx, orc, N, K, W=W)
    X = normal((K, M), 6)
    X[33, 0] = np.nan                       # token 0: NaN everywhere
    X[20, 1] = np.inf                       # token 1: +inf on a +-1 column -> +inf / -inf rows
    X[10, 2] = -np.inf                      # token 2: inf on a 0 column -> NaN
    X[20, 3] = np.inf                       # token 3: +inf and -inf on the same column sign
    X[21, 3] = -np.inf
    X[:, 4] = 0.0                           # token 4: zeros
    X[:, 5] = normal((K,), 7) * np.float32(1e-41)   # token 5: subnormals only
    X[:, 6] = normal((K,), 8) * np.float32(1e-30)
    X[5, 6] = np.float32(3e38)              # token 6: enormous range
    X[:, 7] = normal((K,), 9) * np.float32(1e30)
    got = host(ctx.ternary_matmul_f(rp, dev(tau), dev(X), N, K))
    ref = orc.matmul_q(wq, tau, X, K)
    for m in range(M):
        check(got[:, m:m + 1], ref[:, m:m + 1], TOL)
    assert np.all(np.isnan(got[:, 0])) and np.all(np.isnan(got[:, 2]))
    assert np.all(got[::2, 1] == np.inf) and np.all(got[1::2, 1] == -np.inf)


def test_matmul_f_agrees_with_valu_kernel(ctx, orc):
    """The MFMA path and the reference-layout VALU kernel (nnhip_matmul_q) on the same inputs."""
    N, K, M = 2560, 2560, 16
    wq, tau, rp = case(ctx, orc, N, K, seed=11)
    X = normal((K, M), 12)
    a = host(ctx.ternary_matmul_f(rp, dev(tau), dev(X), N, K))
    b = host(ctx.matmul_q(dev(wq), dev(tau), dev(X), K))
    assert np.max(np.abs(a - b)) <= 1e-4 * max(1.0, float(np.max(np.abs(b))))


def test_matmul_f_rejects_large_k(ctx, nnhip):
    import torch
    rp = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    tau = torch.ones(16, device="cuda")
    B = torch.zeros((131072, 1), device="cuda")
    with pytest.raises(nnhip.NNHipError):
        ctx.ternary_matmul_f(rp, tau, B, 16, 131072)


def transposed_case(ctx, orc, K, M, seed):
    """A container (K, ceil(M/16)) with tau per stored row (BitLinear's W with K = out features,
    M = in features), its bit transpose and the repack of that."""
    W = normal((K, M), seed, 0.0, 0.02)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    A = orc.trit_pack(W, tau)
    At = ctx.trit_transpose(dev(A), M)
    rpT = ctx.repack(At, K)
    return A, tau, At, rpT


@pytest.mark.parametrize("K,M", [(1, 1), (17, 65), (48, 192), (2560, 6912), (300, 33)])
def test_trit_transpose_bits(ctx, orc, K, M):
    """trit (m, k) of the transpose = trit (k, m) of the container; tail codes 2 (trit 0)."""
    say(f"trit_transpose K={K} M={M}")
    W = normal((K, M), K + M, 0.0, 0.02)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    A = orc.trit_pack(W, tau)
    At = ctx.trit_transpose(dev(A), M).cpu().numpy().view(np.uint32)
    assert At.shape == (M, (K + 15) // 16)
    codes = lambda P: ((P[:, :, None] >> (2 * np.arange(16, dtype=np.uint32))) & 3).reshape(P.shape[0], -1)
    ca = codes(A)[:, :M]
    ct = codes(At)
    assert np.array_equal(ct[:, :K], ca.T)
    assert np.all(ct[:, K:] == 2)


@pytest.mark.parametrize("K,M,N", [(2560, 6912, 16), (6912, 2560, 4), (2560, 2560, 1), (640, 2560, 7),
                                   (520, 100, 3), (17, 65, 65), (1000, 300, 40)])
def test_matmul_t_f_gaussian(ctx, orc, K, M, N):
    """dX = (tau o trit(W))^T . dY on the transposed repack (src/ternary_gemm_test.cpp:291-334)."""
    say(f"ternary_matmul_t_f K={K} M={M} N={N}")
    A, tau, _, rpT = transposed_case(ctx, orc, K, M, seed=K + M + N)
    B = normal((K, N), 3 + N)
    B[:, ::3] *= 41.0
    got = host(ctx.ternary_matmul_t_f(rpT, dev(tau), dev(B), M))
    check(got, orc.matmul_q_t(A, tau, B, M), TOL)


def test_matmul_t_f_reference_pattern(ctx, orc):
    """src/ternary_gemm_test.cpp:435-526 patterns with transA (A stored (K, M))."""
    M, K, N = 192, 48, 320
    r = np.arange(K)[:, None]
    c = np.arange(M)[None, :]
    W = (np.float32(0.17) * ((r * 7 + c * 3) % 13).astype(np.float32) - np.float32(0.9)).astype(np.float32)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    A = orc.trit_pack(W, tau)
    rpT = ctx.repack(ctx.trit_transpose(dev(A), M), K)
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    B = (np.float32(0.21) * ((k + 2 * n) % 9).astype(np.float32) - np.float32(0.8)).astype(np.float32)
    got = host(ctx.ternary_matmul_t_f(rpT, dev(tau), dev(B), M))
    check(got, orc.matmul_q_t(A, tau, B, M), TOL)


def test_matmul_t_f_half_and_specials(ctx, orc):
    """f16 activations / outputs, and the IEEE path for non-finite tokens with tau folded in."""
    import torch
    K, M, N = 700, 300, 6
    say("ternary_matmul_t_f f16 and special values")
    W = normal((K, M), 21, 0.0, 0.02)
    W[20, ::2] = 1.0
    W[20, 1::2] = -1.0
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    A = orc.trit_pack(W, tau)
    tau[10] = 0.0                             # stored row 10 scaled by 0: 0 x inf -> NaN
    rpT = ctx.repack(ctx.trit_transpose(dev(A), M), K)
    B = normal((K, N), 22)
    B[33, 0] = np.nan
    B[20, 1] = np.inf                         # +-1 column -> +-inf per output row
    B[10, 2] = -np.inf                        # tau 0 -> NaN for every output row
    B[:, 3] = 0.0
    B[:, 4] *= np.float32(1e30)
    got = host(ctx.ternary_matmul_t_f(rpT, dev(tau), dev(B), M))
    ref = orc.matmul_q_t(A, tau, B, M)
    for n in range(N):
        check(got[:, n:n + 1], ref[:, n:n + 1], TOL)
    Bh = B[:, [3, 5]].astype(np.float16).astype(np.float32)
    got = host(ctx.ternary_matmul_t_f(rpT, dev(tau), dev(Bh).to(torch.float16), M, out_f16=True))
    ref = orc.matmul_q_t(A, tau, Bh, M).astype(np.float16).astype(np.float32)
    check(got, ref, 4e-3)


def test_matmul_t_f_agrees_with_valu_kernel(ctx, orc):
    """MFMA transposed path vs the reference-layout VALU kernel (nnhip_matmul_q_t)."""
    K, M, N = 2560, 2560, 16
    A, tau, _, rpT = transposed_case(ctx, orc, K, M, seed=31)
    B = normal((K, N), 32)
    a = host(ctx.ternary_matmul_t_f(rpT, dev(tau), dev(B), M))
    b = host(ctx.matmul_q_t(dev(A), dev(tau), dev(B), M))
    assert np.max(np.abs(a - b)) <= 1e-4 * max(1.0, float(np.max(np.abs(b))))


def digit_model(trits, X, tau=None, kscale=None):
    """The digit-split product bit for bit, for finite tokens: x (times kscale[k] in f32 when
    given), E = the exponent of max|x| (max < 2^E), X = rint(x 2^(30 - E)) (exact in f32),
    T = sum_k trit X in int64 (the four digit products recombined), y = tau_n * (f32(T) 2^(E - 30))
    in f32. trits (N, K), X (K, M) f32 -> (N, M) f32."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    if kscale is not None:
        X = (kscale.astype(np.float32)[:, None] * X).astype(np.float32)
    t64 = trits.astype(np.int64)
    Y = np.empty((trits.shape[0], X.shape[1]), np.float32)
    for m in range(X.shape[1]):
        col = X[:, m]
        _, E = np.frexp(np.max(np.abs(col)))
        Xi = np.rint(np.ldexp(col, 30 - int(E))).astype(np.int64)
        y = np.ldexp((t64 @ Xi).astype(np.float32), int(E) - 30).astype(np.float32)
        Y[:, m] = y if tau is None else (tau.astype(np.float32) * y).astype(np.float32)
    return Y


def misaligned(t):
    """A copy of t whose data pointer is 4 bytes past a 16-byte boundary: the digit-split product
    then runs as three launches (digits, int8 GEMV on the digit tokens, combine) instead of one."""
    import torch
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


def same_bits(a, b):
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(
        a[~np.isnan(a)].view(np.uint32) if a.dtype == np.float32 else a[~np.isnan(a)],
        b[~np.isnan(b)].view(np.uint32) if b.dtype == np.float32 else b[~np.isnan(b)])


@pytest.mark.parametrize("N,K,M", [(2560, 2560, 1), (6912, 2560, 1), (2560, 6912, 1), (2560, 6912, 2),
                                   (2560, 2560, 3), (2560, 2560, 4), (1000, 4096, 4), (3000, 8192, 1),
                                   (37, 1000, 2), (16, 1024, 1)])
def test_matmul_f_one_launch_bits(ctx, orc, N, K, M):
    """Decode sizes (M <= 4 tokens) run the digit split, the MFMAs and the int64 combine in one
    launch: its outputs equal the three-launch path's and the exact digit model's bit for bit."""
    say(f"ternary_matmul_f one launch N={N} K={K} M={M}")
    wq, tau, rp = case(ctx, orc, N, K, seed=N + 3 * K + M)
    X = normal((K, M), 40 + M)
    X[:, ::2] *= 29.0
    Xd = dev(X)
    assert Xd.data_ptr() % 16 == 0
    one = host(ctx.ternary_matmul_f(rp, dev(tau), Xd, N, K))
    three = host(ctx.ternary_matmul_f(rp, dev(tau), misaligned(Xd), N, K))
    assert same_bits(one, three)
    assert same_bits(one, digit_model(orc.trits_of(wq, K), X, tau=tau))
    one16 = ctx.ternary_matmul_f(rp, dev(tau), Xd, N, K, out_f16=True).cpu().numpy()
    assert np.array_equal(one16.view(np.uint16), one.astype(np.float16).view(np.uint16))


def test_matmul_f_one_launch_specials(ctx, orc):
    """Non-finite and zero tokens in the one-launch kernel: the same IEEE results as the three
    launches, and finite tokens beside them unaffected."""
    N, K, M = 300, 2560, 4
    W = normal((N, K), 51, 0.0, 0.02)
    W[::2, 20] = 1.0
    W[1::2, 20] = -1.0
    W[:, 10] = 0.0
    wq, tau, rp = case(ctx, orc, N, K, W=W)
    X = normal((K, M), 52)
    X[20, 0] = np.inf       # +-1 column -> +-inf rows
    X[10, 1] = -np.inf      # 0 column -> NaN
    X[:, 2] = 0.0
    Xd = dev(X)
    one = host(ctx.ternary_matmul_f(rp, dev(tau), Xd, N, K))
    three = host(ctx.ternary_matmul_f(rp, dev(tau), misaligned(Xd), N, K))
    assert same_bits(one, three)
    assert np.all(one[::2, 0] == np.inf) and np.all(one[1::2, 0] == -np.inf) and np.all(np.isnan(one[:, 1]))
    assert np.all(one[:, 2] == 0.0)
    assert same_bits(one[:, 3:], digit_model(orc.trits_of(wq, K), X[:, 3:], tau=tau))


@pytest.mark.parametrize("K,M,N", [(2560, 2560, 1), (2560, 6912, 2), (1000, 300, 4), (6912, 2560, 1)])
def test_matmul_t_f_one_launch_bits(ctx, orc, K, M, N):
    """The transposed product (tau folded into the digit split per k) in one launch, against the
    three launches and the digit model on the transposed trits."""
    say(f"ternary_matmul_t_f one launch K={K} M={M} N={N}")
    A, tau, At, rpT = transposed_case(ctx, orc, K, M, seed=K + M + 5 * N)
    B = normal((K, N), 60 + N)
    Bd = dev(B)
    one = host(ctx.ternary_matmul_t_f(rpT, dev(tau), Bd, M))
    three = host(ctx.ternary_matmul_t_f(rpT, dev(tau), misaligned(Bd), M))
    assert same_bits(one, three)
    trT = orc.trits_of(At.cpu().numpy().view(np.uint32), K)
    assert same_bits(one, digit_model(trT, B, kscale=tau))


@pytest.mark.parametrize("N,K,M", [(640, 12000, 3), (1000, 8192, 2), (2048, 7000, 4), (48, 30000, 1)])
def test_matmul_f_split_k_bits(ctx, orc, N, K, M):
    """A few long tokens over few rows (M <= 4, K >= 6144, at most 2048 row tiles, beyond the
    one-launch kernel's shapes) run split-k: digits in column chunks, int32 slice sums, and a
    combine adding both; bit for bit the exact digit model, and within the f32 tolerance of the
    oracle's float64 product."""
    say(f"ternary_matmul_f split-k N={N} K={K} M={M}")
    wq, tau, rp = case(ctx, orc, N, K, seed=N + K + M)
    X = normal((K, M), 70 + M)
    X[::3, :] *= 17.0
    got = host(ctx.ternary_matmul_f(rp, dev(tau), dev(X), N, K))
    assert same_bits(got, digit_model(orc.trits_of(wq, K), X, tau=tau))
    check(got, orc.matmul_q(wq, tau, X, K), TOL)


def test_matmul_t_f_split_k_long_reduction(ctx, orc):
    """The dX product with a long reduction (16384 k over 1024 outputs, one token), on the split-k
    path: bit for bit the digit model on the transposed trits with tau folded per k."""
    K, M, N = 16384, 1024, 1
    say(f"ternary_matmul_t_f split-k K={K} M={M} N={N}")
    A, tau, At, rpT = transposed_case(ctx, orc, K, M, seed=77)
    B = normal((K, N), 78)
    got = host(ctx.ternary_matmul_t_f(rpT, dev(tau), dev(B), M))
    trT = orc.trits_of(At.cpu().numpy().view(np.uint32), K)
    assert same_bits(got, digit_model(trT, B, kscale=tau))


def test_matmul_f_split_k_specials(ctx, orc):
    """Non-finite and zero tokens on the split-k path: the IEEE results of the exact path, and the
    finite token beside them the digit model's bits."""
    N, K, M = 300, 9000, 4
    W = normal((N, K), 81, 0.0, 0.02)
    W[::2, 20] = 1.0
    W[1::2, 20] = -1.0
    W[:, 10] = 0.0
    wq, tau, rp = case(ctx, orc, N, K, W=W)
    X = normal((K, M), 82)
    X[20, 0] = np.inf
    X[10, 1] = -np.inf
    X[:, 2] = 0.0
    got = host(ctx.ternary_matmul_f(rp, dev(tau), dev(X), N, K))
    assert np.all(got[::2, 0] == np.inf) and np.all(got[1::2, 0] == -np.inf) and np.all(np.isnan(got[:, 1]))
    assert np.all(got[:, 2] == 0.0)
    assert same_bits(got[:, 3:], digit_model(orc.trits_of(wq, K), X[:, 3:], tau=tau))

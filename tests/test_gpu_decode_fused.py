"""GPU parity of the fused decode-step entry points: the split-k partial GEMV
(nnhip_ternary_matmul_partial) and its epilogue + residual + quantizer kernel
(nnhip_partial_residual_quant_i8), bit for bit against the oracle's integer accumulators and
against the unfused GPU sequence (nnhip_ternary_matmul_add, then nnhip_rmsnorm_quant_i8 /
nnhip_act_quant_i8), whose own parity with the oracle the other GPU tests establish.
"""
import numpy as np
import pytest

from conftest import normal

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def host(t):
    return t.cpu().numpy()


def say(msg):
    print(msg, flush=True)


def case(ctx, orc, N, K, M, seed):
    W = normal((N, K), seed, 0.0, 0.02)
    tau = np.full(N, np.abs(W.astype(np.float64)).mean(), np.float32)
    X = normal((K, M), seed + 1)
    s = orc.act_scale(X)
    wq = orc.trit_pack(W, tau)
    xq = orc.quantize_i8(X, s, True)
    rp = ctx.repack(dev(wq), K)
    xi, s_d, rs = ctx.act_quant_i8(dev(X))
    assert np.array_equal(host(s_d), s)
    return tau, wq, xq, rp, xi, s_d, rs


@pytest.mark.parametrize("N,K,M,slices", [
    (2560, 2560, 16, 4), (2560, 6912, 16, 4), (2560, 6912, 16, 7), (2560, 2560, 16, 2),
    (3840, 2560, 16, 1), (100, 1024, 3, 4), (2561, 6900, 5, 3), (17, 4096, 16, 8), (33, 256, 1, 1),
    (640, 3584, 13, 7),
])
def test_matmul_partial_sums(ctx, orc, N, K, M, slices):
    """sum over the slices of part - 2 rowsum = the oracle's integer accumulator trit . xq."""
    say(f"partial N={N} K={K} M={M} slices={slices}")
    tau, wq, xq, rp, xi, s_d, rs = case(ctx, orc, N, K, M, N + K + M + slices)
    part = host(ctx.ternary_matmul_partial(rp, xi, N, K, M, slices)).astype(np.int64)
    assert part.shape == (slices, M, N)
    total = part.sum(axis=0) - 2 * host(rs).astype(np.int64)[:, None]       # (M, N)
    ref = orc.matmul_q_i8_acc(wq, xq, K, M).astype(np.int64)                  # (N, M)
    assert np.array_equal(total.T, ref)


@pytest.mark.parametrize("N,K,M,slices,bias,res,norm", [
    (2560, 2560, 16, 4, False, True, True),    # C5 w_o: + residual, RMSNorm2
    (2560, 6912, 16, 4, False, True, True),    # C5 fc2: + residual, next block's RMSNorm1
    (2560, 6912, 16, 4, True, True, False),    # bias, plain absmax
    (1000, 2560, 7, 2, True, False, True),     # no residual
    (2561, 6900, 5, 3, False, True, False),
    (6912, 2560, 16, 4, False, False, True),   # K of the next BitLinear = 6912 (14 rounds)
])
def test_partial_residual_quant_equals_unfused(ctx, orc, N, K, M, slices, bias, res, norm):
    say(f"epilogue N={N} K={K} M={M} slices={slices} bias={bias} res={res} norm={norm}")
    import torch
    tau, wq, xq, rp, xi, s_d, rs = case(ctx, orc, N, K, M, 3 * N + K + M)
    b = dev(normal((N,), 7)) if bias else None
    r = dev(normal((N, M), 8)) if res else None
    gamma = dev(1.0 + 0.1 * normal((N,), 9)) if norm else None
    eps = 1e-5
    part = ctx.ternary_matmul_partial(rp, xi, N, K, M, slices)
    x_out = torch.empty((N, M), dtype=torch.float32, device="cuda")
    xi2, s2, rs2 = ctx.partial_residual_quant_i8(part, dev(tau), s_d, rs, N, M, x_out, res=r, bias=b,
                                                 gamma=gamma, eps=eps)
    zero = torch.zeros((N, M), dtype=torch.float32, device="cuda")
    Y = ctx.ternary_matmul_add(rp, dev(tau), xi, s_d, rs, N, K, M, r if res else zero, bias=b)
    assert np.array_equal(host(x_out).view(np.uint32), host(Y).view(np.uint32))
    ref = ctx.rmsnorm_quant_i8(Y, gamma, eps) if norm else ctx.act_quant_i8(Y)
    assert np.array_equal(host(xi2), host(ref[0]))
    assert np.array_equal(host(s2).view(np.uint32), host(ref[1]).view(np.uint32))
    assert np.array_equal(host(rs2), host(ref[2]))


def test_partial_residual_in_place(ctx, orc):
    """x_out aliasing res: the decoder's residual stream updated in place."""
    import torch
    N, K, M, slices = 2560, 2560, 16, 4
    tau, wq, xq, rp, xi, s_d, rs = case(ctx, orc, N, K, M, 77)
    x0 = normal((N, M), 78)
    x = dev(x0)
    part = ctx.ternary_matmul_partial(rp, xi, N, K, M, slices)
    ctx.partial_residual_quant_i8(part, dev(tau), s_d, rs, N, M, x, res=x, gamma=dev(np.ones(N, np.float32)), eps=1e-5)
    Y = ctx.ternary_matmul_add(rp, dev(tau), xi, s_d, rs, N, K, M, dev(x0))
    assert np.array_equal(host(x).view(np.uint32), host(Y).view(np.uint32))


def test_partial_rejects(ctx, nnhip):
    import torch
    xi = torch.zeros((16, 512), dtype=torch.int8, device="cuda")
    rp = torch.zeros(4096, dtype=torch.int32, device="cuda")
    with pytest.raises(nnhip.NNHipError):
        ctx.ternary_matmul_partial(rp, xi, 64, 512, 16, 9)    # slices > 8
    with pytest.raises(nnhip.NNHipError):
        ctx.ternary_matmul_partial(rp, xi, 64, 512, 16, 3)    # 2 k tiles: a slice would be empty
    with pytest.raises(nnhip.NNHipError):
        ctx.ternary_matmul_partial(rp, xi, 64, 512, 17, 1)    # M > 16
    xi27 = torch.zeros((16, 6912), dtype=torch.int8, device="cuda")
    rp27 = torch.zeros(64 * 27 * 256, dtype=torch.int32, device="cuda")
    with pytest.raises(nnhip.NNHipError):
        ctx.ternary_matmul_partial(rp27, xi27, 64, 6912, 16, 8)  # 27 k tiles in 8 slices of 4: the last is empty
    part = torch.zeros((1, 65, 8), dtype=torch.int32, device="cuda")
    f = torch.zeros(8, dtype=torch.float32, device="cuda")
    i = torch.zeros(65, dtype=torch.int32, device="cuda")
    x = torch.zeros((8, 65), dtype=torch.float32, device="cuda")
    with pytest.raises(nnhip.NNHipError):                       # M > 64
        ctx.partial_residual_quant_i8(part, f, torch.zeros(65, device="cuda"), i, 8, 65, x)



# ---------------------------------------------------------------- token-major FFN intermediate

@pytest.mark.parametrize("M,act,bias", [(16, 0, True), (1, 1, False), (7, 0, False)])
def test_glu_tokens_equals_glu(ctx, orc, M, act, bias):
    """nnhip_ternary_matmul_glu_tokens: h token-major (M, F), the transpose of
    nnhip_ternary_matmul_glu's (F, M) bit for bit (C5's fc1: d=2560, F=6912)."""
    say(f"glu tokens M={M} act={act} bias={bias}")
    K, F = 2560, 6912
    W = normal((2 * F, K), 61 + M, 0.0, 0.02)
    tau = np.abs(W.astype(np.float64)).mean(axis=1).astype(np.float32)
    wq = orc.trit_pack(W, tau)
    b = dev(normal((2 * F,), 62)) if bias else None
    wqi, taui, bi = ctx.glu_interleave(dev(wq), dev(tau), b, F, K)
    rp = ctx.repack(wqi, K)
    xi, s_d, rs = ctx.act_quant_i8(dev(normal((K, M), 63 + M)))
    h = host(ctx.ternary_matmul_glu(rp, taui, xi, s_d, rs, F, K, M, act=act, bias=bi))
    ht = host(ctx.ternary_matmul_glu_tokens(rp, taui, xi, s_d, rs, F, K, M, act=act, bias=bi))
    assert ht.shape == (M, F)
    assert np.array_equal(np.ascontiguousarray(ht.T).view(np.uint32), h.view(np.uint32))


@pytest.mark.parametrize("K,M,norm", [(6912, 16, True), (6912, 16, False), (2560, 1, True), (1000, 64, True),
                                      (11264, 5, False), (300, 3, True)])
def test_quant_tokens_equals_quant(ctx, orc, K, M, norm):
    """nnhip_rmsnorm_quant_i8_tokens on X (M, K) token-major: the codes, scales and row sums of
    nnhip_rmsnorm_quant_i8 / nnhip_act_quant_i8 on X transposed, bit for bit."""
    say(f"quant tokens K={K} M={M} norm={norm}")
    X = normal((K, M), 71 + K + M) * np.float32(4.0)
    X[3, 0] = np.float32(1e-3)
    gamma = dev(1.0 + 0.2 * normal((K,), 72)) if norm else None
    ref = ctx.rmsnorm_quant_i8(dev(X), gamma, 1e-5) if norm else ctx.act_quant_i8(dev(X))
    got = ctx.rmsnorm_quant_i8_tokens(dev(np.ascontiguousarray(X.T)), gamma, 1e-5)
    assert np.array_equal(host(got[0]), host(ref[0]))
    assert np.array_equal(host(got[1]).view(np.uint32), host(ref[1]).view(np.uint32))
    assert np.array_equal(host(got[2]), host(ref[2]))


def test_token_major_rejects(ctx, nnhip):
    import torch
    with pytest.raises(nnhip.NNHipError) as e:     # M = 65: past the one-token kernel
        ctx.rmsnorm_quant_i8_tokens(torch.zeros((65, 256), device="cuda"), None, 1e-5)
    assert e.value.status == 5
    with pytest.raises(nnhip.NNHipError) as e:     # K = 12000: more than 22 rounds of 512
        ctx.rmsnorm_quant_i8_tokens(torch.zeros((4, 12000), device="cuda"), None, 1e-5)
    assert e.value.status == 5
    xi = torch.zeros((16, 256), dtype=torch.int8, device="cuda")
    f = torch.ones(16, device="cuda")
    i = torch.zeros(16, dtype=torch.int32, device="cuda")
    rp = torch.zeros(64 * 64, dtype=torch.int32, device="cuda")
    with pytest.raises(nnhip.NNHipError) as e:     # K = 256: not a decode GEMV width
        ctx.ternary_matmul_glu_tokens(rp, torch.ones(32, device="cuda"), xi, f, i, 16, 256, 16)
    assert e.value.status == 5


def test_prefetch_hint_leaves_results(ctx, orc, nnhip):
    """nnhip_ctx_prefetch_next: the quantizer call that takes the ranges (its extra blocks read
    them) gives the bits it gives without them, on every entry point that takes them; the hint
    is consumed by that call, also where the launch cannot carry it (M > 64)."""
    import torch
    N, K, M, slices = 2560, 6912, 16, 4
    W = normal((N, K), 81, 0.0, 0.02)
    tau = np.full(N, np.abs(W.astype(np.float64)).mean(), np.float32)
    rp = ctx.repack(dev(orc.trit_pack(W, tau)), K)
    big = torch.arange(3 * 1024 * 1024 + 5, dtype=torch.int32, device="cuda")  # 12 MiB + 20 B
    ranges = [rp, big[:1000], big, big[16:17]]
    X = dev(normal((K, M), 82) * np.float32(3.0))
    g = dev(1.0 + 0.2 * normal((K,), 83))
    say("prefetch: rmsnorm_quant_i8 / act_quant_i8")
    ref = [host(t) for t in ctx.rmsnorm_quant_i8(X, g, 1e-5)]
    ctx.prefetch_next(ranges)
    got = [host(t) for t in ctx.rmsnorm_quant_i8(X, g, 1e-5)]
    assert all(np.array_equal(a.view(np.uint8), b.view(np.uint8)) for a, b in zip(got, ref))
    ref = [host(t) for t in ctx.act_quant_i8(X)]
    ctx.prefetch_next([big])
    got = [host(t) for t in ctx.act_quant_i8(X)]
    assert all(np.array_equal(a.view(np.uint8), b.view(np.uint8)) for a, b in zip(got, ref))
    say("prefetch: rmsnorm_quant_i8_tokens")
    Xt = dev(np.ascontiguousarray(host(X).T))
    ref = [host(t) for t in ctx.rmsnorm_quant_i8_tokens(Xt, g, 1e-5)]
    ctx.prefetch_next([rp, big])
    got = [host(t) for t in ctx.rmsnorm_quant_i8_tokens(Xt, g, 1e-5)]
    assert all(np.array_equal(a.view(np.uint8), b.view(np.uint8)) for a, b in zip(got, ref))
    say("prefetch: partial_residual_quant_i8")
    xi, s_d, rs = ctx.act_quant_i8(X)
    part = ctx.ternary_matmul_partial(rp, xi, N, K, M, slices)
    r = dev(normal((N, M), 84))
    gn = dev(1.0 + 0.1 * normal((N,), 85))
    x0 = torch.empty((N, M), device="cuda")
    ref = [host(t) for t in ctx.partial_residual_quant_i8(part, dev(tau), s_d, rs, N, M, x0, res=r, gamma=gn,
                                                          eps=1e-5)]
    x1 = torch.empty((N, M), device="cuda")
    ctx.prefetch_next(ranges)
    got = [host(t) for t in ctx.partial_residual_quant_i8(part, dev(tau), s_d, rs, N, M, x1, res=r, gamma=gn,
                                                          eps=1e-5)]
    assert all(np.array_equal(a.view(np.uint8), b.view(np.uint8)) for a, b in zip(got, ref))
    assert np.array_equal(host(x1).view(np.uint32), host(x0).view(np.uint32))
    say("prefetch: taken by a call that cannot carry it, then cleared")
    X2 = dev(normal((512, 128), 86))
    ref = [host(t) for t in ctx.act_quant_i8(X2)]
    ctx.prefetch_next([big])
    got = [host(t) for t in ctx.act_quant_i8(X2)]      # M = 128: register kernel, hint dropped
    assert all(np.array_equal(a.view(np.uint8), b.view(np.uint8)) for a, b in zip(got, ref))
    ctx.prefetch_next([])
    with pytest.raises(nnhip.NNHipError):
        ctx.prefetch_next([big, big, big, big, big])    # more than 4 ranges
    with pytest.raises(nnhip.NNHipError):
        ctx.prefetch_next([big[1:]])                    # not 16-byte aligned
    torch.cuda.synchronize()


@pytest.mark.parametrize("bias", [False, True])
def test_token_major_residual_entries(ctx, orc, bias):
    """The token-major forms of the decoder's residual-stream entry points give the bits of the
    feature-major ones transposed: nnhip_ternary_matmul_add_tokens (o + residual),
    nnhip_partial_residual_quant_i8_tokens (fc2 epilogue + residual + next quantizer, also with
    x_out aliasing res) and nnhip_embedding_gather_tokens (an id out of range gives a NaN row)."""
    import torch
    N, K, M = 2560, 2560, 16
    say(f"token-major residual entries bias={bias}")
    W = normal((N, K), 101, 0.0, 0.02)
    tau = np.full(N, np.abs(W.astype(np.float64)).mean(), np.float32)
    rp = ctx.repack(dev(orc.trit_pack(W, tau)), K)
    xi, s_d, rs = ctx.act_quant_i8(dev(normal((K, M), 102)))
    b = dev(normal((N,), 103)) if bias else None
    res = normal((N, M), 104)
    y = host(ctx.ternary_matmul_add(rp, dev(tau), xi, s_d, rs, N, K, M, dev(res), bias=b))
    yt = host(ctx.ternary_matmul_add(rp, dev(tau), xi, s_d, rs, N, K, M, dev(np.ascontiguousarray(res.T)), bias=b,
                                     tokens=True))
    assert yt.shape == (M, N)
    assert np.array_equal(np.ascontiguousarray(yt.T).view(np.uint32), y.view(np.uint32))
    # fc2-shaped partial sums + epilogue + residual + next RMSNorm quantizer
    N2, K2, S = 2560, 6912, 4
    W2 = normal((N2, K2), 105, 0.0, 0.02)
    tau2 = np.full(N2, np.abs(W2.astype(np.float64)).mean(), np.float32)
    rp2 = ctx.repack(dev(orc.trit_pack(W2, tau2)), K2)
    xi2, s2, rs2 = ctx.act_quant_i8(dev(normal((K2, M), 106)))
    part = ctx.ternary_matmul_partial(rp2, xi2, N2, K2, M, S)
    g = dev(1.0 + 0.1 * normal((N2,), 107))
    b2 = dev(normal((N2,), 108)) if bias else None
    x0 = torch.empty((N2, M), device="cuda")
    ref = [host(t) for t in ctx.partial_residual_quant_i8(part, dev(tau2), s2, rs2, N2, M, x0, res=dev(res), bias=b2,
                                                          gamma=g, eps=1e-5)]
    x1 = dev(np.ascontiguousarray(res.T))            # in place: x_out aliases res
    got = [host(t) for t in ctx.partial_residual_quant_i8(part, dev(tau2), s2, rs2, N2, M, x1, res=x1, bias=b2,
                                                          gamma=g, eps=1e-5, tokens=True)]
    assert all(np.array_equal(a.view(np.uint8), c.view(np.uint8)) for a, c in zip(got, ref))
    assert np.array_equal(np.ascontiguousarray(host(x1).T).view(np.uint32), host(x0).view(np.uint32))
    # embedding rows
    V, d = 97, 2560
    table = dev(normal((V, d), 109))
    ids = dev(np.array([3, 96, 0, 97, 5, -1, 40, 41, 1, 2, 3, 4, 5, 6, 7, 8], np.int32))
    e = host(ctx.embedding_gather(table, ids))
    et = host(ctx.embedding_gather(table, ids, tokens=True))
    assert et.shape == (16, d)
    a, c = np.ascontiguousarray(et.T), e
    assert np.array_equal(np.isnan(a), np.isnan(c)) and np.all(np.isnan(a[:, 3])) and np.all(np.isnan(a[:, 5]))
    assert np.array_equal(a[~np.isnan(a)].view(np.uint32), c[~np.isnan(c)].view(np.uint32))


@pytest.mark.parametrize("d,B,gamma", [(2560, 16, True), (2560, 16, False), (256, 3, True), (6912, 5, True)])
def test_embedding_rmsnorm_quant_fused(ctx, orc, d, B, gamma):
    """nnhip_embedding_rmsnorm_quant_i8_tokens: the gathered rows against the oracle's embedding
    gather, the codes / scales / row sums against the oracle's [RMSNorm ->] absmax int8 of those
    rows, and, with ids out of range (NaN rows), the same bits as the two-launch form
    (nnhip_embedding_gather_tokens, then nnhip_rmsnorm_quant_i8_tokens)."""
    import torch
    say(f"embedding + rmsnorm quant d={d} B={B} gamma={gamma}")
    V, eps = 1000, 1e-5
    table = normal((V, d), 120 + d)
    ids = (np.arange(B, dtype=np.int32) * 37 + 5) % V
    g = (1.0 + 0.1 * normal((d,), 121)).astype(np.float32) if gamma else None
    gd = dev(g) if gamma else None
    x, (xi, s, rs) = ctx.embedding_rmsnorm_quant_i8_tokens(dev(table), dev(ids), gd, eps)
    X = orc.embedding_gather(table, ids)                       # (d, B)
    assert np.array_equal(np.ascontiguousarray(host(x).T).view(np.uint32), X.view(np.uint32))
    if gamma:
        xq_o, s_o = orc.rmsnorm_quant_i8(X, g, eps)
    else:
        s_o = orc.act_scale(X)
        xq_o = orc.quantize_i8(X, s_o, True)
    q = orc.container_to_int8(xq_o, B).T                      # (B, d)
    assert np.array_equal(host(s).view(np.uint32), np.asarray(s_o, np.float32).reshape(-1).view(np.uint32))
    assert np.array_equal(host(xi)[:, :d], q)
    assert np.array_equal(host(rs), q.astype(np.int64).sum(axis=1))
    # NaN rows from ids outside [0, V): the two-launch form's bits
    ids2 = ids.copy()
    ids2[0], ids2[-1] = V, -1
    got_x, got = ctx.embedding_rmsnorm_quant_i8_tokens(dev(table), dev(ids2), gd, eps)
    ref_x = ctx.embedding_gather(dev(table), dev(ids2), tokens=True)
    ref = ctx.rmsnorm_quant_i8_tokens(ref_x, gd, eps)
    torch.cuda.synchronize()
    assert np.array_equal(host(got_x).view(np.uint32), host(ref_x).view(np.uint32))
    assert np.all(np.isnan(host(got_x)[0])) and np.all(np.isnan(host(got_x)[-1]))
    assert all(np.array_equal(host(a).view(np.uint8), host(c).view(np.uint8)) for a, c in zip(got, ref))

"""GPU parity of the gated feed-forward block (config C4): the gated activations (SwiGLU,
ReLU^2-GLU) with this library's fp32 exp, the gate/up interleave of fc1, fc1 with the
activation fused (decode GEMV path and prefill GEMM epilogue), and the whole block
[RMSNorm] -> int8 -> fc1 -> act -> int8 -> fc2, all bit for bit against the CPU oracle.

Reference: FeedForward::forward (include/neuralnet.cpp/compute_layer_feedforward.hpp:182-204),
SwiGLU / ReLU2GLU::forward (compute_layer_mlp.hpp:317-328, :405-414), BitLinear int8 forward
(compute_layer_bitlinear.hpp:441-457).
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
    return a.view(dtype) if dtype is not None else a


def say(msg):
    print(msg, flush=True)


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def special_values():
    v = [0.0, -0.0, 1.0, -1.0, 0.5, 1e-30, -1e-30, 1e-45, 86.9, 87.0, 87.01, -86.9, -87.0, -87.01,
         88.72, -88.72, 99.9, 100.0, 100.01, -100.01, 1e30, -1e30, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38]
    return np.array(v, np.float32)


@pytest.mark.parametrize("act", [0, 1])
def test_glu_bitexact(ctx, orc, act):
    say(f"glu act={act}")
    sp = special_values()
    g = np.concatenate([np.repeat(sp, len(sp)), normal((200_000,), 3, 0.0, 6.0),
                        np.linspace(-90, 90, 100_001, dtype=np.float32)])
    u = np.concatenate([np.tile(sp, len(sp)), normal((200_000,), 4, 0.0, 2.0),
                        uniform((100_001,), 5, -3.0, 3.0)])
    M = 7
    n = (len(g) // M) * M
    Y1 = np.concatenate([g[:n].reshape(-1, M), u[:n].reshape(-1, M)])
    ref = orc.glu(Y1, act)
    got = host(ctx.glu(dev(Y1), act))
    assert same_bits(got, ref)


@pytest.mark.parametrize("F,K", [(12, 40), (300, 257), (13, 16), (6912, 2560)])
def test_glu_interleave(ctx, orc, F, K):
    say(f"glu_interleave F={F} K={K}")
    W = normal((2 * F, K), 100 + F, 0.0, 0.02)
    tau = orc.row_absmean(W)
    wq = orc.trit_pack(W, tau)
    b = normal((2 * F,), 101 + F)
    wo_r, to_r, bo_r = orc.glu_interleave(wq, tau, b, F, K)
    wo, to, bo = ctx.glu_interleave(dev(wq), dev(tau), dev(b), F, K)
    assert np.array_equal(host(wo, np.uint32), wo_r)
    assert same_bits(host(to), to_r) and same_bits(host(bo), bo_r)
    wo2, to2, bo2 = ctx.glu_interleave(dev(wq), dev(tau), None, F, K)
    assert bo2 is None and np.array_equal(host(wo2, np.uint32), wo_r)


def fc1_case(orc, d, F, seed, bias=True):
    W1 = normal((2 * F, d), seed, 0.0, 0.02)
    t1 = orc.row_absmean(W1)
    wq1 = orc.trit_pack(W1, t1)
    b1 = normal((2 * F,), seed + 1, 0.0, 0.5) if bias else None
    return wq1, t1, b1


def prepare_fc1(ctx, wq1, t1, b1, F, d):
    wo, to, bo = ctx.glu_interleave(dev(wq1), dev(t1), dev(b1) if b1 is not None else None, F, d)
    return ctx.repack(wo, d), to, bo


@pytest.mark.parametrize("M", [1, 7, 16, 17, 100, 256, 300])
@pytest.mark.parametrize("act", [0, 1])
def test_matmul_glu(ctx, orc, M, act):
    d, F = 320, 100
    say(f"ternary_matmul_glu d={d} F={F} M={M} act={act}")
    wq1, t1, b1 = fc1_case(orc, d, F, 200 + M)
    X = normal((d, M), 300 + M, 0.0, 1.0)
    s = orc.act_scale(X)
    xq = orc.quantize_i8(X, s, True)
    y1 = orc.add_row_broadcast(orc.matmul_q_i8(wq1, t1, xq, s, d, M), b1)
    ref = orc.glu(y1, act)
    rp, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    xi, sg, rs = ctx.act_quant_i8(dev(X))
    h = host(ctx.ternary_matmul_glu(rp, to, xi, sg, rs, F, d, M, act, bias=bo))
    assert same_bits(h, ref)


@pytest.mark.parametrize("d,F,M", [(2560, 6912, 16), (1024, 100, 5), (2560, 13, 1), (4096, 700, 3)])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("bias", [True, False])
def test_matmul_glu_deep_gemv(ctx, orc, d, F, M, act, bias):
    """Decode fc1 through the deep GEMV with the gated activation in its epilogue (k-tile counts
    4, 10, 16; feature counts not multiples of 8), bit for bit against fc1 + glu."""
    say(f"deep ternary_matmul_glu d={d} F={F} M={M} act={act} bias={bias}")
    wq1, t1, b1 = fc1_case(orc, d, F, 700 + F + M, bias=bias)
    X = normal((d, M), 800 + M, 0.0, 1.0)
    s = orc.act_scale(X)
    xq = orc.quantize_i8(X, s, True)
    y1 = orc.matmul_q_i8(wq1, t1, xq, s, d, M)
    if bias:
        y1 = orc.add_row_broadcast(y1, b1)
    ref = orc.glu(y1, act)
    rp, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    xi, sg, rs = ctx.act_quant_i8(dev(X))
    h = host(ctx.ternary_matmul_glu(rp, to, xi, sg, rs, F, d, M, act, bias=bo))
    assert same_bits(h, ref)


def block_case(orc, d, F, seed):
    wq1, t1, b1 = fc1_case(orc, d, F, seed)
    W2 = normal((d, F), seed + 2, 0.0, 0.02)
    t2 = orc.row_absmean(W2)
    wq2 = orc.trit_pack(W2, t2)
    b2 = normal((d,), seed + 3, 0.0, 0.5)
    return wq1, t1, b1, wq2, t2, b2


@pytest.mark.parametrize("d,F,M", [(96, 40, 1), (256, 136, 16), (320, 100, 64), (512, 344, 300)])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("norm", [True, False])
def test_ffn_block(ctx, orc, d, F, M, act, norm):
    say(f"ffn_glu_i8 d={d} F={F} M={M} act={act} norm={norm}")
    wq1, t1, b1, wq2, t2, b2 = block_case(orc, d, F, 400 + d + M)
    X = normal((d, M), 500 + M, 0.0, 1.0)
    gamma = normal((d,), 501, 1.0, 0.1) if norm else None
    Y_ref, _ = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, b1, wq2, t2, b2, act)
    rp1, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    rp2 = ctx.repack(dev(wq2), F)
    Y = host(ctx.ffn_glu_i8(dev(X), dev(gamma) if gamma is not None else None, 1e-6, F, rp1, to, bo, rp2,
                            dev(t2), dev(b2), act))
    assert same_bits(Y, Y_ref)


def test_ffn_block_c4_sampled_tokens(ctx, orc):
    """Config C4 at full size (d=2560, F=6912, 2048 tokens, RMSNorm eps=1e-6, gamma=1): every
    step is per token, so the oracle run on a sample of token columns gives those columns."""
    d, F, M = 2560, 6912, 2048
    say("ffn_glu_i8 C4 full size, sampled tokens")
    import torch
    g = torch.Generator(device="cuda").manual_seed(7)
    W1 = torch.randn((2 * F, d), device="cuda", generator=g) * 0.02
    W2 = torch.randn((d, F), device="cuda", generator=g) * 0.02
    t1, t2 = ctx.row_absmean(W1), ctx.row_absmean(W2)
    wq1, wq2 = ctx.trit_pack(W1, t1), ctx.trit_pack(W2, t2)
    X = torch.randn((d, M), device="cuda", generator=g)
    gamma = torch.ones(d, device="cuda")
    wo, to, _ = ctx.glu_interleave(wq1, t1, None, F, d)
    rp1, rp2 = ctx.repack(wo, d), ctx.repack(wq2, F)
    Y = host(ctx.ffn_glu_i8(X, gamma, 1e-6, F, rp1, to, None, rp2, t2, None, 0))
    cols = np.array([0, 1, 127, 128, 1000, 1023, 2046, 2047])
    Xs = host(X)[:, cols]
    Y_ref, _ = orc.ffn_glu_i8(Xs, np.ones(d, np.float32), 1e-6, F, host(wq1, np.uint32), host(t1), None,
                              host(wq2, np.uint32), host(t2), None, 0)
    assert same_bits(Y[:, cols], Y_ref)
    assert np.isfinite(Y).all()


def test_ffn_block_repeat_and_special_h(ctx, orc):
    """Consecutive prefill-block calls on one context (a smaller M after a larger one, inputs of
    other magnitudes; the context's workspace is reused) each match the oracle. The last call
    has a fc1 bias with NaN and inf entries, so h holds NaN (ignored by the absmax, quantized to
    0) and inf (scale inf, codes 0)."""
    d, F = 256, 136
    wq1, t1, b1, wq2, t2, b2 = block_case(orc, d, F, 900)
    rp1, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    rp2 = ctx.repack(dev(wq2), F)
    cases = [(300, 1.0, b1), (64, 30.0, b1), (300, 0.01, b1)]
    b_special = b1.copy()
    b_special[[3, 70]] = np.nan
    b_special[[5]] = np.inf
    cases.append((200, 1.0, b_special))
    for i, (M, scale, bias) in enumerate(cases):
        say(f"ffn_glu_i8 repeat call {i}: M={M} scale={scale}")
        X = (normal((d, M), 910 + i, 0.0, 1.0) * np.float32(scale)).astype(np.float32)
        gamma = normal((d,), 920 + i, 1.0, 0.1)
        Y_ref, _ = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, bias, wq2, t2, b2, 0)
        if bias is b1:
            b_dev = bo
        else:
            _, _, b_dev = prepare_fc1(ctx, wq1, t1, bias, F, d)
        Y = host(ctx.ffn_glu_i8(dev(X), dev(gamma), 1e-6, F, rp1, to, b_dev, rp2, dev(t2), dev(b2), 0))
        assert same_bits(Y, Y_ref), f"call {i}"


@pytest.mark.parametrize("tile", [1, 2, 3])
def test_ffn_block_each_tile(ctx, orc, tile):
    """The gated epilogue (h and its per-token absmax) under every prefill GEMM block tile."""
    d, F, M = 320, 100, 150
    say(f"ffn_glu_i8 tile={tile} d={d} F={F} M={M}")
    wq1, t1, b1, wq2, t2, b2 = block_case(orc, d, F, 930)
    X = normal((d, M), 931, 0.0, 1.0)
    gamma = normal((d,), 932, 1.0, 0.1)
    Y_ref, _ = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, b1, wq2, t2, b2, 1)
    rp1, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    rp2 = ctx.repack(dev(wq2), F)
    ctx.set_gemm_tile(tile)
    try:
        Y = host(ctx.ffn_glu_i8(dev(X), dev(gamma), 1e-6, F, rp1, to, bo, rp2, dev(t2), dev(b2), 1))
    finally:
        ctx.set_gemm_tile(0)
    assert same_bits(Y, Y_ref)


@pytest.mark.parametrize("F,M", [(2304, 2048), (2300, 2000)])
def test_ffn_block_split_rows(ctx, orc, F, M):
    """fc1 of F gated features (2F interleaved rows) at about 2048 tokens: on a 256-CU device the
    automatic tile choice runs 256 x 128 blocks over the first 4096 rows (features 0..2047) and a
    smaller tile over the rest (F = 2300, M = 2000: the last features and tokens end inside a
    block). The block against the oracle on every token, h the same bits as under the 256 x 128
    tile alone."""
    d = 256
    say(f"ffn_glu_i8 split rows d={d} F={F} M={M}")
    wq1, t1, b1, wq2, t2, b2 = block_case(orc, d, F, 960)
    X = normal((d, M), 961, 0.0, 1.0)
    gamma = normal((d,), 962, 1.0, 0.1)
    Y_ref, _ = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, b1, wq2, t2, b2, 0)
    rp1, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    rp2 = ctx.repack(dev(wq2), F)
    Y = host(ctx.ffn_glu_i8(dev(X), dev(gamma), 1e-6, F, rp1, to, bo, rp2, dev(t2), dev(b2), 0))
    assert same_bits(Y, Y_ref)
    xi, s, rs = ctx.act_quant_i8(dev(X))
    h = host(ctx.ternary_matmul_glu(rp1, to, xi, s, rs, F, d, M, bias=bo))
    ctx.set_gemm_tile(1)
    try:
        h1 = host(ctx.ternary_matmul_glu(rp1, to, xi, s, rs, F, d, M, bias=bo))
    finally:
        ctx.set_gemm_tile(0)
    assert same_bits(h, h1)


@pytest.mark.parametrize("M", [1, 16, 64, 300])
@pytest.mark.parametrize("act", [0, 1])
def test_ffn_block_subln(ctx, orc, M, act):
    """SubLN (BitNet b1.58): an RMSNorm of the gated output (eps 1e-5) before fc2's quantizer,
    decode and prefill sizes, bit-exact against the oracle."""
    d, F = 256, 136
    say(f"ffn_glu_i8 SubLN d={d} F={F} M={M} act={act}")
    wq1, t1, b1, wq2, t2, b2 = block_case(orc, d, F, 940 + M)
    X = normal((d, M), 941 + M, 0.0, 1.0)
    gamma = normal((d,), 942, 1.0, 0.1)
    gsub = normal((F,), 943, 1.0, 0.1)
    Y_ref, _ = orc.ffn_glu_i8(X, gamma, 1e-6, F, wq1, t1, b1, wq2, t2, b2, act, gamma_sub=gsub, eps_sub=1e-5)
    rp1, to, bo = prepare_fc1(ctx, wq1, t1, b1, F, d)
    rp2 = ctx.repack(dev(wq2), F)
    Y = host(ctx.ffn_glu_i8(dev(X), dev(gamma), 1e-6, F, rp1, to, bo, rp2, dev(t2), dev(b2), act,
                            gamma_sub=dev(gsub), eps_sub=1e-5))
    assert same_bits(Y, Y_ref)

"""GPU parity of the batched prefill (config C5's context): nnhip_kv_cache_fill and the causal
nnhip_attention_prefill against the oracle run as the reference fills a cache, one decode step
per context token (GPTModel::generate's loop of forward_step calls,
include/neuralnet.cpp/compute_layer_gpt.hpp:774-794; AttentionBase::forward_step,
compute_layer_attention.hpp:1003-1091), then the whole prefill of Decoder.prefill.

The cache rows (rotated keys, values) are compared bit for bit. The attention output is compared
within 5e-6 x max(1, max|out|) of the oracle: its dot products and softmax sums are f32 in an
order the reference leaves open, and the prefill kernel accumulates on the fp32 MFMA with an
online softmax.
"""
import math

import numpy as np
import pytest

from conftest import normal

pytestmark = pytest.mark.gpu

ATOL = 5e-6   # x max(1, max|out|)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def say(msg):
    print(msg, flush=True)


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def close(got, ref):
    return float(np.max(np.abs(got - ref))) <= ATOL * max(1.0, float(np.max(np.abs(ref))))


@pytest.mark.parametrize("B,T,H,Hkv,dk,pos0,rope", [
    (3, 100, 8, 2, 128, 0, True),      # tail query block, GQA 4
    (2, 37, 4, 4, 64, 5, False),       # one head per KV head, dk 64, no position encoding
    (1, 64, 8, 1, 128, 60, True),      # 8 heads per KV head, context not a multiple of 32
    (2, 1, 4, 2, 128, 33, True),       # one token: a decode step
    (4, 33, 20, 5, 128, 2000, True),   # config C5 heads near the end of a 2176-row cache
])
def test_prefill_matches_token_by_token(ctx, orc, nnhip, B, T, H, Hkv, dk, pos0, rope):
    """T tokens per sequence at positions pos0 .. pos0+T-1 over a cache holding pos0 rows of history:
    the caches bit for bit and every token's attention against T oracle decode steps."""
    say(f"prefill B={B} T={T} H={H} Hkv={Hkv} dk={dk} pos0={pos0} rope={rope}")
    max_len = 2176 if pos0 >= 2000 else pos0 + T + 7
    seed = 1000 + B + T + H + pos0
    M = B * T
    q = normal((H * dk, M), seed)
    k = normal((Hkv * dk, M), seed + 1)
    v = normal((Hkv * dk, M), seed + 2)
    kc = normal((B, max_len, Hkv * dk), seed + 3)
    vc = normal((B, max_len, Hkv * dk), seed + 4)
    cos, sin = nnhip.rope_table(dk, max_len) if rope else (None, None)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(dk)))
    kc_d, vc_d = dev(kc), dev(vc)
    cd, sd = (None, None) if cos is None else (dev(cos), dev(sin))
    ctx.kv_cache_fill(dev(k), dev(v), B, T, Hkv, dk, pos0, kc_d, vc_d, cd, sd)
    out = host(ctx.attention_prefill(dev(q), kc_d, vc_d, B, T, H, Hkv, dk, pos0, scale, cd, sd))
    kc_o, vc_o = kc.copy(), vc.copy()
    cols = np.arange(B) * T
    for t in range(T):
        ref = orc.attention_decode(q[:, cols + t], k[:, cols + t], v[:, cols + t], H, Hkv, dk,
                                   np.full(B, pos0 + t, np.int32), kc_o, vc_o, scale, cos, sin)
        assert close(out[:, cols + t], ref), f"token {t}"
    assert same_bits(host(kc_d), kc_o), "key cache differs"
    assert same_bits(host(vc_d), vc_o), "value cache differs"


def test_prefill_c5_full_context(ctx, orc, nnhip):
    """Config C5's prefill geometry at full size (16 sequences x 2048 tokens, 20 heads / 5 KV heads
    of 128, 2176-row caches): every cache row of three sequences bit for bit against the oracle's
    rotation, and sampled tokens (both ends of every 32-token block boundary tried, the first and
    last) against the oracle decode step over the prefilled cache."""
    import torch
    B, T, H, Hkv, dk, max_len = 16, 2048, 20, 5, 128, 2176
    say(f"prefill C5 geometry B={B} T={T}")
    M = B * T
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC5F)
    q = torch.randn((H * dk, M), generator=gen, device="cuda")
    k = torch.randn((Hkv * dk, M), generator=gen, device="cuda")
    v = torch.randn((Hkv * dk, M), generator=gen, device="cuda")
    kc = torch.zeros((B, max_len, Hkv * dk), device="cuda")
    vc = torch.zeros((B, max_len, Hkv * dk), device="cuda")
    cos, sin = nnhip.rope_table(dk, max_len)
    cd, sd = dev(cos), dev(sin)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(dk)))
    ctx.kv_cache_fill(k, v, B, T, Hkv, dk, 0, kc, vc, cd, sd)
    out = ctx.attention_prefill(q, kc, vc, B, T, H, Hkv, dk, 0, scale, cd, sd)
    torch.cuda.synchronize()
    kh, vh = host(k), host(v)
    for b in (0, 9, 15):
        kcb, vcb = host(kc[b]), host(vc[b])
        # every row of the sequence: the rotated key and the value of its token
        for t in range(T):
            col = b * T + t
            for g in range(Hkv):
                x = kh[g * dk:(g + 1) * dk, col]
                assert same_bits(kcb[t, g * dk:(g + 1) * dk], orc.rope_apply(x, cos[t], sin[t])), (b, t, g)
            assert same_bits(vcb[t], vh[:, col]), (b, t)
        assert not np.any(kcb[T:]) and not np.any(vcb[T:])
        qs = host(q[:, b * T:(b + 1) * T])
        os_ = host(out[:, b * T:(b + 1) * T])
        for t in (0, 1, 31, 32, 33, 63, 64, 1000, 2046, 2047):
            kco, vco = kcb[None].copy(), vcb[None].copy()
            ref = orc.attention_decode(qs[:, t:t + 1], kh[:, b * T + t:b * T + t + 1], vh[:, b * T + t:b * T + t + 1],
                                       H, Hkv, dk, np.array([t], np.int32), kco, vco, scale, cos, sin)
            assert close(os_[:, t:t + 1], ref), (b, t)


def test_prefill_rejects(ctx, nnhip):
    import torch
    q = torch.zeros((8 * 128, 4), device="cuda")
    kc = torch.zeros((2, 8, 2 * 128), device="cuda")
    with pytest.raises(nnhip.NNHipError):   # pos0 + T beyond max_len
        ctx.attention_prefill(q, kc, kc, 2, 2, 8, 2, 128, 7, 0.1)
    with pytest.raises(nnhip.NNHipError):   # dk 96
        ctx.attention_prefill(q, kc, kc, 2, 2, 8, 2, 96, 0, 0.1)
    with pytest.raises(nnhip.NNHipError):   # 3 heads per KV head
        ctx.attention_prefill(q, kc, kc, 2, 2, 6, 2, 128, 0, 0.1)


# ---------------------------------------------------------------- the whole prefill

def _orc_bitlinear(orc, x, lin, gamma, eps):
    """int8 BitLinear of the oracle: [RMSNorm ->] absmax int8 -> matmul_q_i8 [+ b]."""
    wq, tau, b = lin
    if gamma is None:
        s = orc.act_scale(x)
        xq = orc.quantize_i8(x, s, True)
    else:
        xq, s = orc.rmsnorm_quant_i8(x, gamma, eps)
    y = orc.matmul_q_i8_rowblock(wq, tau, xq, s, x.shape[0], x.shape[1])
    return y if b is None else orc.add_row_broadcast(y, b)


def _gpu_model(ctx, nnhip, cfg, L, B, seed, subln=True, bias=False):
    """Random BitNet-style weights made on the GPU (W ~ N(0, 0.02), per-row absmean, trit_pack,
    which the parity tests pin bit for bit), kept as device Linear objects and downloaded as the
    oracle's reference containers; norm gains ~ N(1, 0.1)."""
    import torch
    from nnhip_py import decoder as dmod
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    d, F, dk = cfg.d, cfg.F, cfg.dk

    def lin(N, K):
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        tau = ctx.row_absmean(W)
        wq = ctx.trit_pack(W, tau)
        b = torch.randn((N,), generator=gen, device="cuda") * 0.1 if bias else None
        del W
        return wq, tau, b

    def gain(n):
        return 1.0 + 0.1 * torch.randn((n,), generator=gen, device="cuda")

    def hostlin(t):
        wq, tau, b = t
        return host(wq).view(np.uint32), host(tau), None if b is None else host(b)

    host_blocks, dev_blocks = [], []
    for _ in range(L):
        t = {n: lin(N, K) for n, N, K in (("q", cfg.H * dk, d), ("k", cfg.Hkv * dk, d), ("v", cfg.Hkv * dk, d),
                                           ("o", d, cfg.H * dk), ("fc1", 2 * F, d), ("fc2", d, F))}
        g = {"g1": gain(d), "g2": gain(d), "ga": gain(d) if subln else None, "gf": gain(F) if subln else None}
        hb = {n: hostlin(t[n]) for n in t}
        hb.update({n: None if g[n] is None else host(g[n]) for n in g})
        host_blocks.append(hb)

        def dl(n, N, K):
            wq, tau, b = t[n]
            return dmod.Linear(ctx.repack(wq, K), tau, b, N, K)

        wo, to, bo = ctx.glu_interleave(t["fc1"][0], t["fc1"][1], t["fc1"][2], F, d)
        fc1 = dmod.Linear(ctx.repack(wo, d), to, bo, nnhip.glu_rows(F), d)
        dev_blocks.append(dmod.Block(g1=g["g1"], q=dl("q", cfg.H * dk, d), k=dl("k", cfg.Hkv * dk, d),
                                     v=dl("v", cfg.Hkv * dk, d), o=dl("o", d, cfg.H * dk), g2=g["g2"], fc1=fc1,
                                     fc2=dl("fc2", d, F), g_attn_sub=g["ga"], g_ffn_sub=g["gf"]))
    emb = torch.randn((cfg.vocab, d), generator=gen, device="cuda")
    gfin = gain(d)
    ht = lin(cfg.vocab, d)
    head_d = dmod.Linear(ctx.repack(ht[0], d), ht[1], None, cfg.vocab, d)
    dec = dmod.Decoder(ctx, cfg, dev_blocks, emb, gfin, head_d, B)
    return dec, host_blocks, host(emb), host(gfin), (hostlin(ht)[0], hostlin(ht)[1], None)


def _prefill_chain(ctx, orc, cfg, dec, hb, emb, gfin, head, B, T, samp, steps, seed, advance=False):
    """Decoder.prefill of T prompt tokens for B sequences, then `steps` decode steps, against the
    oracle chain on the sampled sequences: per block q / k / v and the block output bit for bit,
    the attention within tolerance (the GPU's attention output is fed to the oracle's next stage, so
    the int8 stages stay comparable bit for bit), the caches bit for bit, then the last tokens'
    logits and greedy ids; the decode steps continue from the prefilled caches (GPTBlock::
    forward_step order, compute_layer_gpt.hpp:201-219). advance: the last step runs with
    advance=True and must leave its greedy ids in its own input ids and every position one ahead."""
    import torch
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, cfg.vocab, size=(B, T)).astype(np.int32)
    cols = np.concatenate([np.arange(b * T, (b + 1) * T) for b in samp])
    got = {}

    def hook(i, name, t):
        got[(i, name)] = host(t[:, cols])

    logits_d, next_d = dec.prefill(dev(ids.reshape(-1)), T, 0, hook=hook)
    logits, nxt = host(logits_d), host(next_d)
    cos, sin = orc.rope_table(cfg.dk, cfg.max_len)
    Bs = len(samp)
    kc_o = [np.zeros((Bs, cfg.max_len, cfg.Hkv * cfg.dk), np.float32) for _ in hb]
    vc_o = [np.zeros_like(kc_o[0]) for _ in hb]
    x = orc.embedding_gather(emb, ids[samp].reshape(-1))              # (d, Bs*T), column j*T + t
    tcols = np.arange(Bs) * T
    for l, b in enumerate(hb):
        say(f"prefill chain: block {l}")
        q = _orc_bitlinear(orc, x, b["q"], b["g1"], cfg.eps)
        k = _orc_bitlinear(orc, x, b["k"], b["g1"], cfg.eps)
        v = _orc_bitlinear(orc, x, b["v"], b["g1"], cfg.eps)
        assert same_bits(got[(l, "q")], q) and same_bits(got[(l, "k")], k) and same_bits(got[(l, "v")], v), l
        ag = got[(l, "a")]
        for t in range(T):
            a = orc.attention_decode(q[:, tcols + t], k[:, tcols + t], v[:, tcols + t], cfg.H, cfg.Hkv, cfg.dk,
                                     np.full(Bs, t, np.int32), kc_o[l], vc_o[l], cfg.scale, cos, sin)
            assert close(ag[:, tcols + t], a), (l, t)
        o = _orc_bitlinear(orc, ag, b["o"], b["ga"], cfg.eps)
        r = x + o
        f, _ = orc.ffn_glu_i8(r, b["g2"], cfg.eps, cfg.F, *b["fc1"], *b["fc2"], cfg.act, gamma_sub=b["gf"],
                              eps_sub=cfg.eps)
        x = r + f
        assert same_bits(got[(l, "x")], x), l
    torch.cuda.synchronize()
    for l in range(len(hb)):
        kcg, vcg = host(dec.caches[l][0]), host(dec.caches[l][1])
        assert same_bits(kcg[samp], kc_o[l]) and same_bits(vcg[samp], vc_o[l]), l
    lg = _orc_bitlinear(orc, x[:, tcols + T - 1], head, gfin, cfg.eps)
    assert same_bits(logits[:, samp], lg), "prefill logits differ"
    assert nxt[samp].tolist() == orc.argmax_cols(lg).tolist()
    # decode steps from the prefilled caches
    cur = nxt.astype(np.int32)
    for step in range(steps):
        pos = np.full(B, T + step, np.int32)
        say(f"prefill chain: decode step {step}")
        attn = {}
        adv = advance and step == steps - 1
        cur_d, pos_d = dev(cur), dev(pos)
        logits_d, next_d = dec.step(cur_d, pos_d, T + step + 1,
                                    attn_hook=lambda i, a: attn.__setitem__(i, host(a[:, samp])), advance=adv)
        logits, nxt = host(logits_d), host(next_d)
        if adv:
            assert next_d.data_ptr() == cur_d.data_ptr()
            assert host(pos_d).tolist() == (pos + 1).tolist()
        x = orc.embedding_gather(emb, cur[samp])
        for l, b in enumerate(hb):
            q = _orc_bitlinear(orc, x, b["q"], b["g1"], cfg.eps)
            k = _orc_bitlinear(orc, x, b["k"], b["g1"], cfg.eps)
            v = _orc_bitlinear(orc, x, b["v"], b["g1"], cfg.eps)
            a = orc.attention_decode(q, k, v, cfg.H, cfg.Hkv, cfg.dk, pos[samp], kc_o[l], vc_o[l], cfg.scale, cos, sin)
            assert close(attn[l], a), (step, l)
            o = _orc_bitlinear(orc, attn[l], b["o"], b["ga"], cfg.eps)
            r = x + o
            f, _ = orc.ffn_glu_i8(r, b["g2"], cfg.eps, cfg.F, *b["fc1"], *b["fc2"], cfg.act, gamma_sub=b["gf"],
                                  eps_sub=cfg.eps)
            x = r + f
        lg = _orc_bitlinear(orc, x, head, gfin, cfg.eps)
        assert same_bits(logits[:, samp], lg), f"step {step} logits differ"
        assert nxt[samp].tolist() == orc.argmax_cols(lg).tolist()
        cur = nxt.astype(np.int32)


@pytest.mark.parametrize("subln,bias,act", [(True, False, 0), (False, True, 1)])
def test_decoder_prefill_chain_small(ctx, orc, nnhip, subln, bias, act):
    """A 2-block model (d=256, 4 heads / 2 KV heads of 64, F=320, vocab 97): 3 sequences x 45 prompt
    tokens through Decoder.prefill, then 2 decode steps, every sequence against the oracle chain."""
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=256, H=4, Hkv=2, F=320, vocab=97, max_len=64, act=act, eps=1e-5)
    B, T = 3, 45
    dec, hb, emb, gfin, head = _gpu_model(ctx, nnhip, cfg, 2, B, 0x9F + act, subln=subln, bias=bias)
    _prefill_chain(ctx, orc, cfg, dec, hb, emb, gfin, head, B, T, [0, 1, 2], 2, 11 + act, advance=True)


def test_decoder_prefill_chain_c5(ctx, orc, nnhip):
    """Config C5's model at full size (30 layers, d=2560, 20 heads / 5 KV heads, SwiGLU F=6912 with
    SubLN, vocab 10000, batch 16): a 16-token prompt per sequence through Decoder.prefill, then 2
    decode steps, sequences 0 and 13 against the oracle chain (the batch only shares weights, so
    the others run the same kernels on other columns)."""
    from nnhip_py import decoder as dmod
    cfg = dmod.Config(d=2560, H=20, Hkv=5, F=6912, vocab=10000, max_len=64, act=0, eps=1e-5)
    B, T = 16, 16
    say("building the 30-layer C5 model")
    dec, hb, emb, gfin, head = _gpu_model(ctx, nnhip, cfg, 30, B, 0xC5C5)
    assert dec.logits_t is not None, "the C5 head should produce token-major logits"
    _prefill_chain(ctx, orc, cfg, dec, hb, emb, gfin, head, B, T, [0, 13], 2, 5, advance=True)


@pytest.mark.parametrize("N,K,gated", [(2560, 2560, False), (2560, 6912, False), (6912, 2560, True)])
def test_prefill_gemm_c5_token_count(ctx, orc, nnhip, N, K, gated):
    """The prefill GEMM at config C5's size: 16 sequences x 2048 tokens = 32768 tokens per call, the
    o / q and fc2 shapes (2560 x 2560, 2560 x 6912) and fc1 with the gated epilogue (13824 fused
    gate/up rows over d = 2560 into 6912 features). Against the oracle's CpuEngine restatement
    (src/int8_act_test.cpp:210-236 order): every row on a band of 256 tokens in the middle of the
    call and sampled rows (every 97th, the last) over all 32768 tokens; the scales bit for bit."""
    import torch
    M = 32768
    say(f"prefill GEMM at C5 size N={N} K={K} M={M} gated={gated}")
    rows_w = 2 * N if gated else N
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xC5 + N + K)
    W = torch.randn((rows_w, K), generator=gen, device="cuda") * 0.02
    tau_d = W.abs().mean(dim=1).contiguous()           # per-row absmean, as a converted checkpoint has
    wq_d = ctx.trit_pack(W, tau_d)
    del W
    b = normal((rows_w,), 0xC6 + N, 0.0, 0.1)
    X_d = torch.randn((K, M), generator=gen, device="cuda")
    xi, s_d, rs = ctx.act_quant_i8(X_d)
    X = host(X_d)
    del X_d
    s = orc.act_scale(X)
    assert np.array_equal(host(s_d), s)
    xq = orc.quantize_i8(X, s, True)
    del X
    wq, tau = host(wq_d).view(np.uint32), host(tau_d)
    if gated:
        wo, to, bo = ctx.glu_interleave(wq_d, tau_d, dev(b), N, K)
        Y = host(ctx.ternary_matmul_glu(ctx.repack(wo, K), to, xi, s_d, rs, N, K, M, 0, bias=bo))
    else:
        Y = host(ctx.ternary_matmul(ctx.repack(wq_d, K), tau_d, xi, s_d, rs, N, K, M, bias=dev(b)))

    def ref(rows, m0, m1):
        """oracle output rows `rows` (features when gated) for tokens [m0, m1), m0 % 4 == 0"""
        xs = np.ascontiguousarray(xq[:, m0 // 4:(m1 + 3) // 4])
        if not gated:
            y = orc.matmul_q_i8_rowblock(wq[rows], tau[rows], xs, s[m0:m1], K, m1 - m0)
            return orc.add_row_broadcast(y, b[rows])
        both = np.concatenate([rows, rows + N])           # gate rows, then their up rows
        y1 = orc.add_row_broadcast(orc.matmul_q_i8_rowblock(wq[both], tau[both], xs, s[m0:m1], K, m1 - m0), b[both])
        return orc.glu(y1, 0)

    m0 = 16384 + 128
    band = ref(np.arange(N), m0, m0 + 256)
    assert same_bits(Y[:, m0:m0 + 256], band), "band of 256 tokens differs"
    rows = np.unique(np.concatenate([np.arange(0, N, 97), [N - 1]]))
    assert same_bits(Y[rows], ref(rows, 0, M)), "sampled rows differ"

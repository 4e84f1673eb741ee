"""Pins the oracle's batched decode-step functions (oracle/nn_oracle.c: RoPE table and
rotation, decode attention over a KV cache, embedding gather, greedy argmax) against what the
reference and the mathematics fix: float64 recomputations written independently of the
oracle's loops (complex rotation, textbook softmax attention), closed forms (one cached
position returns v exactly, equal keys give the mean of the values), the grouped-query head map
with distinct KV heads, and the reference's own greedy rule on ties and NaN.
Reference citations are file:line in neuralnet-cpp-dev/neuralnet.cpp v1.18.0.
"""
import math

import numpy as np
import pytest

from conftest import normal, uniform


# ---------------------------------------------------------------- RoPE

def test_rope_table_matches_library_host_table(orc, nnhip):
    """The oracle's table and libnn-hip.so's nnhip_rope_table (both the float formula of
    compute_position_encoding.hpp:64-80) agree bit for bit."""
    for dk, L in ((64, 300), (128, 2200), (256, 40)):
        c0, s0 = orc.rope_table(dk, L)
        c1, s1 = nnhip.rope_table(dk, L)
        assert np.array_equal(c0.view(np.uint32), c1.view(np.uint32))
        assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32))


def test_rope_table_against_float64(orc):
    """cos/sin of pos / 10000^(2j/dk): position 0 is the identity; elsewhere within the float
    rounding of theta (|d theta| <= 2^-23 theta) of float64 values."""
    dk, L = 128, 2200
    c, s = orc.rope_table(dk, L)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    pos = np.arange(L, dtype=np.float64)[:, None]
    j = np.arange(dk // 2, dtype=np.float64)[None, :]
    theta = pos / np.power(10000.0, 2.0 * j / dk)
    bound = 2e-7 + 2.0 ** -22 * theta
    assert np.all(np.abs(c - np.cos(theta)) <= bound)
    assert np.all(np.abs(s - np.sin(theta)) <= bound)
    # a plausible mistake (exponent j/dk instead of 2j/dk) is far outside the bound
    wrong = pos / np.power(10000.0, j / dk)
    assert np.max(np.abs(c - np.cos(wrong))) > 0.1


def test_rope_apply_is_the_llama_rotation(orc):
    """q*cos + rotate_half(q)*sin == the complex rotation (x_j + i x_{j+dk/2}) e^{i theta_j}."""
    dk = 128
    c, s = orc.rope_table(dk, 3000)
    x = normal((dk,), 0xC501)
    for p in (0, 1, 7, 1000, 2999):
        out = orc.rope_apply(x, c[p], s[p]).astype(np.float64)
        z = (x[:dk // 2].astype(np.float64) + 1j * x[dk // 2:].astype(np.float64)) * \
            (c[p].astype(np.float64) + 1j * s[p].astype(np.float64))
        ref = np.concatenate([z.real, z.imag])
        assert np.max(np.abs(out - ref)) <= 4e-7 * np.max(np.abs(x))
    # unit vectors: e_j -> cos at j, sin at j + dk/2 (the sign convention)
    for j in (0, 5, 63):
        e = np.zeros(dk, np.float32)
        e[j] = 1.0
        out = orc.rope_apply(e, c[11], s[11])
        assert out[j] == c[11, j] and out[j + dk // 2] == s[11, j]
        assert np.count_nonzero(out) <= 2


# ---------------------------------------------------------------- decode attention

def _rot64(x, cr, sr):
    h = x.shape[0] // 2
    z = (x[:h] + 1j * x[h:]) * (cr + 1j * sr)
    return np.concatenate([z.real, z.imag])


def _attn64(q, K, V, H, Hkv, dk, pos, cos, sin, scale):
    """Textbook float64 decode attention (independent of the oracle): rotate, GQA map h // R,
    softmax over t <= pos, weighted sum of values."""
    B = q.shape[1]
    R = H // Hkv
    out = np.zeros((H * dk, B))
    for b in range(B):
        p = pos[b]
        for h in range(H):
            g = h // R
            qh = q[h * dk:(h + 1) * dk, b].astype(np.float64)
            if cos is not None:
                qh = _rot64(qh, cos[p].astype(np.float64), sin[p].astype(np.float64))
            Kg = K[b, :p + 1, g * dk:(g + 1) * dk].astype(np.float64)
            Vg = V[b, :p + 1, g * dk:(g + 1) * dk].astype(np.float64)
            sc = (Kg @ qh) * scale
            w = np.exp(sc - sc.max())
            w /= w.sum()
            out[h * dk:(h + 1) * dk, b] = w @ Vg
    return out


def _case(B, H, Hkv, dk, max_len, pos, seed, rope=True):
    q = normal((H * dk, B), seed)
    k = normal((Hkv * dk, B), seed + 1)
    v = normal((Hkv * dk, B), seed + 2)
    kc = normal((B, max_len, Hkv * dk), seed + 3)
    vc = normal((B, max_len, Hkv * dk), seed + 4)
    return q, k, v, kc, vc


@pytest.mark.parametrize("B,H,Hkv,dk,pos,rope", [
    (1, 4, 4, 64, [0], True),
    (2, 8, 2, 128, [5, 130], True),
    (3, 20, 5, 128, [127, 128, 300], True),
    (2, 4, 1, 256, [40, 3], False),
])
def test_attention_decode_against_float64(orc, B, H, Hkv, dk, pos, rope):
    max_len = 320
    q, k, v, kc, vc = _case(B, H, Hkv, dk, max_len, pos, 0xA770 + B)
    cos, sin = orc.rope_table(dk, max_len) if rope else (None, None)
    kc0, vc0 = kc.copy(), vc.copy()
    scale = np.float32(1.0) / np.float32(math.sqrt(dk))
    out = orc.attention_decode(q, k, v, H, Hkv, dk, pos, kc, vc, float(scale), cos, sin)
    # the cache: row pos[b] = rotated new key / the new value, every other row unchanged
    for b in range(B):
        p = pos[b]
        for g in range(Hkv):
            kn = k[g * dk:(g + 1) * dk, b]
            if rope:
                want = orc.rope_apply(kn, cos[p], sin[p])
                assert np.max(np.abs(_rot64(kn.astype(np.float64), cos[p].astype(np.float64),
                                            sin[p].astype(np.float64)) - want)) <= 4e-7 * np.max(np.abs(kn))
            else:
                want = kn
            assert np.array_equal(kc[b, p, g * dk:(g + 1) * dk], want)
            assert np.array_equal(vc[b, p, g * dk:(g + 1) * dk], v[g * dk:(g + 1) * dk, b])
        mask = np.ones(max_len, bool)
        mask[p] = False
        assert np.array_equal(kc[b, mask], kc0[b, mask]) and np.array_equal(vc[b, mask], vc0[b, mask])
    ref = _attn64(q, kc, vc, H, Hkv, dk, pos, cos, sin, float(scale))
    assert np.max(np.abs(out - ref)) <= 2e-6 * max(1.0, np.max(np.abs(ref)))


def test_attention_single_position_returns_v_exactly(orc):
    """pos = 0: softmax over one score is exactly 1, so out = v of the head's KV head; with
    distinct KV heads this pins the grouped-query map h -> h // (H / Hkv)."""
    B, H, Hkv, dk = 2, 6, 3, 64
    q, k, v, kc, vc = _case(B, H, Hkv, dk, 4, [0, 0], 0x51)
    cos, sin = orc.rope_table(dk, 4)
    out = orc.attention_decode(q, k, v, H, Hkv, dk, [0, 0], kc, vc, 0.125, cos, sin)
    for h in range(H):
        g = h // (H // Hkv)
        assert np.array_equal(out[h * dk:(h + 1) * dk], v[g * dk:(g + 1) * dk])
        # the map h % Hkv would read another head for h = 1, 2, 4
        if h % Hkv != g:
            assert not np.array_equal(out[h * dk:(h + 1) * dk], v[(h % Hkv) * dk:(h % Hkv + 1) * dk])


def test_attention_equal_keys_give_the_mean(orc):
    """All cached keys equal (and no rotation): uniform weights, out = mean of the values."""
    B, H, Hkv, dk, p = 1, 2, 1, 64, 99
    q = normal((H * dk, B), 0x61)
    key = normal((dk,), 0x62)
    k = key[:, None].copy()
    v = normal((dk, B), 0x63)
    kc = np.tile(key, (B, 128, 1)).astype(np.float32)
    vc = normal((B, 128, dk), 0x64)
    out = orc.attention_decode(q, k, v, H, Hkv, dk, [p], kc, vc, 0.125)
    mean = vc[0, :p + 1].astype(np.float64).mean(axis=0)
    for h in range(H):
        assert np.max(np.abs(out[h * dk:(h + 1) * dk, 0] - mean)) <= 2e-6


# ---------------------------------------------------------------- gather / greedy

def test_embedding_gather(orc):
    table = normal((50, 24), 0x71)
    ids = np.array([3, 0, 49, 3, -1, 50], np.int32)
    out = orc.embedding_gather(table, ids)
    for b, i in enumerate(ids):
        if 0 <= i < 50:
            assert np.array_equal(out[:, b], table[i])
        else:
            assert np.all(np.isnan(out[:, b]))


def test_argmax_greedy_rule(orc):
    """sample_next_token_'s greedy loop (compute_layer_base.hpp:1152-1160): first index of the
    largest value; NaN never replaces the best, and a NaN at index 0 keeps index 0."""
    L = uniform((1000, 4), 0x81)
    assert orc.argmax_cols(L).tolist() == np.argmax(L, axis=0).tolist()
    L = np.zeros((6, 5), np.float32)
    L[:, 0] = [1, 3, 3, 2, 3, 0]                 # ties -> first
    L[:, 1] = [np.nan, 5, 6, 7, 1, 0]            # NaN at 0 -> 0
    L[:, 2] = [1, np.nan, 2, np.nan, 0, 1]       # NaN elsewhere ignored
    L[:, 3] = -np.inf                            # all equal -> 0
    L[:, 4] = [-1, -2, np.inf, np.inf, 0, 0]
    assert orc.argmax_cols(L).tolist() == [1, 0, 2, 0, 2]


def test_round_f16_matches_numpy(orc):
    """orc_round_f16 (the element of a compute = F16 KV cache) bit for bit against numpy's
    float32 -> float16 conversion (round to nearest, ties to even): every 1031st float32 bit
    pattern, plus every pattern around the f16 overflow threshold, the normal/subnormal boundary
    and the f16 ties of a range of exponents."""
    bits = np.arange(0, 1 << 32, 1031, dtype=np.uint64).astype(np.uint32)
    extra = [np.arange(0x477F0000, 0x47810000, dtype=np.uint32),   # 65280 .. 66048 (overflow)
             np.arange(0x38700000, 0x38900000, dtype=np.uint32),   # around 2^-14
             np.arange(0x33000000, 0x33800000, 997, dtype=np.uint32)]  # around 2^-25
    ties = (np.arange(0x38800000, 0x477FF000, 0x2000, dtype=np.uint64) + 0x1000).astype(np.uint32)  # exact ties
    allb = np.concatenate([bits] + extra + [ties, ties + 1, ties - 1])
    allb = np.concatenate([allb, allb | np.uint32(0x80000000)])
    x = allb.view(np.float32)
    got = orc.round_f16(x)
    with np.errstate(over="ignore", invalid="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))

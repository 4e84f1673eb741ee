"""ctypes binding of oracle/libnnoracle.so (the CPU restatement in nn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline. The shipped library never
uses it. Arrays are numpy; packed containers are uint32 arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnnoracle.so")

_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t

_lib = None


def build() -> None:
    """Compile libnnoracle.so with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def release_lib():
    """The same oracle built with the reference's Release flags (oracle/Makefile), for the timed CPU
    baseline: the x86-64-v4 (AVX-512) build when this host's CPU has the subsets v4 needs, else the
    x86-64-v3 build. Returns (library, "v4" or "v3")."""
    global _rel
    if _rel is None:
        flags = set()
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("flags"):
                        flags = set(line.split(":", 1)[1].split())
                        break
        except OSError:
            pass
        level = "v4" if {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags else "v3"
        path = os.path.join(_HERE, f"libnnoracle_rel_{level}.so")
        if not os.path.exists(path):
            build()
        _rel = (_load(path), level)
    return _rel


_rel = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _load(LIB_PATH)
    return _lib


def _load(path) -> ctypes.CDLL:
    """Load one build of the oracle and declare every entry's signature."""
    L = ctypes.CDLL(path)
    sig = {
        "orc_fill_uniform": (None, [_f32p, _sz, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
        "orc_fill_normal": (None, [_f32p, _sz, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
        "orc_trit_words_per_row": (_sz, [_sz]),
        "orc_trit_code": (ctypes.c_uint32, [ctypes.c_float, ctypes.c_float]),
        "orc_trit_pack": (None, [_f32p, _f32p, _sz, _sz, _u32p]),
        "orc_trit_at": (ctypes.c_int, [_u32p, _sz]),
        "orc_row_absmean": (None, [_f32p, _sz, _sz, _f32p]),
        "orc_i8_words_per_row": (_sz, [_sz]),
        "orc_quantize_one": (ctypes.c_int8, [ctypes.c_float, ctypes.c_float]),
        "orc_col_absmax": (None, [_f32p, _sz, _sz, _f32p]),
        "orc_act_scale": (None, [_f32p, _sz, _sz, _f32p]),
        "orc_quantize_i8": (None, [_f32p, _f32p, _sz, _sz, ctypes.c_int, _u32p]),
        "orc_unpack_i8": (None, [_u32p, _sz, _sz, _f32p]),
        "orc_matmul_q_i8_acc": (None, [_u32p, _u32p, _sz, _sz, _sz, _i32p]),
        "orc_matmul_q_i8": (None, [_u32p, _f32p, _u32p, _f32p, _sz, _sz, _sz, _f32p]),
        "orc_matmul_q_i8_rowblock": (ctypes.c_int, [_u32p, _f32p, _u32p, _f32p, _sz, _sz, _sz, _f32p, ctypes.c_int]),
        "orc_add_row_broadcast": (None, [_f32p, _f32p, _sz, _sz]),
        "orc_matmul_q": (None, [_u32p, _f32p, _f32p, _sz, _sz, _sz, _f32p]),
        "orc_matmul_q_t": (None, [_u32p, _f32p, _f32p, _sz, _sz, _sz, _f32p]),
        "orc_rmsnorm": (None, [_f32p, _f32p, ctypes.c_float, _sz, _sz, _f32p]),
        "orc_layernorm": (None, [_f32p, _f32p, _f32p, ctypes.c_float, _sz, _sz, _f32p]),
        "orc_rmsnorm_quant_i8": (None, [_f32p, _f32p, ctypes.c_float, _sz, _sz, _u32p, _f32p]),
        "orc_exp": (ctypes.c_float, [ctypes.c_float]),
        "orc_exp_array": (None, [_f32p, _sz, _f32p]),
        "orc_glu_one": (ctypes.c_float, [ctypes.c_float, ctypes.c_float, ctypes.c_int]),
        "orc_glu": (None, [_f32p, _sz, _sz, ctypes.c_int, _f32p]),
        "orc_glu_src_row": (ctypes.c_long, [_sz, _sz]),
        "orc_glu_interleave": (None, [_u32p, _f32p, _f32p, _sz, _sz, _u32p, _f32p, _f32p]),
        "orc_ffn_glu_i8": (None, [_f32p, _f32p, ctypes.c_float, _sz, _sz, _sz, ctypes.c_int,
                                  _u32p, _f32p, _f32p, _f32p, ctypes.c_float, _u32p, _f32p, _f32p, ctypes.c_int,
                                  _f32p, _f32p]),
        "orc_rope_table": (None, [_sz, _sz, _f32p, _f32p]),
        "orc_rope_apply": (None, [_f32p, _sz, _f32p, _f32p, _f32p]),
        "orc_attention_decode": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _i32p, _f32p, _f32p, _f32p,
                                        _f32p, _sz, ctypes.c_float, _f32p]),
        "orc_attention_decode_ct": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _i32p, _f32p, _f32p, _f32p,
                                           _f32p, _sz, ctypes.c_float, ctypes.c_int, _f32p]),
        "orc_round_f16": (ctypes.c_float, [ctypes.c_float]),
        "orc_round_f16_n": (None, [_f32p, _sz, _f32p]),
        "orc_embedding_gather": (None, [_f32p, _i32p, _sz, _sz, _sz, _f32p]),
        "orc_argmax": (ctypes.c_int32, [_f32p, _sz, _sz]),
        "orc_repacked_words": (_sz, [_sz, _sz]),
        "orc_repack": (None, [_u32p, _sz, _sz, _u32p]),
        "orc_unrepack": (None, [_u32p, _sz, _sz, _u32p]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    return L


def _p(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


def fill_uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform(_p(out, ctypes.c_float), n, seed, lo, hi)
    return out


def fill_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(_p(out, ctypes.c_float), n, seed, mean, std)
    return out


def trit_words_per_row(K: int) -> int:
    return (K + 15) // 16


def i8_words_per_row(cols: int) -> int:
    return (cols + 3) // 4


def trit_pack(W: np.ndarray, tau: np.ndarray) -> np.ndarray:
    W = _f32(W)
    N, K = W.shape
    tau = _f32(tau).reshape(N)
    out = np.empty((N, trit_words_per_row(K)), np.uint32)
    lib().orc_trit_pack(_p(W, ctypes.c_float), _p(tau, ctypes.c_float), N, K, _p(out, ctypes.c_uint32))
    return out


def row_absmean(W: np.ndarray) -> np.ndarray:
    W = _f32(W)
    N, K = W.shape
    tau = np.empty(N, np.float32)
    lib().orc_row_absmean(_p(W, ctypes.c_float), N, K, _p(tau, ctypes.c_float))
    return tau


def quantize_one(x: float, s: float) -> int:
    return int(lib().orc_quantize_one(x, s))


def col_absmax(X: np.ndarray) -> np.ndarray:
    X = _f32(X)
    r, c = X.shape
    out = np.empty(c, np.float32)
    lib().orc_col_absmax(_p(X, ctypes.c_float), r, c, _p(out, ctypes.c_float))
    return out


def act_scale(X: np.ndarray) -> np.ndarray:
    X = _f32(X)
    r, c = X.shape
    out = np.empty(c, np.float32)
    lib().orc_act_scale(_p(X, ctypes.c_float), r, c, _p(out, ctypes.c_float))
    return out


def quantize_i8(x: np.ndarray, scale: np.ndarray, col_scale: bool = True) -> np.ndarray:
    x = _f32(x)
    rows, cols = x.shape
    scale = _f32(scale).reshape(-1)
    out = np.empty((rows, i8_words_per_row(cols)), np.uint32)
    lib().orc_quantize_i8(_p(x, ctypes.c_float), _p(scale, ctypes.c_float), rows, cols, int(col_scale),
                          _p(out, ctypes.c_uint32))
    return out


def unpack_i8(packed: np.ndarray, cols: int) -> np.ndarray:
    packed = _u32(packed)
    rows = packed.shape[0]
    out = np.empty((rows, cols), np.float32)
    lib().orc_unpack_i8(_p(packed, ctypes.c_uint32), rows, cols, _p(out, ctypes.c_float))
    return out


def matmul_q_i8_acc(wq: np.ndarray, xq: np.ndarray, K: int, M: int) -> np.ndarray:
    wq, xq = _u32(wq), _u32(xq)
    N = wq.shape[0]
    acc = np.empty((N, M), np.int32)
    lib().orc_matmul_q_i8_acc(_p(wq, ctypes.c_uint32), _p(xq, ctypes.c_uint32), N, K, M,
                              _p(acc, ctypes.c_int32))
    return acc


def matmul_q_i8(wq, tau, xq, s, K: int, M: int) -> np.ndarray:
    wq, xq = _u32(wq), _u32(xq)
    N = wq.shape[0]
    tau, s = _f32(tau).reshape(N), _f32(s).reshape(M)
    Y = np.empty((N, M), np.float32)
    lib().orc_matmul_q_i8(_p(wq, ctypes.c_uint32), _p(tau, ctypes.c_float), _p(xq, ctypes.c_uint32),
                          _p(s, ctypes.c_float), N, K, M, _p(Y, ctypes.c_float))
    return Y


def matmul_q_i8_rowblock(wq, tau, xq, s, K: int, M: int, threads: int = 0, L=None) -> np.ndarray:
    """CpuEngine restatement (row-block decode + dense f32 microkernel); L selects another build of
    the oracle (release_lib()[0] for the timed baseline)."""
    wq, xq = _u32(wq), _u32(xq)
    N = wq.shape[0]
    tau, s = _f32(tau).reshape(N), _f32(s).reshape(M)
    Y = np.empty((N, M), np.float32)
    rc = (L or lib()).orc_matmul_q_i8_rowblock(_p(wq, ctypes.c_uint32), _p(tau, ctypes.c_float),
                                        _p(xq, ctypes.c_uint32), _p(s, ctypes.c_float), N, K, M,
                                        _p(Y, ctypes.c_float), threads)
    if rc != 0:
        raise ValueError("rowblock path is exact only for 127*K < 2^24")
    return Y


def matmul_q(wq: np.ndarray, tau: np.ndarray, B: np.ndarray, K: int) -> np.ndarray:
    """Y (N, M) = (tau o trit(wq)) . B in float64, rounded once (ref_gemm, transA = 0)."""
    wq, B = _u32(wq), _f32(B)
    N, M = wq.shape[0], B.shape[1]
    tau = _f32(tau).reshape(N)
    Y = np.empty((N, M), np.float32)
    lib().orc_matmul_q(_p(wq, ctypes.c_uint32), _p(tau, ctypes.c_float), _p(B, ctypes.c_float), N, K, M,
                       _p(Y, ctypes.c_float))
    return Y


def matmul_q_t(A: np.ndarray, tau: np.ndarray, B: np.ndarray, M: int) -> np.ndarray:
    """Y (M, N) = (tau o trit(A))^T . B, A (K, ceil(M/16)) (ref_gemm, transA = 1)."""
    A, B = _u32(A), _f32(B)
    K, N = A.shape[0], B.shape[1]
    tau = _f32(tau).reshape(K)
    Y = np.empty((M, N), np.float32)
    lib().orc_matmul_q_t(_p(A, ctypes.c_uint32), _p(tau, ctypes.c_float), _p(B, ctypes.c_float), K, M, N,
                         _p(Y, ctypes.c_float))
    return Y


def add_row_broadcast(Y: np.ndarray, b: np.ndarray) -> np.ndarray:
    Y = _f32(Y).copy()
    N, M = Y.shape
    b = _f32(b).reshape(N)
    lib().orc_add_row_broadcast(_p(Y, ctypes.c_float), _p(b, ctypes.c_float), N, M)
    return Y


def rmsnorm(X: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    X = _f32(X)
    F, M = X.shape
    gamma = _f32(gamma).reshape(F)
    out = np.empty((F, M), np.float32)
    lib().orc_rmsnorm(_p(X, ctypes.c_float), _p(gamma, ctypes.c_float), eps, F, M, _p(out, ctypes.c_float))
    return out


def layernorm(X: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float) -> np.ndarray:
    """LayerNorm of each token (column) of X (F, M), include/neuralnet.cpp/compute_layer_mlp.hpp:529-545."""
    X = _f32(X)
    F, M = X.shape
    gamma = _f32(gamma).reshape(F)
    beta = _f32(beta).reshape(F)
    out = np.empty((F, M), np.float32)
    lib().orc_layernorm(_p(X, ctypes.c_float), _p(gamma, ctypes.c_float), _p(beta, ctypes.c_float), eps, F, M,
                        _p(out, ctypes.c_float))
    return out


def rmsnorm_quant_i8(X: np.ndarray, gamma: np.ndarray, eps: float):
    X = _f32(X)
    F, M = X.shape
    gamma = _f32(gamma).reshape(F)
    xq = np.empty((F, i8_words_per_row(M)), np.uint32)
    s = np.empty(M, np.float32)
    lib().orc_rmsnorm_quant_i8(_p(X, ctypes.c_float), _p(gamma, ctypes.c_float), eps, F, M,
                               _p(xq, ctypes.c_uint32), _p(s, ctypes.c_float))
    return xq, s


ACT_SWIGLU, ACT_RELU2 = 0, 1


def exp(x) -> np.ndarray:
    """Element-wise orc_exp (this build's fp32 exp, identical to the GPU kernels')."""
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    lib().orc_exp_array(_p(x, ctypes.c_float), x.size, _p(out, ctypes.c_float))
    return out


def glu(Y1: np.ndarray, act: int = ACT_SWIGLU) -> np.ndarray:
    """(2F, M) fused fc1 output -> (F, M) gated activation (gate rows first, then up)."""
    Y1 = _f32(Y1)
    F, M = Y1.shape[0] // 2, Y1.shape[1]
    out = np.empty((F, M), np.float32)
    lib().orc_glu(_p(Y1, ctypes.c_float), F, M, act, _p(out, ctypes.c_float))
    return out


def glu_src_rows(F: int) -> np.ndarray:
    """Reference row of every interleaved row (-1 for padding), length 2*roundup(F, 8)."""
    rows = 2 * ((F + 7) // 8 * 8)
    return np.array([lib().orc_glu_src_row(r, F) for r in range(rows)], np.int64)


def glu_interleave(wq: np.ndarray, tau: np.ndarray, bias, F: int, K: int):
    """Fused gate/up container (2F, ceil(K/16)) -> interleaved container, tau and bias."""
    wq = _u32(wq)
    tau = _f32(tau).reshape(-1)
    rows = 2 * ((F + 7) // 8 * 8)
    wo = np.empty((rows, trit_words_per_row(K)), np.uint32)
    to = np.empty(rows, np.float32)
    bo = np.empty(rows, np.float32)
    bp = _p(_f32(bias).reshape(-1), ctypes.c_float) if bias is not None else None
    lib().orc_glu_interleave(_p(wq, ctypes.c_uint32), _p(tau, ctypes.c_float), bp, F, K,
                             _p(wo, ctypes.c_uint32), _p(to, ctypes.c_float), _p(bo, ctypes.c_float))
    return wo, to, bo


def ffn_glu_i8(X, gamma, eps, F, wq1, tau1, b1, wq2, tau2, b2, act: int = ACT_SWIGLU, threads: int = 0,
               gamma_sub=None, eps_sub: float = 1e-5, L=None):
    """Config C4 block: [RMSNorm] -> int8 -> fc1 (2F) -> gated activation -> [SubLN RMSNorm] ->
    int8 -> fc2. Returns (Y (d, M), h (F, M)); h is the gated output before SubLN."""
    X = _f32(X)
    d, M = X.shape
    Y = np.empty((d, M), np.float32)
    h = np.empty((F, M), np.float32)
    fp = lambda a: None if a is None else _p(_f32(a).reshape(-1), ctypes.c_float)
    keep = [None if a is None else _f32(a).reshape(-1) for a in (gamma, tau1, b1, tau2, b2, gamma_sub)]
    g_, t1, b1_, t2, b2_, gs_ = keep
    wq1, wq2 = _u32(wq1), _u32(wq2)
    (L or lib()).orc_ffn_glu_i8(_p(X, ctypes.c_float), fp(g_), eps, d, F, M, act, _p(wq1, ctypes.c_uint32), fp(t1), fp(b1_),
                         fp(gs_), eps_sub, _p(wq2, ctypes.c_uint32), fp(t2), fp(b2_), threads, _p(h, ctypes.c_float),
                         _p(Y, ctypes.c_float))
    return Y, h


def repacked_words(N: int, K: int) -> int:
    return int(lib().orc_repacked_words(N, K))


def repack(wq: np.ndarray, K: int) -> np.ndarray:
    wq = _u32(wq)
    N = wq.shape[0]
    out = np.empty(repacked_words(N, K), np.uint32)
    lib().orc_repack(_p(wq, ctypes.c_uint32), N, K, _p(out, ctypes.c_uint32))
    return out


def unrepack(rp: np.ndarray, N: int, K: int) -> np.ndarray:
    rp = _u32(rp)
    out = np.empty((N, trit_words_per_row(K)), np.uint32)
    lib().orc_unrepack(_p(rp, ctypes.c_uint32), N, K, _p(out, ctypes.c_uint32))
    return out


# ---- batched decode step (config C5)

def rope_table(dk: int, max_len: int):
    """(cos, sin), each (max_len, dk/2) float32, as RotaryEmbedding::fill_pos_column_."""
    c = np.empty((max_len, dk // 2), np.float32)
    s = np.empty((max_len, dk // 2), np.float32)
    lib().orc_rope_table(dk, max_len, _p(c, ctypes.c_float), _p(s, ctypes.c_float))
    return c, s


def rope_apply(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    """x*cos + rotate_half(x)*sin for one head vector x (dk)."""
    x, c, s = _f32(x), _f32(cos_row), _f32(sin_row)
    out = np.empty_like(x)
    lib().orc_rope_apply(_p(x, ctypes.c_float), x.shape[0], _p(c, ctypes.c_float), _p(s, ctypes.c_float),
                         _p(out, ctypes.c_float))
    return out


def attention_decode(q, k, v, H: int, Hkv: int, dk: int, pos, k_cache, v_cache, scale: float,
                     cos=None, sin=None, cache_f16: bool = False):
    """One decode step for B sequences; q (H*dk, B), k/v (Hkv*dk, B), caches (B, max_len, Hkv*dk)
    are updated IN PLACE (row pos[b] written). Returns out (H*dk, B). cache_f16: the appended rows
    are rounded to f16 before use (the caches of compute = F16, held here as float32 values)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B = q.shape[1]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert k_cache.dtype == np.float32 and k_cache.flags["C_CONTIGUOUS"]
    assert v_cache.dtype == np.float32 and v_cache.flags["C_CONTIGUOUS"]
    max_len = k_cache.shape[1]
    out = np.empty((H * dk, B), np.float32)
    keep = (None if cos is None else _f32(cos), None if sin is None else _f32(sin))
    cp = None if keep[0] is None else _p(keep[0], ctypes.c_float)
    sp = None if keep[1] is None else _p(keep[1], ctypes.c_float)
    lib().orc_attention_decode_ct(_p(q, ctypes.c_float), _p(k, ctypes.c_float), _p(v, ctypes.c_float), B, H, Hkv,
                                  dk, _p(pos, ctypes.c_int32), cp, sp, _p(k_cache, ctypes.c_float),
                                  _p(v_cache, ctypes.c_float), max_len, scale, 1 if cache_f16 else 0,
                                  _p(out, ctypes.c_float))
    return out


def round_f16(x) -> np.ndarray:
    """Elementwise orc_round_f16: the nearest f16 value of each float32 (ties to even), as float32."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_round_f16_n(_p(x, ctypes.c_float), x.size, _p(out, ctypes.c_float))
    return out


def embedding_gather(table: np.ndarray, ids) -> np.ndarray:
    table = _f32(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    V, d = table.shape
    out = np.empty((d, ids.shape[0]), np.float32)
    lib().orc_embedding_gather(_p(table, ctypes.c_float), _p(ids, ctypes.c_int32), V, d, ids.shape[0],
                               _p(out, ctypes.c_float))
    return out


def argmax_cols(L: np.ndarray) -> np.ndarray:
    """Greedy token per column of logits (V, B)."""
    L = _f32(L)
    V, B = L.shape
    flat = L.reshape(-1)
    return np.array([lib().orc_argmax(_p(flat[b:], ctypes.c_float), V, B) for b in range(B)], np.int32)


# ---- helpers on the reference containers (pure numpy; used by tests to cross-check) ----

def container_to_int8(xq: np.ndarray, cols: int) -> np.ndarray:
    """(rows, ceil(cols/4)) u32 container -> (rows, cols) int8."""
    b = _u32(xq).view(np.uint8).reshape(xq.shape[0], -1)[:, :cols]
    return b.view(np.int8).copy()


def trits_of(wq: np.ndarray, K: int) -> np.ndarray:
    """(N, ceil(K/16)) packed words -> (N, K) int8 trits (code - 2)."""
    wq = _u32(wq)
    shifts = (2 * np.arange(16, dtype=np.uint32))
    codes = (wq[:, :, None] >> shifts[None, None, :]) & 3
    return (codes.reshape(wq.shape[0], -1)[:, :K].astype(np.int8) - 2)

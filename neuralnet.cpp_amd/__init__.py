"""Python binding (ctypes) of libnn-hip.so — the MI355X BitLinear W1.58A8 engine.

The product is the C ABI in include/nnhip.h and the C++ nn:: engine layer built into the
same library; this module is plumbing for the tests and bench.py. Device memory comes from
torch (CUDA/HIP tensors), and every call runs on torch's current stream, so it is ordered
with torch's own work. There is no CPU fallback: if libnn-hip.so is missing or no gfx950
device is visible, the calls raise.

The directory name contains a dot, so load it by path:
    spec = importlib.util.spec_from_file_location(
        "nnhip_py", "neuralnet.cpp_amd/__init__.py",
        submodule_search_locations=["neuralnet.cpp_amd"])
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(_HERE, "libnn-hip.so")
HEADER_PATH = os.path.join(ROOT, "include", "nnhip.h")

TILE_K = 256
TILE_ROWS = 16
GEMV_MAX_M = 16


class NNHipError(RuntimeError):
    """A libnn-hip.so call returned a status other than NNHIP_OK."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


def build(jobs: int = 8) -> None:
    """Compile libnn-hip.so in-tree with neuralnet.cpp_amd/Makefile (hipcc, gfx950)."""
    subprocess.run(["make", "-s", "-C", _HERE, f"-j{jobs}"], check=True)


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_st = ctypes.c_int
_f = ctypes.c_float


class GemvDesc(ctypes.Structure):
    _fields_ = [("rp", _vp), ("tau", _vp), ("xi", _vp), ("s", _vp), ("rowsum", _vp),
                ("bias", _vp), ("y", _vp), ("N", ctypes.c_uint64), ("K", ctypes.c_uint64),
                ("M", ctypes.c_uint64)]


# name -> (restype, argtypes); every nnhip_* symbol of include/nnhip.h
SIGNATURES = {
    "nnhip_last_error": (ctypes.c_char_p, []),
    "nnhip_version": (ctypes.c_char_p, []),
    "nnhip_fnv1a64": (ctypes.c_uint64, [_vp, _sz]),
    "nnhip_device_count": (_st, [ctypes.POINTER(ctypes.c_int)]),
    "nnhip_ctx_create": (_st, [ctypes.c_int, ctypes.POINTER(_vp)]),
    "nnhip_ctx_destroy": (_st, [_vp]),
    "nnhip_ctx_set_stream": (_st, [_vp, _vp]),
    "nnhip_ctx_reset_stream": (_st, [_vp]),
    "nnhip_ctx_get_stream": (_st, [_vp, ctypes.POINTER(_vp)]),
    "nnhip_sync": (_st, [_vp]),
    "nnhip_ctx_set_gemm_tile": (_st, [_vp, _st]),
    "nnhip_ctx_prefetch_next": (_st, [_vp, _sz, ctypes.POINTER(_vp), ctypes.POINTER(_sz)]),
    "nnhip_malloc": (_st, [_vp, _sz, ctypes.POINTER(_vp)]),
    "nnhip_free": (_st, [_vp, _vp]),
    "nnhip_memcpy_h2d": (_st, [_vp, _vp, _vp, _sz]),
    "nnhip_memcpy_d2h": (_st, [_vp, _vp, _vp, _sz]),
    "nnhip_memcpy_d2d": (_st, [_vp, _vp, _vp, _sz]),
    "nnhip_fill_u32": (_st, [_vp, _vp, ctypes.c_uint32, _sz]),
    "nnhip_device_name": (_st, [ctypes.c_int, ctypes.c_char_p, _sz]),
    "nnhip_convert_f32_f16": (_st, [_vp, _vp, _sz, _vp]),
    "nnhip_convert_f16_f32": (_st, [_vp, _vp, _sz, _vp]),
    "nnhip_row_absmean": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_trit_pack": (_st, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "nnhip_col_reduce_max": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_abs": (_st, [_vp, _vp, _sz, _vp]),
    "nnhip_scale_inplace": (_st, [_vp, _vp, _sz, _f]),
    "nnhip_act_scale": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_quantize_i8": (_st, [_vp, _vp, _vp, _sz, _sz, ctypes.c_int, _vp]),
    "nnhip_unpack_i8": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_matmul_q_i8": (_st, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_matmul_q_i8_noalloc": (_st, [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_add_row_broadcast": (_st, [_vp, _vp, _vp, _sz, _sz]),
    "nnhip_matmul_q": (_st, [_vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _vp, ctypes.c_int]),
    "nnhip_matmul_q_t": (_st, [_vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _vp, ctypes.c_int]),
    "nnhip_rmsnorm": (_st, [_vp, _vp, _vp, _f, _sz, _sz, _vp]),
    "nnhip_layernorm": (_st, [_vp, _vp, _vp, _vp, _f, _sz, _sz, _vp]),
    "nnhip_repacked_bytes": (_sz, [_sz, _sz]),
    "nnhip_repack_ternary": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_unrepack_ternary": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_act_i8_bytes": (_sz, [_sz, _sz]),
    "nnhip_act_quant_i8": (_st, [_vp, _vp, _sz, _sz, _vp, _vp, _vp, _vp]),
    "nnhip_rmsnorm_quant_i8": (_st, [_vp, _vp, _vp, _f, _sz, _sz, _vp, _vp, _vp, _vp]),
    "nnhip_act_i8_from_container": (_st, [_vp, _vp, _sz, _sz, _vp, _vp]),
    "nnhip_act_i8_to_container": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_ternary_matmul": (_st, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_ternary_matmul_f": (_st, [_vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _vp, ctypes.c_int]),
    "nnhip_ternary_matmul_t_f": (_st, [_vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _vp, ctypes.c_int]),
    "nnhip_trit_transpose": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_stream_xor": (_st, [_vp, _vp, _sz, _vp]),
    "nnhip_device_info": (_st, [ctypes.c_int] + [ctypes.POINTER(ctypes.c_int)] * 4),
    "nnhip_ternary_matmul_add": (_st, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_ternary_matmul_add_tokens": (_st, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_ternary_matmul_partial": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp]),
    "nnhip_partial_residual_quant_i8": (_st, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _f, _vp,
                                              _vp, _vp]),
    "nnhip_partial_residual_quant_i8_tokens": (_st, [_vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _f, _vp,
                                              _vp, _vp]),
    "nnhip_ternary_matmul_n": (_st, [_vp, _sz, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                     ctypes.POINTER(_sz), ctypes.POINTER(_vp), _vp, _vp, _vp, _sz, _sz]),
    "nnhip_ternary_matmul_n_tokens": (_st, [_vp, _sz, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                     ctypes.POINTER(_sz), ctypes.POINTER(_vp), _vp, _vp, _vp, _sz, _sz]),
    "nnhip_ffn_glu_i8_add": (_st, [_vp, _vp, _vp, _f, _sz, _sz, _sz, ctypes.c_int, _vp, _vp, _vp, _vp, _f, _vp, _vp,
                                   _vp, _vp, _vp]),
    "nnhip_group_create": (_st, [_vp, ctypes.POINTER(GemvDesc), _sz, ctypes.POINTER(_vp)]),
    "nnhip_group_run": (_st, [_vp, _vp]),
    "nnhip_group_destroy": (_st, [_vp, _vp]),
    "nnhip_gemv_grid_waves": (_sz, [_vp, _sz]),
    "nnhip_group_info": (_st, [_vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "nnhip_glu": (_st, [_vp, _vp, _sz, _sz, ctypes.c_int, _vp]),
    "nnhip_glu_rows": (_sz, [_sz]),
    "nnhip_glu_interleave": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    "nnhip_ternary_matmul_glu": (_st, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_int, _vp]),
    "nnhip_ternary_matmul_glu_tokens": (_st, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_int,
                                              _vp]),
    "nnhip_rmsnorm_quant_i8_tokens": (_st, [_vp, _vp, _vp, _f, _sz, _sz, _vp, _vp, _vp]),
    "nnhip_embedding_rmsnorm_quant_i8_tokens": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _vp, _f, _vp, _vp, _vp, _vp]),
    "nnhip_ffn_glu_workspace_bytes": (_sz, [_sz, _sz, _sz]),
    "nnhip_ffn_glu_i8": (_st, [_vp, _vp, _vp, _f, _sz, _sz, _sz, ctypes.c_int, _vp, _vp, _vp, _vp, _f, _vp, _vp,
                               _vp, _vp]),
    "nnhip_rope_table": (_st, [_sz, _sz, _vp, _vp]),
    "nnhip_attention_workspace_bytes": (_sz, [_sz, _sz, _sz, _sz, _sz]),
    "nnhip_attention_decode": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp, _sz, _f,
                                     _vp]),
    "nnhip_attention_decode_tokens": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp, _sz,
                                            _f, _vp]),
    "nnhip_attention_decode_h": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp, _sz, _f,
                                       _vp]),
    "nnhip_attention_decode_tokens_h": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp,
                                              _sz, _f, _vp]),
    "nnhip_add": (_st, [_vp, _vp, _vp, _sz, _vp]),
    "nnhip_kv_cache_fill": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _sz]),
    "nnhip_kv_cache_fill_h": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _sz]),
    "nnhip_attention_prefill": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _f, _vp]),
    "nnhip_attention_prefill_h": (_st, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _f, _vp]),
    "nnhip_copy_columns": (_st, [_vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp]),
    "nnhip_embedding_gather": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_embedding_gather_tokens": (_st, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "nnhip_argmax_cols": (_st, [_vp, _vp, _sz, _sz, _vp]),
    "nnhip_argmax_rows": (_st, [_vp, _vp, _sz, _sz, _vp, _vp]),
}

ACT_SWIGLU, ACT_RELU2GLU = 0, 1
# prefill GEMM block tiles (nnhip_ctx_set_gemm_tile)
GEMM_TILE_AUTO, GEMM_TILE_256x128, GEMM_TILE_128x128, GEMM_TILE_64x64 = 0, 1, 2, 3

_lib = None


def lib() -> ctypes.CDLL:
    """Load libnn-hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NNHipError(-1, f"{LIB_PATH} is missing: run __graft_entry__.build() "
                                 "(make -C neuralnet.cpp_amd)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(status: int, fn: str) -> None:
    if status != 0:
        msg = lib().nnhip_last_error().decode(errors="replace")
        raise NNHipError(status, msg or fn)


def fnv1a64(t) -> str:
    """FNV-1a 64 of a tensor's bytes (a device tensor is copied to the host first), as hex: the
    reference layer_bench --hash of an output."""
    import numpy as np
    a = np.ascontiguousarray(t.detach().cpu().numpy() if hasattr(t, "detach") else t)
    return "%016x" % lib().nnhip_fnv1a64(_vp(a.ctypes.data), a.nbytes)


def repacked_bytes(N: int, K: int) -> int:
    return int(lib().nnhip_repacked_bytes(N, K))


def act_i8_bytes(K: int, M: int) -> int:
    return int(lib().nnhip_act_i8_bytes(K, M))


def glu_rows(F: int) -> int:
    return int(lib().nnhip_glu_rows(F))


def rope_table(dk: int, max_len: int):
    """Host RoPE tables (cos, sin), each (max_len, dk/2) float32 numpy (nnhip_rope_table)."""
    import numpy as np
    c = np.empty((max_len, dk // 2), np.float32)
    s = np.empty((max_len, dk // 2), np.float32)
    _check(lib().nnhip_rope_table(dk, max_len, _vp(c.ctypes.data), _vp(s.ctypes.data)), "nnhip_rope_table")
    return c, s


def attention_workspace_bytes(B: int, H: int, Hkv: int, dk: int, len_bound: int) -> int:
    return int(lib().nnhip_attention_workspace_bytes(B, H, Hkv, dk, len_bound))


def device_info(device: int = 0) -> dict:
    """HIP's compute-unit count, peak engine clock, memory clock (kHz) and bus width (bits)."""
    v = [ctypes.c_int(0) for _ in range(4)]
    _check(lib().nnhip_device_info(device, *[ctypes.byref(x) for x in v]), "nnhip_device_info")
    return {"cus": v[0].value, "clock_khz": v[1].value, "mem_clock_khz": v[2].value, "bus_bits": v[3].value}


def device_name(device: int = 0) -> str:
    """HIP's name and architecture of a device (nnhip_device_name)."""
    buf = ctypes.create_string_buffer(256)
    _check(lib().nnhip_device_name(device, buf, 256), "nnhip_device_name")
    return buf.value.decode(errors="replace")


def kp(K: int) -> int:
    return (K + TILE_K - 1) // TILE_K * TILE_K


class Context:
    """One nnhip context (device + stream). Arguments are torch CUDA tensors."""

    def __init__(self, device: int = 0):
        import torch

        self._torch = torch
        if not torch.cuda.is_available():
            raise NNHipError(4, "no GPU visible to torch")
        self.device = device
        h = _vp()
        _check(lib().nnhip_ctx_create(device, ctypes.byref(h)), "nnhip_ctx_create")
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().nnhip_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- helpers
    def _bind_stream(self) -> None:
        s = self._torch.cuda.current_stream(self.device).cuda_stream
        _check(lib().nnhip_ctx_set_stream(self.h, _vp(s)), "nnhip_ctx_set_stream")

    def _dev(self, t, dtype=None, name="tensor"):
        torch = self._torch
        if t is None:
            return None
        if not t.is_cuda:
            raise NNHipError(1, f"{name} must be a device tensor")
        if not t.is_contiguous():
            raise NNHipError(1, f"{name} must be contiguous")
        if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
            raise NNHipError(1, f"{name} has dtype {t.dtype}, expected {dtype}")
        return _vp(t.data_ptr())

    def _empty(self, shape, dtype):
        return self._torch.empty(shape, dtype=dtype, device=f"cuda:{self.device}")

    def sync(self) -> None:
        self._bind_stream()
        _check(lib().nnhip_sync(self.h), "nnhip_sync")

    def set_gemm_tile(self, tile: int) -> None:
        """Force the prefill GEMM block tile (GEMM_TILE_*); GEMM_TILE_AUTO picks per call."""
        _check(lib().nnhip_ctx_set_gemm_tile(self.h, tile), "nnhip_ctx_set_gemm_tile")

    def prefetch_next(self, tensors) -> None:
        """Device tensors (up to 4) that the next per-token quantizer call (act_quant_i8 /
        rmsnorm_quant_i8 at M <= 64, rmsnorm_quant_i8_tokens, partial_residual_quant_i8) also
        reads, so that the kernel after it finds them in the memory-side cache. Results are
        unaffected; an empty list clears them."""
        ts = [t for t in tensors if t is not None]
        if len(ts) > 4:
            raise NNHipError(1, "at most 4 ranges")
        ptrs = (_vp * max(1, len(ts)))(*[self._dev(t, None, "range") for t in ts])
        nb = (_sz * max(1, len(ts)))(*[t.numel() * t.element_size() for t in ts])
        _check(lib().nnhip_ctx_prefetch_next(self.h, len(ts), ptrs, nb), "nnhip_ctx_prefetch_next")

    # -- reference-layout primitives
    def row_absmean(self, W):
        torch = self._torch
        N, K = W.shape
        tau = self._empty((N,), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_row_absmean(self.h, self._dev(W, torch.float32, "W"), N, K,
                                       self._dev(tau)), "nnhip_row_absmean")
        return tau

    def trit_pack(self, W, tau):
        torch = self._torch
        N, K = W.shape
        wq = self._empty((N, (K + 15) // 16), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_trit_pack(self.h, self._dev(W, torch.float32, "W"),
                                     self._dev(tau, torch.float32, "tau"), N, K, self._dev(wq)),
               "nnhip_trit_pack")
        return wq

    def col_reduce_max(self, x):
        torch = self._torch
        rows, cols = x.shape
        out = self._empty((cols,), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_col_reduce_max(self.h, self._dev(x, torch.float32, "x"), rows, cols,
                                          self._dev(out)), "nnhip_col_reduce_max")
        return out

    def abs(self, x, out=None):
        torch = self._torch
        out = self._empty(x.shape, torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_abs(self.h, self._dev(x, torch.float32, "x"), x.numel(), self._dev(out)),
               "nnhip_abs")
        return out

    def scale_inplace(self, x, alpha: float):
        self._bind_stream()
        _check(lib().nnhip_scale_inplace(self.h, self._dev(x, self._torch.float32, "x"), x.numel(),
                                         alpha), "nnhip_scale_inplace")
        return x

    def act_scale(self, X):
        torch = self._torch
        K, M = X.shape
        s = self._empty((M,), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_act_scale(self.h, self._dev(X, torch.float32, "X"), K, M, self._dev(s)),
               "nnhip_act_scale")
        return s

    def quantize_i8(self, x, scale, col_scale: bool = True):
        torch = self._torch
        rows, cols = x.shape
        out = self._empty((rows, (cols + 3) // 4), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_quantize_i8(self.h, self._dev(x, torch.float32, "x"),
                                       self._dev(scale, torch.float32, "scale"), rows, cols,
                                       int(col_scale), self._dev(out)), "nnhip_quantize_i8")
        return out

    def unpack_i8(self, packed, cols: int):
        torch = self._torch
        rows = packed.shape[0]
        out = self._empty((rows, cols), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_unpack_i8(self.h, self._dev(packed, torch.int32, "packed"), rows, cols,
                                     self._dev(out)), "nnhip_unpack_i8")
        return out

    def matmul_q_i8(self, wq, tau, xq, s, K: int, M: int):
        torch = self._torch
        N = wq.shape[0]
        Y = self._empty((N, M), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_matmul_q_i8(self.h, self._dev(wq, torch.int32, "wq"),
                                       self._dev(tau, torch.float32, "tau"),
                                       self._dev(xq, torch.int32, "xq"),
                                       self._dev(s, torch.float32, "s"), N, K, M, self._dev(Y)),
               "nnhip_matmul_q_i8")
        return Y

    def matmul_q_i8_noalloc(self, wq, tau, xq, s, K: int, M: int, out):
        """nnhip_matmul_q_i8 with the library's static per-GPU scratch (no device allocation);
        `out` (N, M) float32 is required, so the call allocates nothing on the device."""
        torch = self._torch
        N = wq.shape[0]
        if tuple(out.shape) != (N, M):
            raise NNHipError(1, f"out has shape {tuple(out.shape)}, expected {(N, M)}")
        self._bind_stream()
        _check(lib().nnhip_matmul_q_i8_noalloc(self.h, self._dev(wq, torch.int32, "wq"),
                                               self._dev(tau, torch.float32, "tau"),
                                               self._dev(xq, torch.int32, "xq"),
                                               self._dev(s, torch.float32, "s"), N, K, M,
                                               self._dev(out, torch.float32, "out")),
               "nnhip_matmul_q_i8_noalloc")
        return out

    def matmul_q(self, wq, tau, B, K: int, out_f16: bool = False, out=None):
        """Y (N, M) = (tau o trit(wq)) . B; B f32 or f16 (K, M); Y f32, or f16 if out_f16."""
        torch = self._torch
        N, M = wq.shape[0], B.shape[1]
        if B.shape[0] != K:
            raise NNHipError(1, f"B has {B.shape[0]} rows, expected K={K}")
        ydt = torch.float16 if out_f16 else torch.float32
        Y = self._empty((N, M), ydt) if out is None else out
        self._dev(Y, ydt, "out")
        if tuple(Y.shape) != (N, M):
            raise NNHipError(1, f"out has shape {tuple(Y.shape)}, expected {(N, M)}")
        self._bind_stream()
        _check(lib().nnhip_matmul_q(self.h, self._dev(wq, torch.int32, "wq"), self._dev(tau, torch.float32, "tau"),
                                    self._dev(B, (torch.float32, torch.float16), "B"),
                                    1 if B.dtype == torch.float16 else 0, N, K, M, self._dev(Y),
                                    1 if out_f16 else 0), "nnhip_matmul_q")
        return Y

    def matmul_q_t(self, A, tau, B, M: int, out_f16: bool = False, out=None):
        """Y (M, N) = (tau o trit(A))^T . B, A (K, ceil(M/16)) packed with tau per stored row."""
        torch = self._torch
        K, N = A.shape[0], B.shape[1]
        if B.shape[0] != K:
            raise NNHipError(1, f"B has {B.shape[0]} rows, expected K={K}")
        ydt = torch.float16 if out_f16 else torch.float32
        Y = self._empty((M, N), ydt) if out is None else out
        self._dev(Y, ydt, "out")
        if tuple(Y.shape) != (M, N):
            raise NNHipError(1, f"out has shape {tuple(Y.shape)}, expected {(M, N)}")
        self._bind_stream()
        _check(lib().nnhip_matmul_q_t(self.h, self._dev(A, torch.int32, "A"), self._dev(tau, torch.float32, "tau"),
                                      self._dev(B, (torch.float32, torch.float16), "B"),
                                      1 if B.dtype == torch.float16 else 0, K, M, N, self._dev(Y),
                                      1 if out_f16 else 0), "nnhip_matmul_q_t")
        return Y

    def add_row_broadcast(self, Y, b):
        torch = self._torch
        N, M = Y.shape
        self._bind_stream()
        _check(lib().nnhip_add_row_broadcast(self.h, self._dev(Y, torch.float32, "Y"),
                                             self._dev(b, torch.float32, "b"), N, M),
               "nnhip_add_row_broadcast")
        return Y

    def rmsnorm(self, X, gamma, eps: float):
        torch = self._torch
        F, M = X.shape
        out = self._empty((F, M), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_rmsnorm(self.h, self._dev(X, torch.float32, "X"),
                                   self._dev(gamma, torch.float32, "gamma"), eps, F, M,
                                   self._dev(out)), "nnhip_rmsnorm")
        return out

    def layernorm(self, X, gamma, beta, eps: float = 1e-5):
        """LayerNorm of each token (column) of X (F, M) with gain gamma (F) and shift beta (F):
        LayerNorm::forward (include/neuralnet.cpp/compute_layer_mlp.hpp:529-545), the SubLN norm type
        FeedForward takes by default. Returns (F, M) float32."""
        torch = self._torch
        F, M = X.shape
        if gamma.numel() != F or beta.numel() != F:
            raise NNHipError(1, f"layernorm: gamma and beta must hold F={F} values "
                                f"(got {gamma.numel()}, {beta.numel()})")
        out = self._empty((F, M), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_layernorm(self.h, self._dev(X, torch.float32, "X"),
                                     self._dev(gamma, torch.float32, "gamma"),
                                     self._dev(beta, torch.float32, "beta"), eps, F, M,
                                     self._dev(out)), "nnhip_layernorm")
        return out

    # -- fast path
    def repack(self, wq, K: int):
        torch = self._torch
        N = wq.shape[0]
        rp = self._empty((repacked_bytes(N, K) // 4,), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_repack_ternary(self.h, self._dev(wq, torch.int32, "wq"), N, K,
                                          self._dev(rp)), "nnhip_repack_ternary")
        return rp

    def unrepack(self, rp, N: int, K: int):
        torch = self._torch
        wq = self._empty((N, (K + 15) // 16), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_unrepack_ternary(self.h, self._dev(rp, torch.int32, "rp"), N, K,
                                            self._dev(wq)), "nnhip_unrepack_ternary")
        return wq

    def _act_out(self, K: int, M: int):
        torch = self._torch
        xi = self._empty((M, kp(K)), torch.int8)
        s = self._empty((M,), torch.float32)
        rs = self._empty((M,), torch.int32)
        return xi, s, rs

    def act_quant_i8(self, X, want_container: bool = False, outs=None):
        """outs: optional preallocated (xi, s, rowsum) to write into."""
        torch = self._torch
        K, M = X.shape
        xi, s, rs = self._act_out(K, M) if outs is None else outs
        xq = self._empty((K, (M + 3) // 4), torch.int32) if want_container else None
        self._bind_stream()
        _check(lib().nnhip_act_quant_i8(self.h, self._dev(X, torch.float32, "X"), K, M,
                                        self._dev(xi), self._dev(s), self._dev(rs),
                                        self._dev(xq) if xq is not None else None),
               "nnhip_act_quant_i8")
        return (xi, s, rs, xq) if want_container else (xi, s, rs)

    def rmsnorm_quant_i8(self, X, gamma, eps: float, want_container: bool = False, outs=None):
        """outs: optional preallocated (xi, s, rowsum) to write into."""
        torch = self._torch
        F, M = X.shape
        xi, s, rs = self._act_out(F, M) if outs is None else outs
        xq = self._empty((F, (M + 3) // 4), torch.int32) if want_container else None
        self._bind_stream()
        _check(lib().nnhip_rmsnorm_quant_i8(self.h, self._dev(X, torch.float32, "X"),
                                            self._dev(gamma, torch.float32, "gamma"), eps, F, M,
                                            self._dev(xi), self._dev(s), self._dev(rs),
                                            self._dev(xq) if xq is not None else None),
               "nnhip_rmsnorm_quant_i8")
        return (xi, s, rs, xq) if want_container else (xi, s, rs)

    def act_from_container(self, xq, K: int, M: int):
        torch = self._torch
        xi, _, rs = self._act_out(K, M)
        self._bind_stream()
        _check(lib().nnhip_act_i8_from_container(self.h, self._dev(xq, torch.int32, "xq"), K, M,
                                                 self._dev(xi), self._dev(rs)),
               "nnhip_act_i8_from_container")
        return xi, rs

    def act_to_container(self, xi, K: int, M: int):
        torch = self._torch
        xq = self._empty((K, (M + 3) // 4), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_act_i8_to_container(self.h, self._dev(xi, torch.int8, "xi"), K, M,
                                               self._dev(xq)), "nnhip_act_i8_to_container")
        return xq

    def ternary_matmul(self, rp, tau, xi, s, rowsum, N: int, K: int, M: int, bias=None, out=None):
        torch = self._torch
        Y = self._empty((N, M), torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ternary_matmul(self.h, self._dev(rp, torch.int32, "rp"),
                                          self._dev(tau, torch.float32, "tau"),
                                          self._dev(xi, torch.int8, "xi"),
                                          self._dev(s, torch.float32, "s"),
                                          self._dev(rowsum, torch.int32, "rowsum"),
                                          self._dev(bias, torch.float32, "bias"), N, K, M,
                                          self._dev(Y, torch.float32, "Y")),
               "nnhip_ternary_matmul")
        return Y

    def ternary_matmul_f(self, rp, tau, B, N: int, K: int, out_f16: bool = False, out=None):
        """Float-activation product on repacked weights: (tau o trit) . B, B (K, M) f32 or f16."""
        torch = self._torch
        M = B.shape[1]
        Y = self._empty((N, M), torch.float16 if out_f16 else torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ternary_matmul_f(self.h, self._dev(rp, torch.int32, "rp"), self._dev(tau, torch.float32, "tau"),
                                            self._dev(B, (torch.float32, torch.float16), "B"),
                                            int(B.dtype == torch.float16), N, K, M,
                                            self._dev(Y, (torch.float32, torch.float16), "Y"), int(out_f16)),
               "nnhip_ternary_matmul_f")
        return Y

    def stream_xor(self, src, out):
        """out (1 int32 word on the device) ^= xor of src's 32-bit words."""
        torch = self._torch
        self._bind_stream()
        _check(lib().nnhip_stream_xor(self.h, self._dev(src), src.numel() * src.element_size(),
                                      self._dev(out, torch.int32, "out")), "nnhip_stream_xor")
        return out

    def trit_transpose(self, A, M: int):
        """A (K, ceil(M/16)) packed -> At (M, ceil(K/16))."""
        torch = self._torch
        K = A.shape[0]
        At = self._empty((M, (K + 15) // 16), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_trit_transpose(self.h, self._dev(A, torch.int32, "A"), K, M, self._dev(At)),
               "nnhip_trit_transpose")
        return At

    def ternary_matmul_t_f(self, rpT, tau, B, M: int, out_f16: bool = False, out=None):
        """(tau o trit(A))^T . B on rpT = repack(transpose(A)); B (K, N); returns (M, N)."""
        torch = self._torch
        K, N = B.shape
        Y = self._empty((M, N), torch.float16 if out_f16 else torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ternary_matmul_t_f(self.h, self._dev(rpT, torch.int32, "rpT"),
                                              self._dev(tau, torch.float32, "tau"),
                                              self._dev(B, (torch.float32, torch.float16), "B"),
                                              int(B.dtype == torch.float16), K, M, N,
                                              self._dev(Y, (torch.float32, torch.float16), "Y"), int(out_f16)),
               "nnhip_ternary_matmul_t_f")
        return Y

    def ternary_matmul_add(self, rp, tau, xi, s, rowsum, N: int, K: int, M: int, res, bias=None, out=None,
                           tokens: bool = False):
        """Y = ternary_matmul(...) + res (res must not alias Y); with tokens, res and Y are (M, N)
        (nnhip_ternary_matmul_add_tokens, decode sizes)."""
        torch = self._torch
        Y = self._empty((M, N) if tokens else (N, M), torch.float32) if out is None else out
        self._bind_stream()
        entry = lib().nnhip_ternary_matmul_add_tokens if tokens else lib().nnhip_ternary_matmul_add
        _check(entry(self.h, self._dev(rp, torch.int32, "rp"),
                                              self._dev(tau, torch.float32, "tau"), self._dev(xi, torch.int8, "xi"),
                                              self._dev(s, torch.float32, "s"),
                                              self._dev(rowsum, torch.int32, "rowsum"),
                                              self._dev(bias, torch.float32, "bias"),
                                              self._dev(res, torch.float32, "res"), N, K, M,
                                              self._dev(Y, torch.float32, "Y")),
               "nnhip_ternary_matmul_add_tokens" if tokens else "nnhip_ternary_matmul_add")
        return Y

    def ternary_matmul_partial(self, rp, xi, N: int, K: int, M: int, slices: int, out=None):
        """Split-k integer partial sums part (slices, M, N) int32 of the ternary GEMV (no epilogue)."""
        torch = self._torch
        part = self._empty((slices, M, N), torch.int32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ternary_matmul_partial(self.h, self._dev(rp, torch.int32, "rp"),
                                                  self._dev(xi, torch.int8, "xi"), N, K, M, slices,
                                                  self._dev(part, torch.int32, "part")),
               "nnhip_ternary_matmul_partial")
        return part

    def partial_residual_quant_i8(self, part, tau, s_in, rowsum_in, N: int, M: int, x_out, res=None, bias=None,
                                  gamma=None, eps: float = 0.0, outs=None, tokens: bool = False):
        """x_out = epilogue(sum of part) [+ bias] [+ res], then [RMSNorm(gamma) ->] int8: returns (xi, s, rowsum).
        With tokens, res and x_out are token-major (M, N)."""
        torch = self._torch
        xi, s, rs = self._act_out(N, M) if outs is None else outs
        self._bind_stream()
        entry = lib().nnhip_partial_residual_quant_i8_tokens if tokens else lib().nnhip_partial_residual_quant_i8
        _check(entry(self.h, self._dev(part, torch.int32, "part"), part.shape[0],
                                                     self._dev(tau, torch.float32, "tau"),
                                                     self._dev(s_in, torch.float32, "s_in"),
                                                     self._dev(rowsum_in, torch.int32, "rowsum_in"),
                                                     self._dev(bias, torch.float32, "bias"),
                                                     self._dev(res, torch.float32, "res"), N, M,
                                                     self._dev(x_out, torch.float32, "x_out"),
                                                     self._dev(gamma, torch.float32, "gamma"), eps,
                                                     self._dev(xi), self._dev(s), self._dev(rs)),
               "nnhip_partial_residual_quant_i8_tokens" if tokens else "nnhip_partial_residual_quant_i8")
        return xi, s, rs

    def ternary_matmul_n(self, problems, xi, s, rowsum, K: int, M: int, tokens: bool = False):
        """problems: list of (rp, tau, bias or None, N, out or None) sharing the input; returns the outputs
        ((N, M) each, or token-major (M, N) with tokens: nnhip_ternary_matmul_n_tokens)."""
        torch = self._torch
        n = len(problems)
        outs = [p[4] if p[4] is not None else self._empty((M, p[3]) if tokens else (p[3], M), torch.float32)
                for p in problems]
        rp = (_vp * n)(*[self._dev(p[0], torch.int32, "rp") for p in problems])
        tau = (_vp * n)(*[self._dev(p[1], torch.float32, "tau") for p in problems])
        bias = (_vp * n)(*[self._dev(p[2], torch.float32, "bias") for p in problems])
        Ns = (_sz * n)(*[p[3] for p in problems])
        Ys = (_vp * n)(*[self._dev(o, torch.float32, "Y") for o in outs])
        self._bind_stream()
        entry = lib().nnhip_ternary_matmul_n_tokens if tokens else lib().nnhip_ternary_matmul_n
        _check(entry(self.h, n, rp, tau, bias, Ns, Ys, self._dev(xi, torch.int8, "xi"),
                     self._dev(s, torch.float32, "s"), self._dev(rowsum, torch.int32, "rowsum"), K, M),
               "nnhip_ternary_matmul_n_tokens" if tokens else "nnhip_ternary_matmul_n")
        return outs

    def ffn_glu_i8_add(self, X, gamma, eps: float, F: int, rp1, tau1, b1, rp2, tau2, b2, res, act: int = ACT_SWIGLU,
                       out=None, gamma_sub=None, eps_sub: float = 1e-5):
        """res + ffn_glu_i8(X, ...) (res must not alias the output)."""
        torch = self._torch
        d, M = X.shape
        Y = self._empty((d, M), torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ffn_glu_i8_add(self.h, self._dev(X, torch.float32, "X"),
                                          self._dev(gamma, torch.float32, "gamma"), eps, d, F, M, act,
                                          self._dev(rp1, torch.int32, "rp1"), self._dev(tau1, torch.float32, "tau1"),
                                          self._dev(b1, torch.float32, "b1"),
                                          self._dev(gamma_sub, torch.float32, "gamma_sub"), eps_sub,
                                          self._dev(rp2, torch.int32, "rp2"), self._dev(tau2, torch.float32, "tau2"),
                                          self._dev(b2, torch.float32, "b2"), self._dev(res, torch.float32, "res"),
                                          self._dev(Y, torch.float32, "Y")), "nnhip_ffn_glu_i8_add")
        return Y

    # -- batched decode step
    def attention_decode(self, q, k, v, H: int, Hkv: int, dk: int, pos, len_bound: int, k_cache, v_cache,
                         scale: float, cos=None, sin=None, out=None, tokens: bool = False):
        """q (H*dk, B), k/v (Hkv*dk, B), pos (B) int32 device, caches (B, max_len, Hkv*dk) updated in
        place (row pos[b]); cos/sin (max_len, dk/2) device tables or None. Returns out (H*dk, B).
        With tokens, q (B, H*dk), k/v (B, Hkv*dk) and out (B, H*dk) (nnhip_attention_decode_tokens).
        float16 caches (compute = F16) run the _h entry points; both caches have one dtype."""
        torch = self._torch
        B = q.shape[0] if tokens else q.shape[1]
        max_len = k_cache.shape[1]
        ct = self._cache_dtype(k_cache, v_cache)
        if out is None:
            out = self._empty((B, H * dk) if tokens else (H * dk, B), torch.float32)
        self._bind_stream()
        name = ("nnhip_attention_decode_tokens" if tokens else "nnhip_attention_decode") + \
            ("_h" if ct == torch.float16 else "")
        _check(getattr(lib(), name)(
            self.h, self._dev(q, torch.float32, "q"), self._dev(k, torch.float32, "k"),
            self._dev(v, torch.float32, "v"), B, H, Hkv, dk, self._dev(pos, torch.int32, "pos"), len_bound,
            self._dev(cos, torch.float32, "cos"), self._dev(sin, torch.float32, "sin"),
            self._dev(k_cache, ct, "k_cache"), self._dev(v_cache, ct, "v_cache"), max_len,
            scale, self._dev(out, torch.float32, "out")), name)
        return out

    def _cache_dtype(self, k_cache, v_cache):
        """The caches' element type: float32, or float16 under compute = F16 (both alike)."""
        torch = self._torch
        if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (torch.float32, torch.float16):
            raise NNHipError(1, f"caches must both be float32 or both float16 (got {k_cache.dtype}, {v_cache.dtype})")
        return k_cache.dtype

    def kv_cache_fill(self, k, v, B: int, T: int, Hkv: int, dk: int, pos0: int, k_cache, v_cache, cos=None, sin=None):
        """Append T tokens of each of B sequences (k / v (Hkv*dk, B*T)) to the caches at rows pos0 + t
        (float16 caches: nnhip_kv_cache_fill_h)."""
        torch = self._torch
        ct = self._cache_dtype(k_cache, v_cache)
        name = "nnhip_kv_cache_fill" + ("_h" if ct == torch.float16 else "")
        self._bind_stream()
        _check(getattr(lib(), name)(self.h, self._dev(k, torch.float32, "k"), self._dev(v, torch.float32, "v"),
                                    B, T, Hkv, dk, pos0, self._dev(cos, torch.float32, "cos"),
                                    self._dev(sin, torch.float32, "sin"), self._dev(k_cache, ct, "k_cache"),
                                    self._dev(v_cache, ct, "v_cache"), k_cache.shape[1]), name)

    def attention_prefill(self, q, k_cache, v_cache, B: int, T: int, H: int, Hkv: int, dk: int, pos0: int,
                          scale: float, cos=None, sin=None, out=None):
        """Causal attention of T tokens per sequence (q (H*dk, B*T)) over caches holding rows [0, pos0 + T)."""
        torch = self._torch
        ct = self._cache_dtype(k_cache, v_cache)
        name = "nnhip_attention_prefill" + ("_h" if ct == torch.float16 else "")
        Y = out if out is not None else self._empty((H * dk, B * T), torch.float32)
        self._bind_stream()
        _check(getattr(lib(), name)(self.h, self._dev(q, torch.float32, "q"), self._dev(k_cache, ct, "k_cache"),
                                    self._dev(v_cache, ct, "v_cache"), B, T, H, Hkv, dk, pos0,
                                    self._dev(cos, torch.float32, "cos"), self._dev(sin, torch.float32, "sin"),
                                    k_cache.shape[1], scale, self._dev(Y, torch.float32, "out")), name)
        return Y

    def copy_columns(self, src, col0: int, stride: int, n: int, out=None):
        """dst (rows, n): column j = src column col0 + j * stride."""
        torch = self._torch
        rows, cols = src.shape
        Y = out if out is not None else self._empty((rows, n), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_copy_columns(self.h, self._dev(src, torch.float32, "src"), rows, cols, col0, stride, n,
                                        self._dev(Y, torch.float32, "dst")), "nnhip_copy_columns")
        return Y

    def to_f16(self, x, out=None):
        """f32 -> binary16 (round to nearest even), as a torch.float16 tensor."""
        torch = self._torch
        Y = out if out is not None else self._empty(tuple(x.shape), torch.float16)
        self._bind_stream()
        _check(lib().nnhip_convert_f32_f16(self.h, self._dev(x, torch.float32, "x"), x.numel(),
                                           self._dev(Y, torch.float16, "out")), "nnhip_convert_f32_f16")
        return Y

    def to_f32(self, x, out=None):
        """binary16 -> f32 (exact)."""
        torch = self._torch
        Y = out if out is not None else self._empty(tuple(x.shape), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_convert_f16_f32(self.h, self._dev(x, torch.float16, "x"), x.numel(),
                                           self._dev(Y, torch.float32, "out")), "nnhip_convert_f16_f32")
        return Y

    def add(self, x, y, out=None):
        torch = self._torch
        if out is None:
            out = self._empty(tuple(x.shape), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_add(self.h, self._dev(x, torch.float32, "x"), self._dev(y, torch.float32, "y"),
                               x.numel(), self._dev(out, torch.float32, "out")), "nnhip_add")
        return out

    def embedding_gather(self, table, ids, out=None, tokens: bool = False):
        """table (V, d), ids (B) int32 device -> (d, B), or (B, d) with tokens."""
        torch = self._torch
        V, d = table.shape
        B = ids.shape[0]
        if out is None:
            out = self._empty((B, d) if tokens else (d, B), torch.float32)
        self._bind_stream()
        entry = lib().nnhip_embedding_gather_tokens if tokens else lib().nnhip_embedding_gather
        _check(entry(self.h, self._dev(table, torch.float32, "table"),
                                            self._dev(ids, torch.int32, "ids"), V, d, B,
                                            self._dev(out, torch.float32, "out")),
               "nnhip_embedding_gather_tokens" if tokens else "nnhip_embedding_gather")
        return out

    def argmax_cols(self, logits, out=None):
        """logits (V, B) -> (B) int32 greedy token ids."""
        torch = self._torch
        V, B = logits.shape
        if out is None:
            out = self._empty((B,), torch.int32)
        self._bind_stream()
        _check(lib().nnhip_argmax_cols(self.h, self._dev(logits, torch.float32, "logits"), V, B,
                                       self._dev(out, torch.int32, "out")), "nnhip_argmax_cols")
        return out

    def argmax_rows(self, logits, out=None, pos=None):
        """token-major logits (B, V) -> (B) int32 greedy token ids; pos (B) int32, when given, is
        advanced by one in the same launch."""
        torch = self._torch
        B, V = logits.shape
        if out is None:
            out = self._empty((B,), torch.int32)
        if pos is not None and tuple(pos.shape) != (B,):
            raise NNHipError(1, f"pos must have shape ({B},)")
        self._bind_stream()
        _check(lib().nnhip_argmax_rows(self.h, self._dev(logits, torch.float32, "logits"), V, B,
                                       self._dev(out, torch.int32, "out"), self._dev(pos, torch.int32, "pos")),
               "nnhip_argmax_rows")
        return out

    # -- gated feed-forward block
    def glu(self, Y1, act: int = ACT_SWIGLU):
        """Y1 (2F, M): gate rows then up rows -> h (F, M)."""
        torch = self._torch
        F, M = Y1.shape[0] // 2, Y1.shape[1]
        h = self._empty((F, M), torch.float32)
        self._bind_stream()
        _check(lib().nnhip_glu(self.h, self._dev(Y1, torch.float32, "Y1"), F, M, act, self._dev(h)), "nnhip_glu")
        return h

    def glu_interleave(self, wq, tau, bias, F: int, K: int):
        """fc1 container (2F, ceil(K/16)) + tau/bias (2F) -> interleaved (wq, tau, bias)."""
        torch = self._torch
        rows = glu_rows(F)
        wo = self._empty((rows, (K + 15) // 16), torch.int32)
        to = self._empty((rows,), torch.float32)
        bo = self._empty((rows,), torch.float32) if bias is not None else None
        self._bind_stream()
        _check(lib().nnhip_glu_interleave(self.h, self._dev(wq, torch.int32, "wq"), self._dev(tau, torch.float32, "tau"),
                                          self._dev(bias, torch.float32, "bias"), F, K, self._dev(wo), self._dev(to),
                                          self._dev(bo) if bo is not None else None), "nnhip_glu_interleave")
        return wo, to, bo

    def ternary_matmul_glu_tokens(self, rp, tau, xi, s, rowsum, F: int, K: int, M: int, act: int = ACT_SWIGLU,
                                  bias=None, out=None):
        """ternary_matmul_glu with h token-major (M, F) (decode sizes)."""
        torch = self._torch
        h = self._empty((M, F), torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ternary_matmul_glu_tokens(self.h, self._dev(rp, torch.int32, "rp"),
                                                     self._dev(tau, torch.float32, "tau"),
                                                     self._dev(xi, torch.int8, "xi"), self._dev(s, torch.float32, "s"),
                                                     self._dev(rowsum, torch.int32, "rowsum"),
                                                     self._dev(bias, torch.float32, "bias"), F, K, M, act,
                                                     self._dev(h, torch.float32, "h")),
               "nnhip_ternary_matmul_glu_tokens")
        return h

    def rmsnorm_quant_i8_tokens(self, X, gamma, eps: float, outs=None):
        """[RMSNorm (gamma, or None) ->] absmax -> int8 of a token-major X (M, K); returns (xi, s, rowsum)."""
        torch = self._torch
        M, K = X.shape
        if outs is None:
            outs = (self._empty((M, kp(K)), torch.int8), self._empty((M,), torch.float32),
                    self._empty((M,), torch.int32))
        xi, s, rs = outs
        self._bind_stream()
        _check(lib().nnhip_rmsnorm_quant_i8_tokens(self.h, self._dev(X, torch.float32, "X"),
                                                   self._dev(gamma, torch.float32, "gamma"), eps, K, M,
                                                   self._dev(xi, torch.int8, "xi"), self._dev(s, torch.float32, "s"),
                                                   self._dev(rs, torch.int32, "rowsum")),
               "nnhip_rmsnorm_quant_i8_tokens")
        return outs

    def embedding_rmsnorm_quant_i8_tokens(self, table, ids, gamma, eps: float, out=None, outs=None):
        """Rows ids[b] of table (V, d) into out (B, d) and their [RMSNorm (gamma, or None) ->] absmax
        -> int8 in the same launch; returns (out, (xi, s, rowsum))."""
        torch = self._torch
        V, d = table.shape
        B = ids.shape[0]
        if out is None:
            out = self._empty((B, d), torch.float32)
        if outs is None:
            outs = (self._empty((B, kp(d)), torch.int8), self._empty((B,), torch.float32),
                    self._empty((B,), torch.int32))
        xi, s, rs = outs
        self._bind_stream()
        _check(lib().nnhip_embedding_rmsnorm_quant_i8_tokens(
            self.h, self._dev(table, torch.float32, "table"), self._dev(ids, torch.int32, "ids"), V, d, B,
            self._dev(gamma, torch.float32, "gamma"), eps, self._dev(out, torch.float32, "out"),
            self._dev(xi, torch.int8, "xi"), self._dev(s, torch.float32, "s"), self._dev(rs, torch.int32, "rowsum")),
            "nnhip_embedding_rmsnorm_quant_i8_tokens")
        return out, outs

    def ternary_matmul_glu(self, rp, tau, xi, s, rowsum, F: int, K: int, M: int, act: int = ACT_SWIGLU,
                           bias=None, out=None):
        torch = self._torch
        h = self._empty((F, M), torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ternary_matmul_glu(self.h, self._dev(rp, torch.int32, "rp"),
                                              self._dev(tau, torch.float32, "tau"), self._dev(xi, torch.int8, "xi"),
                                              self._dev(s, torch.float32, "s"),
                                              self._dev(rowsum, torch.int32, "rowsum"),
                                              self._dev(bias, torch.float32, "bias"), F, K, M, act,
                                              self._dev(h, torch.float32, "h")), "nnhip_ternary_matmul_glu")
        return h

    def ffn_glu_i8(self, X, gamma, eps: float, F: int, rp1, tau1, b1, rp2, tau2, b2, act: int = ACT_SWIGLU,
                   out=None, gamma_sub=None, eps_sub: float = 1e-5):
        """Gated FFN block on X (d, M): [RMSNorm] -> int8 -> fc1 (interleaved) -> act -> [SubLN RMSNorm
        (gamma_sub, eps_sub)] -> int8 -> fc2."""
        torch = self._torch
        d, M = X.shape
        Y = self._empty((d, M), torch.float32) if out is None else out
        self._bind_stream()
        _check(lib().nnhip_ffn_glu_i8(self.h, self._dev(X, torch.float32, "X"), self._dev(gamma, torch.float32, "gamma"),
                                      eps, d, F, M, act, self._dev(rp1, torch.int32, "rp1"),
                                      self._dev(tau1, torch.float32, "tau1"), self._dev(b1, torch.float32, "b1"),
                                      self._dev(gamma_sub, torch.float32, "gamma_sub"), eps_sub,
                                      self._dev(rp2, torch.int32, "rp2"), self._dev(tau2, torch.float32, "tau2"),
                                      self._dev(b2, torch.float32, "b2"), self._dev(Y, torch.float32, "Y")),
               "nnhip_ffn_glu_i8")
        return Y

    def group_create(self, problems):
        """problems: list of dicts with rp, tau, xi, s, rowsum, bias (or None), y, N, K, M."""
        arr = (GemvDesc * len(problems))()
        for i, p in enumerate(problems):
            arr[i] = GemvDesc(p["rp"].data_ptr(), p["tau"].data_ptr(), p["xi"].data_ptr(),
                              p["s"].data_ptr(), p["rowsum"].data_ptr(),
                              p["bias"].data_ptr() if p.get("bias") is not None else None,
                              p["y"].data_ptr(), p["N"], p["K"], p["M"])
        h = _vp()
        self._bind_stream()
        _check(lib().nnhip_group_create(self.h, arr, len(problems), ctypes.byref(h)),
               "nnhip_group_create")
        return h

    def group_run(self, h) -> None:
        self._bind_stream()
        _check(lib().nnhip_group_run(self.h, h), "nnhip_group_run")

    def group_destroy(self, h) -> None:
        self._bind_stream()
        _check(lib().nnhip_group_destroy(self.h, h), "nnhip_group_destroy")

    def group_info(self, h) -> dict:
        """What nnhip_group_create chose: {"lds": True (every launch stages its activations in LDS),
        False (register variant only) or "mixed", "waves": int, "lds_bytes": int}."""
        v, w, b = ctypes.c_int(0), _sz(0), _sz(0)
        _check(lib().nnhip_group_info(h, ctypes.byref(v), ctypes.byref(w), ctypes.byref(b)), "nnhip_group_info")
        lds = {0: False, 1: True}.get(v.value, "mixed")
        return {"lds": lds, "waves": int(w.value), "lds_bytes": int(b.value)}

    def gemv_grid_waves(self, items: int) -> int:
        return int(lib().nnhip_gemv_grid_waves(self.h, items))

"""Batched decode step of a BitNet-b1.58 GPT model over libnn-hip.so's C ABI.

The Python mirror of nn::GPTModel::forward_step (include/neuralnet.cpp/decoder.hpp), used by
the tests and bench.py: the reference's GPTModel::forward_step (compute_layer_gpt.hpp:693-724)
for B sequences, one token each, each at its own position. Every buffer is allocated once at
construction, so one step makes no allocation and can be captured in a graph and replayed.

Per block (GPTBlock::forward_step, compute_layer_gpt.hpp:201-219, all BitLinears in the int8
branch):
    xi = int8(RMSNorm1(x))                        nnhip_rmsnorm_quant_i8
    q, k, v = BitLinear(xi)                       nnhip_ternary_matmul_n (one launch)
    a = attention(q, k, v, caches, pos)           nnhip_attention_decode (RoPE, GQA, append)
    xi = int8([SubLN] a)                          nnhip_rmsnorm_quant_i8 / nnhip_act_quant_i8
    r = x + BitLinear_o(xi)                       nnhip_ternary_matmul_add (residual in the epilogue)
    x = r + FFN(RMSNorm2(r))                      nnhip_ffn_glu_i8_add (norm and residual fused)
then logits = BitLinear_head(int8(RMSNorm_f(x))) and the greedy ids (nnhip_argmax_cols).

Decoder.prefill runs T tokens of every sequence through the same chain at once (M = B*T token
columns: the GEMM path, nnhip_kv_cache_fill and the causal nnhip_attention_prefill), giving each
token the result of its own step() (the reference fills the cache with one forward_step per
context token, compute_layer_gpt.hpp:774-794), and the logits and greedy ids of each sequence's
last token.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional


@dataclass
class Linear:
    """One BitLinear on the device in the fast layout: repacked words, tau, bias (or None)."""
    rp: object
    tau: object
    bias: Optional[object]
    N: int
    K: int


@dataclass
class Block:
    g1: object
    q: Linear
    k: Linear
    v: Linear
    o: Linear
    g2: object
    fc1: Linear            # interleaved gate/up rows (nnhip_glu_interleave), N = glu_rows(F)
    fc2: Linear
    g_attn_sub: Optional[object] = None
    g_ffn_sub: Optional[object] = None


@dataclass
class Config:
    d: int
    H: int
    Hkv: int
    F: int
    vocab: int
    max_len: int
    act: int = 0            # ACT_SWIGLU / ACT_RELU2GLU
    eps: float = 1e-5
    rope: bool = True
    # KV caches in f16 (compute = F16: the reference creates them in the profile's compute
    # precision, compute_layer_gpt.hpp:764-765); the arithmetic stays f32
    cache_f16: bool = False

    @property
    def dk(self) -> int:
        return self.d // self.H

    @property
    def scale(self) -> float:
        import numpy as np
        return float(np.float32(1.0) / np.float32(math.sqrt(self.dk)))


class Decoder:
    """Device state of one model for B sequences: weights, KV caches, RoPE tables and the
    step's scratch buffers."""

    # BitLinears whose packed weights the per-token quantizer before them also reads
    # (nnhip_ctx_prefetch_next), so that their GEMV finds them in the memory-side cache: q/k/v
    # (in the fc2 epilogue kernel of the block before), o (in the attention SubLN quantizer) and
    # fc2 (in the FFN SubLN quantizer), whose quantizers absorb the extra reads (C5 step
    # 2.519 -> 2.498 ms for q/k/v and o; 2.340 -> 2.332 ms for fc2's split-k slices). Also
    # available: "fc1" (in the o epilogue kernel: 2.340 -> 2.350 ms, so off).
    prefetch = ("qkv", "o", "fc2")
    # the fused step keeps its activations token-major, (B, features): q/k/v, the attention
    # output, the residual stream x and the mid-block sum r (nnhip_ternary_matmul_n_tokens,
    # nnhip_attention_decode_tokens, nnhip_embedding_gather_tokens,
    # nnhip_ternary_matmul_add_tokens, nnhip_partial_residual_quant_i8_tokens), so every
    # per-token quantizer and the attention's query staging read contiguous rows
    tokens = True

    def __init__(self, ctx, cfg: Config, blocks: List[Block], emb, g_final, head: Linear, B: int, caches=None):
        import torch

        self.ctx, self.cfg, self.blocks, self.emb, self.g_final, self.head, self.B = \
            ctx, cfg, blocks, emb, g_final, head, B
        dev = f"cuda:{ctx.device}"
        f32 = dict(dtype=torch.float32, device=dev)
        d, H, Hkv, dk = cfg.d, cfg.H, cfg.Hkv, cfg.dk
        if caches is None:
            cdt = dict(dtype=torch.float16 if cfg.cache_f16 else torch.float32, device=dev)
            caches = [(torch.zeros((B, cfg.max_len, Hkv * dk), **cdt), torch.zeros((B, cfg.max_len, Hkv * dk), **cdt))
                      for _ in blocks]
        self.caches = caches
        if cfg.rope:
            c, s = _pkg().rope_table(dk, cfg.max_len)
            self.cos, self.sin = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
        else:
            self.cos = self.sin = None
        kpd = _pkg().kp
        self.x = torch.empty((d, B), **f32)
        self.r = torch.empty((d, B), **f32)
        self.q = torch.empty((H * dk, B), **f32)
        self.k = torch.empty((Hkv * dk, B), **f32)
        self.v = torch.empty((Hkv * dk, B), **f32)
        self.a = torch.empty((H * dk, B), **f32)
        # token-major buffers of the fused step (decode sizes of the one-token quantizer)
        self._tok = self.tokens and B <= 16 and max(d, H * dk) <= 11264
        if self._tok:
            self.q_t = torch.empty((B, H * dk), **f32)
            self.k_t = torch.empty((B, Hkv * dk), **f32)
            self.v_t = torch.empty((B, Hkv * dk), **f32)
            self.a_t = torch.empty((B, H * dk), **f32)
            self.x_t = torch.empty((B, d), **f32)
            self.r_t = torch.empty((B, d), **f32)
        self.xi = torch.empty((B * kpd(max(d, H * dk, cfg.F)),), dtype=torch.int8, device=dev)
        self.s = torch.empty((B,), **f32)
        self.rs = torch.empty((B,), dtype=torch.int32, device=dev)
        self._logits_cols = torch.empty((cfg.vocab, B), **f32)
        self._logits = self._logits_cols
        self.logits_t = None    # token-major (B, vocab) logits of the step, when the head takes them
        self.ids = torch.empty((B,), dtype=torch.int32, device=dev)
        if self._tok and blocks:
            # the token-major q/k/v and o products run on the single-launch decode GEMV only: one
            # call of each on scratch tells whether this model's shapes are taken
            self.xi.zero_()
            self.s.zero_()
            self.rs.zero_()
            blk = blocks[0]
            try:
                self._qkv(blk, True)
                ctx.ternary_matmul_add(blk.o.rp, blk.o.tau, self.xi, self.s, self.rs, blk.o.N, blk.o.K, B,
                                       self.x_t.zero_(), out=self.r_t, tokens=True)
            except _pkg().NNHipError as e:
                if e.status != 5:   # NNHIP_ERR_UNSUPPORTED
                    raise
                self._tok = False
        if self._tok:
            # the head with token-major logits, so that the greedy choice reads each sequence's
            # logits as one row (and advances the positions in the same launch)
            lt = torch.empty((B, cfg.vocab), **f32)
            try:
                ctx.ternary_matmul_n([(head.rp, head.tau, head.bias, head.N, lt)], self.xi, self.s, self.rs, head.K,
                                     B, tokens=True)
                self.logits_t = lt
            except _pkg().NNHipError as e:
                if e.status != 5:
                    raise

    @property
    def logits(self):
        """The last logits written (vocab, B): by prefill(), or by step() (a transposed view of the
        token-major logits when the head produces those)."""
        return self._logits

    def _prefill_buffers(self, M: int):
        """Scratch of a prefill over M = B*T token columns (allocated once per M)."""
        import torch
        if getattr(self, "_pf_M", None) == M:
            return self._pf
        cfg = self.cfg
        dev = f"cuda:{self.ctx.device}"
        f32 = dict(dtype=torch.float32, device=dev)
        d, H, Hkv, dk = cfg.d, cfg.H, cfg.Hkv, cfg.dk
        kpd = _pkg().kp
        self._pf = dict(
            x=torch.empty((d, M), **f32), r=torch.empty((d, M), **f32), q=torch.empty((H * dk, M), **f32),
            k=torch.empty((Hkv * dk, M), **f32), v=torch.empty((Hkv * dk, M), **f32),
            a=torch.empty((H * dk, M), **f32),
            xi=torch.empty((M * kpd(max(d, H * dk)),), dtype=torch.int8, device=dev),
            s=torch.empty((M,), **f32), rs=torch.empty((M,), dtype=torch.int32, device=dev))
        self._pf_M = M
        return self._pf

    def prefill(self, ids, T: int, pos0: int = 0, hook=None):
        """T tokens of each of the B sequences, at positions pos0 .. pos0 + T - 1, through every block
        in one pass: the caches get rows pos0 .. pos0 + T - 1 and every token the result of its own
        step(). ids: (B*T,) int32 device tensor, token column b*T + t. hook(i, name, tensor) sees each
        block's q / k / v / attention output / block output (tests). Returns (logits (vocab, B), greedy
        ids (B,)) of each sequence's last token."""
        cfg, ctx, B = self.cfg, self.ctx, self.B
        M = B * T
        pf = self._prefill_buffers(M)
        outs = (pf["xi"], pf["s"], pf["rs"])
        x, r = pf["x"], pf["r"]

        def quant(t, gamma):
            if gamma is None:
                ctx.act_quant_i8(t, outs=outs)
            else:
                ctx.rmsnorm_quant_i8(t, gamma, cfg.eps, outs=outs)

        def mm(lin, out):
            return ctx.ternary_matmul(lin.rp, lin.tau, pf["xi"], pf["s"], pf["rs"], lin.N, lin.K, M, bias=lin.bias,
                                      out=out)

        ctx.embedding_gather(self.emb, ids, out=x)
        for i, blk in enumerate(self.blocks):
            quant(x, blk.g1)
            mm(blk.q, pf["q"])
            mm(blk.k, pf["k"])
            mm(blk.v, pf["v"])
            kc, vc = self.caches[i]
            ctx.kv_cache_fill(pf["k"], pf["v"], B, T, cfg.Hkv, cfg.dk, pos0, kc, vc, self.cos, self.sin)
            ctx.attention_prefill(pf["q"], kc, vc, B, T, cfg.H, cfg.Hkv, cfg.dk, pos0, cfg.scale, self.cos, self.sin,
                                  out=pf["a"])
            if hook is not None:
                for name in ("q", "k", "v", "a"):
                    hook(i, name, pf[name])
            quant(pf["a"], blk.g_attn_sub)
            o = blk.o
            ctx.ternary_matmul_add(o.rp, o.tau, pf["xi"], pf["s"], pf["rs"], o.N, o.K, M, x, bias=o.bias, out=r)
            ctx.ffn_glu_i8_add(r, blk.g2, cfg.eps, cfg.F, blk.fc1.rp, blk.fc1.tau, blk.fc1.bias, blk.fc2.rp,
                               blk.fc2.tau, blk.fc2.bias, r, cfg.act, out=x, gamma_sub=blk.g_ffn_sub, eps_sub=cfg.eps)
            if hook is not None:
                hook(i, "x", x)
        ctx.copy_columns(x, T - 1, T, B, out=self.x)
        self._quant(self.x, self.g_final)
        self._mm(self.head, self._logits_cols)
        ctx.argmax_cols(self._logits_cols, out=self.ids)
        self._logits = self._logits_cols
        return self._logits, self.ids

    def _mm(self, lin: Linear, out):
        return self.ctx.ternary_matmul(lin.rp, lin.tau, self.xi, self.s, self.rs, lin.N, lin.K, self.B,
                                       bias=lin.bias, out=out)

    def _qkv(self, blk, tokens: bool):
        """q, k, v of the quantized input in one launch (token-major rows with tokens)."""
        outs = (self.q_t, self.k_t, self.v_t) if tokens else (self.q, self.k, self.v)
        self.ctx.ternary_matmul_n([(blk.q.rp, blk.q.tau, blk.q.bias, blk.q.N, outs[0]),
                                   (blk.k.rp, blk.k.tau, blk.k.bias, blk.k.N, outs[1]),
                                   (blk.v.rp, blk.v.tau, blk.v.bias, blk.v.N, outs[2])],
                                  self.xi, self.s, self.rs, blk.q.K, self.B, tokens=tokens)

    def _prefetch(self, kind: str, *lins):
        """Arm the next quantizer call to prefetch these BitLinears' packed weights."""
        if kind in self.prefetch:
            self.ctx.prefetch_next([lin.rp for lin in lins])

    def _quant(self, x, gamma):
        outs = (self.xi, self.s, self.rs)
        if gamma is None:
            self.ctx.act_quant_i8(x, outs=outs)
        else:
            self.ctx.rmsnorm_quant_i8(x, gamma, self.cfg.eps, outs=outs)

    def block_step(self, i: int, pos, len_bound: int, attn_hook=None):
        """Block i on self.x (d, B) in place. attn_hook(i, a) sees the attention output (tests)."""
        cfg, blk, ctx = self.cfg, self.blocks[i], self.ctx
        self._quant(self.x, blk.g1)
        ctx.ternary_matmul_n([(blk.q.rp, blk.q.tau, blk.q.bias, blk.q.N, self.q),
                              (blk.k.rp, blk.k.tau, blk.k.bias, blk.k.N, self.k),
                              (blk.v.rp, blk.v.tau, blk.v.bias, blk.v.N, self.v)],
                             self.xi, self.s, self.rs, blk.q.K, self.B)
        kc, vc = self.caches[i]
        ctx.attention_decode(self.q, self.k, self.v, cfg.H, cfg.Hkv, cfg.dk, pos, len_bound, kc, vc, cfg.scale,
                             self.cos, self.sin, out=self.a)
        if attn_hook is not None:
            attn_hook(i, self.a)
        self._quant(self.a, blk.g_attn_sub)
        o = blk.o
        ctx.ternary_matmul_add(o.rp, o.tau, self.xi, self.s, self.rs, o.N, o.K, self.B, self.x, bias=o.bias,
                               out=self.r)
        ctx.ffn_glu_i8_add(self.r, blk.g2, cfg.eps, cfg.F, blk.fc1.rp, blk.fc1.tau, blk.fc1.bias, blk.fc2.rp,
                           blk.fc2.tau, blk.fc2.bias, self.r, cfg.act, out=self.x, gamma_sub=blk.g_ffn_sub,
                           eps_sub=cfg.eps)

    # split-k slices of fc2 on the fused step path
    slices_fc2 = 4
    # the o projection as split-k slice sums whose per-token epilogue kernel also adds the
    # residual and quantizes for fc1 (0: the whole-K GEMV with the residual, then the quantizer)
    slices_o = 4

    # widest residual stream of the per-token epilogue + quantizer kernel (epilogue_quant_ok)
    fused_max_d = 11264

    def fused_ok(self) -> bool:
        """The fused step path (fc2 split-k, its epilogue, the residual add and the next block's
        RMSNorm -> int8 as one per-token kernel) applies to batches of at most 16 sequences whose
        residual stream fits the per-token kernel (d <= fused_max_d) and whose fc2 (and, on the
        token-major path, o) reductions have a split-k slicing; otherwise step() runs block_step."""
        cfg = self.cfg
        if self.B > 16 or cfg.d > self.fused_max_d:
            return False
        try:
            self._slices(cfg.F, self.slices_fc2)
            if self._tok and self.slices_o > 0:
                self._slices(cfg.H * cfg.dk, self.slices_o)
        except ValueError:
            return False
        return True

    @staticmethod
    def _slices(K: int, want: int) -> int:
        """The largest slice count <= want whose slices of ceil(KT / S) k tiles (KT = ceil(K / 256))
        are all non-empty and at most 14 tiles long."""
        KT = (K + 255) // 256
        for S in range(min(want, 8), 0, -1):
            kts = (KT + S - 1) // S
            if (S - 1) * kts < KT and kts <= 14:
                return S
        raise ValueError(f"no split-k slicing for K={K}")

    def _scratch(self):
        import torch
        if getattr(self, "_part_buf", None) is None:
            dev = f"cuda:{self.ctx.device}"
            S = max(self.slices_fc2, self.slices_o)
            self._part_buf = torch.empty((S, self.B, self.cfg.d), dtype=torch.int32, device=dev)
            self._h_buf = torch.empty((self.cfg.F, self.B), dtype=torch.float32, device=dev)
        return self._part_buf, self._h_buf

    # h token-major between fc1 and the FFN SubLN quantizer: None until the first step tries it
    _glu_tokens: Optional[bool] = None

    def _ffn_gate_quant(self, blk: Block, h):
        """fc1 + gated activation into h, then the FFN SubLN -> int8 into self.xi / s / rs. Where the
        decode GEMV takes fc1 (the library reports the shape as unsupported otherwise) h is written
        token-major, so the quantizer reads each token as one contiguous row; the bits are the
        same either way."""
        cfg, ctx, B, f1 = self.cfg, self.ctx, self.B, blk.fc1
        if self._glu_tokens is not False:
            try:
                ctx.ternary_matmul_glu_tokens(f1.rp, f1.tau, self.xi, self.s, self.rs, cfg.F, cfg.d, B, act=cfg.act,
                                              bias=f1.bias, out=h.view(B, cfg.F))
                self._glu_tokens = True
            except _pkg().NNHipError as e:
                if e.status != 5:   # NNHIP_ERR_UNSUPPORTED
                    raise
                self._glu_tokens = False
        if self._glu_tokens:
            self._prefetch("fc2", blk.fc2)
            ctx.rmsnorm_quant_i8_tokens(h.view(B, cfg.F), blk.g_ffn_sub, cfg.eps, outs=(self.xi, self.s, self.rs))
        else:
            ctx.ternary_matmul_glu(f1.rp, f1.tau, self.xi, self.s, self.rs, cfg.F, cfg.d, B, act=cfg.act,
                                   bias=f1.bias, out=h)
            self._prefetch("fc2", blk.fc2)
            self._quant(h, blk.g_ffn_sub)

    def block_step_fused(self, i: int, pos, len_bound: int, attn_hook=None):
        """Block i with self.xi / s / rs holding int8(RMSNorm1(x)) on entry; on exit self.x holds the
        block output and self.xi / s / rs its quantization for the next block (gamma = next block's
        g1, or g_final after the last block). The same operations, in the same order, as
        block_step followed by the next block's first quantizer."""
        cfg, blk, ctx, B, d = self.cfg, self.blocks[i], self.ctx, self.B, self.cfg.d
        outs = (self.xi, self.s, self.rs)
        self._qkv(blk, self._tok)
        kc, vc = self.caches[i]
        o = blk.o
        if self._tok:
            ctx.attention_decode(self.q_t, self.k_t, self.v_t, cfg.H, cfg.Hkv, cfg.dk, pos, len_bound, kc, vc,
                                 cfg.scale, self.cos, self.sin, out=self.a_t, tokens=True)
            if attn_hook is not None:
                attn_hook(i, self.a_t.t())
            self._prefetch("o", o)
            ctx.rmsnorm_quant_i8_tokens(self.a_t, blk.g_attn_sub, cfg.eps, outs=outs)
        else:
            ctx.attention_decode(self.q, self.k, self.v, cfg.H, cfg.Hkv, cfg.dk, pos, len_bound, kc, vc, cfg.scale,
                                 self.cos, self.sin, out=self.a)
            if attn_hook is not None:
                attn_hook(i, self.a)
            self._prefetch("o", o)
            self._quant(self.a, blk.g_attn_sub)
        self._prefetch("fc1", blk.fc1)
        part, h = self._scratch()
        if self._tok and self.slices_o > 0:
            S = self._slices(o.K, self.slices_o)
            po = ctx.ternary_matmul_partial(o.rp, self.xi, o.N, o.K, B, S, out=part[:S])
            ctx.partial_residual_quant_i8(po, o.tau, self.s, self.rs, d, B, self.r_t, res=self.x_t, bias=o.bias,
                                          gamma=blk.g2, eps=cfg.eps, outs=outs, tokens=True)
        elif self._tok:
            ctx.ternary_matmul_add(o.rp, o.tau, self.xi, self.s, self.rs, o.N, o.K, B, self.x_t, bias=o.bias,
                                   out=self.r_t, tokens=True)
            ctx.rmsnorm_quant_i8_tokens(self.r_t, blk.g2, cfg.eps, outs=outs)
        else:
            ctx.ternary_matmul_add(o.rp, o.tau, self.xi, self.s, self.rs, o.N, o.K, B, self.x, bias=o.bias,
                                   out=self.r)
            self._quant(self.r, blk.g2)
        self._ffn_gate_quant(blk, h)
        f2 = blk.fc2
        S = self._slices(f2.K, self.slices_fc2)
        pf = ctx.ternary_matmul_partial(f2.rp, self.xi, f2.N, f2.K, B, S, out=part[:S])
        g_next = self.blocks[i + 1].g1 if i + 1 < len(self.blocks) else self.g_final
        if i + 1 < len(self.blocks):
            nb = self.blocks[i + 1]
            self._prefetch("qkv", nb.q, nb.k, nb.v)
        else:
            self._prefetch("qkv", self.head)
        if self._tok:
            ctx.partial_residual_quant_i8(pf, f2.tau, self.s, self.rs, d, B, self.x_t, res=self.r_t, bias=f2.bias,
                                          gamma=g_next, eps=cfg.eps, outs=outs, tokens=True)
        else:
            ctx.partial_residual_quant_i8(pf, f2.tau, self.s, self.rs, d, B, self.x, res=self.r, bias=f2.bias,
                                          gamma=g_next, eps=cfg.eps, outs=outs)

    def step(self, ids, pos, len_bound: int, attn_hook=None, advance: bool = False):
        """ids / pos: (B,) int32 device tensors. Returns (logits (vocab, B), greedy ids (B,)).
        advance: the greedy ids are written into ids itself and every pos is advanced by one, so
        that the next call continues the generation (a captured step then replays as is)."""
        ctx = self.ctx
        fused = self.fused_ok()
        if fused and self._tok:
            # the embedding rows and their first quantization in one launch
            if self.blocks:
                self._prefetch("qkv", self.blocks[0].q, self.blocks[0].k, self.blocks[0].v)
            g0 = self.blocks[0].g1 if self.blocks else self.g_final
            ctx.embedding_rmsnorm_quant_i8_tokens(self.emb, ids, g0, self.cfg.eps, out=self.x_t,
                                                  outs=(self.xi, self.s, self.rs))
        else:
            ctx.embedding_gather(self.emb, ids, out=self.x)
        if fused:
            if not self._tok:
                if self.blocks:
                    self._prefetch("qkv", self.blocks[0].q, self.blocks[0].k, self.blocks[0].v)
                self._quant(self.x, self.blocks[0].g1 if self.blocks else self.g_final)
            for i in range(len(self.blocks)):
                self.block_step_fused(i, pos, len_bound, attn_hook)
        else:
            for i in range(len(self.blocks)):
                self.block_step(i, pos, len_bound, attn_hook)
            self._quant(self.x, self.g_final)
        out_ids = ids if advance else self.ids
        if fused and self.logits_t is not None:
            h = self.head
            ctx.ternary_matmul_n([(h.rp, h.tau, h.bias, h.N, self.logits_t)], self.xi, self.s, self.rs, h.K, self.B,
                                 tokens=True)
            ctx.argmax_rows(self.logits_t, out=out_ids, pos=pos if advance else None)
            self._logits = self.logits_t.t()
            return self._logits, out_ids
        self._mm(self.head, self._logits_cols)
        ctx.argmax_cols(self._logits_cols, out=out_ids)
        if advance:
            pos.add_(1)
        self._logits = self._logits_cols
        return self._logits, out_ids


def _pkg():
    import sys
    return sys.modules[__name__.rsplit(".", 1)[0]]


def attention_bytes(B: int, lens, Hkv: int, dk: int, H: int, cache_elem: int = 4) -> int:
    """Algorithmic HBM bytes of one decode attention call: the cached keys and values read
    (lens[b] - 1 rows each, cache_elem bytes per element: 4 in f32 caches, 2 in f16 ones), the
    new key/value (f32) read and their cache rows written, q read and the output written."""
    rows = sum(int(L) - 1 for L in lens)
    return (2 * rows * Hkv * dk * cache_elem + 2 * B * Hkv * dk * 4 + 2 * B * Hkv * dk * cache_elem +
            2 * B * H * dk * 4)

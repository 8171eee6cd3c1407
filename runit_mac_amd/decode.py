"""One greedy decode step of a Qwen2-shape model over the dispatch API.

This is the caller side of the hot path — the per-layer loop of RunIT's
`Executor::forward` / `forward_greedy` (crates/engine/src/forward.rs:1470-1787,
1795-1975) — restated over the C ABI so the GEMV kernels can be measured in
a whole decode step.  Two kernel sequences are provided:

* ``reference``: the reference's own sequence per layer — rms_norm,
  fused_qkv_bias, fused_rope_qk, kv_copy ×2, decode_attention, gemv_add (o),
  rms_norm, fused_ffn, gemv_add (down) — 10 launches per layer;
* ``fused``: the same arithmetic in 5 launches per layer (RMSNorm folded into
  the QKV / FFN / LM-head activation staging; RoPE and the KV-cache write
  folded into attention), captured once into a HIP graph and replayed.

Weights are synthetic (seeded N(0, 0.02) quantised per block, f16 biases
N(0, 0.02), norms 1 + N(0, 0.02)); the KV cache is pre-filled with N(0, 1)
for the positions before the decoded one.

Each projection may take its own block format (``quant``: a Q4_K_M-style mix
keeps V and down in Q6_K): the fused sequence then routes every matrix to the
kernels of its format, as the reference's WeightBuf dispatch does
(forward.rs:70-248).  RMSNorm folds into the Q8_0 and Q4_K_M projections'
activation staging; other formats take it as a launch of its own, and output
projections that are not Q8_0 run after the attention as a second launch.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import dispatch as d


@dataclass(frozen=True)
class DecodeConfig:
    """Qwen2.5-0.5B shapes (config.rs:96-265 reads these from GGUF metadata)."""
    layers: int = 24
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    ff: int = 4864
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1e6
    max_seq: int = 1024

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    def weight_bytes(self, quant: dict | None = None) -> int:
        """Weight bytes read per token (each matrix once), Q8_0 unless
        `quant` names another format for a role."""
        fq = dict(Q8_ALL, **(quant or {}))
        h, q, kv, ff = self.hidden, self.q_dim, self.kv_dim, self.ff
        per_layer = sum(d.weight_bytes(fq[r], n, k) for r, n, k in
                        (("q", q, h), ("k", kv, h), ("v", kv, h), ("o", h, q), ("gate", ff, h),
                         ("up", ff, h), ("down", h, ff)))
        return self.layers * per_layer + d.weight_bytes(fq["lm_head"], self.vocab, h)

    def step_bytes(self, kv_len: int, quant: dict | None = None) -> int:
        """Algorithmic bytes of one step: weights + KV reads + f16 biases and
        f32 norms (activations are a few KB and not counted)."""
        kv = self.layers * 2 * self.kv_heads * kv_len * self.head_dim * 4
        small = self.layers * ((self.q_dim + 2 * self.kv_dim) * 2 + 2 * self.hidden * 4)
        return self.weight_bytes(quant) + kv + small + self.hidden * 4


# Block format per weight role; the embedding table stays Q8_0 (its row is
# read by embed_q8_0_f32).
ROLES = ("q", "k", "v", "o", "gate", "up", "down", "lm_head")
Q8_ALL = {r: "q8_0" for r in ROLES}
# Q4_K_M-style mix: V and down (and the LM head) in Q6_K
Q4K_M = dict(q="q4k", k="q4k", v="q6k", o="q4k", gate="q4k", up="q4k", down="q6k",
             lm_head="q6k")


class Arena:
    """Bump allocator over one device allocation (256-byte aligned pieces)."""

    def __init__(self, ctx: d.HipContext, nbytes: int):
        self.buf = ctx.new_buffer(nbytes)
        self.off = 0

    def take(self, nbytes: int) -> int:
        p = self.buf.ptr + self.off
        self.off += (nbytes + 255) & ~255
        if self.off > self.buf.nbytes:
            raise d.BufferSize(f"buffer size mismatch: expected {self.off} bytes, "
                               f"got {self.buf.nbytes}")
        return p


class DecodeModel:
    """Synthetic Qwen2-shape model resident in one arena, plus the KV cache."""

    def __init__(self, ctx: d.HipContext, cfg: DecodeConfig = DecodeConfig(), seed: int = 7,
                 gguf=None, quant: dict | None = None):
        """Synthetic weights, or (gguf: a runit_mac_amd.gguf.GgufFile) the
        file's tensors: Q8_0 matrices as stored, f32 norms, f32/f16 biases
        converted to f16 (RNE, as upload_weight converts F32, forward.rs:
        442-455), an absent bias as zeros, the LM head tied to token_embd when
        output.weight is absent (forward.rs:1271-1276), and an empty KV cache."""
        self.ctx, self.cfg = ctx, cfg
        c = cfg
        self.quant = fq = dict(Q8_ALL, **(quant or {}))
        if set(fq) != set(ROLES):
            raise ValueError(f"quant roles must be among {ROLES}")
        if gguf is not None and any(f != "q8_0" for f in fq.values()):
            raise ValueError("GGUF models load Q8_0 matrices")
        h, q, kv, ff = c.hidden, c.q_dim, c.kv_dim, c.ff
        wb = lambda n, k, f="q8_0": d.weight_bytes(f, n, k)  # noqa: E731
        per_layer = (wb(q, h, fq["q"]) + wb(kv, h, fq["k"]) + wb(kv, h, fq["v"])
                     + wb(h, q, fq["o"]) + wb(ff, h, fq["gate"]) + wb(ff, h, fq["up"])
                     + wb(h, ff, fq["down"])
                     + 2 * (q + 2 * kv) + 8 * h + 2 * 4 * c.kv_heads * c.max_seq * c.head_dim
                     + 16 * 256)
        tied = (gguf is None or "output.weight" not in gguf) and fq["lm_head"] == "q8_0"
        total = c.layers * per_layer + wb(c.vocab, h) + \
            (0 if tied else wb(c.vocab, h, fq["lm_head"])) + 16 * h + \
            64 * 1024 + 4 * (c.vocab + 8 * ff + 8 * q)
        self.arena = Arena(ctx, total)
        a = self.arena
        s = seed * 1000
        # how every synthetic tensor was generated, in order: (pointer, kind,
        # seed, count, format or (mean, std)) — a host twin rebuilds the same
        # bytes from it (the device generators are pinned to the oracle's)
        self.recipe = []
        lib = d.load_library()

        def upload_host(p, arr):
            arr = np.ascontiguousarray(arr)
            ctx._check(lib.rt_upload(ctx.handle, p, arr.ctypes.data, arr.nbytes))

        def tensor(name, n, k=None, dtypes=()):
            t = gguf.tensor(name)
            shape = (k, n) if k is not None else (n,)
            if t.shape != shape or t.dtype_name not in dtypes:
                raise ValueError(f"{name}: {t.dtype_name} {t.shape}, expected one of {dtypes} "
                                 f"{shape}")
            return t

        def qw(n, k, name=None, fmt="q8_0"):
            nonlocal s
            p = a.take(wb(n, k, fmt))
            if gguf is not None:
                tensor(name, n, k, ("Q8_0",))
                gguf.upload(ctx, name, p)
            else:
                d.synth_weights(ctx, fmt, p, n * k // d.BLOCK[fmt][0], s)
                self.recipe.append((p, "w", s, n * k, fmt))
                s += 1
            return p

        def f32(n, mean, std, name=None):
            nonlocal s
            p = a.take(4 * n)
            if gguf is not None and name is not None:
                t = tensor(name, n, dtypes=("F32", "F16"))
                raw = gguf.tensor_bytes(name)
                v = raw.view(np.float32) if t.dtype_name == "F32" else \
                    raw.view(np.float16).astype(np.float32)
                upload_host(p, v)
            elif gguf is not None:  # KV cache of a loaded model: empty
                ctx._check(lib.rt_memset(ctx.handle, p, 0, 4 * n))
            else:
                d.synth_normal_f32(ctx, p, n, s, mean, std)
                self.recipe.append((p, "f32", s, n, (mean, std)))
                s += 1
            return p

        def f16(n, std, name=None):
            nonlocal s
            p = a.take(2 * n)
            if gguf is not None:
                if name in gguf:
                    t = tensor(name, n, dtypes=("F32", "F16"))
                    raw = gguf.tensor_bytes(name)
                    v = raw.view(np.float16) if t.dtype_name == "F16" else \
                        raw.view(np.float32).astype(np.float16)
                else:
                    v = np.zeros(n, np.float16)
                upload_host(p, v)
            else:
                d.synth_normal_f16(ctx, p, n, s, 0.0, std)
                self.recipe.append((p, "f16", s, n, (0.0, std)))
                s += 1
            return p

        self.layers = []
        for i in range(c.layers):
            b = f"blk.{i}."
            L = dict(wq=qw(q, h, b + "attn_q.weight", fq["q"]),
                     wk=qw(kv, h, b + "attn_k.weight", fq["k"]),
                     wv=qw(kv, h, b + "attn_v.weight", fq["v"]),
                     bq=f16(q, 0.02, b + "attn_q.bias"),
                     bk=f16(kv, 0.02, b + "attn_k.bias"), bv=f16(kv, 0.02, b + "attn_v.bias"),
                     wo=qw(h, q, b + "attn_output.weight", fq["o"]),
                     wg=qw(ff, h, b + "ffn_gate.weight", fq["gate"]),
                     wu=qw(ff, h, b + "ffn_up.weight", fq["up"]),
                     wd=qw(h, ff, b + "ffn_down.weight", fq["down"]),
                     attn_norm=f32(h, 1.0, 0.02, b + "attn_norm.weight"),
                     ffn_norm=f32(h, 1.0, 0.02, b + "ffn_norm.weight"),
                     kc=f32(c.kv_heads * c.max_seq * c.head_dim, 0.0, 1.0),
                     vc=f32(c.kv_heads * c.max_seq * c.head_dim, 0.0, 1.0))
            self.layers.append(L)
        self.final_norm = f32(h, 1.0, 0.02, "output_norm.weight")
        self.embd = qw(c.vocab, h, "token_embd.weight")
        # LM head: tied to token_embd unless the file has output.weight
        self.lm_head = self.embd if tied else qw(c.vocab, h, "output.weight", fq["lm_head"])
        # activations
        self.x = a.take(4 * h)
        self.xn = a.take(4 * h)
        self.q = a.take(4 * q)
        self.k = a.take(4 * kv)
        self.v = a.take(4 * kv)
        self.attn = a.take(4 * q)
        self.act = a.take(4 * ff)
        self.logits = a.take(4 * c.vocab)
        self.token = a.take(256)
        ctx.flush()

    @classmethod
    def from_gguf(cls, ctx: d.HipContext, gguf, max_seq: int = 1024) -> "DecodeModel":
        """A Qwen2-family model from a GGUF file (Q8_0 matrices), with the
        dimensions of ModelConfig.from_metadata (config.rs:96-265)."""
        from .gguf import ModelConfig
        mc = ModelConfig.from_metadata(gguf.metadata, gguf.metadata_types)
        cfg = DecodeConfig(layers=mc.num_hidden_layers, hidden=mc.hidden_size,
                           heads=mc.num_attention_heads, kv_heads=mc.num_key_value_heads,
                           head_dim=mc.head_dim, ff=mc.intermediate_size, vocab=mc.vocab_size,
                           eps=mc.rms_norm_eps, theta=mc.rope_theta, max_seq=max_seq)
        return cls(ctx, cfg, gguf=gguf)

    def set_token(self, tok: int) -> None:
        buf = np.array([tok], np.uint32)  # kept alive across the synchronous copy
        self.ctx._check(d.load_library().rt_upload(self.ctx.handle, self.token,
                                                   buf.ctypes.data, 4))

    def get_token(self) -> int:
        out = np.zeros(1, np.uint32)
        self.ctx._check(d.load_library().rt_download(self.ctx.handle, out.ctypes.data,
                                                     self.token, 4))
        return int(out[0])

    def read(self, ptr: int, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.ctx._check(d.load_library().rt_download(self.ctx.handle, out.ctypes.data, ptr,
                                                     out.nbytes))
        return out

    # ─────────────────────────── step sequences ───────────────────────────

    def step_reference(self, pos: int) -> None:
        """forward.rs:1494-1771, the reference's kernel sequence (Q8_0 models)."""
        if any(f != "q8_0" for f in self.quant.values()):
            raise ValueError("the reference sequence is built for Q8_0 models")
        ctx, c = self.ctx, self.cfg
        h, q_dim, kv_dim = c.hidden, c.q_dim, c.kv_dim
        d.embed_q8_0_f32(ctx, self.embd, self.token, self.x, h)
        for L in self.layers:
            d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, L["attn_norm"], c.eps, h, 1)
            d.fused_qkv_bias_q8_0_f32(ctx, L["wq"], L["wk"], L["wv"], self.xn, self.q, self.k,
                                      self.v, L["bq"], L["bk"], L["bv"], q_dim, kv_dim, h)
            d.fused_rope_qk_f32(ctx, self.q, self.k, c.head_dim, c.heads, c.kv_heads, pos,
                                c.theta)
            d.kv_copy_to_cache_f32(ctx, self.k, L["kc"], pos, c.max_seq, c.head_dim, c.kv_heads)
            d.kv_copy_to_cache_f32(ctx, self.v, L["vc"], pos, c.max_seq, c.head_dim, c.kv_heads)
            d.decode_attention_f32(ctx, self.q, L["kc"], L["vc"], self.attn, 1, pos + 1, c.heads,
                                   c.kv_heads, c.head_dim, c.max_seq)
            d.gemv_q8_0_add_f32_f32in_mr(ctx, L["wo"], self.attn, self.x, self.x, h, q_dim)
            d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, L["ffn_norm"], c.eps, h, 1)
            d.fused_ffn_q8_0_f32(ctx, L["wg"], L["wu"], self.xn, self.act, c.ff, h)
            d.gemv_q8_0_add_f32_f32in_mr(ctx, L["wd"], self.act, self.x, self.x, h, c.ff)
        d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, self.final_norm, c.eps, h, 1)
        d.gemv_q8_0_f32in_f32out_mr(ctx, self.lm_head, self.xn, self.logits, c.vocab, h)
        d.argmax_f32(ctx, self.logits, self.token, c.vocab)

    def _qkv(self, L, x) -> None:
        """Q/K/V (+ bias) of the input x, routed by the projections' formats."""
        c, fq = self.cfg, self.quant
        fqk, fv = fq["q"], fq["v"]
        if fq["k"] != fqk:
            raise ValueError("Q and K must share a format")
        name = (f"fused_qkv_bias_{fqk}_f32" if fv == fqk else f"fused_qkv_bias_{fqk}_{fv}_f32")
        fn = getattr(d, name, None)
        if fn is None:
            raise ValueError(f"no fused Q/K/V for Q/K in {fqk}, V in {fv}")
        fn(self.ctx, L["wq"], L["wk"], L["wv"], x, self.q, self.k, self.v, L["bq"], L["bk"],
           L["bv"], c.q_dim, c.kv_dim, c.hidden)

    def step_fused(self, pos: int) -> None:
        """Same arithmetic, 5 launches per layer for Q8_0 (RMSNorm folded into
        the staging of the next GEMV, attention merged into the output
        projection); other formats add a launch for each RMSNorm and split
        attention from the output projection."""
        ctx, c, fq = self.ctx, self.cfg, self.quant
        h, q_dim, kv_dim = c.hidden, c.q_dim, c.kv_dim
        d.embed_q8_0_f32(ctx, self.embd, self.token, self.x, h)
        for L in self.layers:
            if fq["q"] == fq["k"] == fq["v"] == "q8_0":
                d.rms_norm_fused_qkv_bias_q8_0_f32(ctx, L["wq"], L["wk"], L["wv"], self.x,
                                                   L["attn_norm"], c.eps, self.q, self.k, self.v,
                                                   L["bq"], L["bk"], L["bv"], q_dim, kv_dim, h)
            elif (fq["q"], fq["k"], fq["v"]) == ("q4k", "q4k", "q6k") and h <= 8192:
                d.rms_norm_fused_qkv_bias_q4k_q6k_f32(ctx, L["wq"], L["wk"], L["wv"], self.x,
                                                      L["attn_norm"], c.eps, self.q, self.k,
                                                      self.v, L["bq"], L["bk"], L["bv"], q_dim,
                                                      kv_dim, h)
            else:
                d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, L["attn_norm"], c.eps, h, 1)
                self._qkv(L, self.xn)
            if fq["o"] == "q8_0":
                d.decode_attention_rope_oproj_q8_0_f32(ctx, self.q, self.k, self.v, L["kc"],
                                                       L["vc"], L["wo"], self.x, pos, c.max_seq,
                                                       c.heads, c.kv_heads, c.head_dim,
                                                       c.theta, h)
            else:
                d.decode_attention_rope_f32(ctx, self.q, self.k, self.v, L["kc"], L["vc"],
                                            self.attn, pos, c.max_seq, c.heads, c.kv_heads,
                                            c.head_dim, c.theta)
                getattr(d, f"gemv_{fq['o']}_add_f32_f32in")(ctx, L["wo"], self.attn, self.x,
                                                            self.x, h, q_dim)
            if fq["gate"] != fq["up"]:
                raise ValueError("gate and up must share a format")
            if fq["gate"] in ("q8_0", "q4k"):
                getattr(d, f"rms_norm_fused_ffn_{fq['gate']}_f32")(
                    ctx, L["wg"], L["wu"], self.x, L["ffn_norm"], c.eps, self.act, c.ff, h)
            else:
                d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, L["ffn_norm"], c.eps, h, 1)
                getattr(d, f"fused_ffn_{fq['gate']}_f32")(ctx, L["wg"], L["wu"], self.xn,
                                                          self.act, c.ff, h)
            getattr(d, f"gemv_{fq['down']}_add_f32_f32in")(ctx, L["wd"], self.act, self.x,
                                                           self.x, h, c.ff)
        if fq["lm_head"] in ("q8_0", "q6k"):
            getattr(d, f"rms_norm_gemv_{fq['lm_head']}_f32in_f32out")(
                ctx, self.lm_head, self.x, self.final_norm, c.eps, self.logits, c.vocab, h)
        else:
            d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, self.final_norm, c.eps, h, 1)
            getattr(d, f"gemv_{fq['lm_head']}_f32in_f32out")(ctx, self.lm_head, self.xn,
                                                             self.logits, c.vocab, h)
        d.argmax_f32(ctx, self.logits, self.token, c.vocab)

    def launches_fused(self) -> int:
        """Launches of one fused step."""
        fq, h = self.quant, self.cfg.hidden
        qkv_norm_fused = (fq["q"] == fq["k"] == fq["v"] == "q8_0" or
                          ((fq["q"], fq["k"], fq["v"]) == ("q4k", "q4k", "q6k") and h <= 8192))
        per = (1 if qkv_norm_fused else 2) + 2 + \
            (1 if fq["gate"] in ("q8_0", "q4k") else 2) + 1
        return 1 + self.cfg.layers * per + (1 if fq["lm_head"] in ("q8_0", "q6k") else 2) + 1

    def capture(self, pos: int, fused: bool = True) -> d.Graph:
        """One step captured as a HIP graph (the reference's single command
        buffer per token, context.rs:248-296)."""
        step = self.step_fused if fused else self.step_reference
        step(pos)  # eager first run sizes any workspace before capture
        self.ctx.flush()
        self.ctx.capture_begin()
        step(pos)
        return self.ctx.capture_end()

    def free(self) -> None:
        self.arena.buf.free()

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


# GGUF tensor dtype → block format of the kernels, per layout: real files
# (upstream quantisers) use ggml's layouts; "reference" reads Q4_0 / Q4_K /
# Q5_K / Q6_K with the reference's own decoders (forward.rs:900-1057), which
# differ from ggml's (docs/STATUS_REPORT.md:184).  Q8_0 and Q5_0 agree.
GGUF_FORMATS = {
    "ggml": {"Q8_0": "q8_0", "Q4_0": "q4_0g", "Q4_K": "q4kg", "Q5_0": "q5_0", "Q5_K": "q5kg",
             "Q6_K": "q6kg"},
    "reference": {"Q8_0": "q8_0", "Q4_0": "q4_0", "Q4_K": "q4k", "Q5_0": "q5_0", "Q5_K": "q5k",
                  "Q6_K": "q6k"},
}
# embedding tables may also be plain rows
EMBED_FORMATS = {"F16": "f16", "F32": "f32"}
_MATRIX_ROLES = (("q", "wq", "attn_q"), ("k", "wk", "attn_k"), ("v", "wv", "attn_v"),
                 ("o", "wo", "attn_output"), ("gate", "wg", "ffn_gate"), ("up", "wu", "ffn_up"),
                 ("down", "wd", "ffn_down"))


def _fmt_bytes(fmt: str, n: int, k: int) -> int:
    if fmt in ("f16", "f32"):
        return n * k * (2 if fmt == "f16" else 4)
    return d.weight_bytes(fmt, n, k)


def accept_drafts(argmax_rows, drafts) -> tuple[int, int]:
    """The acceptance loop of verify_draft (forward.rs:2279-2305): row r's
    argmax must equal draft r; the first row that differs ends it with its
    argmax as the correct next token; when every draft is accepted the last
    row's argmax is the next token.  len(argmax_rows) = len(drafts) + 1."""
    if len(argmax_rows) != len(drafts) + 1:
        raise ValueError("one argmax per verified row (prompt token + drafts) expected")
    accepted = 0
    for r, best in enumerate(int(b) for b in argmax_rows):
        if r < len(drafts):
            if best != int(drafts[r]):
                return accepted, best
            accepted += 1
        else:
            return accepted, best
    raise AssertionError("unreachable")


class DecodeModel:
    """Qwen2-shape model resident in one arena, plus the KV cache.

    Every weight matrix carries its own block format (``layers[i]["fmt"]``,
    ``embd_fmt``, ``lm_fmt``), and the step routes each matrix to its
    format's kernels, as the reference's WeightBuf dispatch does per tensor
    (forward.rs:70-248, chosen by dtype in upload_weight_wb, :1137-1222)."""

    def __init__(self, ctx: d.HipContext, cfg: DecodeConfig = DecodeConfig(), seed: int = 7,
                 gguf=None, quant: dict | None = None, layout: str = "ggml"):
        """Synthetic weights (seeded N(0, 0.02) quantised per block; `quant`:
        format per role), or (gguf: a runit_mac_amd.gguf.GgufFile) the file's
        tensors, each routed by its own dtype (Q8_0, Q4_0, Q4_K, Q5_0, Q5_K,
        Q6_K read in `layout`: "ggml" for upstream files, "reference" for the
        reference's decoders), f32 norms, f32/f16 biases converted to f16
        (RNE, as upload_weight converts F32, forward.rs:442-455), an absent
        bias as zeros, the LM head tied to token_embd when output.weight is
        absent (forward.rs:1271-1276), and an empty KV cache."""
        self.ctx, self.cfg = ctx, cfg
        c = cfg
        if gguf is not None and quant is not None:
            raise ValueError("quant applies to synthetic weights; a GGUF file names its dtypes")
        if layout not in GGUF_FORMATS:
            raise ValueError(f"layout must be one of {tuple(GGUF_FORMATS)}")
        self.quant = fq = dict(Q8_ALL, **(quant or {}))
        if set(fq) != set(ROLES):
            raise ValueError(f"quant roles must be among {ROLES}")
        h, q, kv, ff = c.hidden, c.q_dim, c.kv_dim, c.ff
        shapes = {"q": (q, h), "k": (kv, h), "v": (kv, h), "o": (h, q), "gate": (ff, h),
                  "up": (ff, h), "down": (h, ff)}

        def file_fmt(name, n, k, embed=False):
            t = gguf.tensor(name)
            if t.shape != (k, n):
                raise ValueError(f"{name}: shape {t.shape}, expected {(k, n)}")
            table = dict(GGUF_FORMATS[layout], **(EMBED_FORMATS if embed else {}))
            if t.dtype_name not in table:
                raise ValueError(f"{name}: dtype {t.dtype_name} has no GPU path here "
                                 f"(supported: {sorted(table)})")
            return table[t.dtype_name]

        # format of every matrix
        if gguf is not None:
            lfmts = [{role: file_fmt(f"blk.{i}.{base}.weight", *shapes[role])
                      for role, _, base in _MATRIX_ROLES} for i in range(c.layers)]
            self.embd_fmt = file_fmt("token_embd.weight", c.vocab, h, embed=True)
            tied = "output.weight" not in gguf
            self.lm_fmt = self.embd_fmt if tied else file_fmt("output.weight", c.vocab, h)
            if self.lm_fmt in ("f16", "f32"):
                raise ValueError(f"LM head in {self.lm_fmt}: no f16/f32-weight GEMV here")
        else:
            lfmts = [{role: fq[role] for role, _, _ in _MATRIX_ROLES} for _ in range(c.layers)]
            self.embd_fmt = "q8_0"
            tied = fq["lm_head"] == "q8_0"
            self.lm_fmt = fq["lm_head"]
        per_layer = [sum(_fmt_bytes(L[r], *shapes[r]) + 256 for r in shapes) for L in lfmts]
        small = 2 * (q + 2 * kv) + 8 * h + 2 * 4 * c.kv_heads * c.max_seq * c.head_dim + 16 * 256
        total = sum(per_layer) + c.layers * small + _fmt_bytes(self.embd_fmt, c.vocab, h) + \
            (0 if tied else _fmt_bytes(self.lm_fmt, c.vocab, h)) + 16 * h + \
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

        def tensor(name, n, dtypes=()):
            t = gguf.tensor(name)
            if t.shape != (n,) or t.dtype_name not in dtypes:
                raise ValueError(f"{name}: {t.dtype_name} {t.shape}, expected one of {dtypes} "
                                 f"{(n,)}")
            return t

        def qw(n, k, name, fmt):
            nonlocal s
            p = a.take(_fmt_bytes(fmt, n, k))
            if gguf is not None:
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
            F = lfmts[i]
            L = dict(wq=qw(q, h, b + "attn_q.weight", F["q"]),
                     wk=qw(kv, h, b + "attn_k.weight", F["k"]),
                     wv=qw(kv, h, b + "attn_v.weight", F["v"]),
                     bq=f16(q, 0.02, b + "attn_q.bias"),
                     bk=f16(kv, 0.02, b + "attn_k.bias"), bv=f16(kv, 0.02, b + "attn_v.bias"),
                     wo=qw(h, q, b + "attn_output.weight", F["o"]),
                     wg=qw(ff, h, b + "ffn_gate.weight", F["gate"]),
                     wu=qw(ff, h, b + "ffn_up.weight", F["up"]),
                     wd=qw(h, ff, b + "ffn_down.weight", F["down"]),
                     attn_norm=f32(h, 1.0, 0.02, b + "attn_norm.weight"),
                     ffn_norm=f32(h, 1.0, 0.02, b + "ffn_norm.weight"),
                     kc=f32(c.kv_heads * c.max_seq * c.head_dim, 0.0, 1.0),
                     vc=f32(c.kv_heads * c.max_seq * c.head_dim, 0.0, 1.0))
            self.layers.append(L)
        self.fmts = lfmts
        self.final_norm = f32(h, 1.0, 0.02, "output_norm.weight")
        self.embd = qw(c.vocab, h, "token_embd.weight", self.embd_fmt)
        # LM head: tied to token_embd unless the file has output.weight
        self.lm_head = self.embd if tied else qw(c.vocab, h, "output.weight", self.lm_fmt)
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
        # Σx² partial sums (one per 4 elements of x) handed from the launch
        # that updates x to the norm-fused launch that reads it
        self.ssq = [a.take(4 * ((h + 3) // 4)) for _ in range(2)]
        self.hand_off_norm = True  # (False: every norm-fused launch reduces x itself)
        self._launches = None
        ctx.flush()

    @classmethod
    def from_gguf(cls, ctx: d.HipContext, gguf, max_seq: int = 1024,
                  layout: str = "ggml") -> "DecodeModel":
        """A Qwen2-family model from a GGUF file, with the dimensions of
        ModelConfig.from_metadata (config.rs:96-265); every matrix keeps the
        file's dtype (in `layout`) and runs on that format's kernels."""
        from .gguf import ModelConfig
        mc = ModelConfig.from_metadata(gguf.metadata, gguf.metadata_types)
        cfg = DecodeConfig(layers=mc.num_hidden_layers, hidden=mc.hidden_size,
                           heads=mc.num_attention_heads, kv_heads=mc.num_key_value_heads,
                           head_dim=mc.head_dim, ff=mc.intermediate_size, vocab=mc.vocab_size,
                           eps=mc.rms_norm_eps, theta=mc.rope_theta, max_seq=max_seq)
        return cls(ctx, cfg, gguf=gguf, layout=layout)

    def weight_bytes(self) -> int:
        """Weight bytes read per token: every matrix once, in its own format."""
        c = self.cfg
        h, q, kv, ff = c.hidden, c.q_dim, c.kv_dim, c.ff
        shapes = {"q": (q, h), "k": (kv, h), "v": (kv, h), "o": (h, q), "gate": (ff, h),
                  "up": (ff, h), "down": (h, ff)}
        return sum(_fmt_bytes(F[r], *shapes[r]) for F in self.fmts for r in shapes) + \
            _fmt_bytes(self.lm_fmt, c.vocab, h)

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
        if self.embd_fmt != "q8_0" or self.lm_fmt != "q8_0" or \
                any(f != "q8_0" for F in self.fmts for f in F.values()):
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

    # Routing of one layer's launches by its matrices' formats (the WeightBuf
    # match arms of forward.rs:1543-1568, 1684-1702): each returns the number
    # of launches it issues.
    def _plan_qkv(self, F) -> str:
        fqk, fk, fv = F["q"], F["k"], F["v"]
        h = self.cfg.hidden
        if fqk == fk == fv == "q8_0":
            return "norm_q8_0"
        if (fqk, fk, fv) == ("q4k", "q4k", "q6k") and h <= 8192:
            return "norm_q4k_q6k"
        if fqk == fk and hasattr(d, f"fused_qkv_bias_{fqk}_f32") and fv == fqk:
            return "fused"
        if fqk == fk and hasattr(d, f"fused_qkv_bias_{fqk}_{fv}_f32"):
            return "fused_mixed"
        return "separate"

    def _qkv(self, L, F, x) -> int:
        """Q/K/V (+ bias) of the normalised input x: one fused launch where a
        kernel covers the formats, else the reference's fallback of three
        GEMVs each followed by add_f16_into_f32 (forward.rs:1561-1568)."""
        c, ctx = self.cfg, self.ctx
        plan = self._plan_qkv(F)
        args = (L["wq"], L["wk"], L["wv"], x, self.q, self.k, self.v, L["bq"], L["bk"], L["bv"],
                c.q_dim, c.kv_dim, c.hidden)
        if plan == "fused":
            getattr(d, f"fused_qkv_bias_{F['q']}_f32")(ctx, *args)
            return 1
        if plan == "fused_mixed":
            getattr(d, f"fused_qkv_bias_{F['q']}_{F['v']}_f32")(ctx, *args)
            return 1
        for role, w, b, out, n in (("q", "wq", "bq", self.q, c.q_dim),
                                   ("k", "wk", "bk", self.k, c.kv_dim),
                                   ("v", "wv", "bv", self.v, c.kv_dim)):
            getattr(d, f"gemv_{F[role]}_f32in_f32out")(ctx, L[w], x, out, n, c.hidden)
            d.add_f16_into_f32(ctx, L[b], out, n)
        return 6

    def step_fused(self, pos: int) -> int:
        """One greedy step: embedding, per layer Q/K/V (+ bias), RoPE + KV
        write + attention, O (+ residual), gate/up/SiLU, down (+ residual);
        final norm, LM head, argmax.  RMSNorm folds into the next launch's
        staging for the Q8_0 and Q4_K_M projections, the attention's split
        merge into the Q8_0 and Q4_K output projections; other formats take
        them as launches of their own.  Returns the number of launches (as
        the library counted them)."""
        ctx, c = self.ctx, self.cfg
        h, q_dim = c.hidden, c.q_dim
        n0 = d.launch_count(ctx)
        n = 1
        d.embed_f32(ctx, self.embd_fmt, self.embd, self.token, self.x, h)
        # Q8_0 layers of a model whose x fits 256 partial sums hand the RMSNorm
        # factor from the launch that updates x (O, down) to the norm-fused
        # launch after it (gate+up, the next layer's Q/K/V)
        nparts = (h + 3) // 4
        ssq_x = None  # partial sums of the current x, if a launch wrote them
        for L, F in zip(self.layers, self.fmts):
            plan = self._plan_qkv(F)
            q8 = (self.hand_off_norm and nparts <= 256
                  and F["o"] == F["gate"] == F["up"] == F["down"] == "q8_0")
            if plan == "norm_q8_0" and ssq_x is not None:
                d.rms_norm_fused_qkv_bias_q8_0_f32_ssq(
                    ctx, L["wq"], L["wk"], L["wv"], self.x, L["attn_norm"], c.eps, self.q,
                    self.k, self.v, L["bq"], L["bk"], L["bv"], q_dim, c.kv_dim, h, ssq_x, nparts)
                n += 1
            elif plan == "norm_q8_0":
                d.rms_norm_fused_qkv_bias_q8_0_f32(ctx, L["wq"], L["wk"], L["wv"], self.x,
                                                   L["attn_norm"], c.eps, self.q, self.k, self.v,
                                                   L["bq"], L["bk"], L["bv"], q_dim, c.kv_dim, h)
                n += 1
            elif plan == "norm_q4k_q6k":
                d.rms_norm_fused_qkv_bias_q4k_q6k_f32(ctx, L["wq"], L["wk"], L["wv"], self.x,
                                                      L["attn_norm"], c.eps, self.q, self.k,
                                                      self.v, L["bq"], L["bk"], L["bv"], q_dim,
                                                      c.kv_dim, h)
                n += 1
            else:
                d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, L["attn_norm"], c.eps, h, 1)
                n += 1 + self._qkv(L, F, self.xn)
            ssq_x = None
            if q8:
                d.decode_attention_rope_oproj_q8_0_f32_ssq(
                    ctx, self.q, self.k, self.v, L["kc"], L["vc"], L["wo"], self.x, pos,
                    c.max_seq, c.heads, c.kv_heads, c.head_dim, c.theta, h, self.ssq[0])
                ssq_x = self.ssq[0]
            elif F["o"] in ("q8_0", "q4k", "q4kg"):
                getattr(d, f"decode_attention_rope_oproj_{F['o']}_f32")(
                    ctx, self.q, self.k, self.v, L["kc"], L["vc"], L["wo"], self.x, pos,
                    c.max_seq, c.heads, c.kv_heads, c.head_dim, c.theta, h)
            else:
                d.decode_attention_rope_f32(ctx, self.q, self.k, self.v, L["kc"], L["vc"],
                                            self.attn, pos, c.max_seq, c.heads, c.kv_heads,
                                            c.head_dim, c.theta)
                getattr(d, f"gemv_{F['o']}_add_f32_f32in")(ctx, L["wo"], self.attn, self.x,
                                                           self.x, h, q_dim)
            n += 2
            if q8 and ssq_x is not None:
                d.rms_norm_fused_ffn_q8_0_f32_ssq(ctx, L["wg"], L["wu"], self.x, L["ffn_norm"],
                                                  c.eps, self.act, c.ff, h, ssq_x, nparts)
                n += 1
            elif F["gate"] == F["up"] and F["gate"] in ("q8_0", "q4k"):
                getattr(d, f"rms_norm_fused_ffn_{F['gate']}_f32")(
                    ctx, L["wg"], L["wu"], self.x, L["ffn_norm"], c.eps, self.act, c.ff, h)
                n += 1
            else:
                d.rms_norm_f32_f32_f32g(ctx, self.x, self.xn, L["ffn_norm"], c.eps, h, 1)
                n += 1
                if F["gate"] == F["up"] and hasattr(d, f"fused_ffn_{F['gate']}_f32"):
                    getattr(d, f"fused_ffn_{F['gate']}_f32")(ctx, L["wg"], L["wu"], self.xn,
                                                              self.act, c.ff, h)
                    n += 1
                else:
                    raise ValueError(f"gate {F['gate']} / up {F['up']}: no fused gate+up+SiLU")
            if q8:
                d.gemv_q8_0_add_f32_f32in_ssq(ctx, L["wd"], self.act, self.x, self.x, h, c.ff,
                                              self.ssq[1])
                ssq_x = self.ssq[1]
            else:
                getattr(d, f"gemv_{F['down']}_add_f32_f32in")(ctx, L["wd"], self.act, self.x,
                                                              self.x, h, c.ff)
                ssq_x = None
            n += 1
        n += self._lm_head(self.x)
        d.argmax_f32(ctx, self.logits, self.token, c.vocab)
        # launches as the library counted them (a fused call may fall back to
        # its unfused sequence)
        self._launches = d.launch_count(ctx) - n0
        return self._launches

    def launches_fused(self) -> int:
        """Launches of one fused step, as the last step_fused issued them (the
        attention + output projection pair counted as two)."""
        if self._launches is None:
            raise RuntimeError("no fused step has run yet")
        return self._launches

    def plan_persistent(self, pos: int) -> d.DecodeStep:
        """The step at `pos` as one persistent launch (k_decode_step_q8_0:
        embedding and every layer, weights of each phase requested before the
        grid barrier that precedes it) + the norm-fused LM head + argmax.
        Q8_0 models with head size 64."""
        if self.embd_fmt != "q8_0" or self.lm_fmt != "q8_0" or \
                any(f != "q8_0" for F in self.fmts for f in F.values()):
            raise ValueError("the persistent step is built for Q8_0 models")
        c = self.cfg
        layers = (d.StepLayer * c.layers)()
        for i, L in enumerate(self.layers):
            for k_dev, k_c in (("wq", "wq"), ("wk", "wk"), ("wv", "wv"), ("wo", "wo"), ("wg", "wg"),
                               ("wu", "wu"), ("wd", "wd"), ("bq", "bq"), ("bk", "bk"),
                               ("bv", "bv"), ("attn_norm", "attn_norm"),
                               ("ffn_norm", "ffn_norm"), ("kc", "k_cache"), ("vc", "v_cache")):
                setattr(layers[i], k_c, L[k_dev])
        model = d.StepModel(c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim, c.ff, c.vocab,
                            c.max_seq, c.eps, c.theta, layers, self.embd, self.lm_head,
                            self.final_norm, self.token, self.logits)
        step = d.DecodeStep(self.ctx, model, pos)
        step._layers = layers
        return step

    # ───────────────────────── batched verify ─────────────────────────

    def _verify_arena(self, rows: int, logits: bool = True) -> dict:
        """Activation buffers of an M-row pass, [rows][dim] f32, allocated
        once per largest M seen (with the [rows][vocab] logits only when a
        caller needs every row's logits: not for prefill)."""
        v = getattr(self, "_vbufs", None)
        if v is not None and v["rows"] >= rows and (v["has_logits"] or not logits):
            return v
        if v is not None:
            # the old arena stays allocated until free(): a graph captured
            # over it (verify_pass is capturable) keeps valid pointers
            rows = max(rows, v["rows"])
            self._retired_arenas = getattr(self, "_retired_arenas", []) + [v["arena"]]
        c = self.cfg
        dims = dict(x=c.hidden, xn=c.hidden, q=c.q_dim, k=c.kv_dim, v=c.kv_dim, att=c.q_dim,
                    p=c.hidden, g=c.ff, u=c.ff)
        if logits:
            dims["logits"] = c.vocab
        dims.update(tok=1, idx=1)
        a = Arena(self.ctx, sum(((4 * rows * n + 255) & ~255) for n in dims.values()))
        v = {k: a.take(4 * rows * n) for k, n in dims.items()}
        v.update(rows=rows, arena=a, has_logits=logits)
        self._vbufs = v
        return v

    def verify_forward(self, tokens, start_pos: int, form: str | None = None) -> dict:
        """verify_draft's batched forward (forward.rs:2141-2273) on the GPU:
        the M tokens embedded together; per layer Q/K/V (+ bias) of the
        normalised rows, batched RoPE at start_pos.., the M keys / values
        written to the cache, causal attention (row r at position
        start_pos + r sees the cache up to there), O (+ residual), gate+up+SiLU
        of the normalised rows, down (+ residual); the final norm and the LM
        head, and the per-row first-max argmax.  Every projection runs in its
        matrix's own format (see verify_pass for the two forms).  Returns the
        activation buffers (``logits``: [M][vocab], ``idx``: [M] argmax)."""
        ctx, c = self.ctx, self.cfg
        ids = np.asarray(tokens).astype(np.int64, casting="same_kind").ravel()
        if ids.size == 0:
            raise ValueError("verify: empty sequence")
        # the embedding kernel indexes the table with the id unchecked: a
        # negative or past-the-vocabulary id is refused before any upload
        if np.any(ids < 0) or np.any(ids >= c.vocab):
            raise ValueError(f"verify: token id out of range [0, {c.vocab})")
        toks = ids.astype(np.uint32)
        M = int(toks.size)
        if start_pos + M > c.max_seq:
            raise ValueError(f"verify: start_pos {start_pos} + {M} tokens exceed the KV cache "
                             f"({c.max_seq})")
        if self.lm_fmt in ("f16", "f32"):
            raise ValueError(f"LM head in {self.lm_fmt}: no f16/f32-weight GEMM here")
        B = self._verify_arena(M)
        lib = d.load_library()
        ctx._check(lib.rt_upload(ctx.handle, B["tok"], toks.ctypes.data, toks.nbytes))
        return self.verify_pass(M, start_pos, form)

    # Batches of up to VERIFY_ROWS_MAX rows of a model with a hidden size of at
    # most 1024 take the multi-row GEMVs (weights read once per 8 rows, norms /
    # biases / SiLU / residuals fused in; at the 0.5B shapes, 8 rows: 12.4 µs
    # for gate+up+SiLU, 9.1 µs for O + residual).  Larger models and longer
    # batches take the batched GEMMs, which are faster there (the 7B Q4_K
    # gate+up at 8 rows: 72.8 µs as multi-row GEMVs; the whole 0.5B pass at
    # 4 / 8 / 16 rows: 1.54 / 1.59 / 1.71 ms on the GEMMs, 1.37 / 1.75 / 3.01
    # ms on the multi-row GEMVs, even at about 6).
    VERIFY_ROWS_MAX = 5
    VERIFY_ROWS_MAX_HIDDEN = 1024

    def verify_pass(self, M: int, start_pos: int, form: str | None = None,
                    last_only: bool = False) -> dict:
        """The launches of verify_forward for the M token ids already in the
        verify buffers (``tok``): no host transfer, so it can be captured.
        form: "rows" (multi-row GEMVs) or "gemm" (batched GEMMs + separate
        norm / bias / SiLU / residual kernels, the reference's sequence);
        default by M."""
        ctx, c = self.ctx, self.cfg
        B = self._verify_arena(M, logits=not last_only)
        h, qd, kvd, hd, ff = c.hidden, c.q_dim, c.kv_dim, c.head_dim, c.ff
        X, XN, Xo = B["x"], B["xn"], B["p"]
        form = form or ("rows" if M <= self.VERIFY_ROWS_MAX and h <= self.VERIFY_ROWS_MAX_HIDDEN
                        else "gemm")
        if form not in ("rows", "gemm"):
            raise ValueError("form must be 'rows' or 'gemm'")
        d.embed_rows_f32(ctx, self.embd_fmt, self.embd, B["tok"], X, h, M)

        for L, F in zip(self.layers, self.fmts):
            if form == "rows":
                # Q/K/V (+ bias) of the normalised rows, one call per format
                for fmt in dict.fromkeys((F["q"], F["k"], F["v"])):
                    sel = lambda role, key: L[key] if F[role] == fmt else None
                    d.qkv_bias_rows_f32(ctx, fmt, sel("q", "wq"), sel("k", "wk"), sel("v", "wv"), X,
                                        B["q"] if F["q"] == fmt else None,
                                        B["k"] if F["k"] == fmt else None,
                                        B["v"] if F["v"] == fmt else None,
                                        sel("q", "bq"), sel("k", "bk"), sel("v", "bv"), M, qd, kvd, h,
                                        gamma=L["attn_norm"], eps=c.eps)
                d.rope_kv_write_batch_f32(ctx, B["q"], B["k"], B["v"], L["kc"], L["vc"], hd, c.heads,
                                          c.kv_heads, start_pos, c.theta, M, c.max_seq)
            else:
                # Q/K/V (+ bias) of the normalised rows: one preparation of
                # RMSNorm(X)·γ for the three GEMMs; the biases, RoPE and the
                # cache writes in their sums
                d.gemm_qkv_rope_f32(ctx, (F["q"], F["k"], F["v"]), L["wq"], L["wk"], L["wv"],
                                    L["bq"], L["bk"], L["bv"], X, L["attn_norm"], c.eps, XN,
                                    B["q"], B["k"], B["v"], L["kc"], L["vc"], M, h, qd, kvd, hd,
                                    start_pos, c.theta, c.max_seq)
            if form == "rows":
                d.flash_attention_f32(ctx, B["q"], L["kc"], L["vc"], B["att"], 1, M, start_pos + M,
                                      c.heads, c.kv_heads, hd, c.max_seq, q_start=start_pos)
                d.gemv_rows_add_f32(ctx, F["o"], L["wo"], B["att"], X, X, M, h, qd)
                if F["gate"] != F["up"]:
                    raise ValueError(f"gate {F['gate']} / up {F['up']}: no fused gate+up+SiLU")
                d.fused_ffn_rows_f32(ctx, F["gate"], L["wg"], L["wu"], X, B["g"], M, ff, h,
                                     gamma=L["ffn_norm"], eps=c.eps)
                d.gemv_rows_add_f32(ctx, F["down"], L["wd"], B["g"], X, X, M, h, ff)
            else:
                # the attention, O + residual (into Xo), norm, gate/up + SiLU,
                # down + residual (back into X): the attention's key-range
                # partials merged and each K-split sum folded into the next
                # projection's operand preparation
                d.gemm_attn_ffn_block_f32(ctx, B["q"], L["kc"], L["vc"], start_pos + M, c.heads,
                                          c.kv_heads, hd, c.max_seq, start_pos, B["att"],
                                          (F["o"], F["gate"], F["up"], F["down"]), L["wo"],
                                          L["wg"], L["wu"], L["wd"], X, Xo, L["ffn_norm"], c.eps,
                                          B["g"], B["u"], XN, M, h, ff)
        if last_only:
            # prefill: the final norm and the LM head on the last row only, into
            # the decode buffers (logits, token = its argmax) so that decoding
            # continues at position start_pos + M
            self._lm_head(X + 4 * (M - 1) * h)
            d.argmax_f32(ctx, self.logits, self.token, c.vocab)
        elif form == "rows":
            d.gemv_rows_f32(ctx, self.lm_fmt, self.lm_head, X, B["logits"], M, c.vocab, h,
                            gamma=self.final_norm, eps=c.eps)
        else:
            d.gemm_set_f32(ctx, [self.lm_fmt], [self.lm_head], [B["logits"]], [c.vocab], X, M, h,
                           gamma=self.final_norm, eps=c.eps, xn=XN)
        if not last_only:
            d.argmax_rows_first_f32(ctx, B["logits"], B["idx"], M, c.vocab)
        return B

    def _lm_head(self, x) -> int:
        """Final RMSNorm + LM head of one hidden row x into self.logits (the
        norm fused into the GEMV's staging for Q8_0 / Q6_K heads); returns the
        number of launches."""
        c, ctx = self.cfg, self.ctx
        if self.lm_fmt in ("q8_0", "q6k"):
            getattr(d, f"rms_norm_gemv_{self.lm_fmt}_f32in_f32out")(
                ctx, self.lm_head, x, self.final_norm, c.eps, self.logits, c.vocab, c.hidden)
            return 1
        d.rms_norm_f32_f32_f32g(ctx, x, self.xn, self.final_norm, c.eps, c.hidden, 1)
        getattr(d, f"gemv_{self.lm_fmt}_f32in_f32out")(ctx, self.lm_head, self.xn, self.logits,
                                                       c.vocab, c.hidden)
        return 2

    def prefill(self, tokens) -> np.ndarray:
        """prefill.rs:29-257: the whole prompt in one batched pass from
        position 0 (every KV position written, causal attention), then the
        final norm and the LM head on the last token only.  Returns that
        token's logits; the greedy next token is left in the decode token
        buffer, so step_fused(len(tokens)) continues the sequence."""
        ids = np.asarray(tokens).astype(np.int64, casting="same_kind").ravel()
        if ids.size == 0:
            raise ValueError("prefill: empty prompt")
        if np.any(ids < 0) or np.any(ids >= self.cfg.vocab):
            raise ValueError("prefill: token id out of range")
        toks = ids.astype(np.uint32)
        M = int(toks.size)
        if M > self.cfg.max_seq:
            raise ValueError(f"prefill: {M} tokens exceed the KV cache ({self.cfg.max_seq})")
        B = self._verify_arena(M, logits=False)
        self.ctx._check(d.load_library().rt_upload(self.ctx.handle, B["tok"], toks.ctypes.data,
                                                   toks.nbytes))
        self.verify_pass(M, 0, last_only=True)
        self.ctx.flush()
        return self.read(self.logits, self.cfg.vocab)

    def verify_draft(self, prompt_token: int, draft_tokens, start_pos: int):
        """forward.rs:2118-2309: run [prompt_token, *draft_tokens] at
        start_pos.. in one batched pass, then accept drafts while each equals
        the argmax of the row before it.  Returns (accepted, correct_next):
        the first rejected row's argmax, or the last row's when every draft
        was accepted.  The cache holds the keys / values of all M rows; the
        caller's next position is start_pos + accepted + 1 (the reference's
        kv.set_seq_len)."""
        drafts = [int(t) for t in draft_tokens]
        B = self.verify_forward([int(prompt_token)] + drafts, start_pos)
        M = len(drafts) + 1
        idx = np.zeros(M, np.uint32)
        self.ctx._check(d.load_library().rt_download(self.ctx.handle, idx.ctypes.data, B["idx"],
                                                     idx.nbytes))
        return accept_drafts(idx, drafts)

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
        if getattr(self, "_vbufs", None) is not None:
            self._vbufs["arena"].buf.free()
            self._vbufs = None
        for a in getattr(self, "_retired_arenas", []):
            a.buf.free()
        self._retired_arenas = []
        self.arena.buf.free()

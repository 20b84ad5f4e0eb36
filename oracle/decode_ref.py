"""TEST INFRASTRUCTURE ONLY: CPU oracle for one greedy decode step of
welvet's transformer decoder, in float64 numpy. Importable from tests/ and
bench.py's cpu_baseline leg; the product package never imports it.

It follows the reference's host path for one new token at position `pos`
(model/transformer/forward.go:26-90) and rounds to float32 where the
reference stores float32 tensors:
  * RMSNorm (layers/rmsnorm/cpu.go:70-85): f64 sum of squares, inv = 1/sqrt(
    sumSq/dim + eps), y = f32((x*inv)*gamma).
  * Dense projections: the reference's packed GEMV accumulates exactly
    dequantized weights in f64 and rounds once to f32, i.e. f32(Unpack(W) @ x).
  * MHA (layers/mha/cpu.go:163-215): Q, K, V rows widened to f64; RoPE
    rotate-half on Q and K (layers/mha/rope.go:6-21, angle = pos /
    theta^(2d/hd)); K and V appended to the f64 cache at row pos % max_seq;
    attention (layers/mha/attn.go:40-118): scores q.k*scale over kPos <= pos,
    max-subtracted softmax, sum p*v, all f64; output rounded to f32; then O.
  * Residual adds in f32 (forward.go:63,76).
  * SwiGLU (layers/swiglu/cpu.go:21-56): silu(gate)*up, down.
  * Final RMSNorm, LM head, argmax (lowest index on ties).
"""
from __future__ import annotations

import numpy as np

import oracle

F32 = np.float32


def rmsnorm(x32: np.ndarray, gamma: np.ndarray | None, eps: float) -> np.ndarray:
    """layers/rmsnorm/cpu.go:70-85."""
    x = x32.astype(np.float64)
    inv = 1.0 / np.sqrt(np.dot(x, x) / x.size + eps)
    xh = x * inv
    return (xh if gamma is None else xh * gamma.astype(np.float64)).astype(F32)


def rope(vec: np.ndarray, pos: int, n_heads: int, hd: int, theta: float) -> None:
    """layers/mha/rope.go:6-21, in place on an f64 vector of n_heads*hd."""
    half = hd // 2
    d = np.arange(half, dtype=np.float64)
    angle = float(pos) / np.power(theta, (2.0 * d) / float(hd))
    c, s = np.cos(angle), np.sin(angle)
    v = vec.reshape(n_heads, hd)
    v0, v1 = v[:, :half].copy(), v[:, half:].copy()
    v[:, :half] = v0 * c - v1 * s
    v[:, half:] = v0 * s + v1 * c


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, kv_len: int, n_heads: int, n_kv: int, hd: int
              ) -> np.ndarray:
    """layers/mha/attn.go:40-118 for one query position with every kPos < kv_len allowed."""
    g = n_heads // n_kv
    out = np.zeros(n_heads * hd)
    scale = 1.0 / np.sqrt(float(hd))
    for h in range(n_heads):
        kvh = h // g
        K = kc[:kv_len, kvh * hd:(kvh + 1) * hd]
        V = vc[:kv_len, kvh * hd:(kvh + 1) * hd]
        sc = K @ q[h * hd:(h + 1) * hd] * scale
        e = np.exp(sc - sc.max())
        p = e / e.sum()
        out[h * hd:(h + 1) * hd] = p @ V
    return out


def silu_mul(g32: np.ndarray, u32: np.ndarray) -> np.ndarray:
    """layers/swiglu/cpu.go:41-53: f32(silu(gate) * up)."""
    g = g32.astype(np.float64)
    return (g / (1.0 + np.exp(-g)) * u32.astype(np.float64)).astype(F32)


class DenseW:
    """A packed projection as the oracle multiplies it: f64 Unpack(W)."""

    def __init__(self, packed):
        p = oracle.Packed(packed.fmt, packed.rows, packed.cols, packed.raw, packed.scales, packed.meta,
                          packed.block_weights, getattr(packed, "mins", None))
        self.w = oracle.unpack(p).reshape(packed.rows, packed.cols).astype(np.float64)

    def __call__(self, x32: np.ndarray) -> np.ndarray:
        return (self.w @ x32.astype(np.float64)).astype(F32)


class DecodeRef:
    """Holds the oracle's model state: weights, norms, f64 KV caches."""

    def __init__(self, cfg, layers, lm_head, final_norm, embedding):
        # layers: list of (dict name -> DenseW for q,k,v,o,gate,up,down, attn_norm, ffn_norm)
        self.cfg = cfg
        self.layers = layers
        self.lm = lm_head
        self.final_norm = final_norm
        self.emb = embedding
        self.kc = [np.zeros((cfg.max_seq, cfg.kv_dim)) for _ in layers]
        self.vc = [np.zeros((cfg.max_seq, cfg.kv_dim)) for _ in layers]

    def set_kv(self, layer: int, first_pos: int, k: np.ndarray, v: np.ndarray) -> None:
        n = k.size // self.cfg.kv_dim
        self.kc[layer][first_pos:first_pos + n] = np.asarray(k, np.float64).reshape(n, -1)
        self.vc[layer][first_pos:first_pos + n] = np.asarray(v, np.float64).reshape(n, -1)

    def prefill(self, tokens, pos0: int = 0):
        """ForwardTokens over a prompt block (forward.go:26-90 with seqLen =
        len(tokens)): every op is row-wise except attention, whose causal mask
        (layers/mha/attn.go:52-56, kPos <= qPos) limits row s to the cache rows
        up to its own position, which hold exactly the K and V of the rows
        before it (layers/mha/cpu.go:178-193). So the block equals these
        per-position steps; returns the last row's (f32 logits, argmax)."""
        out = None
        for i, t in enumerate(tokens):
            out = self.step(int(t), pos0 + i)
        return out

    def step(self, token: int, pos: int):
        """One decode step; returns (f32 logits, argmax token)."""
        c = self.cfg
        h = self.emb[min(max(token, 0), c.vocab - 1)].astype(F32).copy()
        for L, (w, an, fn) in enumerate(self.layers):
            n1 = rmsnorm(h, an, c.rms_eps)
            q = w["q"](n1).astype(np.float64)
            k = w["k"](n1).astype(np.float64)
            v = w["v"](n1).astype(np.float64)
            rope(q, pos, c.n_heads, c.head_dim, c.rope_theta)
            rope(k, pos, c.n_kv_heads, c.head_dim, c.rope_theta)
            self.kc[L][pos % c.max_seq] = k
            self.vc[L][pos % c.max_seq] = v
            att = attention(q, self.kc[L], self.vc[L], pos + 1, c.n_heads, c.n_kv_heads, c.head_dim).astype(F32)
            h = (h + w["o"](att)).astype(F32)
            n2 = rmsnorm(h, fn, c.rms_eps)
            hm = silu_mul(w["gate"](n2), w["up"](n2))
            h = (h + w["down"](hm)).astype(F32)
        if self.final_norm is not None:
            h = rmsnorm(h, self.final_norm, c.rms_eps)
        logits = self.lm(h)
        return logits, int(np.argmax(logits))

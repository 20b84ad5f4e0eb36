"""Device decode step (wv_decoder_*): welvet's transformer ForwardTokens for one
new token (model/transformer/forward.go:26-90) over resident blobs, greedy."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import DeviceBlob, check, lib


class DecoderConfig(ctypes.Structure):
    _fields_ = [("n_layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("n_heads", ctypes.c_int32),
                ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("ffn", ctypes.c_int32),
                ("vocab", ctypes.c_int32), ("max_seq", ctypes.c_int32), ("rope_theta", ctypes.c_double),
                ("rms_eps", ctypes.c_double)]


@dataclass
class Config:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_seq: int
    rope_theta: float = 5e5
    rms_eps: float = 1e-5

    def c(self) -> DecoderConfig:
        return DecoderConfig(self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn,
                             self.vocab, self.max_seq, self.rope_theta, self.rms_eps)

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim


class Decoder:
    """Owns a wv_decoder handle. The device blobs given to set_layer and
    set_output are referenced by the decoder's kernels, so the Decoder keeps
    those DeviceBlob objects alive until free() (or until a later set_layer /
    set_output replaces them): a caller may pass freshly uploaded blobs
    without holding them itself."""

    def __init__(self, cfg: Config):
        self.cfg = cfg
        self._layer_blobs: dict[int, list[DeviceBlob]] = {}
        self._lm: DeviceBlob | None = None
        h = ctypes.c_uint64()
        c = cfg.c()
        check(lib().wv_decoder_create(ctypes.byref(c), ctypes.byref(h)))
        self.handle = h.value

    def set_layer(self, layer: int, blobs: list[DeviceBlob], attn_norm: np.ndarray, ffn_norm: np.ndarray) -> None:
        hs = (ctypes.c_uint64 * 7)(*[b.handle for b in blobs])
        an = np.ascontiguousarray(attn_norm, np.float32)
        fn = np.ascontiguousarray(ffn_norm, np.float32)
        check(lib().wv_decoder_set_layer(self.handle, layer, hs, an.ctypes.data, fn.ctypes.data))
        self._layer_blobs[layer] = list(blobs)

    def set_output(self, lm_head: DeviceBlob, final_norm: np.ndarray | None, embedding: np.ndarray) -> None:
        fn = None if final_norm is None else np.ascontiguousarray(final_norm, np.float32)
        emb = np.ascontiguousarray(embedding, np.float32)
        check(lib().wv_decoder_set_output(self.handle, lm_head.handle, None if fn is None else fn.ctypes.data,
                                          emb.ctypes.data))
        self._lm = lm_head

    def set_kv(self, layer: int, first_pos: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        n = k.size // self.cfg.kv_dim
        check(lib().wv_decoder_set_kv(self.handle, layer, first_pos, n, k.ctypes.data, v.ctypes.data))

    def use_graph(self, enable: bool = True) -> None:
        check(lib().wv_decoder_use_graph(self.handle, 1 if enable else 0))

    def generate(self, token: int, pos: int, n_steps: int, advance_pos: bool = True, want_logits: bool = False):
        toks = np.zeros(max(n_steps, 1), np.int32)
        logits = np.zeros(self.cfg.vocab, np.float32) if want_logits else None
        check(lib().wv_decoder_generate(self.handle, token, pos, n_steps, 1 if advance_pos else 0, toks.ctypes.data,
                                        None if logits is None else logits.ctypes.data))
        return (toks[:n_steps], logits) if want_logits else toks[:n_steps]

    def prefill(self, tokens, pos0: int = 0, want_logits: bool = False):
        """ForwardTokens over a prompt block at positions pos0.. (wv_decoder_prefill):
        fills the KV caches on the device and returns the last row's argmax (and logits)."""
        ids = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        nxt = ctypes.c_int32()
        logits = np.zeros(self.cfg.vocab, np.float32) if want_logits else None
        check(lib().wv_decoder_prefill(self.handle, ids.ctypes.data if ids.size else None, ids.size, pos0,
                                       ctypes.byref(nxt), None if logits is None else logits.ctypes.data))
        return (nxt.value, logits) if want_logits else nxt.value

    def free(self) -> None:
        if self.handle:
            check(lib().wv_decoder_free(self.handle))
            self.handle = 0
        self._layer_blobs.clear()
        self._lm = None

    def __del__(self):
        try:
            if self.handle:
                lib().wv_decoder_free(self.handle)
                self.handle = 0
        except Exception:
            pass

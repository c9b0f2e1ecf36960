"""The synthetic decoder of include/q8decoder.h: a dense llama-style model whose
every projection runs on the Q8_0 matmul path (the reference's Model,
apps/engine/src/model.rs:652-1235, over random-init weights generated on the
device).

    dec = Decoder(gpu, DecoderConfig(...), seed=1)
    first = dec.forward(prompt_ids)       # prefill, greedy next token
    rest = dec.generate(127)              # decode steps, fed back on the device
"""
from __future__ import annotations

import ctypes

import numpy as np

from .q8 import DecoderConfig, DecoderStats, DeviceWeight, Gpu, _check, lib

Q, K, V, O, GATE, UP, DOWN, OUTPUT = range(8)


def config(**kw) -> DecoderConfig:
    """A DecoderConfig from keyword fields (eps and rope_base default to the
    reference's 1e-6 and 10000, model.rs:96-97; n_rot to head_dim)."""
    c = DecoderConfig()
    kw.setdefault("eps", 1e-6)
    kw.setdefault("rope_base", 10000.0)
    kw.setdefault("n_rot", kw.get("head_dim", 64))
    kw.setdefault("n_head_kv", kw.get("n_head"))
    for name, value in kw.items():
        setattr(c, name, value)
    return c


class Decoder:
    def __init__(self, gpu: Gpu, cfg: DecoderConfig, seed: int = 0x5EED):
        h = ctypes.c_void_p()
        _check(lib().q8_decoder_create_synthetic(gpu.handle, ctypes.byref(cfg), seed, ctypes.byref(h)))
        self.gpu, self.cfg, self.handle = gpu, cfg, h.value

    def close(self):
        if self.handle:
            lib().q8_decoder_destroy(self.handle)
            self.handle = None

    def reset(self):
        _check(lib().q8_decoder_reset(self.handle))

    @property
    def position(self) -> int:
        p = ctypes.c_int()
        _check(lib().q8_decoder_position(self.handle, ctypes.byref(p)))
        return p.value

    def forward(self, tokens) -> int:
        ids = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt = ctypes.c_uint32()
        _check(lib().q8_decoder_forward(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size,
                                        ctypes.byref(nxt)))
        return int(nxt.value)

    def generate(self, steps: int) -> np.ndarray:
        out = np.zeros(max(steps, 0), dtype=np.uint32)
        _check(lib().q8_decoder_generate(self.handle, steps, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty(self.cfg.n_vocab, dtype=np.float32)
        _check(lib().q8_decoder_logits(self.handle, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out.size))
        return out

    def weight(self, layer: int, which: int = 0) -> DeviceWeight:
        h = ctypes.c_void_p()
        _check(lib().q8_decoder_weight(self.handle, layer, which, ctypes.byref(h)))
        c = self.cfg
        hd = c.n_head * c.head_dim
        kv = c.n_head_kv * c.head_dim
        if layer < 0:
            k, out = c.n_embd, c.n_vocab
        else:
            k, out = {Q: (c.n_embd, hd), K: (c.n_embd, kv), V: (c.n_embd, kv), O: (hd, c.n_embd),
                      GATE: (c.n_embd, c.n_ff), UP: (c.n_embd, c.n_ff), DOWN: (c.n_ff, c.n_embd)}[which]
        return DeviceWeight(h.value, k, out)

    def graph_stats(self) -> dict:
        """Graphs held, captured and dropped, and eager passes (q8_decoder_graph_stats)."""
        st = DecoderStats()
        _check(lib().q8_decoder_graph_stats(self.handle, ctypes.byref(st)))
        return {f: getattr(st, f) for f, _ in st._fields_}

    def norm(self, layer: int, which: int = 0) -> np.ndarray:
        p = ctypes.POINTER(ctypes.c_float)()
        _check(lib().q8_decoder_norm(self.handle, layer, which, ctypes.byref(p)))
        return np.ctypeslib.as_array(p, shape=(self.cfg.n_embd,)).copy()

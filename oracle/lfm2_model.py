"""CPU oracle of the LFM2 token pass -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference executor's `append_tokens` and
`sample_epilogue` (crates/executor-core/src/lfm2/executor/execution.rs:35-571)
composed of the oracle's per-operation restatements (oracle/), so that the
HIP model pass can be compared with the reference's arithmetic on the same
weights and tokens.  Used only by tests/ and by the CPU-baseline leg of the
benchmark, never by the product path.

With `threads` > 1 (the parity tests), packed products run on the
row-parallel oracle without the per-call finite scans and attention on the
score-cached one; both are pinned bit-identical to the single-threaded
restatements (tests/test_oracle.py, tests/test_dense_oracle.py), which is
what makes full LFM2 shapes affordable.  With `threads` = 1 (the CPU
baseline), every operation is the single-threaded restatement of
backend-cpu, admission scans included, as the reference runs it
(crates/backend-cpu/src/lib.rs:3-4).  Pair and SwiGLU products are composed
from single products and swiglu, which the oracle tests pin bitwise to the
composite restatements (packed_pair_validation.rs:169-208).

`timings`, when a dict, accumulates the seconds spent per operation kind.
"""
from __future__ import annotations

import os
import time

import numpy as np

import oracle
from runtime_amd.lfm2 import (CONV, CONV_IN, CONV_KERNEL, CONV_OUT, EMBEDDING_NORM, FFN_NORM,
                              FFN_W1, FFN_W2, FFN_W3, KEY, KEY_NORM, OPERATOR_NORM, OUTPUT,
                              QUERY, QUERY_NORM, TOKEN_EMBEDDING, VALUE, Lfm2Config)


THREADS = max(1, min(16, os.cpu_count() or 1))


class OracleLfm2:
    def __init__(self, cfg: Lfm2Config, weights: dict, threads: int = THREADS,
                 timings: dict | None = None):
        self.cfg = cfg
        self.w = weights
        self.threads = threads
        self.timings = timings
        self.reset()

    def _timed(self, kind, fn, *args, **kwargs):
        if self.timings is None:
            return fn(*args, **kwargs)
        t0 = time.perf_counter()
        out = fn(*args, **kwargs)
        self.timings[kind] = self.timings.get(kind, 0.0) + time.perf_counter() - t0
        return out

    def _packed_linear(self, x, codes, scales, kind="packed_linear"):
        if self.threads > 1:
            fn = oracle.packed_linear_threaded
            return self._timed(kind, fn, x, codes, scales, threads=self.threads)
        return self._timed(kind, oracle.packed_linear, x, codes, scales)

    def snapshot(self) -> dict:
        """A copy of the prefix state (lengths, histories, caches, logits)."""
        return {"length": self.length, "history": {i: h.copy() for i, h in self.history.items()},
                "key": {i: c.copy() for i, c in self.key.items()},
                "value": {i: c.copy() for i, c in self.value.items()},
                "cache_len": dict(self.cache_len),
                "logits": None if self.logits is None else self.logits.copy()}

    def restore(self, state: dict) -> None:
        self.length = state["length"]
        self.history = {i: h.copy() for i, h in state["history"].items()}
        self.key = {i: c.copy() for i, c in state["key"].items()}
        self.value = {i: c.copy() for i, c in state["value"].items()}
        self.cache_len = dict(state["cache_len"])
        self.logits = None if state["logits"] is None else state["logits"].copy()

    def reset(self):
        cfg = self.cfg
        self.length = 0
        self.history = {i: np.zeros((cfg.conv_width - 1, cfg.hidden), dtype=np.float32)
                        for i, k in enumerate(cfg.layers) if k == CONV}
        self.key = {i: np.zeros((cfg.max_tokens, cfg.kv_width), dtype=np.float32)
                    for i, k in enumerate(cfg.layers) if k != CONV}
        self.value = {i: np.zeros((cfg.max_tokens, cfg.kv_width), dtype=np.float32)
                      for i, k in enumerate(cfg.layers) if k != CONV}
        self.cache_len = {i: 0 for i, k in enumerate(cfg.layers) if k != CONV}
        self.logits = None

    def _w(self, role, layer=0):
        return self.w[(role, layer)]

    def _packed(self, role, layer):
        return len(self._w(role, layer)) == 2

    def _same_format(self, a, b, layer):
        wa, wb = self._w(a, layer), self._w(b, layer)
        return len(wa) == 2 and len(wb) == 2 and wa[0].shape[1] == wb[0].shape[1]

    def linear(self, x, role, layer=0, kind="linear"):
        """weight_linear (execution.rs:12-25)."""
        t = self._w(role, layer)
        if len(t) == 2:
            return self._packed_linear(x, t[0], t[1], kind)
        return self._timed(kind, oracle.linear, x, t[0])

    def _ffn(self, index, ffn_input):
        rows = ffn_input.shape[0]
        pair = self._same_format(FFN_W1, FFN_W3, index)
        if rows >= 96 and pair and self._packed(FFN_W2, index):
            g, u = self._w(FFN_W1, index), self._w(FFN_W3, index)
            gate = self._packed_linear(ffn_input, g[0], g[1], "ffn gate/up")
            up = self._packed_linear(ffn_input, u[0], u[1], "ffn gate/up")
            hidden = self._timed("swiglu", oracle.swiglu, gate, up)
            d = self._w(FFN_W2, index)
            return self._packed_linear(hidden, d[0], d[1], "ffn down")
        if pair:
            g, u = self._w(FFN_W1, index), self._w(FFN_W3, index)
            gate = self._packed_linear(ffn_input, g[0], g[1], "ffn gate/up")
            up = self._packed_linear(ffn_input, u[0], u[1], "ffn gate/up")
        else:
            gate = self.linear(ffn_input, FFN_W1, index, "ffn gate/up")
            up = self.linear(ffn_input, FFN_W3, index, "ffn gate/up")
        hidden = self._timed("swiglu", oracle.swiglu, gate, up)
        if self._packed(FFN_W2, index):
            d = self._w(FFN_W2, index)
            return self._packed_linear(hidden, d[0], d[1], "ffn down")
        return self.linear(hidden, FFN_W2, index, "ffn down")

    def append(self, tokens, produce_logits=True):
        cfg = self.cfg
        ids = np.asarray(tokens, dtype=np.int64).reshape(-1)
        rows = ids.size
        positions = np.arange(self.length, self.length + rows, dtype=np.uint64)
        emb = self._w(TOKEN_EMBEDDING)
        if len(emb) == 2:
            x = self._timed("embedding gather", oracle.packed_gather_rows, emb[0], emb[1], ids)
        else:
            x = self._timed("embedding gather", oracle.gather_rows, emb[0], ids)
        u = self._timed("norms", oracle.row_rms_norm, x, self._w(OPERATOR_NORM, 0)[0],
                        cfg.block_norm_epsilon)
        for index, kind in enumerate(cfg.layers):
            if kind == CONV:
                projection = self.linear(u, CONV_IN, index, "conv in projection")
                convolved, self.history[index] = self._timed(
                    "short convolution", oracle.gated_short_convolution, projection,
                    self._w(CONV_KERNEL, index)[0], self.history[index], cfg.hidden,
                    cfg.conv_width)
                op = self.linear(convolved, CONV_OUT, index, "conv out projection")
            else:
                q = self.linear(u, QUERY, index, "q/k/v projections")
                if self._same_format(KEY, VALUE, index):
                    kw, vw = self._w(KEY, index), self._w(VALUE, index)
                    k = self._packed_linear(u, kw[0], kw[1], "q/k/v projections")
                    v = self._packed_linear(u, vw[0], vw[1], "q/k/v projections")
                else:
                    k = self.linear(u, KEY, index, "q/k/v projections")
                    v = self.linear(u, VALUE, index, "q/k/v projections")
                q_rope, k_rope = self._timed(
                    "qk norm + rope", oracle.qk_norm_rope,
                    q, k, self._w(QUERY_NORM, index)[0], self._w(KEY_NORM, index)[0], positions,
                    cfg.attention_heads, cfg.key_value_heads, cfg.head_dim,
                    np.float32(cfg.rope_theta), np.float32(cfg.block_norm_epsilon))
                attention, self.key[index], self.value[index], self.cache_len[index] = \
                    self._timed("attention", oracle.causal_gqa,
                                q_rope, k_rope, v, self.key[index], self.value[index],
                                self.cache_len[index], cfg.attention_heads,
                                cfg.key_value_heads, cfg.head_dim,
                                threads=self.threads if self.threads > 1 else 0, in_place=True)
                op = self.linear(attention, OUTPUT, index, "attention out projection")
            residual, ffn_input = self._timed(
                "norms", oracle.add_row_rms_norm,
                x, op, self._w(FFN_NORM, index)[0], np.float32(cfg.block_norm_epsilon))
            last = index + 1 == len(cfg.layers)
            if last and rows > 1:
                ffn_input, residual = ffn_input[-1:], residual[-1:]
            down = self._ffn(index, ffn_input)
            if last:
                norm, eps = self._w(EMBEDDING_NORM)[0], cfg.norm_epsilon
            else:
                norm, eps = self._w(OPERATOR_NORM, index + 1)[0], cfg.block_norm_epsilon
            x, u = self._timed("norms", oracle.add_row_rms_norm, residual, down, norm,
                               np.float32(eps))
        if produce_logits:
            self.logits = self.linear(u, TOKEN_EMBEDDING, 0, "lm head")
        self.length += rows
        return self.logits

    def sample(self) -> float:
        return float(self._timed("argmax", oracle.argmax, self.logits)[0])

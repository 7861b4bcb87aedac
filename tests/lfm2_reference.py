"""CPU oracle of the LFM2 token pass -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference executor's `append_tokens` and
`sample_epilogue` (crates/executor-core/src/lfm2/executor/execution.rs:35-571)
composed of the oracle's per-operation restatements (oracle/), so that the
HIP model pass can be compared with the reference's arithmetic on the same
weights and tokens.

Packed products run on the row-parallel oracle and attention on the
score-cached one; both are pinned bit-identical to the single-threaded
restatements (tests/test_oracle.py, tests/test_dense_oracle.py), which is
what makes full LFM2 shapes affordable.  Pair and SwiGLU products are
composed from single products and swiglu, which the oracle tests pin
bitwise to the composite restatements (packed_pair_validation.rs:169-208).
"""
from __future__ import annotations

import os

import numpy as np

import oracle
from runtime_amd.lfm2 import (CONV, CONV_IN, CONV_KERNEL, CONV_OUT, EMBEDDING_NORM, FFN_NORM,
                              FFN_W1, FFN_W2, FFN_W3, KEY, KEY_NORM, OPERATOR_NORM, OUTPUT,
                              QUERY, QUERY_NORM, TOKEN_EMBEDDING, VALUE, Lfm2Config)


THREADS = max(1, min(16, os.cpu_count() or 1))


def _linear(x, codes, scales):
    return oracle.packed_linear_threaded(x, codes, scales, threads=THREADS)


class OracleLfm2:
    def __init__(self, cfg: Lfm2Config, weights: dict):
        self.cfg = cfg
        self.w = weights
        self.reset()

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

    def linear(self, x, role, layer=0):
        """weight_linear (execution.rs:12-25)."""
        t = self._w(role, layer)
        if len(t) == 2:
            return _linear(x, t[0], t[1])
        return oracle.linear(x, t[0])

    def _ffn(self, index, ffn_input):
        rows = ffn_input.shape[0]
        pair = self._same_format(FFN_W1, FFN_W3, index)
        if rows >= 96 and pair and self._packed(FFN_W2, index):
            g, u = self._w(FFN_W1, index), self._w(FFN_W3, index)
            hidden = oracle.swiglu(_linear(ffn_input, g[0], g[1]), _linear(ffn_input, u[0], u[1]))
            d = self._w(FFN_W2, index)
            return _linear(hidden, d[0], d[1])
        if pair:
            g, u = self._w(FFN_W1, index), self._w(FFN_W3, index)
            gate, up = _linear(ffn_input, g[0], g[1]), _linear(ffn_input, u[0], u[1])
        else:
            gate = self.linear(ffn_input, FFN_W1, index)
            up = self.linear(ffn_input, FFN_W3, index)
        if self._packed(FFN_W2, index):
            d = self._w(FFN_W2, index)
            return _linear(oracle.swiglu(gate, up), d[0], d[1])
        return self.linear(oracle.swiglu(gate, up), FFN_W2, index)

    def append(self, tokens, produce_logits=True):
        cfg = self.cfg
        ids = np.asarray(tokens, dtype=np.int64).reshape(-1)
        rows = ids.size
        positions = np.arange(self.length, self.length + rows, dtype=np.uint64)
        emb = self._w(TOKEN_EMBEDDING)
        x = (oracle.packed_gather_rows(emb[0], emb[1], ids) if len(emb) == 2
             else oracle.gather_rows(emb[0], ids))
        u = oracle.row_rms_norm(x, self._w(OPERATOR_NORM, 0)[0], cfg.block_norm_epsilon)
        for index, kind in enumerate(cfg.layers):
            if kind == CONV:
                projection = self.linear(u, CONV_IN, index)
                convolved, self.history[index] = oracle.gated_short_convolution(
                    projection, self._w(CONV_KERNEL, index)[0], self.history[index], cfg.hidden,
                    cfg.conv_width)
                op = self.linear(convolved, CONV_OUT, index)
            else:
                q = self.linear(u, QUERY, index)
                if self._same_format(KEY, VALUE, index):
                    kw, vw = self._w(KEY, index), self._w(VALUE, index)
                    k, v = _linear(u, kw[0], kw[1]), _linear(u, vw[0], vw[1])
                else:
                    k, v = self.linear(u, KEY, index), self.linear(u, VALUE, index)
                q_rope, k_rope = oracle.qk_norm_rope(
                    q, k, self._w(QUERY_NORM, index)[0], self._w(KEY_NORM, index)[0], positions,
                    cfg.attention_heads, cfg.key_value_heads, cfg.head_dim,
                    np.float32(cfg.rope_theta), np.float32(cfg.block_norm_epsilon))
                attention, self.key[index], self.value[index], self.cache_len[index] = \
                    oracle.causal_gqa(q_rope, k_rope, v, self.key[index], self.value[index],
                                      self.cache_len[index], cfg.attention_heads,
                                      cfg.key_value_heads, cfg.head_dim, threads=THREADS,
                                      in_place=True)
                op = self.linear(attention, OUTPUT, index)
            residual, ffn_input = oracle.add_row_rms_norm(
                x, op, self._w(FFN_NORM, index)[0], np.float32(cfg.block_norm_epsilon))
            last = index + 1 == len(cfg.layers)
            if last and rows > 1:
                ffn_input, residual = ffn_input[-1:], residual[-1:]
            down = self._ffn(index, ffn_input)
            if last:
                norm, eps = self._w(EMBEDDING_NORM)[0], cfg.norm_epsilon
            else:
                norm, eps = self._w(OPERATOR_NORM, index + 1)[0], cfg.block_norm_epsilon
            x, u = oracle.add_row_rms_norm(residual, down, norm, np.float32(eps))
        if produce_logits:
            self.logits = self.linear(u, TOKEN_EMBEDDING)
        self.length += rows
        return self.logits

    def sample(self) -> float:
        return float(oracle.argmax(self.logits)[0])

"""GPU parity of the LFM2 token pass (runtime_amd/csrc/lfm2.cpp) against the
CPU oracle of the reference executor's pass (oracle/lfm2_model.py).

Small models of the LFM2 layout (convolution and attention blocks, tied
embedding) in several weight-format mixes: the prefill logits, then greedy
decode teacher-forced with the GPU's own tokens so that a near tie cannot
cascade (per-step logits within max|d|/max|cpu| <= 1e-3, and the reference
device rule), the fused-FFN prefill (>= 96 rows), and the device-side greedy
loop against step-by-step sampling.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle.lfm2_model import OracleLfm2
from runtime_amd import convert
from runtime_amd.lfm2 import ATTENTION, CONV, Lfm2Config, Lfm2Model, synthetic_weights
from tests.conftest import assert_close, max_rel_err

pytestmark = pytest.mark.gpu

MIXES = {
    "mixed": {"embedding": "int8", "conv": "nf4", "attention": "nf4", "ffn": "ternary"},
    "ternary": {"embedding": "ternary", "conv": "ternary", "attention": "ternary",
                "ffn": "ternary"},
    "dense-conv-int8": {"embedding": None, "conv": None, "attention": "int8", "ffn": "int8"},
}


def say(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def tiny(mix: str) -> Lfm2Config:
    return Lfm2Config(hidden=256, intermediate=512, attention_heads=4, key_value_heads=2,
                      vocab=1000, layers=[CONV, ATTENTION, CONV, ATTENTION], max_tokens=160,
                      formats=dict(MIXES[mix]))


def build(backend, mix):
    cfg = tiny(mix)
    model = Lfm2Model(backend, cfg)
    host = synthetic_weights(model, seed=0x1F2_0000 + len(mix), norms="random", keep_host=True)
    return cfg, model, OracleLfm2(cfg, host)


def check_logits(got, want):
    assert max_rel_err(got, want) <= 1e-3
    assert_close(got, want)


@pytest.mark.parametrize("mix", list(MIXES))
def test_prefill_then_teacher_forced_decode(backend, path, mix):
    # Device-id steps of a fully packed model take the fused decode step
    # (auto: transforms in the GEMV kernels; split: in the prologue
    # kernels); fma and the dense-conv mix run the op-by-op pass.
    say("lfm2 decode", mix, path)
    cfg, model, ref = build(backend, mix)
    prompt = convert.token_ids(7, 0x7043_0001, cfg.vocab)
    model.append(prompt)
    check_logits(backend.read(model.logits), ref.append(prompt))
    for step in range(6):
        model.sample()
        token = backend.read(model.sampled)[0]
        want_token = ref.sample()
        assert np.isfinite(token)
        # Greedy agreement unless the oracle's top two logits nearly tie.
        top = np.sort(ref.logits.reshape(-1))[-2:]
        if top[1] - top[0] > 1e-4 * max(1.0, abs(top[1])):
            assert token == want_token, (step, token, want_token)
        model.append(model.sampled)          # the device id feeds the gather
        check_logits(backend.read(model.logits), ref.append([int(token)]))
    assert model.length == ref.length == 13
    model.close()


@pytest.mark.parametrize("mix", ["mixed", "ternary"])
def test_decode_past_several_key_ranges(backend, path, mix):
    # 140 cached keys: the decode attention kernel splits them into three
    # 64-key ranges, whose records the separate combine launch merges.
    say("lfm2 long decode", mix, path)
    cfg, model, ref = build(backend, mix)
    prompt = convert.token_ids(140, 0x7043_0004, cfg.vocab)
    model.append(prompt)
    check_logits(backend.read(model.logits), ref.append(prompt))
    for _ in range(4):
        model.sample()
        token = backend.read(model.sampled)[0]
        model.append(model.sampled)
        check_logits(backend.read(model.logits), ref.append([int(token)]))
    model.close()


@pytest.mark.parametrize("mix", ["mixed", "dense-conv-int8"])
def test_fused_ffn_prefill(backend, mix):
    # >= 96 rows with a packed FFN takes packed_swiglu_pair + packed_linear
    # (execution.rs:307-384); the last layer still runs on one row.
    say("lfm2 prefill 100", mix)
    cfg, model, ref = build(backend, mix)
    prompt = convert.token_ids(100, 0x7043_0002, cfg.vocab)
    model.append(prompt)
    check_logits(backend.read(model.logits), ref.append(prompt))
    model.close()


def test_generate_matches_stepwise_sampling(backend):
    say("lfm2 generate")
    cfg, model, _ = build(backend, "mixed")
    prompt = convert.token_ids(9, 0x7043_0003, cfg.vocab)
    model.append(prompt)
    ids = backend.read(model.generate(8))
    model.reset()
    model.append(prompt)
    stepwise = []
    for _ in range(8):
        model.sample()
        stepwise.append(backend.read(model.sampled)[0])
        model.append(model.sampled)
    assert ids.tolist() == stepwise
    assert model.length == 9 + 8
    model.close()


def test_snapshot_restores_and_stays_unchanged(backend):
    """A stored prefix continues exactly like the model it was taken from,
    any number of times, and decoding from it leaves it unchanged
    (Lfm2Prefix / fork, executor.rs:249-281, prefix_task.rs:158)."""
    say("lfm2 snapshot")
    cfg, model, ref = build(backend, "mixed")
    prompt = convert.token_ids(70, 0x7043_0008, cfg.vocab)
    model.append(prompt)
    ref.append(prompt)
    prefix = model.snapshot()
    saved = ref.snapshot()
    assert prefix.length == 70
    first = backend.read(model.generate(6))
    first_logits = backend.read(model.logits)
    # Diverge: teacher-force other tokens, then fork from the prefix again.
    model.restore(prefix)
    for token in convert.token_ids(5, 0x7043_0009, cfg.vocab):
        model.append([int(token)])
    assert model.length == 75
    for _ in range(2):
        model.restore(prefix)
        assert model.length == 70
        assert backend.read(model.generate(6)).tobytes() == first.tobytes()
        assert backend.read(model.logits).tobytes() == first_logits.tobytes()
    # The restored state matches the oracle continued from its own copy.
    model.restore(prefix)
    ref.restore(saved)
    for token in first[:3]:
        model.append([int(token)])
        check_logits(backend.read(model.logits), ref.append([int(token)]))
    # A prefix belongs to its model.
    from runtime_amd.backend import ExecutorError
    other = Lfm2Model(backend, cfg)
    with pytest.raises(ExecutorError) as info:
        other.restore(prefix)
    assert info.value.message == "prefix belongs to another model"
    other.close()
    prefix.close()
    model.close()


def test_append_admission(backend):
    cfg, model, _ = build(backend, "mixed")
    from runtime_amd.backend import ExecutorError
    with pytest.raises(ExecutorError) as info:
        model.append([cfg.vocab])
    assert info.value.message == "valid token ID exceeds loaded model vocabulary"
    with pytest.raises(ExecutorError) as info:
        model.append([])
    assert info.value.message == "token pass requires at least one token"
    with pytest.raises(ExecutorError) as info:
        model.append(np.zeros(cfg.max_tokens + 1, dtype=np.uint32))
    assert info.value.message == "append exceeds configured logical prefix capacity"
    assert model.length == 0
    model.close()

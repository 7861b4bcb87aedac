"""safetensors bundles into device buffers (include/minifield_loader.h).

- The reference's ternary-v1-001 container through the split-stream upload
  and the HIP gather, bit for bit against its vectors.
- Rejects before any upload: INT8 code 0x80 (loader.rs:1154-1162), a
  non-finite F16 scale, a missing or an undeclared tensor, a wrong shape.
- A whole LFM2 model loaded from a bundle equals the same weights attached
  directly, logits bit for bit.
"""
from __future__ import annotations

import json
import sys

import numpy as np
import pytest

import oracle
from runtime_amd import convert
from runtime_amd.backend import ExecutorError
from runtime_amd.lfm2 import (ATTENTION, CONV, Lfm2Config, Lfm2Model, attach,
                              synthetic_host_weights)
from runtime_amd.loader import SafetensorsFile, load_lfm2, lfm2_tensor_names, write_lfm2_bundle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def say(*parts):
    print("[case]", *parts, flush=True)
    sys.stdout.flush()


def total(report) -> int:
    return (report.resident_weight_bytes + report.cache_bytes + report.scratch_bytes +
            report.staged_branch_bytes + report.pending_operation_bytes)


def test_reference_container_through_the_gpu_gather(backend, golden_dir):
    say("loader: ternary-v1-001 container")
    from safetensors.numpy import load_file
    path = golden_dir / "ternary-v1-001" / "packed.safetensors"
    doc = json.loads((golden_dir / "ternary-v1-001" / "vectors.json").read_text())
    expected = np.array([v["expected_dequant"] for v in doc["vectors"]], dtype=np.float32)
    host = load_file(str(path))
    with SafetensorsFile(path) as f:
        codes, scales = f.upload_packed(backend, "demo.weight")
        dense = f.upload_dense(backend, "dense.weight")
    assert backend.packed_prepared(codes, scales)
    # The F32 scales are the loader's f16 -> f32 of the file values.
    assert backend.read(scales).tobytes() == \
        convert.f16_to_f32(host["demo.weight.scales"]).tobytes()
    assert backend.read(dense).tobytes() == host["dense.weight"].tobytes()
    out = backend.allocate_f32((5, 128))
    backend.packed_gather_rows(out, codes, scales, [0, 1, 2, 3, 4])
    assert backend.read(out).tobytes() == expected.tobytes()
    x = convert.normal((3, 128), 0xAC70B00)
    xb = backend.upload_f32(x.shape, x)
    y = backend.allocate_f32((3, 5))
    backend.packed_linear(y, xb, codes, scales)
    want = oracle.packed_linear(x, host["demo.weight.codes"],
                                convert.f16_to_f32(host["demo.weight.scales"]))
    assert_close(backend.read(y), want)


def bundle(tmp_path, tensors, metadata=None, name="b.safetensors"):
    from safetensors.numpy import save_file
    path = tmp_path / name
    save_file(tensors, str(path), metadata=metadata)
    return path


def test_rejects_before_upload(backend, tmp_path):
    say("loader: rejects")
    rng = np.random.default_rng(3)
    codes = rng.integers(-127, 128, size=(8, 256)).astype(np.int8).view(np.uint8)
    scales = np.full((8, 2), 0.01, np.float16)
    bad = codes.copy()
    bad[5, 17] = 0x80
    inf = scales.copy()
    inf[2, 1] = np.inf
    path = bundle(tmp_path, {"ok.codes": codes, "ok.scales": scales, "bad.codes": bad,
                             "bad.scales": scales, "inf.codes": codes, "inf.scales": inf,
                             "x": np.array([1.0, np.nan], np.float32)})
    with SafetensorsFile(path) as f:
        before = total(backend.resource_report())
        for base, variant in (("bad", "InvalidArgument"), ("inf", "BackendFailure")):
            with pytest.raises(ExecutorError) as e:
                f.upload_packed(backend, base)
            assert e.value.variant == variant
            assert total(backend.resource_report()) == before
        with pytest.raises(ExecutorError) as e:
            f.upload_dense(backend, "x")
        assert e.value.variant == "BackendFailure"
        with pytest.raises(ExecutorError) as e:
            f.upload_packed(backend, "missing")
        assert e.value.variant == "MissingRequiredTensor"
        c, s = f.upload_packed(backend, "ok")
        out = backend.allocate_f32((8, 256))
        backend.packed_gather_rows(out, c, s, list(range(8)))
        want = oracle.packed_gather_rows(codes, convert.f16_to_f32(scales), np.arange(8))
        assert backend.read(out).tobytes() == want.tobytes()


def tiny_cfg():
    return Lfm2Config(hidden=256, intermediate=512, attention_heads=4, key_value_heads=2,
                      vocab=1000, layers=[CONV, ATTENTION, CONV, ATTENTION], max_tokens=64,
                      formats={"embedding": "int8", "conv": "nf4", "attention": "ternary",
                               "ffn": "ternary"})


def test_lfm2_bundle_equals_directly_attached_weights(backend, tmp_path):
    say("loader: LFM2 bundle")
    cfg = tiny_cfg()
    host = {(r, l): a for r, l, a in synthetic_host_weights(cfg, seed=0x5EED1F10,
                                                            norms="random")}
    # One dense matmul role too (the mixed format's f32 override).
    from runtime_amd.lfm2 import CONV_OUT
    host[(CONV_OUT, 2)] = (convert.normal((256, 256), 0x5EED1F11, sigma=0.02),)
    path = tmp_path / "model.safetensors"
    write_lfm2_bundle(path, cfg, host)
    direct = Lfm2Model(backend, cfg)
    for (role, layer), arrays in host.items():
        attach(direct, role, layer, arrays)
    loaded = Lfm2Model(backend, cfg)
    with SafetensorsFile(path) as f:
        load_lfm2(loaded, f)
    prompt = convert.token_ids(12, 0x7043_0010, cfg.vocab)
    for model in (direct, loaded):
        model.append(prompt)
    assert backend.read(loaded.logits).tobytes() == backend.read(direct.logits).tobytes()
    for _ in range(3):
        for model in (direct, loaded):
            model.sample()
            model.append(model.sampled)
        assert backend.read(loaded.logits).tobytes() == backend.read(direct.logits).tobytes()
    direct.close()
    loaded.close()


def test_lfm2_bundle_inventory_rejects(backend, tmp_path):
    say("loader: LFM2 inventory")
    from safetensors.numpy import load_file, save_file
    cfg = tiny_cfg()
    host = {(r, l): a for r, l, a in synthetic_host_weights(cfg, seed=0x5EED1F20)}
    path = tmp_path / "model.safetensors"
    write_lfm2_bundle(path, cfg, host)
    tensors = load_file(str(path))
    with SafetensorsFile(path) as f:
        metadata = {k: f.metadata(k) for k in ("format", "tensor_quantization", "group_size")}

    def expect(mutated, variant):
        p = tmp_path / "mutant.safetensors"
        save_file(mutated, str(p), metadata=metadata)
        model = Lfm2Model(backend, cfg)
        before = total(backend.resource_report())
        with SafetensorsFile(p) as f, pytest.raises(ExecutorError) as e:
            load_lfm2(model, f)
        assert e.value.variant == variant
        assert total(backend.resource_report()) == before  # nothing uploaded
        model.close()

    name = lfm2_tensor_names(cfg)
    missing = dict(tensors)
    del missing["model.layers.1.self_attn.k_layernorm.weight"]
    expect(missing, "MissingRequiredTensor")
    extra = dict(tensors)
    extra["model.layers.9.extra.weight"] = np.zeros(4, np.float32)
    expect(extra, "UnexpectedTensor")
    wrong = dict(tensors)
    wrong["model.embedding_norm.weight"] = np.zeros(255, np.float32)
    expect(wrong, "InvalidShape")
    width = dict(tensors)  # nf4-declared role stored with a ternary width
    key = name[(5, 0)] + ".codes"  # CONV_IN of layer 0
    width[key] = np.zeros((768, 64), np.uint8)
    expect(width, "InvalidShape")


def test_lfm2_reload_releases_and_a_failed_load_changes_nothing(tmp_path):
    """Loading a bundle again replaces the previous load's buffers instead of
    keeping them charged; a load that fails partway (a resource limit hit
    while uploading) leaves the model's weights as they were, and a fresh
    model then loads within the same limit."""
    say("loader: reload and failed load")
    from runtime_amd.backend import HipBackend, Limits
    cfg = tiny_cfg()
    host = {(r, l): a for r, l, a in synthetic_host_weights(cfg, seed=0x5EED1F30,
                                                            norms="random")}
    path = tmp_path / "model.safetensors"
    write_lfm2_bundle(path, cfg, host)
    prompt = convert.token_ids(12, 0x7043_0011, cfg.vocab)

    probe = HipBackend(0)
    try:
        model = Lfm2Model(probe, cfg)
        with SafetensorsFile(path) as f:
            load_lfm2(model, f)
        weights = probe.resource_report().resident_weight_bytes
        model.append(prompt)
        want = probe.read(model.logits)
        footprint = total(probe.resource_report())
        for _ in range(2):  # reloads keep one load's weights resident
            with SafetensorsFile(path) as f:
                load_lfm2(model, f)
            assert probe.resource_report().resident_weight_bytes == weights
        model.reset()
        model.append(prompt)
        assert probe.read(model.logits).tobytes() == want.tobytes()
        model.close()
    finally:
        probe.close()

    backend = HipBackend(0, limits=Limits(max_total_bytes=footprint + weights // 2))
    try:
        model = Lfm2Model(backend, cfg)
        with SafetensorsFile(path) as f:
            load_lfm2(model, f)
        model.append(prompt)
        assert backend.read(model.logits).tobytes() == want.tobytes()
        with SafetensorsFile(path) as f, pytest.raises(ExecutorError) as e:
            load_lfm2(model, f)  # needs a second set of weights beside the first
        assert e.value.variant == "ResourceLimit"
        assert backend.resource_report().resident_weight_bytes == weights
        model.reset()
        model.append(prompt)
        assert backend.read(model.logits).tobytes() == want.tobytes()
        model.close()
        fresh = Lfm2Model(backend, cfg)
        with SafetensorsFile(path) as f:
            load_lfm2(fresh, f)
        fresh.append(prompt)
        assert backend.read(fresh.logits).tobytes() == want.tobytes()
        fresh.close()
    finally:
        backend.close()

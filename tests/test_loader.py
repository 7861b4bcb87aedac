"""The safetensors header checks and per-role scheme resolution of
include/minifield_loader.h, on the CPU (no device work).

Cases follow the reference's loader boundary tests
(crates/executor-core/tests/loader_boundaries.rs) and the rules of
parse_safetensors_header (crates/executor-core/src/loader/header.rs), plus
the committed ternary-v1-001 container.
"""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from runtime_amd.backend import ExecutorError
from runtime_amd.loader import SafetensorsFile


def asset(tmp_path, header: str, payload: bytes = b"", name="t.safetensors"):
    raw = header.encode()
    path = tmp_path / name
    path.write_bytes(struct.pack("<Q", len(raw)) + raw + payload)
    return path


def variant(tmp_path, header, payload=b""):
    with pytest.raises(ExecutorError) as e:
        SafetensorsFile(asset(tmp_path, header, payload))
    return e.value.variant, e.value.message


def test_reference_container_opens(golden_dir):
    with SafetensorsFile(golden_dir / "ternary-v1-001" / "packed.safetensors") as f:
        assert sorted(f.names()) == ["demo.weight.codes", "demo.weight.scales", "dense.weight"]
        assert f.info("demo.weight.codes") == ("U8", (5, 32))
        assert f.info("demo.weight.scales") == ("F16", (5, 1))
        assert f.info("dense.weight") == ("F32", (5,))
        assert f.metadata("format") == "minifield.ternary.v1"
        assert f.metadata("group_size") == "128"
        assert f.matmul_scheme("demo.weight") == "ternary"
        with pytest.raises(ExecutorError) as e:
            f.info("demo.weight")
        assert e.value.variant == "MissingRequiredTensor"


def test_empty_tensor_at_a_shared_range_start_in_either_order(tmp_path):
    empty = '"empty":{"dtype":"F32","shape":[0],"data_offsets":[0,0]}'
    nonempty = '"weight":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}'
    for header in ("{%s,%s}" % (empty, nonempty), "{%s,%s}" % (nonempty, empty)):
        with SafetensorsFile(asset(tmp_path, header, bytes(4))) as f:
            assert sorted(f.names()) == ["empty", "weight"]


def test_overlapping_ranges_reject_in_either_order(tmp_path):
    a = '"first":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}'
    b = '"second":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}'
    for header in ("{%s,%s}" % (a, b), "{%s,%s}" % (b, a)):
        assert variant(tmp_path, header, bytes(4))[0] == "InvalidLayout"


@pytest.mark.parametrize("header,payload,want", [
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[4,0]}}', bytes(4), "InvalidLayout"),
    ('{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', bytes(4), "InvalidLayout"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', bytes(0), "OutOfBounds"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}', bytes(8), "InvalidLayout"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', bytes(8), "InvalidLayout"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},'
     '"w":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}', bytes(8), "DuplicateName"),
    ('{"w":{"dtype":"F32","dtype":"F32","shape":[1],"data_offsets":[0,4]}}', bytes(4),
     "DuplicateName"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4],"extra":1}}', bytes(4),
     "InvalidArgument"),
    ('{"w":{"dtype":"F64","shape":[1],"data_offsets":[0,8]}}', bytes(8), "Unsupported"),
    ('{"w":{"dtype":"I32","shape":[1],"data_offsets":[0,4]}}', bytes(4), "InvalidDType"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0]}}', bytes(4), "InvalidArgument"),
    ('{"w":{"dtype":"F32","shape":[1,1,1,1,1],"data_offsets":[0,4]}}', bytes(4),
     "InvalidShape"),
    ('{"w":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', bytes(4), "InvalidArgument"),
    ('{"w":{"dtype":"F32","shape":[1.0],"data_offsets":[0,4]}}', bytes(4), "InvalidArgument"),
    ('{"w":{"shape":[1],"data_offsets":[0,4]}}', bytes(4), "InvalidArgument"),
    ('{"__metadata__":{"format":1}}', b"", "InvalidArgument"),
    ('{"__metadata__":{"a":"x","a":"y"}}', b"", "DuplicateName"),
    ('{} x', b"", "InvalidArgument"),
    ('[]', b"", "InvalidArgument"),
    ('{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}', bytes(4), "InvalidArgument"),
])
def test_header_rejects(tmp_path, header, payload, want):
    assert variant(tmp_path, header, payload)[0] == want


def test_header_padding_and_limits(tmp_path):
    # Trailing spaces pad headers; the length prefix bounds the header.
    with SafetensorsFile(asset(tmp_path, "{}    ")) as f:
        assert f.names() == []
    path = tmp_path / "short.safetensors"
    path.write_bytes(struct.pack("<Q", 100) + b"{}")
    with pytest.raises(ExecutorError) as e:
        SafetensorsFile(path)
    assert e.value.variant == "OutOfBounds"
    path.write_bytes(struct.pack("<Q", 0))
    with pytest.raises(ExecutorError) as e:
        SafetensorsFile(path)
    assert e.value.variant == "ResourceLimit"
    with pytest.raises(ExecutorError) as e:
        SafetensorsFile(asset(tmp_path, "{}" + " " * 64), max_header_bytes=16)
    assert e.value.variant == "ResourceLimit"
    path.write_bytes(b"\x01\x02")
    with pytest.raises(ExecutorError) as e:
        SafetensorsFile(path)
    assert e.value.variant == "InvalidArgument"


def test_metadata_and_escaped_names(tmp_path):
    header = json.dumps({"__metadata__": {"format": "pt", "note": "café"},
                         "aé\"b": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}})
    with SafetensorsFile(asset(tmp_path, header, b"\x01\x02")) as f:
        assert f.metadata("note") == "café"
        assert f.metadata("missing") is None
        assert f.names() == ["aé\"b"]


def scheme_file(tmp_path, metadata):
    header = json.dumps({"__metadata__": metadata}) if metadata is not None else "{}"
    return SafetensorsFile(asset(tmp_path, header))


@pytest.mark.parametrize("marker,want", [(None, "dense"), ("pt", "dense"),
                                         ("minifield.ternary.v1", "ternary"),
                                         ("minifield.nf4.v1", "nf4"),
                                         ("minifield.int8.v1", "int8"),
                                         ("minifield.mixed.v1", "dense")])
def test_bundle_format_markers(tmp_path, marker, want):
    meta = {} if marker is None else {"format": marker}
    with scheme_file(tmp_path, meta) as f:
        assert f.matmul_scheme("model.layers.0.feed_forward.w1.weight") == want


@pytest.mark.parametrize("marker", ["unknown", "minifield.ternary.v2", "minifield.nf4.v2",
                                    "minifield.mixed.v2"])
def test_unknown_format_markers_reject(tmp_path, marker):
    with scheme_file(tmp_path, {"format": marker}) as f:
        with pytest.raises(ExecutorError) as e:
            f.matmul_scheme("x")
        assert e.value.variant == "Unsupported"


def test_tensor_quantization_overrides(tmp_path):
    levels = {"a": "ternary-v1", "b": "nf4-v1", "c": "int8-v1", "d": "f16", "e": "bf16"}
    with scheme_file(tmp_path, {"format": "minifield.mixed.v1",
                                "tensor_quantization": json.dumps(levels)}) as f:
        assert [f.matmul_scheme(n) for n in "abcdez"] == ["ternary", "nf4", "int8", "dense",
                                                           "dense", "dense"]
    with scheme_file(tmp_path, {"format": "minifield.ternary.v1",
                                "tensor_quantization": json.dumps({"a": "f32"})}) as f:
        assert (f.matmul_scheme("a"), f.matmul_scheme("b")) == ("dense", "ternary")
    for bad in ("not json", json.dumps({"a": "q4"}), json.dumps({"a": 1}), "[]",
                '{"a": "nf4-v1",}', '{"a": "nf4-v1"} x'):
        with scheme_file(tmp_path, {"format": "minifield.mixed.v1",
                                    "tensor_quantization": bad}) as f:
            with pytest.raises(ExecutorError) as e:
                f.matmul_scheme("a")
            assert e.value.variant == "InvalidArgument"


@pytest.mark.parametrize("levels", [{"a": "nf4-v1", "b": "q4"}, {"a": "nf4-v1", "b": 1},
                                    {"a": "nf4-v1", "b": None},
                                    {"a": "nf4-v1", "b": {"nested": [1, 2.5e-3, True]}}])
def test_tensor_quantization_checks_every_entry(tmp_path, levels):
    """quantization_from_entries (weights.rs:116-135) rejects the whole map
    when any entry is not a known level string, whichever tensor is looked
    up; a non-string level gets the level message, not a JSON error."""
    with scheme_file(tmp_path, {"format": "minifield.mixed.v1",
                                "tensor_quantization": json.dumps(levels)}) as f:
        for name in ("a", "b", "z"):
            with pytest.raises(ExecutorError) as e:
                f.matmul_scheme(name)
            assert e.value.variant == "InvalidArgument"
            assert "level must be ternary-v1" in str(e.value)


def test_tensor_quantization_repeated_name_keeps_the_last(tmp_path):
    with scheme_file(tmp_path, {"format": "minifield.mixed.v1",
                                "tensor_quantization": '{"a": "nf4-v1", "a": "int8-v1"}'}) as f:
        assert f.matmul_scheme("a") == "int8"


def test_bundle_writer_layout(tmp_path):
    """write_lfm2_bundle names and dtypes as the converter writes them."""
    from runtime_amd.lfm2 import ATTENTION, CONV, Lfm2Config, synthetic_host_weights
    from runtime_amd.loader import lfm2_tensor_names, write_lfm2_bundle
    cfg = Lfm2Config(hidden=256, intermediate=512, attention_heads=4, key_value_heads=2,
                     vocab=300, layers=[CONV, ATTENTION], max_tokens=32,
                     formats={"embedding": "int8", "conv": "nf4", "attention": None,
                              "ffn": "ternary"})
    host = {(r, l): a for r, l, a in synthetic_host_weights(cfg, norms="random")}
    path = tmp_path / "model.safetensors"
    write_lfm2_bundle(path, cfg, host)
    with SafetensorsFile(path) as f:
        assert f.metadata("format") == "minifield.mixed.v1"
        names = lfm2_tensor_names(cfg)
        assert f.info("model.embed_tokens.weight.codes") == ("U8", (300, 256))
        assert f.info("model.embed_tokens.weight.scales") == ("F16", (300, 2))
        assert f.matmul_scheme("model.embed_tokens.weight") == "int8"
        assert f.info("model.layers.0.conv.in_proj.weight.codes") == ("U8", (768, 128))
        assert f.matmul_scheme("model.layers.1.self_attn.q_proj.weight") == "dense"
        assert f.info("model.layers.1.self_attn.q_proj.weight") == ("F32", (256, 256))
        assert f.info("model.layers.0.conv.conv.weight") == ("F32", (256, 1, 3))
        assert f.info("model.layers.0.feed_forward.w2.weight.codes") == ("U8", (256, 128))
        assert len(f.names()) == len(names) + sum(len(host[k]) == 2 for k in names)

"""The native safetensors reader (ming_st_*, the container that
Tensors.load reads through mlx_load_safetensors, src/ming_model.zig:316-350)
against files written by the `safetensors` package, and its handling of
malformed files.  Host only: no GPU call.

Pins: every entry's name, dtype, shape, absolute offset and size equal an
independent read of the same header with Python's json module, and the bytes
at that offset equal the tensor's bytes; malformed headers are refused with
a status and a message (never a crash)."""
import importlib
import json
import struct

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def ming():
    return importlib.import_module("ming-tts-serve_amd")


def independent_index(path):
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    hdr.pop("__metadata__", None)
    return raw, 8 + n, hdr


def test_index_matches_the_writer(ming, tmp_path):
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(0)
    tensors = {
        "model.model.embed_tokens.weight": torch.randn(8, 64, generator=g).to(torch.bfloat16),
        "model.model.layers.0.self_attn.q_proj.weight": torch.randint(0, 2**31, (16, 8), generator=g,
                                                                      dtype=torch.int64).to(torch.uint32),
        "model.model.layers.0.self_attn.q_proj.scales": torch.randn(16, 1, generator=g).to(torch.bfloat16),
        "flowloss.cfm.model.rotary_embed.inv_freq": torch.rand(32, generator=g),
        "ids": torch.arange(5, dtype=torch.int32),
        "half": torch.randn(3, 4, generator=g).half(),
        "big": torch.arange(6, dtype=torch.int64).reshape(1, 2, 3),
        "bytes": torch.arange(7, dtype=torch.uint8),
        "scalar": torch.tensor(3.5, dtype=torch.float32),
        'quote"and\\slash': torch.zeros(2, dtype=torch.float32),
    }
    path = tmp_path / "m.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt", "note": 'a {nested} "string"'})
    raw, data_off, hdr = independent_index(path)
    idx = {e["name"]: e for e in ming.st_index(path)}
    assert set(idx) == set(tensors)
    for name, meta in hdr.items():
        e = idx[name]
        assert e["dtype"] == meta["dtype"], name
        assert e["shape"] == meta["shape"], name
        b0, b1 = meta["data_offsets"]
        assert e["offset"] == data_off + b0 and e["nbytes"] == b1 - b0, name
        t = tensors[name].contiguous().reshape(-1)
        want = t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.uint32 else t.numpy().tobytes()
        assert raw[e["offset"]:e["offset"] + e["nbytes"]] == want, name


def write_raw(path, header: bytes, data: bytes, n=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if n is None else n))
        f.write(header)
        f.write(data)


BAD = {
    "short": (b"", b"", 0),
    "length_past_end": (b"{}", b"", 1 << 20),
    "not_an_object": (b"[1, 2]", b"", None),
    "truncated_json": (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]', b"\0" * 4, None),
    "offsets_past_data": (b'{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', b"\0" * 4, None),
    "size_mismatch": (b'{"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}', b"\0" * 8, None),
    "reversed_offsets": (b'{"a": {"dtype": "F32", "shape": [0], "data_offsets": [4, 0]}}', b"\0" * 8, None),
    "unknown_dtype": (b'{"a": {"dtype": "Q7", "shape": [1], "data_offsets": [0, 1]}}', b"\0", None),
    "missing_field": (b'{"a": {"dtype": "F32", "data_offsets": [0, 4]}}', b"\0" * 4, None),
    "duplicate_name": (b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}, '
                       b'"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}', b"\0\0", None),
    "negative_dim": (b'{"a": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}}', b"\0", None),
    "huge_dim": (b'{"a": {"dtype": "F64", "shape": [4611686018427387904, 8], "data_offsets": [0, 8]}}', b"\0" * 8,
                 None),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_malformed_files_are_refused(ming, tmp_path, case):
    header, data, n = BAD[case]
    path = tmp_path / f"{case}.safetensors"
    if case == "short":
        path.write_bytes(b"\x01\x02")
    else:
        write_raw(path, header, data, n)
    with pytest.raises(ming.MingError) as e:
        ming.st_index(path)
    assert e.value.status in (ming.MING_E_SHAPE, ming.MING_E_ARG)
    assert len(str(e.value)) > 10


def test_missing_file(ming, tmp_path):
    with pytest.raises(ming.MingError) as e:
        ming.st_index(tmp_path / "nope.safetensors")
    assert e.value.status == ming.MING_E_ARG


def test_empty_and_metadata_only(ming, tmp_path):
    p = tmp_path / "e.safetensors"
    write_raw(p, b'{"__metadata__": {"k": "v"}}', b"")
    assert ming.st_index(p) == []
    write_raw(p, b"{}", b"")
    assert ming.st_index(p) == []

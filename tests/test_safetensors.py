"""safetensors reader (sltx_st_*) on the CPU: header parsing and host reads.

Pinned against the reference's own fixture (fixtures/mlx_pass2_noise.safetensors,
committed under tests/golden/ as data), against the `safetensors` package's
reader, and against hand-written files covering every dtype TensorDType knows
(SafeTensors.swift:15-31), the cases the reference skips (unknown dtypes,
"__metadata__"), and corrupt files it would read out of bounds.
"""
import json
import os
import struct

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def write_st(path, tensors, metadata=None, pad=True):
    """tensors: name -> (dtype string, shape, raw bytes).  Layout of
    saveSafetensors (SafeTensors.swift:217-240): LE u64 header length, JSON,
    space padding to 8 bytes, data."""
    header, blob = {}, b""
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape),
                        "data_offsets": [len(blob), len(blob) + len(raw)]}
        blob += raw
    if metadata is not None:
        header["__metadata__"] = metadata
    h = json.dumps(header).encode()
    if pad:
        h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + blob)
    return path


def test_reference_fixture(pkg):
    from safetensors.numpy import load_file
    path = os.path.join(GOLDEN, "mlx_pass2_noise.safetensors")
    f = pkg.SafeTensorsFile(path)
    assert list(f.tensors) == ["noise"]
    info = f.tensors["noise"]
    assert (info.dtype, info.shape, info.offset, info.byte_count) == \
        ("F32", (1, 128, 2, 32, 32), 0, 1048576)
    assert np.array_equal(f.read_host("noise"), load_file(path)["noise"])


def test_every_dtype_and_sorted_names(pkg, tmp_path):
    rng = np.random.default_rng(0)
    arrays = {
        "w.f32": ("F32", rng.standard_normal((3, 5)).astype(np.float32)),
        "a.f16": ("F16", rng.standard_normal((7,)).astype(np.float16)),
        "c.bf16": ("BF16", rng.integers(0, 65535, (2, 2, 2)).astype(np.uint16)),
        "q.i8": ("I8", rng.integers(-128, 127, (4, 4)).astype(np.int8)),
        "b.u8": ("U8", rng.integers(0, 255, (9,)).astype(np.uint8)),
        "z.i32": ("I32", rng.integers(-2**31, 2**31 - 1, (3, 1)).astype(np.int32)),
        "m.u32": ("U32", rng.integers(0, 2**32 - 1, (2, 6), dtype=np.uint64).astype(np.uint32)),
        "empty": ("F16", np.zeros((0, 5), np.float16)),
    }
    path = write_st(tmp_path / "all.safetensors",
                    {k: (dt, a.shape, a.tobytes()) for k, (dt, a) in arrays.items()},
                    metadata={"format": "mlx"})
    f = pkg.SafeTensorsFile(path)
    assert list(f.tensors) == sorted(arrays)
    for name, (dt, a) in arrays.items():
        info = f.tensors[name]
        assert info.dtype == dt and info.shape == a.shape and info.byte_count == a.nbytes
        assert np.array_equal(f.read_host(name), a)


def test_matches_safetensors_package(pkg, tmp_path):
    from safetensors.numpy import load_file, save_file
    rng = np.random.default_rng(1)
    src = {"model.layers.0.mlp.up_proj.weight":
           rng.integers(0, 2**32 - 1, (64, 32), dtype=np.uint64).astype(np.uint32),
           "model.layers.0.mlp.up_proj.scales": rng.standard_normal((64, 4)).astype(np.float16),
           "model.norm.weight": rng.standard_normal(256).astype(np.float32)}
    path = str(tmp_path / "pkg.safetensors")
    save_file(src, path, metadata={"format": "pt"})
    ref = load_file(path)
    f = pkg.SafeTensorsFile(path)
    assert set(f.tensors) == set(ref)
    for k, v in ref.items():
        assert np.array_equal(f.read_host(k), v)


def test_skips_like_the_reference(pkg, tmp_path):
    """Unknown dtypes and non-tensor entries are skipped (SafeTensors.swift:57-78);
    "__metadata__" may be an object or null."""
    a = np.arange(4, dtype=np.float32)
    for meta in ({"k": "v"}, None):
        tensors = {"keep": ("F32", a.shape, a.tobytes()),
                   "f64": ("F64", (2,), np.zeros(2).tobytes()),
                   "u16": ("U16", (2,), np.zeros(2, np.uint16).tobytes())}
        path = write_st(tmp_path / "skip.safetensors", tensors, metadata=meta)
        if meta is None:   # write "__metadata__": null explicitly
            raw = open(path, "rb").read()
            hlen = struct.unpack("<Q", raw[:8])[0]
            h = json.loads(raw[8:8 + hlen])
            h["__metadata__"] = None
            hb = json.dumps(h).encode()
            hb += b" " * ((8 - len(hb) % 8) % 8)
            open(path, "wb").write(struct.pack("<Q", len(hb)) + hb + raw[8 + hlen:])
        f = pkg.SafeTensorsFile(path)
        assert list(f.tensors) == ["keep"]
        assert np.array_equal(f.read_host("keep"), a)


def _bad(pkg, path, frag):
    with pytest.raises(pkg.SltxError) as ei:
        pkg.SafeTensorsFile(str(path))
    assert ei.value.code == pkg.SLTX_ERR_INVALID
    assert frag in str(ei.value)


def test_corrupt_files_are_rejected(pkg, tmp_path):
    a = np.arange(6, dtype=np.float32)
    good = write_st(tmp_path / "g.safetensors", {"t": ("F32", (6,), a.tobytes())})
    raw = open(good, "rb").read()
    hlen = struct.unpack("<Q", raw[:8])[0]
    _bad(pkg, tmp_path / "missing.safetensors", "cannot open")
    (tmp_path / "short.safetensors").write_bytes(b"\x01\x02")
    _bad(pkg, tmp_path / "short.safetensors", "too short")
    (tmp_path / "hlen.safetensors").write_bytes(struct.pack("<Q", 10 ** 6) + raw[8:])
    _bad(pkg, tmp_path / "hlen.safetensors", "header length")
    (tmp_path / "json.safetensors").write_bytes(struct.pack("<Q", 5) + b"{oops" + raw[8 + hlen:])
    _bad(pkg, tmp_path / "json.safetensors", "not a JSON object")
    (tmp_path / "trunc.safetensors").write_bytes(raw[:-4])
    _bad(pkg, tmp_path / "trunc.safetensors", "outside the file")
    write_st(tmp_path / "size.safetensors", {"t": ("F32", (5,), a.tobytes())})
    _bad(pkg, tmp_path / "size.safetensors", "do not match")
    write_st(tmp_path / "dims.safetensors", {"t": ("U8", (1,) * 9, b"\x00")})
    _bad(pkg, tmp_path / "dims.safetensors", "more than 8")
    write_st(tmp_path / "neg.safetensors", {"t": ("U8", (-1,), b"")})
    _bad(pkg, tmp_path / "neg.safetensors", "bad shape")
    # a name repeated in the header is ambiguous: rejected, not deduplicated
    hdr = (b'{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},'
           b'"t":{"dtype":"F32","shape":[2],"data_offsets":[8,16]}}')
    hdr += b" " * ((8 - len(hdr) % 8) % 8)
    (tmp_path / "dup.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + a[:4].tobytes())
    _bad(pkg, tmp_path / "dup.safetensors", "duplicate tensor name")


def test_read_host_capacity_and_names(pkg, tmp_path):
    import ctypes
    a = np.arange(8, dtype=np.int32)
    path = write_st(tmp_path / "c.safetensors", {"t": ("I32", (8,), a.tobytes())})
    f = pkg.SafeTensorsFile(path)
    buf = np.zeros(4, np.int32)
    L = pkg.lib()
    assert L.sltx_st_read_host(f._h, b"t", buf.ctypes.data, buf.nbytes) == -1
    assert "capacity" in pkg.last_error()
    assert L.sltx_st_read_host(f._h, b"nope", buf.ctypes.data, buf.nbytes) == -1
    assert "not found" in pkg.last_error()
    assert L.sltx_st_name(f._h, 0) == b"t" and L.sltx_st_name(f._h, 1) is None
    c = pkg.CStInfo()
    assert L.sltx_st_info_of(f._h, b"t", ctypes.byref(c)) == 0 and c.nbytes == 32


def test_model_config_keys(pkg):
    from swiftltx_amd.weights import ModelConfig
    d = {"hidden_size": 3072, "intermediate_size": 8192, "num_hidden_layers": 28,
         "num_attention_heads": 24, "num_key_value_heads": 8, "vocab_size": 128256,
         "max_position_embeddings": 131072, "rms_norm_eps": 1e-5, "rope_theta": 500000.0,
         "head_dim": 128, "tie_word_embeddings": True,
         "quantization": {"group_size": 64, "bits": 4},
         "rope_scaling": {"factor": 32.0, "rope_type": "llama3"}}
    c = ModelConfig.from_dict(d)
    assert (c.hidden_size, c.head_dim, c.kv_repeat_factor) == (3072, 128, 3)
    assert c.quantization.group_size == 64 and c.tie_word_embeddings
    d.pop("head_dim")
    assert ModelConfig.from_dict(d).head_dim == 128

"""Checkpoint reading on the host (no GPU): the safetensors repository
(src/model/safetensors.zig:17-220) and the config.json checks
(src/model/config.zig:34-157, src/model/mtp.zig:318-345).

The test writer (helpers.write_safetensors) and the C++ reader are both
checked against the independent `safetensors` package: files it writes are
read here, and files the test writer makes are read by it.
"""
import json
import struct

import numpy as np
import pytest

from helpers import qwen35_config, write_checkpoint, write_safetensors
from peregrine_amd._lib import PrgError
from peregrine_amd.checkpoint import Safetensors, read_config, verify_config, verify_mtp_config

NOT_FOUND, MALFORMED, UNSUPPORTED, INVALID_ARG = 8, 9, 10, 1


def _err(excinfo, code, name):
    assert excinfo.value.code == code, str(excinfo.value)
    assert name in str(excinfo.value), str(excinfo.value)


def _index(d, weight_map):
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


# ------------------------------------------------------------- repository ---
def test_reads_files_written_by_the_safetensors_package(tmp_path):
    sn = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(0)
    arrays = {"w": rng.integers(0, 2**32, size=(4, 8), dtype=np.uint32),
              "f": rng.standard_normal(3).astype(np.float32),
              "h": rng.integers(0, 2**16, size=(2, 2, 2), dtype=np.uint16),
              "scalar": np.array(7, dtype=np.int64)}
    sn.save_file(arrays, str(tmp_path / "one.safetensors"), metadata={"format": "mlx"})
    _index(tmp_path, {k: "one.safetensors" for k in arrays})
    with Safetensors(tmp_path) as st:
        assert st.names() == sorted(arrays)
        assert st.shards() == ["one.safetensors"]
        for k, a in arrays.items():
            ti = st.info(k)
            assert ti.shape == a.shape and ti.nbytes == a.nbytes
            assert ti.dtype == {"uint32": "U32", "float32": "F32", "uint16": "U16", "int64": "I64"}[a.dtype.name]
            np.testing.assert_array_equal(st.read(k), a)


def test_package_reads_the_test_writer(tmp_path):
    sn = pytest.importorskip("safetensors.numpy")
    a = np.arange(24, dtype=np.uint32).reshape(3, 8)
    b = np.linspace(-1, 1, 5, dtype=np.float32)
    write_safetensors(tmp_path / "x.safetensors", {"a": ("U32", a.shape, a), "b": ("F32", b.shape, b)},
                      metadata={"format": "mlx"})
    got = sn.load_file(str(tmp_path / "x.safetensors"))
    np.testing.assert_array_equal(got["a"], a)
    np.testing.assert_array_equal(got["b"], b)


def test_shards_are_the_sorted_unique_index_values(tmp_path):
    """discoverShards (safetensors.zig:144-177): unique weight_map values,
    sorted bytewise; every shard's header joins one tensor table."""
    rng = np.random.default_rng(1)
    tensors = {f"t{i}": ("U32", (2, i + 1), rng.integers(0, 2**32, size=(2, i + 1), dtype=np.uint32))
               for i in range(7)}
    where = write_checkpoint(tmp_path, tensors, n_shards=3)
    with Safetensors(tmp_path) as st:
        shards = st.shards()
        assert shards == sorted(set(where.values()))
        assert st.names() == sorted(tensors)
        for n, (_, _, a) in tensors.items():
            assert shards[st.info(n).shard] == where[n]
            np.testing.assert_array_equal(st.read(n), a)


def test_unicode_names_and_ignored_metadata(tmp_path):
    a = np.arange(4, dtype=np.uint16)
    write_safetensors(tmp_path / "s.safetensors", {"café.\U0001F600": ("BF16", (4,), a)},
                      metadata={"format": "mlx", "nested": "x"})
    _index(tmp_path, {"café.\U0001F600": "s.safetensors"})
    with Safetensors(tmp_path) as st:
        assert st.names() == ["café.\U0001F600"]
        np.testing.assert_array_equal(st.read("café.\U0001F600"), a)


def test_missing_index_and_shard(tmp_path):
    with pytest.raises(PrgError) as e:
        Safetensors(tmp_path)
    _err(e, NOT_FOUND, "FileNotFound")
    _index(tmp_path, {"a": "absent.safetensors"})
    with pytest.raises(PrgError) as e:
        Safetensors(tmp_path)
    _err(e, NOT_FOUND, "FileNotFound")


@pytest.mark.parametrize("index,name", [
    ("[]", "MalformedIndex"),
    ('{"metadata": {}}', "MalformedIndex"),
    ('{"weight_map": {"a": 3}}', "MalformedIndex"),
    ('{"weight_map": {}}', "NoShardsFound"),
    ('{"weight_map": {"a": "../escape.safetensors"}}', "MalformedIndex"),
    ('{"weight_map": {"a": "x.safetensors",}}', "MalformedIndex"),
])
def test_malformed_index(tmp_path, index, name):
    (tmp_path / "model.safetensors.index.json").write_text(index)
    with pytest.raises(PrgError) as e:
        Safetensors(tmp_path)
    _err(e, MALFORMED, name)


def _raw_shard(tmp_path, blob: bytes):
    (tmp_path / "s.safetensors").write_bytes(blob)
    _index(tmp_path, {"a": "s.safetensors"})


def _hdr(obj) -> bytes:
    h = json.dumps(obj).encode()
    return struct.pack("<Q", len(h)) + h


@pytest.mark.parametrize("blob,name", [
    (b"\x01\x02\x03", "TruncatedHeader"),                                     # < 8 bytes
    (struct.pack("<Q", 100) + b"{}", "TruncatedHeader"),                      # header past EOF
    (struct.pack("<Q", 2) + b"[]", "MalformedHeader"),                        # not an object
    (struct.pack("<Q", 5) + b"{\"a\":", "MalformedHeader"),                   # bad JSON
    (_hdr({"a": {"dtype": "U32", "shape": [2]}}), "MalformedHeader"),         # no data_offsets
    (_hdr({"a": {"dtype": "U32", "shape": [-2], "data_offsets": [0, 8]}}), "MalformedHeader"),
    (_hdr({"a": {"dtype": "U32", "shape": [2], "data_offsets": [0]}}), "MalformedHeader"),
    (_hdr({"a": {"dtype": "U32", "shape": [2], "data_offsets": [0, 8.5]}}), "MalformedHeader"),
])
def test_malformed_shard(tmp_path, blob, name):
    _raw_shard(tmp_path, blob)
    with pytest.raises(PrgError) as e:
        Safetensors(tmp_path)
    _err(e, MALFORMED, name)


def test_tensor_bounds_checked_on_access(tmp_path):
    """tensorRange (safetensors.zig:123-141): begin <= end and the range inside
    the file, checked when a tensor is looked up or read; offsets past 2^53
    are parsed exactly and rejected, not rounded."""
    big = 2**60 + 1
    _raw_shard(tmp_path, _hdr({"a": {"dtype": "U32", "shape": [2], "data_offsets": [0, 8]},
                               "b": {"dtype": "U32", "shape": [2], "data_offsets": [8, 4]},
                               "c": {"dtype": "U32", "shape": [2], "data_offsets": [big, big + 8]}})
               + b"\0" * 8)
    with Safetensors(tmp_path) as st:
        assert st.info("a").nbytes == 8
        for n in ("b", "c"):
            with pytest.raises(PrgError) as e:
                st.info(n)
            _err(e, MALFORMED, "MalformedHeader")
        with pytest.raises(PrgError) as e:
            st.info("zz")
        _err(e, NOT_FOUND, "TensorNotFound")


def test_read_requires_exact_buffer(tmp_path):
    import ctypes as C

    from peregrine_amd._lib import lib

    a = np.arange(8, dtype=np.uint32)
    write_safetensors(tmp_path / "s.safetensors", {"a": ("U32", (8,), a)})
    _index(tmp_path, {"a": "s.safetensors"})
    with Safetensors(tmp_path) as st:
        buf = np.zeros(64, np.uint8)
        rc = lib.prg_safetensors_read(st.handle, b"a", buf.ctypes.data_as(C.c_void_p), C.c_uint64(16))
        assert rc == INVALID_ARG and b"InvalidTensorBuffer" in lib.prg_last_error()


# ----------------------------------------------------------------- config ---
def _cfg_dir(tmp_path, cfg) -> str:
    (tmp_path / "config.json").write_text(json.dumps(cfg) if not isinstance(cfg, str) else cfg)
    return str(tmp_path)


def test_verify_accepts_exact_9b(tmp_path):
    """config.zig:141-143."""
    verify_config(_cfg_dir(tmp_path, qwen35_config()))


def test_verify_rejects_non_q4(tmp_path):
    """config.zig:145-150."""
    with pytest.raises(PrgError) as e:
        verify_config(_cfg_dir(tmp_path, qwen35_config(bits=8)))
    _err(e, UNSUPPORTED, "UnsupportedQuantization")


def test_verify_rejects_non_9b(tmp_path):
    """config.zig:152-157."""
    with pytest.raises(PrgError) as e:
        verify_config(_cfg_dir(tmp_path, qwen35_config(hidden=1024)))
    _err(e, UNSUPPORTED, "NotQwen35_9B")


@pytest.mark.parametrize("cfg,code,name", [
    (qwen35_config(group=32), UNSUPPORTED, "UnsupportedQuantization"),
    (qwen35_config(mode="mxfp4"), UNSUPPORTED, "UnsupportedQuantization"),
    (qwen35_config(model_type="qwen3_next"), UNSUPPORTED, "UnsupportedArchitecture"),
    (qwen35_config(num_key_value_heads=3), UNSUPPORTED, "InvalidConfig"),
    (qwen35_config(num_attention_heads=0), UNSUPPORTED, "InvalidConfig"),
    (qwen35_config(full_attention_interval=0), UNSUPPORTED, "InvalidConfig"),
    (qwen35_config(rope_parameters={"partial_rotary_factor": 0.0}), UNSUPPORTED, "InvalidConfig"),
    (qwen35_config(rope_parameters={"partial_rotary_factor": 1.5}), UNSUPPORTED, "InvalidConfig"),
    (qwen35_config(vocab_size=151936), UNSUPPORTED, "NotQwen35_9B"),
    (qwen35_config(hidden_size=-4096), MALFORMED, "InvalidNumber"),
    ({"text_config": {"model_type": "qwen3_5_text"}, "quantization": {"group_size": 64, "bits": 4,
                                                                      "mode": "affine"}},
     MALFORMED, "MissingField"),
    ('{"text_config": ', MALFORMED, "SyntaxError"),
])
def test_verify_rejections(tmp_path, cfg, code, name):
    with pytest.raises(PrgError) as e:
        verify_config(_cfg_dir(tmp_path, cfg))
    _err(e, code, name)


def test_verify_missing_config(tmp_path):
    with pytest.raises(PrgError) as e:
        verify_config(str(tmp_path))
    _err(e, NOT_FOUND, "FileNotFound")


def test_partial_rotary_default_and_rounding(tmp_path):
    """rotary_dim = round(factor * head_dim) with factor defaulting to 0.25
    (config.zig:22-24, 54-55): an absent rope_parameters is the 9B's 64."""
    cfg = qwen35_config()
    del cfg["text_config"]["rope_parameters"]
    verify_config(_cfg_dir(tmp_path, cfg))
    # 0.2501 * 256 = 64.03 -> 64
    verify_config(_cfg_dir(tmp_path, qwen35_config(rope_parameters={"partial_rotary_factor": 0.2501})))


def _mtp_cfg(**over):
    c = {"model_type": "qwen3_5_mtp",
         "text_config": {"model_type": "qwen3_5_text", "hidden_size": 4096, "intermediate_size": 12288,
                         "mtp_num_hidden_layers": 1, "num_attention_heads": 16, "num_key_value_heads": 4,
                         "head_dim": 256, "vocab_size": 248320},
         "quantization": {"group_size": 64, "bits": 4, "mode": "affine"}}
    for k, v in over.items():
        if k in c["text_config"]:
            c["text_config"][k] = v
        else:
            c[k] = v
    return c


def test_verify_mtp(tmp_path):
    """mtp.zig:318-345: the sidecar config, with quantization_config as the
    fallback when quantization.bits is absent."""
    verify_mtp_config(_cfg_dir(tmp_path, _mtp_cfg()))
    c = _mtp_cfg()
    c["quantization_config"] = c.pop("quantization")
    verify_mtp_config(_cfg_dir(tmp_path, c))
    for over, name in [({"model_type": "qwen3_5"}, "UnsupportedArchitecture"),
                       ({"mtp_num_hidden_layers": 2}, "UnsupportedArchitecture"),
                       ({"quantization": {"group_size": 64, "bits": 8, "mode": "affine"}},
                        "UnsupportedQuantization"),
                       ({"head_dim": 128}, "NotQwen35_9B")]:
        with pytest.raises(PrgError) as e:
            verify_mtp_config(_cfg_dir(tmp_path, _mtp_cfg(**over)))
        _err(e, UNSUPPORTED, name)


def test_read_config(tmp_path):
    c = read_config(_cfg_dir(tmp_path, qwen35_config()))
    assert (c.num_layers, c.hidden, c.intermediate, c.vocab, c.full_attention_interval, c.mtp_layers) == \
        (32, 4096, 12288, 248320, 4, 0)
    assert abs(c.rms_eps - 1e-6) < 1e-12
    c = read_config(_cfg_dir(tmp_path, qwen35_config(hidden=1024, intermediate=2048, layers=4, vocab=4096,
                                                     rms_norm_eps=1e-5)))
    assert (c.num_layers, c.hidden, c.intermediate, c.vocab) == (4, 1024, 2048, 4096)
    assert abs(c.rms_eps - 1e-5) < 1e-10
    for over in [{"head_dim": 128}, {"linear_num_value_heads": 16},
                 {"rope_parameters": {"partial_rotary_factor": 0.25, "rope_theta": 10000}}]:
        with pytest.raises(PrgError) as e:
            read_config(_cfg_dir(tmp_path, qwen35_config(**over)))
        _err(e, UNSUPPORTED, "UnsupportedArchitecture")

"""The quantized package payload on the host: .npy payload files with SHA-256
checksums (models/tensor_data_io.py), the package metadata and its validation
(models/quantized_package_io.py), the writer (models/quantized_package_writer.py)
and the layer package (models/quantized_layer_package.py) -- against the
reference tests' known answers (tests/test_tensor_data_io.py,
tests/test_quantized_package_writer.py, tests/test_quantized_package_io.py),
numpy's own .npy encoding and hashlib, and a write -> load round trip.  No GPU."""

import hashlib
import io
import json

import numpy as np
import pytest
import torch

from mk import llama_layer_ops as ll
from mk import quantized_layer_package as qlp
from mk import quantized_package_io as qpio
from mk import quantized_package_writer as qpw
from mk import tensor_data_io as tdio
from mk.quantize_weights import QuantizationConfig, quantize_weight_groupwise


def test_checksum_known_answers(tmp_path):
    p = tmp_path / "a.bin"
    p.write_bytes(b"hello world")
    # the reference test's known answer (tests/test_tensor_data_io.py:23-31)
    assert tdio.compute_file_checksum(p) == "b94d27b9934d3e08a52e52d7da7dabfac484efe37a5380ee9088f7ace2efcde9"
    p.write_bytes(b"hello")
    assert len(tdio.compute_file_checksum(p, "sha1")) == 40 and len(tdio.compute_file_checksum(p, "md5")) == 32
    p.write_bytes(b"")
    assert tdio.compute_file_checksum(p) == hashlib.sha256(b"").hexdigest()
    big = bytes(range(256)) * 1000  # crosses the 64 KiB read size
    p.write_bytes(big)
    assert tdio.compute_file_checksum(p) == hashlib.sha256(big).hexdigest()


@pytest.mark.parametrize("arr", [np.array([[1.0, 2.0], [3.0, 4.0]], np.float32), np.array([1, 2, 3], np.int32),
                                 np.arange(24, dtype=np.float16).reshape(2, 3, 4), np.zeros((0, 5), np.uint8)])
def test_npy_bytes_and_header(tmp_path, arr):
    info = tdio.save_tensor_npy(arr, tmp_path / "sub" / "nested" / "t.npy")
    buf = io.BytesIO()
    np.save(buf, arr)  # the file is numpy's own encoding of the array
    raw = (tmp_path / "sub" / "nested" / "t.npy").read_bytes()
    assert raw == buf.getvalue()
    assert info.checksum == hashlib.sha256(raw).hexdigest()
    assert (info.shape, info.dtype, info.nbytes) == (arr.shape, str(arr.dtype), arr.nbytes)
    assert tdio.tensor_shape(info.file_path) == arr.shape and tdio.tensor_dtype(info.file_path) == str(arr.dtype)
    assert tdio.tensor_nbytes(info.file_path) == arr.nbytes
    np.testing.assert_array_equal(tdio.load_tensor_npy(info.file_path), arr)
    got = tdio.load_tensor_to_device(info.file_path, "cpu", expected_shape=arr.shape, expected_checksum=info.checksum)
    assert np.array_equal(got.numpy(), arr)


def test_torch_tensors_and_errors(tmp_path):
    t = torch.arange(6, dtype=torch.int16).reshape(2, 3)
    info = tdio.save_tensor_npy(t, tmp_path / "t.npy")
    assert info.dtype == "int16" and info.shape == (2, 3)
    with pytest.raises(TypeError, match="bfloat16"):
        tdio.save_tensor_npy(t.to(torch.bfloat16), tmp_path / "b.npy")
    with pytest.raises((FileNotFoundError, OSError)):
        tdio.load_tensor_npy(tmp_path / "missing.npy")
    assert tdio.validate_tensor_file(tmp_path / "missing.npy") == [f"file not found: {tmp_path / 'missing.npy'}"]
    issues = tdio.validate_tensor_file(info.file_path, expected_shape=(3, 2), expected_dtype="float32",
                                       expected_checksum="0" * 64)
    assert [m.split(" for ")[0] for m in issues] == ["shape mismatch", "dtype mismatch", "checksum mismatch"]
    (tmp_path / "junk.npy").write_bytes(b"not an npy file")
    assert tdio.validate_tensor_file(tmp_path / "junk.npy")[0].startswith("failed to read shape")
    with pytest.raises(ValueError, match="shape mismatch"):
        tdio.load_tensor_to_device(info.file_path, "cpu", expected_shape=(6,))


def _cfg(layers=2):
    return ll.LlamaLikeConfig(hidden_size=64, intermediate_size=128, num_attention_heads=4, num_key_value_heads=2,
                              head_dim=16, num_hidden_layers=layers, max_position_embeddings=64,
                              vocab_size=96).validate()


def _layer(cfg, idx, bits, g, seed, with_zeros=False):
    gen = torch.Generator().manual_seed(seed)
    qc = QuantizationConfig(bits=bits, group_size=g)

    def lin(key, n, k):
        q = quantize_weight_groupwise(torch.randn(n, k, generator=gen) * 0.05, qc, backend="reference")
        s = q.scales.numpy()
        # stored zeros: the symmetric zero point, as an explicit array
        z = np.full(s.shape, 8.0 if bits == 4 else 128.0, np.float16) if with_zeros else None
        return qlp.QuantizedLinearPackage(name=f"layers.{idx}.{key}", weight=q.packed_weight.numpy(), scales=s,
                                          zeros=z, bits=bits, group_size=g, original_shape=(n, k))

    H, I = cfg.hidden_size, cfg.intermediate_size
    return qlp.QuantizedLlamaLayerPackage(
        layer_idx=idx, input_layernorm_weight=(1 + 0.1 * torch.randn(H, generator=gen)).half().numpy(),
        post_attention_layernorm_weight=(1 + 0.1 * torch.randn(H, generator=gen)).half().numpy(),
        qkv=lin("qkv", cfg.qkv_output_dim(), H), o_proj=lin("o_proj", H, H), gate_proj=lin("gate_proj", I, H),
        up_proj=lin("up_proj", I, H), down_proj=lin("down_proj", H, I))


def test_layer_package_shapes_and_kernel_weights():
    cfg = _cfg(1)
    pkg = _layer(cfg, 0, 4, 32, 1)
    sh = pkg.shapes()
    assert sh["qkv"]["weight"] == (cfg.qkv_output_dim(), 32) and sh["down_proj"]["scales"] == (64, 4)
    assert sh["input_layernorm_weight"] == (64,) and sh["qkv"]["zeros"] is None
    kw = pkg.to_kernel_weights(cfg)
    assert kw.bits == 4 and kw.group_size == 32
    # symmetric packages get the zero point the kernels expect: 8 for q4
    assert kw.qkv_zeros.shape == pkg.qkv.scales.shape and np.all(kw.qkv_zeros == 8.0)
    assert qlp.QuantizedLinearPackage("x", None, torch.ones(2, 3, dtype=torch.float16), None, 8, 32,
                                      (2, 96)).kernel_zeros().eq(128).all()
    with pytest.raises(ValueError, match="qkv_w must have shape"):
        pkg.to_kernel_weights(_cfg(1).__class__(**{**cfg.to_dict(), "num_key_value_heads": 4}))


def test_metadata_roundtrip_and_validation(tmp_path):
    cfg = _cfg(2)
    layers = [_layer(cfg, i, 4, 32, 10 + i) for i in range(2)]
    pkg = qpio.package_from_quantized_layers(cfg, layers, bits=4, group_size=32, metadata={"src": "t"})
    assert pkg.num_layers() == 2 and pkg.tensor_count() == 14
    qkv = pkg.layers[0].tensors["qkv"]
    # the fused qkv's original shape is (q + 2 kv output dims, hidden)
    assert qkv.original_shape == (cfg.qkv_output_dim(), 64) and qkv.packed_shape == (128, 32)
    assert pkg.layers[0].tensors["input_layernorm"].bits == 0 and pkg.config == cfg.to_dict()
    assert pkg.quantization == {"bits": 4, "group_size": 32, "symmetric": True, "with_zeros": False}
    pkg.validate()
    pkg.save_json(tmp_path / "p" / "package.json")
    back = qpio.QuantizedCheckpointPackage.load_json(tmp_path / "p" / "package.json")
    assert back.to_dict() == pkg.to_dict()
    d = json.loads((tmp_path / "p" / "package.json").read_text())
    assert isinstance(d["layers"][0]["tensors"]["qkv"]["original_shape"], list)
    s = pkg.summary()
    assert s["num_layers"] == 2 and s["per_layer"]["1"]["down_proj"] == [64, 128] and s["bits"] == 4
    # validation rules (models/quantized_package_io.py:219-284)
    bad = qpio.QuantizedCheckpointPackage.from_dict(pkg.to_dict())
    bad.layers[1].layer_idx = 0
    with pytest.raises(ValueError, match="duplicate layer_idx"):
        bad.validate()
    bad.layers[1].layer_idx = 3
    with pytest.raises(ValueError, match="contiguous"):
        bad.validate()
    bad = qpio.QuantizedCheckpointPackage.from_dict(pkg.to_dict())
    bad.layers[0].tensors["qkv"].bits = 3
    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        bad.validate()
    bad = qpio.QuantizedCheckpointPackage.from_dict(pkg.to_dict())
    bad.layers[0].tensors["input_layernorm"].bits = 4
    with pytest.raises(ValueError, match="unquantized norm"):
        bad.validate()
    bad = qpio.QuantizedCheckpointPackage.from_dict(pkg.to_dict())
    del bad.layers[0].tensors["up_proj"]
    with pytest.raises(ValueError, match="missing required tensor key"):
        bad.validate()
    bad.validate(allow_partial=True)
    with pytest.raises(ValueError, match="at least one layer"):
        qpio.QuantizedCheckpointPackage().validate()
    with pytest.raises(ValueError, match="format_version"):
        qpio.QuantizedCheckpointPackage(format_version="").validate()


def test_writer_config_and_report():
    assert qpw.PackageWriterConfig().validate().tensor_subdir == "tensors"
    with pytest.raises(ValueError, match="checksum_algorithm"):
        qpw.PackageWriterConfig(checksum_algorithm="crc").validate()
    with pytest.raises(ValueError, match="tensor_subdir"):
        qpw.PackageWriterConfig(tensor_subdir="").validate()
    qpw.PackageWriterReport(ok=True).raise_for_errors()
    with pytest.raises(ValueError, match="something failed"):
        qpw.PackageWriterReport(ok=False, errors=["something failed"]).raise_for_errors()


@pytest.mark.parametrize("bits,with_zeros", [(4, False), (8, True)])
def test_write_then_load_stack(tmp_path, bits, with_zeros):
    cfg = _cfg(2)
    layers = [_layer(cfg, i, bits, 32, 20 + i, with_zeros) for i in range(2)]
    pkg = qpio.package_from_quantized_layers(cfg, layers, bits=bits, group_size=32, with_zeros=with_zeros)
    pkg.global_tensors["norm"] = qpio.QuantizedTensorMetadata("norm", "norm", 0, 0, (64,), (64,), (0,))
    pkg.global_tensors["embedding"] = qpio.QuantizedTensorMetadata("embedding", "embedding", 0, 0, (96, 64),
                                                                   (96, 64), (0,))
    emb = np.random.default_rng(0).standard_normal((96, 64)).astype(np.float16)
    norm = np.linspace(0.5, 1.5, 64).astype(np.float16)
    out = tmp_path / "pkg"
    dry = qpw.QuantizedPackageWriter().write_package(pkg, layers, out, dry_run=True,
                                                     global_tensors={"norm": norm, "embedding": emb})
    assert dry.ok and dry.tensor_count == 16
    assert not out.exists()
    rep = qpw.QuantizedPackageWriter().write_tensors(pkg, layers, out, global_tensors={"norm": norm,
                                                                                       "embedding": emb})
    rep.raise_for_errors()
    assert rep.ok and rep.tensor_count == 16 and rep.package_path == str(out / "package.json")
    qkv = pkg.layers[0].tensors["qkv"]
    # names relative to the tensor folder, as the reference writer records them
    assert qkv.data_file == "layers.0.qkv.weight.npy" and qkv.scales_file == "layers.0.qkv.scales.npy"
    assert (qkv.zeros_file is not None) == with_zeros
    assert qkv.checksum == hashlib.sha256((out / "tensors" / qkv.data_file).read_bytes()).hexdigest()
    loaded = qpio.QuantizedCheckpointPackage.load_json(out / "package.json")
    assert loaded.has_tensor_data() and loaded.to_dict() == pkg.to_dict()
    assert loaded.validate_tensor_files(out / "tensors", check_checksums=True) == []
    assert any("file not found" in m for m in loaded.validate_tensor_files(out))
    # a corrupted payload fails its checksum on load
    cfg_back, stack = qpio.load_quantized_stack(out, "cpu")
    assert cfg_back == cfg and stack.num_layers() == 2
    for i, lp in enumerate(layers):
        kw = stack.layers[i]
        assert np.array_equal(kw.qkv_w.numpy(), lp.qkv.weight) and kw.qkv_w.dtype == torch.uint8
        assert np.array_equal(kw.down_scales.numpy(), lp.down_proj.scales.astype(np.float16))
        zp = lp.gate_proj.kernel_zeros()
        assert np.array_equal(kw.gate_zeros.numpy(), np.asarray(zp, np.float16))
        assert np.array_equal(kw.input_layernorm_weight.numpy(), lp.input_layernorm_weight)
    assert np.array_equal(stack.embedding.numpy(), emb) and np.array_equal(stack.final_norm_weight.numpy(), norm)
    f = out / "tensors" / "layers.1.up_proj.weight.npy"
    raw = bytearray(f.read_bytes())
    raw[-1] ^= 1
    f.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="checksum mismatch"):
        qpio.load_quantized_stack(out, "cpu")
    qpio.load_quantized_stack(out, "cpu", check_checksums=False)


def test_writer_reports_missing_layer(tmp_path):
    cfg = _cfg(2)
    layers = [_layer(cfg, i, 4, 32, 30 + i) for i in range(2)]
    pkg = qpio.package_from_quantized_layers(cfg, layers)
    rep = qpw.QuantizedPackageWriter().write_tensors(pkg, layers[:1], tmp_path)
    assert not rep.ok and rep.errors == ["layer 1: no QuantizedLlamaLayerPackage provided"]
    assert not (tmp_path / "package.json").exists() and rep.package_path == str(tmp_path / "package.json")

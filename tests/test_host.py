"""Host-side checks that need no GPU.

* the C ABI: every entry point declared in include/mk_hip.h is exported by
  libmk_hip.so, bound by mk._lib with the same arity, and rejects invalid
  arguments with MK_ERR_INVALID before touching the device;
* the Python API's validation (exception types and message prefixes of the
  reference) and its refusal to run a HIP backend on host tensors;
* the torch ``reference`` backends on host tensors against the oracle (the
  drop-in's reference path is part of the API).
"""

import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest
import torch

import mk.gqa_ops as gqa
import mk.paged_kv_ops as pk
import mk.paged_quantized_kv_ops as pq
import mk.quant_ops as qo
from mk import _lib
from oracle import paged as op
from oracle import quant as oq
from tests._data import assert_close

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mk_hip.h")


def _header_decls():
    """{name: parameter count} for every ``int|int64_t|size_t mk_*(...)`` declaration."""
    text = open(HEADER).read()
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int64_t|size_t)\s+(mk_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_header_and_binding_agree():
    decls = _header_decls()
    assert len(decls) >= 20
    assert set(decls) == set(_lib.SIGNATURES)
    for name, n in decls.items():
        assert len(_lib.SIGNATURES[name]) == n, name


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _header_decls():
        assert hasattr(lib, name), name
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(_lib.library_path())], capture_output=True, text=True,
                             check=True).stdout
        exported = {ln.split()[-1] for ln in out.splitlines() if " T mk_" in ln}
        assert exported == set(_header_decls()), exported ^ set(_header_decls())


def test_abi_version_and_workspace():
    lib = _lib.load()
    assert lib.mk_abi_version() == _lib.ABI_VERSION == 2
    # split-KV partials: B*Hq*splits*(D+2) fp32, never 0 for a real shape
    ws = _lib.workspace_bytes(16, 32, 8, 128, 512, 16)
    assert ws > 0 and ws % 4 == 0
    assert _lib.workspace_bytes(1, 8, 8, 64, 1, 16) >= 0



def test_invalid_arguments_are_rejected_on_the_host():
    lib = _lib.load()
    assert lib.mk_pack_q4(None, None, 1, 2, None) == _lib.MK_ERR_INVALID
    assert lib.mk_q4_matvec(None, None, None, None, None, None, None, 1, 64, 64, 32, 0, 0, None) == _lib.MK_ERR_INVALID
    assert lib.mk_block_table_lookup(None, None, None, None, 1, 1, 16, None) == _lib.MK_ERR_INVALID
    assert lib.mk_swiglu(None, None, None, 4, 0, None) == _lib.MK_ERR_INVALID


def test_launch_maps_status_to_runtime_error(monkeypatch):
    class Fake:
        def mk_fake(self, *args):
            return _lib.MK_ERR_UNSUPPORTED

    monkeypatch.setattr(_lib, "_lib", Fake())
    monkeypatch.setattr(torch.cuda, "device", lambda d: __import__("contextlib").nullcontext())

    class S:
        cuda_stream = 0

    monkeypatch.setattr(torch.cuda, "current_stream", lambda d=None: S())
    with pytest.raises(RuntimeError, match="unsupported"):
        _lib.launch("mk_fake", torch.device("cuda:0"))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("MK_HIP_LIBRARY", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.NativeLibraryError):
        _lib.load()


# ------------------------------------------------------------------ API validation


def _q4_case(rng, N=32, K=64, g=32):
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    packed = torch.from_numpy(oq.pack_q4(codes))
    s = torch.from_numpy((rng.random((N, K // g)) * 0.1 + 0.01).astype(np.float32))
    z = torch.from_numpy(rng.integers(0, 16, size=(N, K // g)).astype(np.float32))
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32)).to(torch.float16)
    return x, packed, s, z, codes


def test_matvec_validation_errors():
    rng = np.random.default_rng(1)
    x, w, s, z, _ = _q4_case(rng)
    with pytest.raises(TypeError, match="x dtype must be float16 or bfloat16"):
        qo.q4_matvec_decode(x.float(), w, s, z)
    with pytest.raises(ValueError, match="scales must have shape"):
        qo.q4_matvec_decode(x, w, s[:, :1], z)
    with pytest.raises(ValueError, match="packed_w implies K"):
        qo.q4_matvec_decode(x[:, :32], w, s, z)
    with pytest.raises(ValueError, match="backend must be one of"):
        qo.q4_matvec_decode(x, w, s, z, backend="cuda")
    with pytest.raises(ValueError, match="ROCm device"):
        qo.q4_matvec_decode(x, w, s, z, backend="metal")
    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        qo.groupwise_dequant(w, s, z, bits=3)


def test_ci_safe_mode_routes_to_reference(monkeypatch):
    rng = np.random.default_rng(2)
    x, w, s, z, _ = _q4_case(rng)
    monkeypatch.setenv("MLX_METAL_CI_SAFE_MODE", "1")
    got = qo.q4_matvec_decode(x, w, s, z, backend="metal")  # host tensors: only the reference path can run
    ref = qo.reference_q4_matvec_decode(x, w, s, z)
    assert torch.equal(got, ref)


def test_gqa_head_validation():
    with pytest.raises(ValueError):
        gqa.validate_gqa_heads(6, 4)
    assert gqa.gqa_group_size(32, 8) == 4
    assert [gqa.q_head_to_kv_head(h, 32, 8) for h in (0, 3, 4, 31)] == [0, 0, 1, 7]


def test_quantized_kv_config_validation():
    with pytest.raises(ValueError):
        pq.PagedQuantizedKVConfig(bits=3).validate()
    with pytest.raises(NotImplementedError):
        pq.PagedQuantizedKVConfig(bits=8, symmetric=False).validate()
    with pytest.raises(NotImplementedError):
        pq.PagedQuantizedKVConfig(bits=8, with_zeros=True).validate()
    with pytest.raises(ValueError, match="layout"):
        pq.PagedQuantizedKVConfig(layout="contiguous").validate()


# ------------------------------------------------------------------ reference backends vs oracle


def test_reference_pack_and_dequant_bit_exact():
    assert qo.pack_q4(torch.tensor([[1, 2]], dtype=torch.uint8)).tolist() == [[0x21]]
    assert qo.pack_q4(torch.tensor([[15, 0, 3]], dtype=torch.uint8)).tolist() == [[0x0F, 0x03]]
    rng = np.random.default_rng(3)
    x, w, s, z, codes = _q4_case(rng, N=16, K=96, g=32)
    got = qo.reference_dequant_q4(w, s, z, group_size=32).numpy()
    assert np.array_equal(got.view(np.uint16), oq.dequant_q4(w.numpy(), s.numpy(), z.numpy(), 32).view(np.uint16))
    q8 = rng.integers(0, 256, size=(16, 96), dtype=np.uint8)
    s8 = (rng.random((16, 3)) * 0.05).astype(np.float32)
    got8 = qo.reference_dequant_q8(torch.from_numpy(q8), torch.from_numpy(s8), None, group_size=32).numpy()
    assert np.array_equal(got8.view(np.uint16), oq.dequant_q8(q8, s8, None, 32).view(np.uint16))


@pytest.mark.parametrize("bits", [4, 8])
def test_reference_matvec_matches_oracle(bits):
    rng = np.random.default_rng(4 + bits)
    N, K, g = 64, 256, 64
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    codes, scales = oq.quantize_weight_groupwise(W, bits, g)
    zeros = np.full(scales.shape, 8.0 if bits == 4 else 128.0, np.float32)
    x = rng.standard_normal((3, K)).astype(np.float16)
    fn = qo.reference_q4_matvec_decode if bits == 4 else qo.reference_q8_matvec_decode
    got = fn(torch.from_numpy(x), torch.from_numpy(codes), torch.from_numpy(scales.astype(np.float32)),
             torch.from_numpy(zeros), group_size=g)
    ref = (oq.q4_matvec if bits == 4 else oq.q8_matvec)(x, codes, scales.astype(np.float32), zeros, g)
    assert_close(got.float().numpy(), ref.astype(np.float32), what=f"reference q{bits} matvec")


def test_reference_paged_ops_match_oracle():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, D, P, mb = 3, 8, 2, 64, 16, 4
    NP = B * mb
    Kp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    lengths = np.array([1, 37, 64], np.int32)
    pos = np.array([0, 17, 63], np.int32)
    t = torch.from_numpy
    page, off = pk.reference_block_table_lookup(t(bt), t(pos), P)
    rp, ro = op.block_table_lookup(bt, pos, P)
    assert np.array_equal(page.numpy(), rp) and np.array_equal(off.numpy(), ro)
    kn = rng.standard_normal((B, 1, Hkv, D)).astype(np.float16)
    vn = rng.standard_normal((B, 1, Hkv, D)).astype(np.float16)
    K2, V2 = pk.reference_paged_kv_cache_update(t(Kp), t(Vp), t(kn), t(vn), t(bt), t(pos))
    RK, RV = op.paged_kv_update(Kp, Vp, kn, vn, bt, pos)
    assert np.array_equal(K2.numpy(), RK) and np.array_equal(V2.numpy(), RV)
    q = rng.standard_normal((B, 1, Hq, D)).astype(np.float16)
    got = gqa.reference_paged_gqa_decode_attention(t(q), t(Kp), t(Vp), t(bt), t(lengths))
    ref = op.paged_attention(q[:, 0], Kp, Vp, bt, lengths)
    assert_close(got[:, 0].float().numpy(), ref, what="reference paged GQA attention")


@pytest.mark.parametrize("bits", [4, 8])
def test_host_quantize_kv_pages_bit_exact(bits):
    rng = np.random.default_rng(20 + bits)
    NP, P, Hkv, D, g = 3, 4, 2, 96, 32
    Kp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    bt = torch.arange(NP, dtype=torch.int32).reshape(1, NP)
    cfg = pq.PagedQuantizedKVConfig(bits=bits, page_size=P, group_size=g)
    c = pq.quantize_kv_pages(torch.from_numpy(Kp), torch.from_numpy(Vp), bt, torch.tensor([NP * P]), cfg)
    kq, vq, ks, vs = op.quantize_pages(Kp, Vp, g, bits)
    assert np.array_equal(c.k_pages_q.numpy(), kq) and np.array_equal(c.v_pages_q.numpy(), vq)
    assert np.array_equal(c.k_scales.numpy().view(np.uint16), ks.view(np.uint16))
    assert np.array_equal(c.v_scales.numpy().view(np.uint16), vs.view(np.uint16))
    # byte accounting (tests/test_paged_quantized_kv_memory.py of the reference)
    cr = c.compression_ratio(2)
    assert 1.0 < cr < 10.0
    expect = sum(a.numel() * a.element_size() for a in (c.k_pages_q, c.v_pages_q, c.k_scales, c.v_scales, bt,
                                                         c.lengths))
    assert c.memory_bytes() == expect


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_layout_checked_before_launch(bits):
    # metadata that overstates pages / page size / Hkv, or codes and scales in
    # another layout, must raise ValueError on the host before any pointer is
    # handed to a kernel (host tensors: reaching require_device would raise a
    # different ValueError, about the device).
    import dataclasses

    NP, P, Hkv, D, g, B, Hq = 4, 4, 2, 64, 32, 2, 4
    Kp = torch.randn(NP, P, Hkv, D).to(torch.float16)
    cfg = pq.PagedQuantizedKVConfig(bits=bits, page_size=P, group_size=g)
    bt = torch.arange(NP, dtype=torch.int32).reshape(B, NP // B)
    c = pq.quantize_kv_pages(Kp, Kp.clone(), bt, torch.tensor([5, 8], dtype=torch.int32), cfg)
    q = torch.randn(B, 1, Hq, D).to(torch.float16)
    backend = f"metal_q{bits}"
    other = 4 if bits == 8 else 8
    cases = {
        "page_size": dataclasses.replace(c, page_size=2 * P, original_page_shape=(NP, 2 * P, Hkv, D)),
        "Hkv": dataclasses.replace(c, original_page_shape=(NP, P, 2 * Hkv, D)),
        "group": dataclasses.replace(c, group_size=g // 2),
        "codes": dataclasses.replace(c, k_pages_q=c.k_pages_q[..., : c.k_pages_q.shape[-1] // 2].contiguous(),
                                     v_pages_q=c.v_pages_q[..., : c.v_pages_q.shape[-1] // 2].contiguous()),
        "pages": dataclasses.replace(c, k_scales=c.k_scales[:2].contiguous(), v_scales=c.v_scales[:2].contiguous()),
    }
    for what, bad in cases.items():
        with pytest.raises(ValueError, match="must have shape|disagrees|must be"):
            pq.paged_quantized_kv_gqa_decode_attention(q, bad, backend=backend)
    # the layout check also guards the in-place new-token write
    qkv = torch.randn(B, (Hq + 2 * Hkv) * D).to(torch.float16)
    cos = torch.ones(16, D // 2)
    sin = torch.zeros(16, D // 2)
    for what, bad in cases.items():
        if what == "Hkv":
            continue  # original_page_shape check of the update names (Hkv, D) itself
        with pytest.raises(ValueError):
            pq.paged_quantized_kv_update_from_qkv(qkv, bad, cos, sin, [0, 1], num_attention_heads=Hq,
                                                  num_key_value_heads=Hkv, head_dim=D)
    # a cache tagged with the other bit width is caught too
    with pytest.raises(ValueError):
        pq.paged_quantized_kv_gqa_decode_attention(q, dataclasses.replace(c, bits=other), backend=f"metal_q{other}")


def test_q4_packed_shape_odd_d():
    Kp = torch.randn(2, 4, 2, 17).to(torch.float16)
    cfg = pq.PagedQuantizedKVConfig(bits=4, page_size=4, group_size=32)
    c = pq.quantize_kv_pages(Kp, Kp.clone(), torch.arange(2, dtype=torch.int32).reshape(1, 2),
                             torch.tensor([8]), cfg)
    assert tuple(c.k_pages_q.shape) == (2, 4, 2, 9)
    assert tuple(c.k_scales.shape) == (2, 4, 2, 1)


def test_ctypes_pointer_helper():
    assert _lib.ptr(None) is None
    t = torch.zeros(4)
    assert _lib.ptr(t) == t.data_ptr()
    assert isinstance(ctypes.c_void_p(_lib.ptr(t)).value, int)


# ------------------------------------------------------------------ weight quantizer (host paths)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k,g", [(8, 64, 32), (5, 67, 64), (3, 33, 7), (4, 4096, 64)])
def test_weight_quantizer_reference_backend_matches_oracle(bits, n, k, g):
    import mk.quantize_weights as qw

    rng = np.random.default_rng(bits * 1000 + k + g)
    W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    W[0, :g] = 0.0  # an all-zero group: scale = eps
    r = qw.quantize_weight_groupwise(torch.from_numpy(W), qw.QuantizationConfig(bits=bits, group_size=g,
                                                                                 dtype="float32"),
                                     backend="reference")
    p, s = oq.quantize_weight_groupwise(W, bits, g)
    assert np.array_equal(r.packed_weight.numpy(), p)
    assert np.array_equal(r.scales.numpy().view(np.uint32), s.view(np.uint32))
    assert r.zeros is None and r.original_shape == (n, k)
    assert torch.all(r.kernel_zeros() == (8.0 if bits == 4 else 128.0))


def test_weight_quantizer_validation():
    import mk.quantize_weights as qw

    with pytest.raises(ValueError, match="bits must be 4 or 8"):
        qw.QuantizationConfig(bits=3).validate()
    with pytest.raises(ValueError, match="dtype must be one of"):
        qw.QuantizationConfig(dtype="int8").validate()
    with pytest.raises(NotImplementedError):
        qw.quantize_weight_groupwise(torch.zeros(2, 4), qw.QuantizationConfig(symmetric=False))
    with pytest.raises(ValueError, match="rank-2"):
        qw.quantize_weight_groupwise(torch.zeros(4), qw.QuantizationConfig())
    with pytest.raises(ValueError, match="ROCm device"):
        qw.quantize_weight_groupwise(torch.zeros(2, 64), qw.QuantizationConfig())


def test_loader_rejects_another_abi_version(monkeypatch):
    """A library built for another ABI version fails at load, not at a call."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", _lib.ABI_VERSION + 1)
    with pytest.raises(_lib.NativeLibraryError, match="ABI version"):
        _lib.load()

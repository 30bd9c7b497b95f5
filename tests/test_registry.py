"""Backend registry and autotune store (CPU).

Mirrors tests/test_backend_registry.py and tests/test_autotune_ops.py of the
reference for the ops this package registers.
"""

import json

import pytest

import mk.autotune_ops as at
import mk.backend_registry as reg


def test_list_ops_covers_the_hot_path():
    ops = reg.list_ops()
    for name in ("paged_decode_attention", "paged_gqa_decode_attention", "q4_matvec_decode", "q8_matvec_decode",
                 "quantized_mlp_block", "paged_quantized_kv_decode_attention"):
        assert name in ops
    assert ops == sorted(ops)


def test_candidates_reference_and_validate():
    assert reg.get_candidate_backends("q4_matvec_decode") == ["metal", "metal_parallel", "metal_tiled"]
    assert reg.get_reference_backend("q4_matvec_decode") == "reference"
    assert reg.validate_backend("q4_matvec_decode", "reference") == "reference"
    assert reg.validate_backend("q4_matvec_decode", "metal_tiled") == "metal_tiled"
    with pytest.raises(ValueError, match="Unsupported backend"):
        reg.validate_backend("q4_matvec_decode", "not_a_backend")
    with pytest.raises(KeyError, match="Unknown op"):
        reg.get_candidate_backends("fast_attention")


def test_registry_entry_is_a_copy():
    e = reg.get_registry_entry("quantized_mlp_block")
    e["candidate_backends"].append("x")
    assert "x" not in reg.get_candidate_backends("quantized_mlp_block")
    # every registered function resolves to a real attribute of this package
    import importlib

    for op in reg.list_ops():
        mod, fn = reg.get_registry_entry(op)["function"].rsplit(".", 1)
        assert callable(getattr(importlib.import_module(mod), fn))


def test_experimental_flags():
    assert reg.is_experimental_backend("metal_tiled")
    assert reg.is_experimental_backend("fused_experimental")
    assert not reg.is_experimental_backend("metal")


def test_filter_d64_d128():
    b = ["metal", "metal_d64", "metal_d128"]
    assert reg.filter_backends_for_shape("paged_decode_attention", {"D": 64}, "float16", b) == ["metal", "metal_d64"]
    assert reg.filter_backends_for_shape("paged_decode_attention", {"D": 128}, "float16", b) == ["metal", "metal_d128"]


def test_filter_quantized_mlp_fused_experimental():
    b = ["reference", "tiled", "fused_experimental"]
    assert "fused_experimental" in reg.filter_backends_for_shape("quantized_mlp_block", {"bits": 4}, "float16", b)
    assert "fused_experimental" not in reg.filter_backends_for_shape("quantized_mlp_block", {"bits": 4}, "bfloat16", b)
    assert "fused_experimental" not in reg.filter_backends_for_shape("quantized_mlp_block", {"bits": 3}, "float16", b)


def test_filter_paged_quantized():
    b = ["reference", "metal_q8", "metal_q4"]
    shp = {"Hq": 32, "Hkv": 8, "D": 128}
    assert reg.filter_backends_for_shape("paged_quantized_kv_decode_attention", {**shp, "bits": 8}, "float16", b) == [
        "reference", "metal_q8"]
    assert reg.filter_backends_for_shape("paged_quantized_kv_decode_attention", {**shp, "bits": 4}, "float16", b) == [
        "reference", "metal_q4"]
    bad = {"Hq": 6, "Hkv": 4, "D": 128}
    assert reg.filter_backends_for_shape("paged_quantized_kv_decode_attention", bad, "float16", b) == ["reference"]
    big = {"Hq": 8, "Hkv": 8, "D": 256}
    assert reg.filter_backends_for_shape("paged_quantized_kv_decode_attention", big, "float16", b) == ["reference"]
    with pytest.raises(ValueError):
        reg.filter_backends_for_shape("paged_quantized_kv_decode_attention", shp, "float16", ["metal"])


def test_filter_paged_gqa_heads():
    b = ["reference", "metal"]
    assert reg.filter_backends_for_shape("paged_gqa_decode_attention", {"Hq": 32, "Hkv": 8}, "float16", b) == b
    assert reg.filter_backends_for_shape("paged_gqa_decode_attention", {"Hq": 3, "Hkv": 2}, "float16", b) == [
        "reference"]


# ------------------------------------------------------------------ autotune store


def test_tuning_key_is_deterministic_and_order_free():
    shape = {"B": 1, "D": 64, "H": 8}
    extra = {"length": 128, "group_size": 32}
    k1 = at.make_tuning_key("paged_decode_attention", shape, "float16", extra=extra)
    k2 = at.make_tuning_key("paged_decode_attention", dict(reversed(list(shape.items()))), "float16",
                            extra=dict(reversed(list(extra.items()))))
    assert k1 == k2
    payload = json.loads(k1)
    assert payload["system"]["gpu_arch"] == "gfx950"
    assert list(payload["shape"]) == sorted(shape)


def test_dtype_normalisation():
    import torch

    k1 = at.make_tuning_key("q4_matvec_decode", {"N": 1}, torch.float16)
    k2 = at.make_tuning_key("q4_matvec_decode", {"N": 1}, "float16")
    assert k1 == k2


def test_save_load_roundtrip_and_bare_mapping(tmp_path):
    p = tmp_path / "a.json"
    payload = {"version": 1, "entries": {"k": {"best_backend": "metal"}}}
    at.save_autotune_results(payload, path=p)
    assert at.load_autotune_results(path=p) == payload
    p.write_text(json.dumps({"k": {"best_backend": "metal"}}))
    assert at.load_autotune_results(path=p) == payload
    assert at.load_autotune_results(path=tmp_path / "missing.json") == {"version": 1, "entries": {}}


def test_record_and_lookup(tmp_path):
    p = tmp_path / "a.json"
    shape = {"B": 1, "MAX_S": 128, "H": 8, "D": 64, "length": 128}
    e = at.record_best_backend("paged_decode_attention", shape, "float16", "metal_threadgroup",
                               {"metal_threadgroup": {"mean_ms": 1.2}, "metal": {"mean_ms": 1.5}}, path=p,
                               extra={"length": 128})
    assert e["status"] == "ok" and e["timings"]["metal"]["mean_ms"] == 1.5
    assert at.lookup_best_backend("paged_decode_attention", shape, "float16", path=p,
                                  extra={"length": 128}) == "metal_threadgroup"
    with pytest.raises(KeyError):
        at.lookup_best_backend("paged_decode_attention", shape, "float16", path=p)  # extra differs
    # a bare figure is stored under the winner's name
    e2 = at.record_best_backend("q4_matvec_decode", {"N": 1}, "float16", "metal", 0.5, path=p)
    assert e2["timings"] == {"metal": 0.5}


def test_select_prefers_saved_then_caller_default_then_builtin(tmp_path):
    p = tmp_path / "a.json"
    shape = {"B": 1, "K": 4096, "N": 4096, "group_size": 64}
    assert at.select_backend("q4_matvec_decode", shape, "float16", path=p) == "metal_parallel"
    assert at.select_backend("q4_matvec_decode", shape, "float16", path=p, default_backend="metal") == "metal"
    at.record_best_backend("q4_matvec_decode", shape, "float16", "metal_tiled", {"metal_tiled": {"mean_ms": 0.1}},
                           path=p)
    assert at.select_backend("q4_matvec_decode", shape, "float16", path=p) == "metal_tiled"
    with pytest.raises(KeyError, match="No conservative default"):
        at.select_backend("paged_quantized_kv_decode_attention", shape, "float16", path=p)


def test_select_require_tuned_raises(tmp_path):
    with pytest.raises(KeyError, match="No saved autotune backend"):
        at.select_backend("q4_matvec_decode", {"B": 1}, "float16", path=tmp_path / "m.json", require_tuned=True)


def test_explain_backend_choice(tmp_path):
    p = tmp_path / "a.json"
    shape = {"B": 1, "K": 512, "N": 512, "group_size": 32}
    assert "conservative default" in at.explain_backend_choice("q4_matvec_decode", shape, "float16", path=p)
    at.record_best_backend("q4_matvec_decode", shape, "float16", "metal_tiled", {"metal_tiled": {"mean_ms": 0.5}},
                           path=p, extra={"bits": 4})
    assert "autotuned backend" in at.explain_backend_choice("q4_matvec_decode", shape, "float16", path=p,
                                                            extra={"bits": 4})
    with pytest.raises(KeyError):
        at.explain_backend_choice("q4_matvec_decode", {"B": 9}, "float16", path=p, require_tuned=True)

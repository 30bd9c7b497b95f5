"""Host side of the speculative verify drop-in (ops/speculative_verify_ops.py):
config and result rules, acceptance helpers (models/speculative_decoding.py:
163-228, with the reference tests' cases), the torch reference verify
attention against the oracle, and the row tables the HIP path uses.  No GPU."""

import numpy as np
import pytest
import torch

import mk.speculative_verify_ops as sv
from oracle import paged as op
from tests._data import assert_close


def test_config_validation_and_dict():
    cfg = sv.ParallelVerificationConfig().validate()
    assert cfg.to_dict() == {"draft_length": 4, "mode": "greedy_exact", "backend_preset": "fused_experimental",
                             "cache_layout": "contiguous", "use_prefill_for_draft": True, "return_logits": True,
                             "commit_cache": False}
    sv.ParallelVerificationConfig(cache_layout="paged").validate()
    with pytest.raises(ValueError, match="draft_length must be positive"):
        sv.ParallelVerificationConfig(draft_length=0).validate()
    with pytest.raises(ValueError, match="mode must be 'greedy_exact'"):
        sv.ParallelVerificationConfig(mode="sample").validate()
    with pytest.raises(NotImplementedError, match="cache_layout"):
        sv.ParallelVerificationConfig(cache_layout="ring").validate()


def test_accept_mask_prefix_and_replacement():
    # exact matching stops at the first mismatch; later matches do not count
    assert sv.compute_accept_mask([1, 2, 3, 4], [1, 2, 9, 4]) == [True, True, False, False]
    assert sv.compute_accept_mask([1, 2, 3, 4], [1, 2, 9, 4], require_exact_match=False) == [True, True, False, True]
    assert sv.compute_accept_mask([5, 6], [5]) == [True, False]  # missing targets reject
    assert sv.compute_accept_mask([], [1]) == []
    assert sv.accepted_prefix_length([True, True, False, True]) == 2
    vr = sv.verify_draft_tokens([1, 2, 3], [1, 7, 8])
    assert (vr.accepted_count, vr.rejected_count, vr.replacement_token_id) == (1, 2, 7)
    assert vr.all_committed_tokens() == [1, 7] and vr.rejected_tokens() == [2, 3]
    full = sv.verify_draft_tokens([1, 2], [1, 2])
    assert full.replacement_token_id is None and full.all_committed_tokens() == [1, 2]
    res = sv.ParallelVerificationPassResult([1, 2, 3], [1, 7, 8], [True, False, False], 1, replacement_token_id=7)
    assert res.accepted_tokens() == [1] and res.committed_tokens() == [1, 7]
    assert res.to_verification_result().accepted_count == 1
    empty = sv.parallel_verify_tokens(context_token_ids=[1], proposed_token_ids=[])
    assert empty.accepted_count == 0 and empty.metadata["verification_path"] == "no_proposed_tokens"
    with pytest.raises(ValueError, match="stack_cache is required"):
        sv.parallel_verify_tokens(context_token_ids=[1], proposed_token_ids=[3])


def test_target_tokens_first_maximum():
    lg = [np.array([0.0, 3.0, 3.0, 1.0]), torch.tensor([[2.0, -1.0]])]
    assert sv.target_tokens_from_verification_logits(lg, proposed_token_ids=[0, 0]) == [1, 0]
    with pytest.raises(ValueError, match="greedy_exact"):
        sv.target_tokens_from_verification_logits(lg, proposed_token_ids=[0, 0], mode="top_k")


def test_embed_proposed_tokens():
    emb = torch.arange(12, dtype=torch.float32).reshape(6, 2)
    x = sv.embed_proposed_tokens([4, 0, 5], emb)
    assert tuple(x.shape) == (1, 3, 2) and x[0, 0].tolist() == [8.0, 9.0]
    with pytest.raises(NotImplementedError):
        sv.embed_proposed_tokens([1], emb, B=2)
    with pytest.raises(ValueError, match="non-empty"):
        sv.embed_proposed_tokens([], emb)


@pytest.mark.parametrize("W", [1, 3, 5])
def test_reference_verify_attention_matches_oracle(W):
    rng = np.random.default_rng(60 + W)
    B, Hq, Hkv, D, P, mb = 3, 8, 2, 16, 4, 5
    Kp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((B * mb, P, Hkv, D)).astype(np.float16)
    bt = rng.permutation(B * mb).astype(np.int32).reshape(B, mb)
    q = rng.standard_normal((B, W, Hq, D)).astype(np.float16)
    lengths = np.array([20, W + 1, max(1, W - 1)])
    t = torch.from_numpy
    got = sv.paged_verify_attention(t(q), t(Kp), t(Vp), t(bt), t(lengths), backend="reference")
    assert_close(got, op.paged_verify_attention(q, Kp, Vp, bt, lengths), what=f"reference verify W={W}")


def test_rows_cache_repeats_tables_once():
    """The stack verify pass writes row b * W + w through table row b
    (repeated W times); layers that share a block table share one
    repetition."""
    from mk.llama_stack_ops import LlamaStackCache

    bt = torch.tensor([[3, 4], [7, 8]], dtype=torch.int32)
    K = torch.zeros(9, 4, 2, 8, dtype=torch.float16)
    cache = LlamaStackCache([(K, K, bt), (K, K, bt)], "paged", 8, 4)
    rows = sv._rows_cache(cache, 2, 3)
    (_, _, r0), (_, _, r1) = rows.layer_caches
    assert r0.tolist() == [[3, 4]] * 3 + [[7, 8]] * 3
    assert r1 is r0
    assert np.array_equal(r0.numpy()[::3], bt.numpy())  # the attention's per-sequence rows


def test_hip_verify_path_needs_a_device():
    """The HIP verify attention refuses host tensors (no CPU fallback)."""
    q = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    K = torch.zeros(4, 16, 8, 64, dtype=torch.float16)
    bt = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises((RuntimeError, ValueError)):
        sv.paged_verify_attention(q, K, K, bt, 64)


def test_row_mapping_constant_divides_exactly():
    """The verify kernels map a wave's virtual head h0 + j (j < 16) to its row
    without a per-lane division: with x = h0 % W + j < W + 16, x // W is
    (x * ceil(2^16 / W)) >> 16 for every width the entry points accept
    (1..64); the entry points reject W = 65 and up.  Checked here against
    integer division over the whole range; the identity has margin above the
    accepted widths and first fails at W = 257."""
    def ok(W):
        magic = (65536 + W - 1) // W
        return all((x * magic) >> 16 == x // W for x in range(W + 16))

    assert all(ok(W) for W in range(1, 65))
    assert next(W for W in range(65, 1025) if not ok(W)) == 257

"""HIP paged KV plumbing and paged decode attention vs the oracle."""

import math

import numpy as np
import pytest
import torch

import mk.gqa_ops as gqa
import mk.paged_kv_ops as pk
import mk.paged_quantized_kv_ops as pq
from oracle import paged as op
from tests._data import assert_close, to_dev

pytestmark = pytest.mark.gpu


def _case(seed, B, Hq, Hkv, D, P, mb, lengths=None, dtype=np.float16, extra_pages=3):
    rng = np.random.default_rng(seed)
    NP = B * mb + extra_pages
    Kp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float32)
    Vp = rng.standard_normal((NP, P, Hkv, D)).astype(np.float32)
    bt = rng.permutation(NP)[:B * mb].astype(np.int32).reshape(B, mb)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    if lengths is None:
        lengths = rng.integers(1, mb * P + 1, size=B)
    return q, Kp, Vp, bt, np.asarray(lengths, dtype=np.int32)


def _t(a, dev, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(dev)


# ------------------------------------------------------------ lookup / update

def test_block_table_lookup_bit_exact(dev):
    for B, MAX_S, P, pos in ((1, 16, 4, 3), (2, 32, 8, [2, 17]), (16, 8192, 16, None)):
        bt = np.random.default_rng(1).permutation(B * (MAX_S // P)).astype(np.int32).reshape(B, -1)
        if pos is None:
            pos = np.random.default_rng(2).integers(0, MAX_S, size=B).tolist()
        page, off = pk.block_table_lookup(to_dev(bt, dev), pos, P, backend="metal")
        rp, ro = op.block_table_lookup(bt, np.broadcast_to(np.asarray(pos), (B,)), P)
        assert np.array_equal(page.cpu().numpy(), rp) and np.array_equal(off.cpu().numpy(), ro)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,MAX_S,P,H,D,pos", [(1, 16, 4, 2, 16, 3), (2, 32, 8, 4, 32, [2, 17]),
                                               (2, 32, 4, 4, 64, [0, 31]), (16, 8192, 16, 8, 128, None)])
def test_paged_update_bit_exact(dev, dtype, B, MAX_S, P, H, D, pos):
    rng = np.random.default_rng(80)
    NP = B * (MAX_S // P)
    Kp = _t(rng.standard_normal((NP, P, H, D)), dev, dtype)
    Vp = _t(rng.standard_normal((NP, P, H, D)), dev, dtype)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, -1)
    if pos is None:
        pos = rng.integers(0, MAX_S, size=B).tolist()
    k = _t(rng.standard_normal((B, H, D)), dev, dtype)
    v = _t(rng.standard_normal((B, 1, H, D)), dev, dtype)
    K0, V0 = Kp.clone(), Vp.clone()
    K1, V1 = pk.paged_kv_cache_update(Kp, Vp, k, v, to_dev(bt, dev), pos)
    assert K1 is Kp and V1 is Vp  # in place
    rK, rV = op.paged_kv_update(K0.float().cpu().numpy(), V0.float().cpu().numpy(), k.float().cpu().numpy(),
                                v[:, 0].float().cpu().numpy(), bt, np.broadcast_to(np.asarray(pos), (B,)))
    assert np.array_equal(K1.float().cpu().numpy(), rK) and np.array_equal(V1.float().cpu().numpy(), rV)


def test_paged_update_collision_later_b_wins(dev):
    P, H, D = 4, 2, 8
    Kp = torch.zeros((4, P, H, D), dtype=torch.float16, device=dev)
    Vp = torch.zeros_like(Kp)
    bt = torch.tensor([[1, 2], [1, 3], [0, 3]], dtype=torch.int32, device=dev)
    k = torch.arange(3, dtype=torch.float16, device=dev).reshape(3, 1, 1).expand(3, H, D).contiguous() + 1
    pk.paged_kv_cache_update(Kp, Vp, k, k, bt, [2, 2, 6])  # b0, b1 -> (1,2); b2 -> (3,2)
    assert torch.all(Kp[1, 2] == 2) and torch.all(Kp[3, 2] == 3) and int((Kp != 0).sum()) == 2 * H * D


# ------------------------------------------------------------ fp16 paged attention

# The short-context plan runs while B x 32-position blocks per table row x
# units (kv heads x blocks of 16 query heads) is at most SP_MAX_WAVE_BLOCKS,
# or twice that with rows of at most SP_SHORT_ROW_BLOCKS blocks; its arrival
# counters (4 bytes each, 2 x SP_MAX_WAVE_BLOCKS of them) lead the workspace.
SP_MAX_WAVE_BLOCKS = 16384
SP_SHORT_ROW_BLOCKS = 128


def _stream_width(B, units, P, mb):
    """Pages per table row that put a call on the stream plan: rows longer
    than SP_SHORT_ROW_BLOCKS blocks and B x blocks x units past
    SP_MAX_WAVE_BLOCKS."""
    return max(mb, -(-(SP_SHORT_ROW_BLOCKS + 1) * 32 // P), -(-(SP_MAX_WAVE_BLOCKS + 1) * 32 // (B * units * P)) + 1)


def _pad_table(bt, NP, width, seed):
    """The block table widened to ``width`` pages per sequence with random
    valid page ids past the used ones: a wide table moves the attention from
    the short-context plan (laid out from the table width) to the stream
    plan without changing the result."""
    extra = np.random.default_rng(seed).integers(0, NP, size=(bt.shape[0], width - bt.shape[1]))
    return np.concatenate([bt, extra.astype(np.int32)], axis=1)



ATTN_CASES = [
    # (B, Hq, Hkv, D, P, max_blocks)   fast path D in {64,128}; generic otherwise
    (2, 4, 4, 64, 4, 8),
    (2, 4, 2, 128, 8, 6),
    (3, 4, 1, 64, 16, 5),
    (2, 32, 8, 128, 16, 40),
    (1, 8, 8, 128, 16, 300),
    (2, 64, 2, 64, 16, 20),
    (2, 4, 2, 16, 4, 8),
    (2, 2, 1, 96, 8, 6),
    (1, 3, 3, 17 * 2, 4, 4),
    # 12 kv heads: two workgroups per (sequence, split), the second half full
    (3, 24, 12, 128, 16, 30),
    # MQA, 32 query heads on one kv head: two 16-head column blocks
    (2, 32, 1, 64, 32, 12),
    # page size 64: tiles inside pages, splits not page-aligned
    (2, 8, 2, 128, 64, 40),
    # many sequences: the pair scan spans several 64-lane chunks
    (130, 8, 2, 64, 16, 3),
]


@pytest.mark.parametrize("B,Hq,Hkv,D,P,mb", ATTN_CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_gqa_attention(dev, B, Hq, Hkv, D, P, mb, dtype):
    q, Kp, Vp, bt, lengths = _case(B * 100 + D + mb, B, Hq, Hkv, D, P, mb)
    qt, Kt, Vt = _t(q, dev, dtype), _t(Kp, dev, dtype), _t(Vp, dev, dtype)
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(lengths, dev))
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    tol = 1e-2 if dtype == torch.float16 else 3e-2
    assert_close(got[:, 0], ref, rtol=tol, atol=1e-3 if dtype == torch.float16 else 4e-3,
                 what=f"B{B} Hq{Hq} Hkv{Hkv} D{D} P{P}")


@pytest.mark.parametrize("P", [16, 8])
def test_paged_attention_many_short_sequences(dev, P):
    """Pairs of the stream plan that cross many sequences: 70 sequences
    (two 64-lane chunks), most of them a block or less, empty ones between,
    so a pair spans more sequences than the q operands staged per wave."""
    B, Hq, Hkv, D = 70, 8, 2, 128
    mb = 128 // P  # 128 positions per sequence at most
    pattern = [0, 1, 5, 31, 32, 33, 0, 2, 64, 17, 0, 0, 3, 100]
    lengths = [pattern[i % len(pattern)] for i in range(B)]
    lengths[5] = mb * P  # one full-length sequence
    q, Kp, Vp, bt, lengths = _case(77 + P, B, Hq, Hkv, D, P, mb, lengths=lengths)
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got, ref, rtol=1e-2, atol=1e-3, what=f"short sequences P{P}")
    assert torch.all(got[lengths == 0] == 0)


def test_paged_attention_pairs_at_block_cap(dev):
    """A context long enough that equal pairs would exceed the blocks one wave
    can address: the plan adds pairs beyond one round of resident waves."""
    # MQA with 256 query heads: 16 waves per pair, so one round holds few pairs
    B, Hq, Hkv, D, P = 2, 256, 1, 64, 16
    mb = 10000  # 160000 positions per sequence
    q, Kp, Vp, bt, lengths = _case(91, B, Hq, Hkv, D, P, mb, lengths=[mb * P, mb * P - 77])
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got, ref, rtol=1e-2, atol=1e-3, what="long context")


@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("lengths", [[64], [2047], [2048], [2049], [95, 1, 2000], [8191], [8224]])
def test_paged_attention_short_context_split(dev, lengths, wide):
    """Short total contexts.  With the table as wide as the longest sequence
    they take the short-context plan (one, two or three blocks per split,
    one or several workgroups per sequence).  With a wide table they take the
    stream plan, whose pairs shorten (down to two 32-position blocks) so that
    32 of them run; the block totals straddle the points where that minimum
    changes (64 and 256 blocks), and a single pair covering its whole sequence
    is written without the merge."""
    B, Hq, Hkv, D, P = len(lengths), 32, 8, 128, 16
    mb = (max(lengths) + P - 1) // P
    q, Kp, Vp, bt, lengths = _case(31 + sum(lengths), B, Hq, Hkv, D, P, mb, lengths=lengths)
    btw = _pad_table(bt, Kp.shape[0], _stream_width(B, 8, P, mb), 10) if wide else bt
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(btw, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got, ref, rtol=1e-2, atol=1e-3, what=f"short context {lengths.tolist()}")


def test_paged_attention_graph_replays(dev):
    """The one-kernel attention captured in a HIP graph: every replay, with
    eager calls and synchronisations between them, equals the eager result."""
    q, Kp, Vp, bt, lengths = _case(12, 6, 32, 8, 128, 16, 60, lengths=[960, 17, 500, 0, 959, 333])
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    btd, lnd = to_dev(bt, dev), to_dev(lengths, dev)
    run = lambda: gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, btd, lnd)
    st = torch.cuda.Stream(device=qt.device)
    st.wait_stream(torch.cuda.current_stream(qt.device))
    with torch.cuda.stream(st):
        eager = run()
    torch.cuda.current_stream(qt.device).wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        captured = run()
    for i in range(3):
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        _ = run().float().sum().item()  # eager work between replays


def test_paged_attention_edge_lengths(dev):
    q, Kp, Vp, bt, _ = _case(5, 4, 8, 2, 128, 16, 70)
    lengths = np.array([0, 1, 17, 70 * 16], np.int32)
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(lengths, dev))[:, 0]
    assert torch.all(got[0] == 0)
    first = Kt.new_empty((8, 128))
    for h in range(8):
        first[h] = Vt[bt[1, 0], 0, h // 4]
    assert torch.equal(got[1], first)
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got, ref, what="edge lengths")


def test_paged_attention_invalid_pages_skipped(dev):
    q, Kp, Vp, bt, lengths = _case(6, 2, 4, 2, 64, 8, 6, lengths=[48, 40])
    bt = bt.copy()
    bt[0, 2] = -1
    bt[1, 4] = Kp.shape[0] + 5
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got, ref, what="invalid pages")


@pytest.mark.parametrize("backend", ["metal", "metal_threadgroup", "metal_d64", "auto"])
def test_paged_decode_attention_mha(dev, backend):
    q, Kp, Vp, bt, lengths = _case(9, 2, 4, 4, 64, 4, 8)
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = pk.paged_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), lengths.tolist(), backend=backend)
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got[:, 0], ref, what=backend)
    with pytest.raises(ValueError, match="metal_d128"):
        pk.paged_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), lengths.tolist(), backend="metal_d128")


STREAM_CASES = [
    # (B, Hq, Hkv, D, P, used pages, lengths or None)
    (2, 32, 8, 128, 16, 40, None),
    (3, 24, 12, 128, 16, 30, None),
    (2, 32, 1, 64, 32, 12, None),
    (2, 8, 2, 128, 64, 40, None),
    (70, 8, 2, 128, 16, 8, [0, 1, 5, 31, 32, 33, 0, 2, 64, 17, 0, 0, 3, 100] * 5),
]


@pytest.mark.parametrize("B,Hq,Hkv,D,P,mb,lengths", STREAM_CASES)
def test_paged_attention_stream_plan(dev, B, Hq, Hkv, D, P, mb, lengths):
    """Shapes the short-context plan would take, run on the stream plan through
    a block table wide enough (_stream_width)."""
    q, Kp, Vp, bt, lengths = _case(200 + B + D, B, Hq, Hkv, D, P, mb, lengths=lengths)
    units = Hkv * ((Hq // Hkv + 15) // 16)
    width = _stream_width(B, units, P, mb)
    btw = _pad_table(bt, Kp.shape[0], width, 9)
    qt, Kt, Vt = (_t(a, dev, torch.float16) for a in (q, Kp, Vp))
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(btw, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    assert_close(got, ref, rtol=1e-2, atol=1e-3, what=f"stream plan B{B} Hq{Hq} Hkv{Hkv} D{D} P{P}")


def _counters_zero(dev):
    from mk import _lib
    buf = _lib._WORKSPACES[("attention", torch.device(dev).index, torch.cuda.current_stream(dev).cuda_stream)]
    return bool(torch.all(buf[:8 * SP_MAX_WAVE_BLOCKS] == 0).item())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_attention_short_plan_calls_in_a_row(dev, dtype):
    """Short-context plan: sequences spread over several workgroups merge
    through the arrival counters, which every call leaves at zero -- calls in
    a row on one workspace, with other lengths and other shapes between, all
    match the oracle, and the counters read zero after each."""
    cases = [
        (1, 32, 8, 128, 16, 137, [2049]),          # B = 1 decode at ~2k: one block per split
        (1, 32, 8, 128, 16, 137, [2176]),
        (1, 32, 8, 128, 16, 512, [8192]),           # one 8k sequence
        (4, 32, 8, 128, 16, 137, [2049, 33, 2176, 1000]),  # two blocks per split
        (3, 32, 8, 128, 16, 512, [4096, 8192, 31]),  # three blocks per split
        (2, 32, 8, 64, 32, 64, [2048, 1]),
        (16, 32, 8, 128, 16, 137, [2100 - 7 * i for i in range(16)]),  # five blocks per split
        (32, 32, 8, 128, 16, 137, [2112 - 3 * i for i in range(32)]),  # short rows: the wider limit
        (1, 32, 8, 128, 16, 137, [2049]),
    ]
    for i, (B, Hq, Hkv, D, P, mb, lengths) in enumerate(cases):
        q, Kp, Vp, bt, ln = _case(300 + i, B, Hq, Hkv, D, P, mb, lengths=lengths)
        qt, Kt, Vt = (_t(a, dev, dtype) for a in (q, Kp, Vp))
        got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(ln, dev))[:, 0]
        ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(),
                                 bt, ln)
        tol = (1e-2, 1e-3) if dtype == torch.float16 else (3e-2, 4e-3)
        assert_close(got, ref, rtol=tol[0], atol=tol[1], what=f"call {i}: B{B} D{D} lengths {lengths}")
        assert _counters_zero(dev), f"arrival counters left non-zero after call {i}"


@pytest.mark.parametrize("seed", range(12))
def test_paged_attention_random_shapes(dev, seed):
    """Seeded random geometries against the oracle, over both plans: batch,
    GQA group (MHA .. MQA, one or two 16-head blocks), D 64 / 128, page size
    16 / 32 / 64, fp16 / bf16, lengths from 0 to the table's end, and a table
    sometimes much wider than the longest sequence."""
    rng = np.random.default_rng(1000 + seed)
    Hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 8, 32]))
    Hq, D, P = Hkv * G, int(rng.choice([64, 128])), int(rng.choice([16, 32, 64]))
    B = int(rng.integers(1, 12))
    mb = int(rng.integers(1, 2048 // P + 1))
    lengths = rng.integers(0, mb * P + 1, size=B)
    lengths[rng.integers(0, B)] = mb * P
    if seed % 3 == 0:
        lengths[rng.integers(0, B)] = 0
    dtype = torch.float16 if seed % 2 == 0 else torch.bfloat16
    q, Kp, Vp, bt, lengths = _case(2000 + seed, B, Hq, Hkv, D, P, mb, lengths=lengths)
    units = Hkv * ((G + 15) // 16)
    width = _stream_width(B, units, P, mb) if seed % 4 == 1 else mb
    btw = _pad_table(bt, Kp.shape[0], width, 11) if width > mb else bt
    qt, Kt, Vt = _t(q, dev, dtype), _t(Kp, dev, dtype), _t(Vp, dev, dtype)
    print(f"random attention seed {seed}: B={B} Hq={Hq} Hkv={Hkv} D={D} P={P} mb={mb} width={width} {dtype}",
          flush=True)
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(btw, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.float().cpu().numpy(), Vt.float().cpu().numpy(), bt,
                             lengths)
    tol = (1e-2, 1e-3) if dtype == torch.float16 else (3e-2, 4e-3)
    assert_close(got, ref, rtol=tol[0], atol=tol[1], what=f"random seed {seed}")
    assert torch.all(got[lengths == 0] == 0)


def test_config3_full_size(dev):
    """B=16, 32/8 heads, D=128, P=16, lengths U[512,8192],
    permuted block table -- full size against the oracle."""
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D, P, mb = 16, 32, 8, 128, 16, 512
    lengths = rng.integers(512, 8193, size=B).astype(np.int32)
    NP = B * mb
    bt = np.random.default_rng(4).permutation(NP).astype(np.int32).reshape(B, mb)
    Kt = torch.randn((NP, P, Hkv, D), generator=torch.Generator().manual_seed(6)).to(torch.float16).to(dev)
    Vt = torch.randn((NP, P, Hkv, D), generator=torch.Generator().manual_seed(7)).to(torch.float16).to(dev)
    qt = torch.randn((B, Hq, D), generator=torch.Generator().manual_seed(5)).to(torch.float16).to(dev)
    got = gqa.paged_gqa_decode_attention(qt[:, None], Kt, Vt, to_dev(bt, dev), to_dev(lengths, dev))[:, 0]
    ref = op.paged_attention(qt.float().cpu().numpy(), Kt.cpu().numpy(), Vt.cpu().numpy(), bt, lengths)
    assert_close(got, ref, what="config 3")


# ------------------------------------------------------------ fused split + RoPE + update

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,Hq,Hkv,D,P,mb", [(2, 4, 2, 16, 4, 4), (4, 32, 8, 128, 16, 8), (3, 8, 8, 64, 16, 3)])
def test_qkv_rope_update_bit_exact(dev, dtype, B, Hq, Hkv, D, P, mb):
    rng = np.random.default_rng(50 + D)
    NP = B * mb
    Kp = _t(rng.standard_normal((NP, P, Hkv, D)), dev, dtype)
    Vp = _t(rng.standard_normal((NP, P, Hkv, D)), dev, dtype)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = rng.integers(0, mb * P, size=B)
    qkv = _t(rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)), dev, dtype)
    cos, sin = op.rope_tables(mb * P, D, 500000.0)
    K0, V0 = Kp.float().cpu().numpy(), Vp.float().cpu().numpy()
    out, K1, V1 = gqa.paged_gqa_decode_block_from_qkv(
        qkv, Kp, Vp, to_dev(bt, dev), torch.from_numpy(cos), torch.from_numpy(sin), to_dev(pos, dev),
        num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D)
    npdt = np.float16 if dtype == torch.float16 else np.float32
    x = qkv[:, 0].float().cpu().numpy().astype(npdt)
    rq, rK, rV = op.qkv_rope_paged_update(x, cos, sin, pos, bt, K0.astype(npdt), V0.astype(npdt), Hq, Hkv, D)
    if dtype == torch.bfloat16:
        from oracle.quant import round_bf16
        rK = round_bf16(op.qkv_rope_paged_update(x, cos, sin, pos, bt, K0, V0, Hq, Hkv, D)[1])
    assert np.array_equal(K1.float().cpu().numpy(), rK.astype(np.float32))
    assert np.array_equal(V1.float().cpu().numpy(), rV.astype(np.float32))
    ref = op.paged_attention(_rope_q(x, cos, sin, pos, Hq, D, dtype), K1.float().cpu().numpy(),
                             V1.float().cpu().numpy(), bt, pos + 1)
    assert_close(out[:, 0], ref, rtol=1e-2 if dtype == torch.float16 else 3e-2,
                 atol=1e-3 if dtype == torch.float16 else 4e-3, what="block attention")


@pytest.mark.parametrize("D", [128, 64])
def test_qkv_rope_update_collisions_and_skips(dev, D):
    """Batch rows that target one cache slot (the later row's K/V must land)
    -- the vectorised kernel's staged slot table against the oracle's loop
    over b."""
    rng = np.random.default_rng(77 + D)
    B, Hq, Hkv, P, mb = 7, 8, 2, 16, 4
    NP = B * mb
    Kp = _t(rng.standard_normal((NP, P, Hkv, D)), dev, torch.float16)
    Vp = _t(rng.standard_normal((NP, P, Hkv, D)), dev, torch.float16)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = rng.integers(0, mb * P, size=B)
    bt[3] = bt[1]
    pos[3] = pos[1]          # rows 1 and 3 collide: row 3 wins
    bt[5] = bt[2]
    pos[5] = pos[2]
    bt[6] = bt[2]
    pos[6] = pos[2]          # rows 2, 5, 6 collide: row 6 wins
    qkv = _t(rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)), dev, torch.float16)
    cos, sin = op.rope_tables(mb * P, D, 500000.0)
    K0, V0 = Kp.float().cpu().numpy().astype(np.float16), Vp.float().cpu().numpy().astype(np.float16)
    _, K1, V1 = gqa.paged_gqa_decode_block_from_qkv(
        qkv, Kp, Vp, to_dev(bt, dev), torch.from_numpy(cos), torch.from_numpy(sin), to_dev(pos, dev),
        num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D)
    x = qkv[:, 0].cpu().numpy()
    _, rK, rV = op.qkv_rope_paged_update(x, cos, sin, pos, bt, K0, V0, Hq, Hkv, D)
    assert np.array_equal(K1.cpu().numpy(), rK) and np.array_equal(V1.cpu().numpy(), rV)


def _rope_q(x, cos, sin, pos, Hq, D, dtype):
    q = x[:, :Hq * D].reshape(x.shape[0], Hq, D).astype(np.float32)
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    r = op.apply_rope(q, c, s)
    if dtype == torch.float16:
        return r.astype(np.float16).astype(np.float32)
    from oracle.quant import round_bf16
    return round_bf16(r)


# ------------------------------------------------------------ quantized KV

@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("B,Hq,Hkv,D,P,mb,g", [(2, 4, 2, 64, 4, 4, 32), (2, 32, 8, 128, 16, 40, 64),
                                               (2, 32, 8, 64, 16, 40, 64), (2, 4, 1, 16, 4, 4, 16),
                                               (1, 8, 8, 128, 16, 300, 64)])
def test_quantized_attention(dev, bits, B, Hq, Hkv, D, P, mb, g):
    q, Kp, Vp, bt, lengths = _case(70 + D + mb, B, Hq, Hkv, D, P, mb)
    K16, V16 = Kp.astype(np.float16), Vp.astype(np.float16)
    kq, vq, ks, vs = op.quantize_pages(K16, V16, g, bits)
    cache = pq.PagedQuantizedKVCache(k_pages_q=to_dev(kq, dev), v_pages_q=to_dev(vq, dev), k_scales=to_dev(ks, dev),
                                     v_scales=to_dev(vs, dev), block_table=to_dev(bt, dev),
                                     lengths=to_dev(lengths, dev), bits=bits, page_size=P, group_size=g,
                                     original_page_shape=K16.shape)
    qt = _t(q, dev, torch.float16)
    got = pq.paged_quantized_kv_gqa_decode_attention(qt[:, None], cache, backend=f"metal_q{bits}")
    ref = op.quantized_paged_attention(qt.float().cpu().numpy(), kq, vq, ks, vs, bt, lengths, g, bits)
    assert_close(got[:, 0], ref, what=f"q{bits} D{D}")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("amp", [1.0, 1e-3])
def test_quantized_attention_length_one_is_exact_dequant(dev, bits, D, amp):
    """With one position the softmax weight is exactly 1, so each head's
    output is its kv head's dequantized V row: (code - 128|8) * s rounded to
    fp16 once (dequantize_kv_pages, ops/paged_quantized_kv_ops.py:295-341),
    bit for bit -- also for groups of amplitude 1e-3 (fp16 scales below
    2^-10).  Then the same small-amplitude cache at full lengths, at
    tolerance relative to the output's size."""
    B, Hq, Hkv, P, mb, g = 3, 8, 2, 16, 6, 64
    q, Kp, Vp, bt, _ = _case(120 + D + bits, B, Hq, Hkv, D, P, mb)
    K16, V16 = (Kp * amp).astype(np.float16), (Vp * amp).astype(np.float16)
    kq, vq, ks, vs = op.quantize_pages(K16, V16, g, bits)
    lengths = np.ones(B, np.int32)
    cache = pq.PagedQuantizedKVCache(k_pages_q=to_dev(kq, dev), v_pages_q=to_dev(vq, dev), k_scales=to_dev(ks, dev),
                                     v_scales=to_dev(vs, dev), block_table=to_dev(bt, dev),
                                     lengths=to_dev(lengths, dev), bits=bits, page_size=P, group_size=g,
                                     original_page_shape=K16.shape)
    qt = _t(q, dev, torch.float16)
    got = pq.paged_quantized_kv_gqa_decode_attention(qt[:, None], cache, backend=f"metal_q{bits}")[:, 0]
    _, Vd = op.dequantize_pages(kq, vq, ks, vs, g, bits, D)
    want = np.stack([Vd[bt[b, 0], 0][np.arange(Hq) // (Hq // Hkv)] for b in range(B)])
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))
    full = np.full(B, mb * P - 5, np.int32)
    cache.lengths = to_dev(full, dev)
    got = pq.paged_quantized_kv_gqa_decode_attention(qt[:, None], cache, backend=f"metal_q{bits}")[:, 0]
    ref = op.quantized_paged_attention(qt.float().cpu().numpy(), kq, vq, ks, vs, bt, full, g, bits)
    rms = float(np.sqrt(np.mean(ref * ref)))
    assert_close(got.float().cpu().numpy() / rms, ref / rms, what=f"q{bits} D{D} amplitude {amp}")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("D", [128, 64])
def test_config4_full_context(dev, bits, D):
    """B = 8 sequences of 32768 positions, 32/8 heads,
    P = 16, g = 64, q8 / q4 pages quantized on the device (mk_quantize_kv,
    bit-exact against the oracle's quantizer elsewhere), permuted block table.
    At this size the stream plan runs pairs at the 32-block cap (q8 at its
    4-block minimum split) and 32 partials per sequence.  The last sequence
    stops 77 positions short of the table.  The float64 reference is computed
    per sequence over that sequence's pages only, to bound host memory."""
    B, Hq, Hkv, P, g, mb = 8, 32, 8, 16, 64, 2048
    print(f"config 4 full context q{bits} D{D}", flush=True)
    NP = B * mb
    gen = torch.Generator(device=dev).manual_seed(40 + bits + D)
    K = torch.randn((NP, P, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.float16)
    V = torch.randn((NP, P, Hkv, D), generator=gen, device=dev, dtype=torch.float32).to(torch.float16)
    bt = np.random.default_rng(41).permutation(NP).astype(np.int32).reshape(B, mb)
    lengths = np.full(B, mb * P, np.int32)
    lengths[-1] -= 77
    cfg = pq.PagedQuantizedKVConfig(bits=bits, page_size=P, group_size=g)
    cache = pq.quantize_kv_pages(K, V, to_dev(bt, dev), to_dev(lengths, dev), cfg)
    del K, V
    q = torch.randn((B, 1, Hq, D), generator=gen, device=dev, dtype=torch.float32).to(torch.float16)
    got = pq.paged_quantized_kv_gqa_decode_attention(q, cache, backend=f"metal_q{bits}")[:, 0].float().cpu().numpy()
    kq, vq = cache.k_pages_q.cpu().numpy(), cache.v_pages_q.cpu().numpy()
    ks, vs = cache.k_scales.cpu().numpy(), cache.v_scales.cpu().numpy()
    qn = q[:, 0].float().cpu().numpy()
    ident = np.arange(mb, dtype=np.int32)[None]
    for b in range(B):
        pages = bt[b]
        ref = op.quantized_paged_attention(qn[b:b + 1], kq[pages], vq[pages], ks[pages], vs[pages], ident,
                                           lengths[b:b + 1], g, bits)
        assert_close(got[b:b + 1], ref, what=f"config 4 q{bits} D{D} sequence {b}")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("D,g", [(128, 64), (64, 64), (16, 8)])
def test_quantize_pages_matches_oracle(dev, bits, D, g):
    rng = np.random.default_rng(90)
    K = rng.standard_normal((6, 4, 2, D)).astype(np.float16)
    V = rng.standard_normal((6, 4, 2, D)).astype(np.float16)
    bt = np.arange(6, dtype=np.int32).reshape(2, 3)
    c = pq.quantize_kv_pages(to_dev(K, dev), to_dev(V, dev), to_dev(bt, dev), to_dev(np.array([12, 12]), dev),
                             pq.PagedQuantizedKVConfig(bits=bits, page_size=4, group_size=g))
    kq, vq, ks, vs = op.quantize_pages(K, V, g, bits)
    assert np.array_equal(c.k_pages_q.cpu().numpy(), kq) and np.array_equal(c.v_pages_q.cpu().numpy(), vq)
    assert np.array_equal(c.k_scales.cpu().numpy(), ks) and np.array_equal(c.v_scales.cpu().numpy(), vs)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("B,Hq,Hkv,D,P,mb,g", [(2, 4, 2, 64, 4, 4, 32), (8, 32, 8, 128, 16, 8, 64),
                                               (3, 32, 8, 64, 16, 5, 64)])
def test_quantized_fused_update_bit_exact(dev, bits, B, Hq, Hkv, D, P, mb, g):
    rng = np.random.default_rng(95 + D)
    NP = B * mb
    K16 = rng.standard_normal((NP, P, Hkv, D)).astype(np.float16)
    kq, vq, ks, vs = op.quantize_pages(K16, K16[::-1].copy(), g, bits)
    bt = rng.permutation(NP).astype(np.int32).reshape(B, mb)
    pos = rng.integers(0, mb * P, size=B)
    qkv = rng.standard_normal((B, 1, (Hq + 2 * Hkv) * D)).astype(np.float16)
    cos, sin = op.rope_tables(mb * P, D, 500000.0)
    cache = pq.PagedQuantizedKVCache(k_pages_q=to_dev(kq, dev), v_pages_q=to_dev(vq, dev), k_scales=to_dev(ks, dev),
                                     v_scales=to_dev(vs, dev), block_table=to_dev(bt, dev),
                                     lengths=to_dev(pos + 1, dev), bits=bits, page_size=P, group_size=g,
                                     original_page_shape=K16.shape)
    q_out, cache = pq.paged_quantized_kv_update_from_qkv(
        to_dev(qkv, dev), cache, torch.from_numpy(cos), torch.from_numpy(sin), pos.tolist(),
        num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=D)
    rq, rkq, rvq, rks, rvs = op.qkv_rope_paged_update_quant(qkv[:, 0], cos, sin, pos, bt, kq, vq, ks, vs, Hq, Hkv,
                                                            D, g, bits)
    assert np.array_equal(q_out[:, 0].cpu().numpy(), rq)
    assert np.array_equal(cache.k_pages_q.cpu().numpy(), rkq) and np.array_equal(cache.v_pages_q.cpu().numpy(), rvq)
    assert np.array_equal(cache.k_scales.cpu().numpy(), rks) and np.array_equal(cache.v_scales.cpu().numpy(), rvs)
    got = pq.paged_quantized_kv_gqa_decode_attention(q_out, cache, backend=f"metal_q{bits}")
    ref = op.quantized_paged_attention(rq.astype(np.float32), rkq, rvq, rks, rvs, bt, pos + 1, g, bits)
    assert_close(got[:, 0], ref, what="attention after fused write")

"""mk_paged_decode_attention_noalloc (fixed device scratch) against
mk_paged_decode_attention (caller workspace): bit-identical outputs on two
calls in a row, the second smaller, and the size limit rejected before launch."""

import numpy as np
import pytest
import torch

from mk import _lib

pytestmark = pytest.mark.gpu


def _inputs(seed, dev, B, Hq, Hkv, D, P, mb, dtype):
    g = torch.Generator().manual_seed(seed)
    NP = B * mb + 2
    q = torch.randn(B, Hq, D, generator=g).to(dtype).to(dev)
    Kp = torch.randn(NP, P, Hkv, D, generator=g).to(dtype).to(dev)
    Vp = torch.randn(NP, P, Hkv, D, generator=g).to(dtype).to(dev)
    bt = torch.randperm(NP, generator=g)[:B * mb].to(torch.int32).reshape(B, mb).to(dev)
    lengths = torch.randint(1, mb * P + 1, (B,), generator=g).to(torch.int32).to(dev)
    return q, Kp, Vp, bt, lengths


def _both(dev, B, Hq, Hkv, D, P, mb, dtype, seed):
    q, Kp, Vp, bt, lengths = _inputs(seed, dev, B, Hq, Hkv, D, P, mb, dtype)
    NP = Kp.shape[0]
    dt = _lib.dtype_code(dtype)
    scale = float(D) ** -0.5
    print(f"no-alloc case B={B} Hq={Hq} Hkv={Hkv} D={D} P={P} mb={mb} {dtype} seed={seed}", flush=True)
    ref = torch.empty_like(q)
    ws, nbytes = _lib.attention_workspace(dev, B, Hq, Hkv, D, mb, P)
    _lib.launch("mk_paged_decode_attention", dev, q.data_ptr(), Kp.data_ptr(), Vp.data_ptr(), bt.data_ptr(),
                lengths.data_ptr(), ref.data_ptr(), B, Hq, Hkv, D, P, mb, NP, scale, dt,
                None if ws is None else ws.data_ptr(), nbytes)
    out = torch.full_like(q, float("nan"))
    _lib.launch("mk_paged_decode_attention_noalloc", dev, q.data_ptr(), Kp.data_ptr(), Vp.data_ptr(),
                bt.data_ptr(), lengths.data_ptr(), out.data_ptr(), B, Hq, Hkv, D, P, mb, NP, scale, dt)
    torch.cuda.synchronize(dev)
    return ref, out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_matches_workspace_entry_point(dev, dtype):
    # config-3 shape (Hq 32 / Hkv 8 / D 128, P 16) at B 16 x 8192, then a
    # smaller call (B 3, D 64, shorter table) that reuses the same scratch
    for B, Hq, Hkv, D, P, mb, seed in ((16, 32, 8, 128, 16, 512, 1), (3, 8, 2, 64, 16, 40, 2)):
        ref, out = _both(dev, B, Hq, Hkv, D, P, mb, dtype, seed)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (B, D)


def test_noalloc_rejects_oversized_call_before_launch(dev):
    # B 2048 x 512 blocks needs ~300 MiB of partials: status MK_ERR_SCRATCH,
    # nothing launched.  The tensors are still valid for the claimed shape
    # (every table entry names page 0, every length is 1).
    B, Hq, Hkv, D, P, mb = 2048, 32, 8, 128, 16, 512
    assert _lib.workspace_bytes(B, Hq, Hkv, D, mb, P) > (16 << 20)
    q = torch.zeros(B, Hq, D, dtype=torch.float16, device=dev)
    Kp = torch.zeros(1, P, Hkv, D, dtype=torch.float16, device=dev)
    bt = torch.zeros(B, mb, dtype=torch.int32, device=dev)
    lengths = torch.ones(B, dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    lib = _lib.load()
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.mk_paged_decode_attention_noalloc(q.data_ptr(), Kp.data_ptr(), Kp.data_ptr(), bt.data_ptr(),
                                                   lengths.data_ptr(), out.data_ptr(), B, Hq, Hkv, D, P, mb, 1,
                                                   0.1, _lib.DT_F16, stream)
    assert rc == _lib.MK_ERR_SCRATCH
    with pytest.raises(RuntimeError, match="no-allocation scratch"):
        _lib.launch("mk_paged_decode_attention_noalloc", dev, q.data_ptr(), Kp.data_ptr(), Kp.data_ptr(),
                    bt.data_ptr(), lengths.data_ptr(), out.data_ptr(), B, Hq, Hkv, D, P, mb, 1, 0.1, _lib.DT_F16)
    torch.cuda.synchronize(dev)
    assert not torch.any(out != 0)

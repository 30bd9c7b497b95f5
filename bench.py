"""Benchmark of the quantized decode hot path on one MI355X.

Timed workload (the configuration the metric is quoted on):
one q4 quantized-MLP decode step at Llama-3-8B shapes -- hidden 4096,
intermediate 14336, group 64, fp16 scales and zero points, batch M=1:
    residual add + RMSNorm + gate/up q4 matvec + SwiGLU
                                (mk_q4_rmsnorm_gate_up, 2 x 14336x4096, one kernel)
    down q4 matvec + residual   (mk_q4_matvec, 4096x14336)
Each step uses the next of several distinct weight sets (>= 512 MB in total)
so the 256 MB Infinity Cache cannot serve the weights.  The steps are
replayed from HIP graphs holding one pass over the weight sets, so host
launch overhead is not in the timed region.

value = algorithmic HBM bytes of the step (packed codes + fp16 scales/zeros +
activations in/out) / measured step time, in GB/s.  The JSON line also
carries:
  roofline      -- the dominant kernel (norm + q4 gate/up) timed alone with
                   HIP events, against the 8 TB/s HBM peak;
  cpu_baseline  -- the numpy oracle (the reference's array path restated)
                   timed on this host for a bounded sample of the same step;
  extra         -- the q4 GEMVs of the step on their own (gate/up + SwiGLU,
                   down; config 1's 4096x4096 matvec), M=4/8/32 and q8
                   variants, paged GQA decode attention at
                   BASELINE config 3 and at short contexts, config 4 (q8/q4
                   KV), the speculative-verify attention at config-3 geometry
                   (W = 2/4/8 rows, MFMA TFLOP/s beside HBM GB/s) and the
                   config-5 decode stack (tok/s and HBM fraction).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-metal-kernels_amd"))

PEAK_GBS = 8000.0
HIDDEN, INTER, GROUP = 4096, 14336, 64
DOMINANT_KERNEL = "gemv_dot_kernel<4, 2, 2, true, 1, 4>"  # residual + RMSNorm + q4 gate/up + SwiGLU, M = 1
COPY_KERNEL_HINT = "copy"                      # torch's device-to-device copy kernel
TRAFFIC_SUMMARY = "gemv_dot_q4_rmsnorm_gate_up_M1_traffic.json"
ATTN_TRAFFIC_SUMMARY = "paged_attn_config3_fp16_traffic.json"


WORKLOADS = ("config3", "attn_short", "config4", "verify", "gemv", "mlp_m4", "mlp_m8", "mlp_m32", "mlp_q8", "stack")
PEAK_MFMA_F16_TFLOPS = 2500.0  # dense fp16 MFMA peak of MI355X


def _parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--sets", type=int, default=6, help="distinct weight sets rotated through (>= 512 MB total)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the M=4/8, q8 and attention extras")
    ap.add_argument("--decode-stack-only", action="store_true",
                    help="run only the config-5 decode stack extra and print its JSON (same as --workload stack)")
    ap.add_argument("--workload", choices=WORKLOADS, default=None,
                    help="run one workload alone and print its JSON (for profiling): config3 (paged fp16 "
                         "attention), attn_short (fp16 attention at B=1 2k / 8k and B=4 2k), config4 (q8/q4 KV "
                         "attention), gemv (config 2's q4 gate/up + SwiGLU and down GEMVs and config 1's "
                         "matvec, M=1, without the block's norm and residual), mlp_m4 / mlp_m8 / mlp_m32 "
                         "(batched q4 MLP steps), mlp_q8 (q8 MLP step, M=1), stack (config-5 decode stack)")
    ap.add_argument("--cases", default=None,
                    help="with --workload verify: comma-separated widths (default 2,4,8); with --workload "
                         "attn_short: comma-separated case names (B1_ctx2048, B1_ctx8192, B4_ctx2048)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="first run a plain device copy of this many MiB (counter calibration)")
    ap.add_argument("--summarize-counters", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE run, "
                         "WRITE_SIZE run, both with --calib-copy-mb) into the traffic summary and exit")
    ap.add_argument("--summary-out", default=os.path.join(ROOT, "profiles", TRAFFIC_SUMMARY))
    ap.add_argument("--summary-kernel", default=DOMINANT_KERNEL,
                    help="kernel-name substring the traffic summary is for (default: the MLP front kernel)")
    ap.add_argument("--summary-workload", default="config2 residual+RMSNorm+gate/up 2x14336x4096 q4 g64 M=1")
    ap.add_argument("--summary-grid", type=int, default=0,
                    help="with --summarize-counters: only attention dispatches of this grid size (threads)")
    ap.add_argument("--summary-bytes", type=int, default=0,
                    help="algorithmic bytes per launch of that kernel (default: the MLP front's)")
    ap.add_argument("--summarize-pmc", nargs=4, metavar=("CSV", "OUT_MD", "TITLE", "COMMAND"),
                    help="turn one rocprofv3 --pmc counter_collection.csv (SQ counters) into a markdown "
                         "summary for the kernels named by --summary-kernel (';'-separated substrings) and exit")
    ap.add_argument("--summarize-stats", nargs=4, metavar=("CSV", "OUT_MD", "TITLE", "COMMAND"),
                    help="turn one rocprofv3 --kernel-trace --stats kernel_stats.csv into a markdown table for the "
                         "kernels named by --summary-kernel (';'-separated substrings) and exit")
    return ap.parse_args()


# ----------------------------------------------------------------- inputs


def quantize_on_gpu(W, bits, g):
    """Symmetric groupwise quantization (models/quantize_weights.py:164-203
    semantics) done with torch ops on the device, for synthetic weights."""
    import torch

    N, K = W.shape
    limit = 7 if bits == 4 else 127
    zp = 8 if bits == 4 else 128
    Wg = W.float().reshape(N, K // g, g)
    scale = torch.clamp(Wg.abs().amax(dim=-1) / limit, min=1e-8)
    q = torch.clamp(torch.round(Wg / scale[..., None]), -limit, limit).to(torch.int32) + zp
    q = q.reshape(N, K).to(torch.uint8)
    if bits == 4:
        q = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    s = scale.to(torch.float16).contiguous()
    z = torch.full_like(s, float(zp))
    return q, s, z


def make_mlp_set(dev, bits, seed):
    import torch

    gen = torch.Generator(device=dev).manual_seed(seed)
    mats = []
    for n, k in ((INTER, HIDDEN), (INTER, HIDDEN), (HIDDEN, INTER)):
        W = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * 0.02
        mats.append(quantize_on_gpu(W, bits, GROUP))
        del W
    return mats


def mlp_bytes(M, bits):
    """Algorithmic HBM bytes of one MLP step: front = residual add + RMSNorm +
    gate/up + SwiGLU (codes, scales, zero points; x, residual, norm weight
    read; z, normed, mlp written), down = down projection + residual (codes,
    scales, zero points; mlp and z read, out written)."""
    G_h, G_i = HIDDEN // GROUP, INTER // GROUP
    code = bits / 8
    front = 2 * (INTER * HIDDEN * code + INTER * G_h * 4) + 3 * M * HIDDEN * 2 + 2 * M * HIDDEN * 2 + M * INTER * 2
    down = HIDDEN * INTER * code + HIDDEN * G_i * 4 + M * INTER * 2 + 2 * M * HIDDEN * 2
    return int(front), int(down)


# ----------------------------------------------------------------- timing helpers


def capture(fns):
    """One HIP graph that runs every callable of ``fns`` in order."""
    import torch

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for fn in fns:
            fn()  # warm the allocator outside the graph
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):  # the warm-up stream: its cached workspaces carry over
        for fn in fns:
            fn()
    torch.cuda.synchronize()
    return g


def time_steps(fns, steps, warmup):
    """Run exactly ``steps`` calls of the callables ``fns`` (round-robin)
    after ``warmup`` untimed ones; returns ms per call.

    The calls are replayed from HIP graphs that each hold one pass over all
    of ``fns`` (plus one graph for the remainder), so the host's graph-launch
    cost is paid once per pass, not once per call.  The timed region is
    bracketed by ``torch.cuda.synchronize()`` and HIP events on the stream
    the graphs are launched on."""
    import torch

    n = len(fns)
    full = capture(fns)
    rem = capture(fns[: steps % n]) if steps % n else None
    for _ in range(max(1, -(-warmup // n))):
        full.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps // n):
        full.replay()
    if rem is not None:
        rem.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# ----------------------------------------------------------------- workloads


def mlp_step_fns(sets, M, bits, dev):
    import torch

    import mk.quant_ops as qo

    x = torch.randn((M, 1, HIDDEN), device=dev).to(torch.float16)
    res = torch.randn((M, 1, HIDDEN), device=dev).to(torch.float16)
    nw = torch.ones(HIDDEN, device=dev, dtype=torch.float16)
    outs = {}

    def make(ws):
        (gw, gs, gz), (uw, us, uz), (dw, ds, dz) = ws

        def step():
            z, _, mlp = qo.q_rmsnorm_gate_up_swiglu(x, res, nw, gw, uw, gs, us, gz, uz, bits=bits, group_size=GROUP)
            _, out = qo.q_matvec_residual(mlp, dw, ds, dz, z, bits=bits, group_size=GROUP)
            outs["out"] = out

        def front():
            qo.q_rmsnorm_gate_up_swiglu(x, res, nw, gw, uw, gs, us, gz, uz, bits=bits, group_size=GROUP)

        return step, front

    return [make(ws) for ws in sets], (x, res, nw)


def attention_config3(dev, steps, warmup):
    """B=16, Hq 32 / Hkv 8, D=128, P=16, lengths U[512,8192]
    (seed 3), block table a seeded permutation (seed 4); fp16 K/V ~ N(0,1).
    Rotates two cache copies (>= 256 MB each) to defeat the Infinity Cache."""
    import numpy as np
    import torch

    import mk.gqa_ops as gqa

    B, Hq, Hkv, D, P, mb = 16, 32, 8, 128, 16, 512
    rng = np.random.default_rng(3)
    lengths = rng.integers(512, 8193, size=B).astype(np.int32)
    NP = B * mb
    bt = torch.from_numpy(np.random.default_rng(4).permutation(NP).astype(np.int32).reshape(B, mb)).to(dev)
    ln = torch.from_numpy(lengths).to(dev)
    q = torch.randn((B, 1, Hq, D), device=dev).to(torch.float16)
    caches = []
    for c in range(3):
        Kp = torch.randn((NP, P, Hkv, D), device=dev).to(torch.float16)
        Vp = torch.randn((NP, P, Hkv, D), device=dev).to(torch.float16)
        caches.append((Kp, Vp))
    fns = [lambda K=K, V=V: gqa.paged_gqa_decode_attention(q, K, V, bt, ln) for K, V in caches]
    ms = time_steps(fns, steps, warmup)
    tot = int(lengths.sum())
    nbytes = tot * Hkv * D * 2 * 2 + sum(math.ceil(int(n) / P) for n in lengths) * 4 + B * Hq * D * 2 * 2 + B * 4
    del caches, fns
    torch.cuda.empty_cache()
    achieved = nbytes / (ms * 1e-3) / 1e9
    return {
        "workload": "config3_paged_gqa_fp16_B16_ctx_U512_8192",
        "tokens_per_s": B / (ms * 1e-3),
        "us_per_call": ms * 1e3,
        "kv_tokens": tot,
        "ns_per_kv_token": ms * 1e6 / tot,
        "hbm_gbs": achieved,
        "frac_of_peak": achieved / PEAK_GBS,
        "bytes": nbytes,
        # the call is the split-context kernel plus the partial merge; both
        # run on the stream the graph is launched on and are timed together
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": load_traffic(ATTN_TRAFFIC_SUMMARY),
                     "kernel": "paged_attn_kernel<f16,128,0,false,true> + paged_attn_merge_kernel<f16,128>",
                     "bytes_per_launch": nbytes, "us_per_launch": round(ms * 1e3, 3)},
    }


def attention_short(dev, steps=200, warmup=20, cases=None):
    """Short total contexts (the one-kernel short-context plan): one sequence
    of 2048 and of 8192 positions, and four of ~2k -- Hq 32 / Hkv 8, D=128,
    P=16, fp16 K/V ~ N(0,1), a seeded permuted block table as wide as the
    longest sequence.  Enough cache copies rotate through the calls (>= 256 MB
    in all) that every call reads its K/V from HBM, as a decode step does
    after the other layers' traffic."""
    import numpy as np
    import torch

    import mk.gqa_ops as gqa

    Hq, Hkv, D, P = 32, 8, 128, 16
    out = {}
    for name, lengths in (("B1_ctx2048", [2048]), ("B1_ctx8192", [8192]), ("B4_ctx2048", [2048, 2049, 2100, 2176])):
        if cases and name not in cases:
            continue
        B = len(lengths)
        mb = -(-max(lengths) // P)
        NP = B * mb
        bt = torch.from_numpy(np.random.default_rng(4).permutation(NP).astype(np.int32).reshape(B, mb)).to(dev)
        ln = torch.tensor(lengths, dtype=torch.int32, device=dev)
        q = torch.randn((B, 1, Hq, D), device=dev).to(torch.float16)
        copy_bytes = NP * P * Hkv * D * 2 * 2
        ncopy = max(2, -(-(256 << 20) // copy_bytes))
        caches = [(torch.randn((NP, P, Hkv, D), device=dev).to(torch.float16),
                   torch.randn((NP, P, Hkv, D), device=dev).to(torch.float16)) for _ in range(ncopy)]
        fns = [lambda K=K, V=V: gqa.paged_gqa_decode_attention(q, K, V, bt, ln) for K, V in caches]
        ms = time_steps(fns, max(steps, ncopy), warmup)
        tot = int(sum(lengths))
        nbytes = tot * Hkv * D * 2 * 2 + sum(-(-n // P) for n in lengths) * 4 + B * Hq * D * 2 * 2 + B * 4
        achieved = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_call": round(ms * 1e3, 3), "bytes": nbytes, "hbm_gbs": round(achieved, 1),
                     "frac_of_peak": round(achieved / PEAK_GBS, 4), "cache_copies": ncopy}
        del caches, fns
        torch.cuda.empty_cache()
    return out


def attention_config4(dev, steps=30, warmup=5):
    """paged GQA decode over q8 and q4 KV, B=8 at context
    32768, Hq 32 / Hkv 8, D in (128, 64), P=16, groups of 64 with fp16 scales;
    random codes and scales (the kernel's work does not depend on the values),
    a seeded random block table.  Bytes = the codes and scales of every
    position read."""
    import torch

    import mk.paged_quantized_kv_ops as pq

    B, Hq, Hkv, P, ctx, g = 8, 32, 8, 16, 32768, 64
    mb = ctx // P
    NP = B * mb
    out = {"workload": "config4_paged_gqa_q8_q4_B8_ctx32768_g64"}
    for D in (128, 64):
        for bits in (8, 4):
            cols = D if bits == 8 else D // 2
            nbytes = B * ctx * Hkv * 2 * (cols + (D // g) * 2)
            # a cache smaller than 1.5x the 256 MB Infinity Cache is rotated
            # with further copies, so every call reads its codes from HBM
            ncopy = max(1, -(-(384 << 20) // nbytes))
            gen = torch.Generator(device=dev)
            gen.manual_seed(7)
            bt = torch.randperm(NP, device=dev, generator=gen).to(torch.int32).reshape(B, mb)
            ln = torch.full((B,), ctx, dtype=torch.int32, device=dev)
            caches = []
            for _ in range(ncopy):
                kq = torch.randint(0, 256, (NP, P, Hkv, cols), dtype=torch.uint8, device=dev, generator=gen)
                vq = torch.randint(0, 256, (NP, P, Hkv, cols), dtype=torch.uint8, device=dev, generator=gen)
                ks = (torch.rand((NP, P, Hkv, D // g), device=dev, generator=gen) * 0.2 + 0.05).half()
                vs = (torch.rand((NP, P, Hkv, D // g), device=dev, generator=gen) * 0.2 + 0.05).half()
                caches.append(pq.PagedQuantizedKVCache(k_pages_q=kq, v_pages_q=vq, k_scales=ks, v_scales=vs,
                                                       block_table=bt, lengths=ln, bits=bits, page_size=P,
                                                       group_size=g, original_page_shape=(NP, P, Hkv, D)))
            q = torch.randn((B, 1, Hq, D), device=dev).half()
            fns = [lambda c=c: pq.paged_quantized_kv_gqa_decode_attention(q, c, backend=f"metal_q{bits}")
                   for c in caches]
            ms = time_steps(fns, max(steps, ncopy), warmup)
            out[f"D{D}_q{bits}"] = {"us_per_call": ms * 1e3, "tokens_per_s": B / (ms * 1e-3),
                                   "hbm_gbs": nbytes / (ms * 1e-3) / 1e9,
                                   "frac_of_peak": nbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, "bytes": nbytes,
                                   "cache_copies": ncopy}
            del caches, fns
            torch.cuda.empty_cache()
    return out


def attention_verify(dev, steps=60, warmup=10, widths=(2, 4, 8)):
    """Speculative verify at config-3 geometry: B=16, Hq 32 / Hkv 8, D=128,
    P=16, lengths U[512, 8192] (seed 3, counting the W drafts), W draft
    rows per sequence.  mk_paged_verify_attention reads each K/V byte once
    for the W rows (W * 4 MFMA columns per kv head); for comparison the
    same rows run as B * W sequences of the decode kernel sharing their
    table rows (the KV read W times).  Two cache copies of >= 256 MB rotate.
    Bytes = KV of every position read once + q and out; MFMA work = the
    QK^T and PV products of every row over its visible positions."""
    import numpy as np
    import torch

    import mk.gqa_ops as gqa
    import mk.speculative_verify_ops as sv

    B, Hq, Hkv, D, P, mb = 16, 32, 8, 128, 16, 512
    lengths = np.random.default_rng(3).integers(512, 8193, size=B).astype(np.int32)
    NP = B * mb
    bt = torch.from_numpy(np.random.default_rng(4).permutation(NP).astype(np.int32).reshape(B, mb)).to(dev)
    ln = torch.from_numpy(lengths).to(dev)
    caches = [(torch.randn((NP, P, Hkv, D), device=dev).to(torch.float16),
               torch.randn((NP, P, Hkv, D), device=dev).to(torch.float16)) for _ in range(2)]
    tot = int(lengths.sum())
    out = {"workload": "verify_paged_gqa_fp16_B16_ctx_U512_8192"}
    for W in widths:
        q = torch.randn((B, W, Hq, D), device=dev).to(torch.float16)
        fns = [lambda K=K, V=V: sv.paged_verify_attention(q, K, V, bt, ln) for K, V in caches]
        ms = time_steps(fns, steps, warmup)
        # the W rows as B * W decode sequences (row w: length - (W - 1 - w))
        rows_bt = bt.repeat_interleave(W, dim=0)
        rows_ln = (ln[:, None] - torch.arange(W - 1, -1, -1, device=dev, dtype=torch.int32)[None, :]).reshape(-1)
        q3 = q.reshape(B * W, 1, Hq, D)
        fr = [lambda K=K, V=V: gqa.paged_gqa_decode_attention(q3, K, V, rows_bt, rows_ln) for K, V in caches]
        ms_rows = time_steps(fr, steps, warmup)
        nbytes = tot * Hkv * D * 2 * 2 + sum(-(-int(n) // P) for n in lengths) * 4 + B * W * Hq * D * 2 * 2 + B * 4
        vis = sum(int(n) - (W - 1 - w) for n in lengths for w in range(W))  # positions seen, over all rows
        flops = 4.0 * vis * Hq * D
        gbs = nbytes / (ms * 1e-3) / 1e9
        tfl = flops / (ms * 1e-3) / 1e12
        out[f"W{W}"] = {"us_per_call": round(ms * 1e3, 3), "tokens_per_s": B * W / (ms * 1e-3),
                        "hbm_gbs": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4), "bytes": nbytes,
                        "mfma_tflops": round(tfl, 2), "mfma_frac": round(tfl / PEAK_MFMA_F16_TFLOPS, 5),
                        "rows_as_sequences_us": round(ms_rows * 1e3, 3),
                        "speedup_vs_rows_as_sequences": round(ms_rows / ms, 3)}
        del fns, fr, q, q3, rows_bt, rows_ln
    del caches
    torch.cuda.empty_cache()
    return out


def decode_stack_config5(dev, batches=(1, 32), steps=128, ctx=2048):
    """Llama-3-8B shape (32 layers, hidden 4096, 32/8
    heads of 128, intermediate 14336), every projection and the head q4 g64
    (random N(0, 0.02) weights quantized on the device), paged fp16 KV with
    P=16 pre-filled with N(0, 1) for a 2048-token prompt (prefill is outside
    the hot path), then ``steps`` greedy decode steps, each one HIP graph
    replay.  tok/s = B * steps / wall time of the replays."""
    import torch

    import mk.llama_layer_ops as ll
    import mk.llama_stack_ops as ls

    cfg = ll.llama3_8b_like()
    w = ls.create_random_quantized_llama_stack_weights(cfg, bits=4, group_size=GROUP, device=dev, seed=8)
    cos, sin = ll.build_rope_tables(cfg, device=dev)
    G_h = cfg.hidden_size // GROUP
    layer_bytes = sum(n * k // 2 + n * (k // GROUP) * 4 for n, k in (
        (cfg.qkv_output_dim(), cfg.hidden_size), (cfg.hidden_size, cfg.hidden_size),
        (cfg.intermediate_size, cfg.hidden_size), (cfg.intermediate_size, cfg.hidden_size),
        (cfg.hidden_size, cfg.intermediate_size)))
    head_bytes = cfg.vocab_size * cfg.hidden_size // 2 + cfg.vocab_size * G_h * 4
    out = {"workload": "config5_llama3_8b_q4g64_paged_fp16_ctx2048", "steps": steps,
           "weight_bytes_per_step": cfg.num_hidden_layers * layer_bytes + head_bytes}
    gen = torch.Generator(device=dev)
    gen.manual_seed(9)
    for B in batches:
        cache = ls.init_llama_stack_cache(cfg, B, ctx + steps + 2, cache_layout="paged", dtype=torch.float16,
                                          page_size=16, device=dev)
        for K, V, _ in cache.layer_caches:
            K.normal_(generator=gen)
            V.normal_(generator=gen)
        tokens = torch.randint(0, cfg.vocab_size, (B,), generator=gen, device=dev)
        pos = torch.full((B,), ctx, dtype=torch.int32, device=dev)
        graph = ls.DecodeGraph(w, cache, cos, sin, cfg, tokens, pos)  # one eager step, then the capture
        graph.step()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(steps):
            graph.step()
        ev1.record()
        torch.cuda.synchronize()
        ms = ev0.elapsed_time(ev1) / steps
        kv = B * cfg.num_hidden_layers * (ctx + steps // 2) * cfg.num_key_value_heads * cfg.head_dim * 2 * 2
        step_bytes = out["weight_bytes_per_step"] + kv
        out[f"batch{B}"] = {"tokens_per_s": B / (ms * 1e-3), "ms_per_step": ms,
                            "hbm_gbs": step_bytes / (ms * 1e-3) / 1e9,
                            "frac_of_peak": step_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS}
        del graph, cache
        torch.cuda.empty_cache()
    del w
    torch.cuda.empty_cache()
    return out


# ----------------------------------------------------------------- CPU baseline


def cpu_baseline(sets, x_res_nw, budget_s=20.0):
    """The numpy oracle's MLP step (dequantize to fp16, fp32 matmul -- the
    reference's pure-array path) on this host, one weight set, bounded."""
    import numpy as np

    from oracle import quant as oq

    try:
        from threadpoolctl import threadpool_info

        blas = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:  # noqa: BLE001
        blas = 1
    (gw, gs, gz), (uw, us, uz), (dw, ds, dz) = sets[0]
    cpu = lambda t: t.cpu().numpy()
    g = (cpu(gw), cpu(gs).astype(np.float32), cpu(gz).astype(np.float32))
    u = (cpu(uw), cpu(us).astype(np.float32), cpu(uz).astype(np.float32))
    d = (cpu(dw), cpu(ds).astype(np.float32), cpu(dz).astype(np.float32))
    x, res, nw = (cpu(t) for t in x_res_nw)
    x2, r2 = x.reshape(-1, HIDDEN), res.reshape(-1, HIDDEN)
    oq.mlp_block(x2, r2, nw, g, u, d, bits=4, group_size=GROUP)  # warm
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        oq.mlp_block(x2, r2, nw, g, u, d, bits=4, group_size=GROUP)
        times.append(time.perf_counter() - t0)
        if len(times) >= 20:
            break
    med = sorted(times)[len(times) // 2]
    return med, len(times), blas


def cpu_model():
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo),
    with its family / model / stepping: a hypervisor may shorten the name (to
    "AMD EPYC", say), and those three numbers still name the core."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block is enough
                key, _, val = line.partition(":")
                fields[key.strip().lower()] = val.strip()
    except OSError:
        pass
    name = fields.get("model name")
    if not name:
        import platform

        return platform.processor() or "unknown"
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_other_configs(budget_s=6.0):
    """The oracle on this host for BASELINE configs 1 and 3, bounded samples:
    config 1 = one q4 matvec 4096 x 4096, g64, M=1 (median of up to 10 runs);
    config 3 = paged GQA decode attention (Hq 32 / Hkv 8, D=128, P=16) over
    the first two of config 3's sequences (lengths U[512,8192], seed 3),
    scaled to all 16 by KV tokens."""
    import numpy as np

    from oracle import paged as op
    from oracle import quant as oq

    out = {}
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 16, size=(HIDDEN, HIDDEN // 2), dtype=np.uint8) | \
        (rng.integers(0, 16, size=(HIDDEN, HIDDEN // 2), dtype=np.uint8) << 4)
    sc = rng.uniform(0.002, 0.004, size=(HIDDEN, HIDDEN // GROUP)).astype(np.float16).astype(np.float32)
    z = np.full(sc.shape, 8.0, np.float32)
    x = rng.standard_normal((1, HIDDEN)).astype(np.float16)
    oq.q4_matvec(x, codes, sc, z, GROUP)
    times, t_end = [], time.perf_counter() + budget_s
    while (time.perf_counter() < t_end or len(times) < 2) and len(times) < 10:
        t0 = time.perf_counter()
        oq.q4_matvec(x, codes, sc, z, GROUP)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    nbytes = HIDDEN * HIDDEN // 2 + 2 * HIDDEN * (HIDDEN // GROUP) * 2 + 2 * HIDDEN * 2
    out["config1_q4_matvec_4096x4096_M1"] = {"ms_per_call": med * 1e3, "gbs": nbytes / med / 1e9,
                                             "sample": f"{len(times)} calls, median"}
    lengths = np.random.default_rng(3).integers(512, 8193, size=16)
    Hq, Hkv, D, P = 32, 8, 128, 16
    n = lengths[:2]
    mb = int(np.ceil(n.max() / P))
    Kp = rng.standard_normal((2 * mb, P, Hkv, D)).astype(np.float16)
    Vp = rng.standard_normal((2 * mb, P, Hkv, D)).astype(np.float16)
    bt = np.arange(2 * mb, dtype=np.int32).reshape(2, mb)
    q = rng.standard_normal((2, Hq, D)).astype(np.float16)
    t0 = time.perf_counter()
    op.paged_attention(q, Kp, Vp, bt, n)
    dt = (time.perf_counter() - t0) * float(lengths.sum()) / float(n.sum())
    out["config3_paged_gqa_B16"] = {"ms_per_call": dt * 1e3, "tokens_per_s": 16 / dt,
                                    "sample": f"sequences 0-1 ({int(n.sum())} of {int(lengths.sum())} KV positions), "
                                              "scaled by KV positions"}
    return out


# ----------------------------------------------------------------- counters


def _demangled(name):
    """Kernel names as rocprofv3 writes them, without the anonymous-namespace
    prefix (mangled names are matched as they are)."""
    return name.replace("(anonymous namespace)::", "")


def _counter_rows(path, counter):
    import csv

    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name") == counter:
                rows.append((r.get("Kernel_Name", ""), float(r["Counter_Value"])))
    return rows


READ_REQ_COUNTERS = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum")


def _dispatch_bytes(path, counter, grid=0):
    """(kernel name, bytes) per dispatch: from WRITE_SIZE / FETCH_SIZE (KiB),
    or for reads from the L2->fabric request counts by size
    (32 n32 + 64 n64 + 128 n128; the FETCH_SIZE expression reads 128-byte
    requests through TCC_BUBBLE, which does not always count them).  A
    non-zero ``grid`` keeps only the attention dispatches of that grid size
    (threads), so workloads that launch one kernel at several sizes can be
    told apart."""
    import csv

    per = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            d = per.setdefault(r["Dispatch_Id"], {"kernel": r.get("Kernel_Name", ""),
                                                  "grid": int(r.get("Grid_Size") or 0)})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    out = []
    for d in per.values():
        if grid and d["grid"] != grid and "gemv" not in d["kernel"] and "paged" in d["kernel"]:
            continue
        if counter in d:
            out.append((d["kernel"], d[counter] * 1024.0))
        elif counter == "FETCH_SIZE" and "TCC_EA0_RDREQ_128B_sum" in d:
            n32, n64, n128 = (d.get(c, 0.0) for c in READ_REQ_COUNTERS[1:])
            out.append((d["kernel"], 32 * n32 + 64 * n64 + 128 * n128))
    return out


def summarize_counters(fetch_csv, write_csv, out_path, copy_mb, kernel=DOMINANT_KERNEL, workload=None,
                       algo_bytes=0, grid=0):
    """HBM traffic per launch of ``kernel``: reads from one --pmc pass
    (FETCH_SIZE, or the read-request counts by size), writes from a WRITE_SIZE
    pass.  The plain copy of ``copy_mb`` MiB run by --calib-copy-mb reads and
    writes exactly that many bytes; its reading is reported beside the
    kernel's (``copy_ratio`` = counted / true) as the check of the counter."""
    copy_bytes = copy_mb * (1 << 20)
    out = {"kernel": kernel, "workload": workload, "algorithmic_bytes": None, "copy_bytes": copy_bytes}
    for name, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _dispatch_bytes(path, name, grid)
        dom = [v for k, v in rows if kernel in _demangled(k)]
        # the calibration copy: copy-kernel dispatches whose count is nearest
        # the copy's size
        cop = [v for k, v in rows if COPY_KERNEL_HINT in k.lower() and "gemv" not in k]
        if not dom or not cop:
            raise SystemExit(f"{name}: kernel rows not found in {path}")
        near = min(cop, key=lambda v: abs(math.log(max(v, 1.0) / copy_bytes)))
        per_launch = sum(dom) / len(dom)
        by_size = name == "FETCH_SIZE" and not _has_counter(path, "FETCH_SIZE")
        out[name] = {"source": "TCC_EA0_RDREQ_{32B,64B,128B}_sum" if by_size else name,
                     "dispatches": len(dom), "copy_ratio": round(near / copy_bytes, 4),
                     "bytes_per_launch": int(per_launch)}
    out["traffic_bytes_per_launch"] = out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"]
    algo = algo_bytes or mlp_bytes(1, 4)[0]
    out["algorithmic_bytes"] = algo
    out["traffic_over_algorithmic"] = round(out["traffic_bytes_per_launch"] / algo, 4)
    with open(out_path, "w") as f:
        json.dump(out, f, indent=2)
    print(json.dumps(out))


def _has_counter(path, counter):
    return bool(_counter_rows(path, counter))


SIMDS = 256 * 4          # MI355X: 256 CUs x 4 SIMDs
CLOCK_GHZ = 2.4          # MI355X peak engine clock
VALU_CYCLES = 4          # a wave64 VALU instruction occupies a 16-lane SIMD for 4 cycles


def summarize_pmc(csv_path, kernels, title, command, out_path=""):
    """Markdown summary of SQ counters per dispatch (averaged over dispatches)
    for each kernel-name substring in ``kernels``, with the busy fractions they
    imply: MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x cycles), VALU busy =
    SQ_INSTS_VALU x 4 / (SIMDs x cycles), cycles = dispatch duration x clock."""
    import csv

    per = {}
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            name = _demangled(r["Kernel_Name"])
            key = next((k for k in kernels if k in name), None)
            if key is None:
                continue
            d = per.setdefault(key, {}).setdefault(r["Dispatch_Id"], {"ns": 0})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    lines = [f"# {title}", "", "Command (from the repository root on an MI355X box, ROCm 7.2):", "",
             f"    {command}", "",
             "then, to write this file:", "",
             f"    python3 bench.py --summarize-pmc {csv_path} {out_path} '<title>' '<command>' "
             f"--summary-kernel '{';'.join(kernels)}'", "",
             f"Averages per dispatch; busy fractions over {SIMDS} SIMDs at {CLOCK_GHZ} GHz for the "
             "dispatch's duration (VALU: 4 cycles per wave64 instruction).", ""]
    for key in kernels:
        disp = list(per.get(key, {}).values())
        if not disp:
            raise SystemExit(f"no dispatches of {key!r} in {csv_path}")
        names = sorted({n for d in disp for n in d if n != "ns"})
        avg = {n: sum(d.get(n, 0.0) for d in disp) / len(disp) for n in names}
        ns = sorted(d["ns"] for d in disp)[len(disp) // 2]
        cyc = SIMDS * ns * CLOCK_GHZ
        lines += [f"## `{key}`", "", f"{len(disp)} dispatches, median duration {ns / 1e3:.2f} us", "",
                  "| counter | per dispatch |", "|---|---:|"]
        lines += [f"| {n} | {avg[n]:,.0f} |" for n in names]
        if "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
            lines.append(f"| MFMA busy (derived) | {avg['SQ_VALU_MFMA_BUSY_CYCLES'] / cyc:.3f} |")
        if "SQ_INSTS_VALU" in avg:
            lines.append(f"| VALU busy (derived) | {avg['SQ_INSTS_VALU'] * VALU_CYCLES / cyc:.3f} |")
        if "SQ_WAVES" in avg and "SQ_INSTS_VALU" in avg:
            lines.append(f"| VALU instructions per wave | {avg['SQ_INSTS_VALU'] / avg['SQ_WAVES']:,.0f} |")
        lines.append("")
    return "\n".join(lines)


def summarize_stats(csv_path, kernels, title, command, out_path=""):
    """Markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv,
    restricted to the kernels whose names contain one of ``kernels``."""
    import csv

    lines = [f"# {title}", "", "Command (from the repository root on an MI355X box, ROCm 7.2):", "",
             f"    {command}", "", "then, to write this file:", "",
             f"    python3 bench.py --summarize-stats {csv_path} {out_path} '<title>' '<command>' "
             f"--summary-kernel '{';'.join(kernels)}'", "",
             "| kernel | calls | avg us | min us | max us |", "|---|---:|---:|---:|---:|"]
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            name = _demangled(r["Name"])
            if any(k in name for k in kernels):
                lines.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                             f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} |")
    return "\n".join(lines) + "\n"


def load_traffic(name=TRAFFIC_SUMMARY):
    """Measured HBM bytes per launch from a traffic summary in profiles/, or None."""
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


# ----------------------------------------------------------------- main


def mlp_extra(dev, sets, M, bits, steps, warmup=12):
    """One batched / q8 MLP step (same kernels as the timed step) -> dict."""
    import torch

    s8 = [make_mlp_set(dev, 8, 200 + i) for i in range(4)] if bits == 8 else None
    f8, _ = mlp_step_fns(s8 if bits == 8 else sets, M, bits, dev)
    m_ms = time_steps([step for step, _ in f8], steps, warmup)
    bb = sum(mlp_bytes(M, bits))
    del f8, s8
    torch.cuda.empty_cache()
    return {"us_per_step": m_ms * 1e3, "hbm_gbs": bb / (m_ms * 1e-3) / 1e9,
            "frac_of_peak": bb / (m_ms * 1e-3) / 1e9 / PEAK_GBS, "bytes": bb}


def gemv_extra(dev, sets, steps, warmup=12):
    """Config 2's q4 GEMVs at M = 1 on their own, without the MLP block's
    residual + RMSNorm: the fused gate/up + SwiGLU (2 x 14336 x 4096) and the
    down projection (4096 x 14336), each over the rotating weight sets; and
    config 1's 4096 x 4096 matvec over enough weight copies (~300 MB) that no
    call is served by the Infinity Cache.  Bytes: codes, fp16 scales and zero
    points, x read, y written."""
    import torch

    import mk.quant_ops as qo

    G_h, G_i = HIDDEN // GROUP, INTER // GROUP
    x = torch.randn((1, HIDDEN), device=dev).to(torch.float16)
    m = torch.randn((1, INTER), device=dev).to(torch.float16)
    fns = [lambda ws=ws: qo.q_gate_up_swiglu(x, ws[0][0], ws[1][0], ws[0][1], ws[1][1], ws[0][2], ws[1][2], bits=4,
                                             group_size=GROUP) for ws in sets]
    fns_d = [lambda ws=ws: qo.q4_matvec_decode(m, ws[2][0], ws[2][1], ws[2][2], group_size=GROUP) for ws in sets]
    res = {}
    for name, f, nb in (("gate_up_swiglu", fns, 2 * (INTER * HIDDEN // 2 + INTER * G_h * 4) + HIDDEN * 2 + INTER * 2),
                        ("down", fns_d, HIDDEN * INTER // 2 + HIDDEN * G_i * 4 + INTER * 2 + HIDDEN * 2)):
        ms = time_steps(f, steps, warmup)
        res[name] = {"us_per_call": ms * 1e3, "hbm_gbs": nb / (ms * 1e-3) / 1e9,
                     "frac_of_peak": nb / (ms * 1e-3) / 1e9 / PEAK_GBS, "bytes": nb}
    gen = torch.Generator(device=dev).manual_seed(1)
    c1 = []
    for _ in range(32):
        W = torch.randn((HIDDEN, HIDDEN), generator=gen, device=dev, dtype=torch.float32) * 0.02
        c1.append(quantize_on_gpu(W, 4, GROUP))
        del W
    fns_1 = [lambda w=w: qo.q4_matvec_decode(x, w[0], w[1], w[2], group_size=GROUP) for w in c1]
    b1 = HIDDEN * HIDDEN // 2 + HIDDEN * G_h * 4 + 2 * HIDDEN * 2
    ms = time_steps(fns_1, max(steps, 2 * len(fns_1)), warmup)
    res["config1_4096x4096"] = {"us_per_call": ms * 1e3, "hbm_gbs": b1 / (ms * 1e-3) / 1e9,
                                "frac_of_peak": b1 / (ms * 1e-3) / 1e9 / PEAK_GBS, "bytes": b1}
    del c1, fns, fns_d, fns_1
    torch.cuda.empty_cache()
    return res


def run_workload(name, dev, args):
    """One workload alone (single-workload profiling runs)."""
    if name == "config3":
        return attention_config3(dev, max(50, args.steps // 3), 10)
    if name == "config4":
        return attention_config4(dev)
    if name == "verify":
        widths = tuple(int(w) for w in args.cases.split(",")) if args.cases else (2, 4, 8)
        return attention_verify(dev, widths=widths)
    if name == "attn_short":
        cases = args.cases.split(",") if args.cases else None
        return {"workload": "paged_gqa_fp16_short_contexts", **attention_short(dev, cases=cases)}
    if name == "stack":
        return decode_stack_config5(dev)
    sets = [make_mlp_set(dev, 4, 100 + i) for i in range(args.sets)]
    if name == "gemv":
        return {"workload": "q4_gemv_M1", **gemv_extra(dev, sets, max(60, args.steps // 3))}
    if name == "mlp_q8":
        return {"workload": "q8_mlp_M1", **mlp_extra(dev, sets, 1, 8, max(60, args.steps // 3))}
    M = int(name.split("_m")[1])
    return {"workload": f"q4_mlp_M{M}", **mlp_extra(dev, sets, M, 4, max(60, args.steps // 3))}


def main():
    args = _parse()
    if args.summarize_stats:
        csv_path, out_path, title, command = args.summarize_stats
        text = summarize_stats(csv_path, args.summary_kernel.split(";"), title, command, out_path)
        with open(out_path, "w") as f:
            f.write(text)
        print(text)
        return
    if args.summarize_pmc:
        csv_path, out_path, title, command = args.summarize_pmc
        text = summarize_pmc(csv_path, args.summary_kernel.split(";"), title, command, out_path)
        with open(out_path, "w") as f:
            f.write(text)
        print(text)
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters, args.summary_out, args.calib_copy_mb or 256,
                           kernel=args.summary_kernel, workload=args.summary_workload, algo_bytes=args.summary_bytes,
                           grid=args.summary_grid)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU; multi-GPU runs are not part of it",
                          "requested_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from mk import _lib

    dev = torch.device("cuda:0")
    _lib.load()
    torch.manual_seed(0)
    if args.calib_copy_mb:
        src = torch.empty(args.calib_copy_mb << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.decode_stack_only:
        args.workload = "stack"
    if args.workload:
        print(json.dumps(run_workload(args.workload, dev, args)), flush=True)
        return

    sets = [make_mlp_set(dev, 4, 100 + i) for i in range(args.sets)]
    set_bytes = sum(t.numel() * t.element_size() for ws in sets for m in ws for t in m)
    fns, x_res_nw = mlp_step_fns(sets, 1, 4, dev)
    # timed region: exactly `steps` MLP steps
    ms = time_steps([step for step, _ in fns], args.steps, args.warmup)
    b_front, b_down = mlp_bytes(1, 4)
    step_bytes = b_front + b_down
    value = step_bytes / (ms * 1e-3) / 1e9

    # dominant kernel alone (same stream, HIP events over the timed region)
    ms_front = time_steps([front for _, front in fns], args.steps, args.warmup)
    achieved = b_front / (ms_front * 1e-3) / 1e9

    extra = {}
    if not args.no_extra:
        for bits, M in ((4, 4), (4, 8), (4, 32), (8, 1)):
            extra[f"q{bits}_mlp_M{M}"] = mlp_extra(dev, sets, M, bits, max(60, args.steps // 3))
        extra["q4_gemv_M1"] = gemv_extra(dev, sets, max(60, args.steps // 3))
        torch.cuda.empty_cache()
        extra["paged_attention"] = attention_config3(dev, max(50, args.steps // 3), 10)
        extra["paged_attention_short"] = attention_short(dev)
        extra["quantized_attention"] = attention_config4(dev)
        extra["verify_attention"] = attention_verify(dev)
        extra["decode_stack"] = decode_stack_config5(dev)

    cpu = None
    if not args.no_cpu:
        med, reps, blas = cpu_baseline(sets, x_res_nw)
        cpu = {
            "value": step_bytes / med / 1e9,
            "unit": "GB/s",
            "cores": blas,
            "kind": "port",
            "sample": f"{reps} q4 MLP decode steps (M=1, 4096/14336, g64) of the numpy oracle, median "
                      f"{med * 1e3:.1f} ms/step; BLAS threads {blas}, host cpu_count {os.cpu_count()}",
            "cpu_model": cpu_model(),
            "other_configs": cpu_other_configs(),
        }

    line = {
        "metric": "q4 GEMV HBM GB/s (% of peak) + paged GQA decode tok/s at Llama-3-8B shapes",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (random N(0,0.02) weights quantized q4 g64 on device; random activations)",
        "config": {"workload": "config2_q4_mlp_decode_step_M1", "hidden": HIDDEN, "intermediate": INTER,
                   "group_size": GROUP, "M": 1, "weight_sets": args.sets, "weight_set_bytes_total": set_bytes,
                   "step_bytes": step_bytes, "frac_of_peak": round(value / PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": load_traffic(),
                     "kernel": "gemv_dot_kernel<4,2,2,true,1,4> residual+RMSNorm+q4 gate/up+SwiGLU 2x14336x4096 M=1",
                     "bytes_per_launch": b_front, "us_per_launch": round(ms_front * 1e3, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()

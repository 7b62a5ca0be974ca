#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Default workload (the N=1 `value`): single-layer paged decode at the Qwen3
serving shape -- 256 sequences, 16 query / 8 KV heads, head_dim 128, bf16,
context ~ U[1024, 2047] after the store, KV block 256 with block tables drawn
from one shuffled shared pool.  One step = store one new K/V token per
sequence through the paged append, then attend (flash_attn_with_kvcache with
k=/v=).  `value` is the step's algorithmic HBM bytes (K/V context read once,
q read, output written, new K/V read and stored) divided by the step time,
inputs resident in HBM.

Also reported on the same line:
  roofline      the decode attention launch alone (aac_decode_paged): HIP
                events on the launch stream around back-to-back launches,
                divided by their count (every per-launch figure below is
                timed the same way), against 8 TB/s HBM;
  decode_slot   the same store+attend step through the reference's own cache
                layout (slot caches [256, 2064, 8, 128] picked by
                cache_batch_idx, as model/model.py:233-240 calls it);
  decode_long   long-context GQA-4 decode (64 sequences, 32 query / 8 KV heads,
                context ~ U[16384, 32768]): the split-K decode plus its
                log-sum-exp reduction, HIP events, against 8 TB/s HBM;
  tp2_rank      the decode and prefill kernels at one rank's share of TP=2
                (8 query / 4 KV heads), the shape one GPU runs when the heads
                are split across two (no collective is run or timed);
  kv_transfer   KV export (gather of one 2048-token request's 28 layers from the
                paged cache into one contiguous buffer) and import, against
                8 TB/s; the host-inclusive request export (PCIe) beside it;
  prefill       varlen causal prefill, 8 x 1024 tokens, 16/8 heads, bf16, with
                the paged store in the same call, as TFLOP/s against the
                2.5 PFLOP/s dense bf16 MFMA peak (roofline of that kernel),
                and torch's own flash attention (SDPA, flash backend) on the
                same shape for reference;
  prefill_one_request  one 2048-token request: too few work items for the
                CUs, so each item's key range is split over two workgroups
                (the same call unsplit beside it);
  prefill_long  the same kernel on 8 x 8192 causal tokens: its steady-state
                rate, where per-item start and epilogue costs are small;
  prefill_engine  the prefill call the engine makes for 256 fresh 1024-token
                requests: 256 x 1024 causal tokens with the paged store,
                about 64 work items per CU;
  decode_fp32_small  the fp32 decode of the CPU-runnable case (4 seqs,
                contexts 17/64/200/511) on the GPU, with its host figure;
  e2e           random-init Qwen3-0.6B, 256 requests x 1024 input / 1024
                output tokens under the continuous-batching engine: output
                tok/s (generated tokens / wall clock from submit to the last
                token) and total tok/s (prompt + generated), as
                benchmark_tp.py:93-99 defines them;
  cpu_baseline  the reference's semantics in fp32 torch on the host cores
                (oracle/torch_path.py: index_copy_ store + attention; threads
                = the cores this process may use, capped by OMP_NUM_THREADS),
                3 warm-ups then the median of 5: the decode step of the
                headline workload here, the prefill and long-context decode
                legs' own figures inside them; oracle_1core is the numpy
                float64 oracle on one core.  e2e.cpu_baseline is a complete
                small generation run on the host (oracle/qwen3_ref.py, 8
                requests x 128 in / 32 out); e2e.cpu_decode_step_extrapolated
                one decoder layer's decode step for all 256 sequences times
                28 layers plus lm_head.

`python bench.py --gpus N --steps K --warmup W`; only N=1 is supported (one
GPU), N>1 exits with a message.  Before its timed region every leg runs W
warm-up iterations and then keeps its kernels running back to back for
--warmup-seconds (default 1 s): the GPU's clocks fall while the host prepares
a leg's inputs and climb back only under sustained load (8 x 1024 prefill:
55 us right after an idle spell, 44 us after a few seconds of load), so the
timed region measures the sustained rate a busy server sees.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_PROFILE = "profiles/decode_256seq_ctx1k-2k_bf16_traffic.md"
CACHE_LAYOUT_NOTE = ("K/V caches placed as the engine's PagedKVCache places them "
                     "(paged.alloc_kv_cache: V 512 B past K modulo 1 KiB)")
TRAFFIC_PREFILL = "profiles/prefill_8x1024_bf16_traffic.md"
TRAFFIC_PREFILL_LONG = "profiles/prefill_8x8192_bf16_traffic.md"
TRAFFIC_PREFILL_ENGINE = "profiles/prefill_engine_256x1024_bf16_traffic.md"
TRAFFIC_DECODE_LONG = "profiles/decode_long_64seq_ctx16k-32k_bf16_traffic.md"
TRAFFIC_KV_EXPORT = "profiles/kv_export_2048tok_28layers_bf16_traffic.md"
DEVICE_PROFILE = "profiles/device_mi355x.md"


def measured_traffic(profile=TRAFFIC_PROFILE, key="traffic_bytes_per_launch"):
    """Bytes per launch moved between L2 and memory, from a committed counter
    summary (FETCH_SIZE / WRITE_SIZE scaled by the same counters on a plain
    copy of known size), or None when the summary is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), profile)
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--warmup-seconds", type=float, default=1.0,
                   help="back-to-back warm-up time per leg before its timed region")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--partition", type=int, default=0, help="decode partition tokens (0=auto)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--prefill-seqs", type=int, default=8, help="prefill segments (default 8)")
    p.add_argument("--prefill-len", type=int, default=1024, help="tokens per segment (default 1024)")
    p.add_argument("--prefill-noncausal", action="store_true", help="prefill without the causal mask")
    p.add_argument("--no-long", action="store_true", help="skip the long-context GQA-4 decode leg")
    p.add_argument("--no-slot", action="store_true", help="skip the slot-layout decode leg")
    p.add_argument("--no-prefill-long", action="store_true", help="skip the 8 x 8192 prefill leg")
    p.add_argument("--no-prefill-engine", action="store_true",
                   help="skip the 256 x 1024 prefill leg (the engine's prefill call)")
    p.add_argument("--no-kv", action="store_true", help="skip the KV export/import leg")
    p.add_argument("--no-tp2", action="store_true", help="skip the TP=2 per-rank shape leg")
    p.add_argument("--no-e2e", action="store_true", help="skip the end-to-end engine leg")
    p.add_argument("--e2e-seqs", type=int, default=256)
    p.add_argument("--e2e-in", type=int, default=1024)
    p.add_argument("--e2e-out", type=int, default=1024)
    p.add_argument("--only", choices=["decode", "decode_fp32_small", "decode_slot", "decode_long",
                                      "tp2_rank", "kv_transfer",
                                      "prefill", "prefill_one", "prefill_long", "prefill_engine", "e2e"],
                   default=None,
                   help="run one leg only (for profiling)")
    return p.parse_args()


# ----------------------------------------------------------------------------
# decode: 256 seqs x ctx U[1024, 2047]
# ----------------------------------------------------------------------------
def make_decode_inputs(torch, dev, seed, B=256, hq=16, hkv=8, d=128, bs=256, ctx_lo=1024,
                       ctx_hi=2048, layout="engine"):
    """Synthetic decode inputs.  layout "engine": the K/V caches placed as the
    engine's cache places them (paged.alloc_kv_cache: the V cache 512 bytes
    past its K cache modulo 1 KiB); "separate": two separate allocations, as
    the reference's two torch.zeros (model/model.py:328-335)."""
    rs = np.random.RandomState(seed)
    ctx = rs.randint(ctx_lo, ctx_hi, B).astype(np.int32)      # after the store
    need = [int(-(-c // bs)) for c in ctx]
    pool = sum(need)
    perm = rs.permutation(pool).astype(np.int32)
    width = max(need)
    bt = np.zeros((B, width), np.int32)
    k0 = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    if layout == "engine":
        from awesome_acceleration_amd import paged
        kc, vc = paged.alloc_kv_cache(pool, bs, hkv, d, dtype=bf, device=dev)
        kc.copy_(torch.randn((pool, bs, hkv, d), generator=g, device=dev))
        vc.copy_(torch.randn((pool, bs, hkv, d), generator=g, device=dev))
    else:
        kc = torch.randn((pool, bs, hkv, d), generator=g, device=dev).to(bf)
        vc = torch.randn((pool, bs, hkv, d), generator=g, device=dev).to(bf)
    q = torch.randn((B, 1, hq, d), generator=g, device=dev).to(bf)
    kn = torch.randn((B, 1, hkv, d), generator=g, device=dev).to(bf)
    vn = torch.randn((B, 1, hkv, d), generator=g, device=dev).to(bf)
    return dict(ctx=ctx, bt=bt, kc=kc, vc=vc, q=q, kn=kn, vn=vn, B=B, hq=hq, hkv=hkv, d=d, bs=bs,
                v_minus_k_mod_1k=(vc.data_ptr() - kc.data_ptr()) % 1024,
                bt_g=torch.from_numpy(bt).to(dev),
                seqlens_g=torch.from_numpy(ctx - 1).to(dev),
                ctx_g=torch.from_numpy(ctx).to(dev))


def decode_bytes(x):
    kv = int(x["ctx"].sum()) * x["hkv"] * x["d"] * 2 * 2
    qo = 2 * x["B"] * x["hq"] * x["d"] * 2
    store = 2 * x["B"] * x["hkv"] * x["d"] * 2 * 2  # new k/v read + written
    return kv + qo, kv + qo + store


def launch_avg(torch, fn, n):
    """Average duration of one launch of ``fn`` (seconds): HIP events on the
    current stream around ``n`` back-to-back launches, so the per-launch host
    dispatch latency overlaps the previous launch as in a running engine."""
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(n):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n / 1e3


def warm(torch, fns, seconds):
    """Run ``fns`` in turn back to back for ``seconds`` of wall time (untimed),
    so the clocks reach their sustained level under this load."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            for fn in fns:
                fn()
        torch.cuda.synchronize()


def bench_decode(torch, fai, dev, args, hq=16, hkv=8):
    x = make_decode_inputs(torch, dev, args.seed, hq=hq, hkv=hkv)
    attend_bytes, step_bytes = decode_bytes(x)
    maxctx = int(x["ctx"].max())

    def step():
        return fai.flash_attn_with_kvcache(
            x["q"], x["kc"], x["vc"], k=x["kn"], v=x["vn"], cache_seqlens=x["seqlens_g"],
            block_table=x["bt_g"], causal=False, max_context_len=maxctx)

    q3 = x["q"].view(x["B"], x["hq"], x["d"])
    out3 = torch.empty_like(q3)

    def attend():
        return fai.decode_paged(q3, x["kc"], x["vc"], x["bt_g"], x["ctx_g"],
                                max_context_len=maxctx, partition_tokens=args.partition,
                                out=out3)

    for _ in range(args.warmup):
        step()
        attend()
    warm(torch, [step, attend], args.warmup_seconds)
    # whole step (store + attend), wall clock
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t_step = (time.perf_counter() - t0) / args.steps
    # the attention launch alone, HIP events on the launch stream
    t_att = launch_avg(torch, attend, args.steps)
    achieved = attend_bytes / t_att / 1e9
    t_sep = separate_caches_time(torch, fai, x, maxctx, args)
    return dict(
        t_step=t_step, step_bytes=step_bytes, attend_bytes=attend_bytes, t_attend=t_att,
        achieved=achieved, x=x, t_attend_separate=t_sep)


def separate_caches_time(torch, fai, x, maxctx, args):
    """The same attention over copies of the caches in two separate
    allocations (the reference's placement), for comparison: HIP-event time
    per launch and the V cache's offset from the K cache modulo 1 KiB."""
    kc, vc = x["kc"].clone(), x["vc"].clone()
    q3 = x["q"].view(x["B"], x["hq"], x["d"])
    out3 = torch.empty_like(q3)

    def attend():
        return fai.decode_paged(q3, kc, vc, x["bt_g"], x["ctx_g"], max_context_len=maxctx,
                                partition_tokens=getattr(args, "partition", 0), out=out3)

    warm(torch, [attend], min(args.warmup_seconds, 0.5))
    t = launch_avg(torch, attend, args.steps)
    off = (vc.data_ptr() - kc.data_ptr()) % 1024
    del kc, vc
    torch.cuda.empty_cache()
    return t, off


# ----------------------------------------------------------------------------
# the CPU-runnable fp32 decode case: 4 seqs, contexts {17, 64, 200, 511}
# ----------------------------------------------------------------------------
def bench_decode_fp32_small(torch, fai, dev, args):
    """The fp32 single-layer decode of the golden fixture's shape (batch 4,
    16 / 8 heads, contexts 17 / 64 / 200 / 511 after the store, block 256,
    blocks from a permuted 16-block pool): store + attend through
    flash_attn_with_kvcache on the GPU, per call."""
    B, hq, hkv, d, bs, pool = 4, 16, 8, 128, 256, 16
    ctx = np.array([17, 64, 200, 511], np.int32)
    rs = np.random.RandomState(args.seed)
    perm = rs.permutation(pool).astype(np.int32)
    bt = np.zeros((B, 2), np.int32)
    k0 = 0
    for b in range(B):
        n = -(-int(ctx[b]) // bs)
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n
    g = torch.Generator(device=dev).manual_seed(args.seed)
    kc = torch.randn((pool, bs, hkv, d), generator=g, device=dev)
    vc = torch.randn((pool, bs, hkv, d), generator=g, device=dev)
    q = torch.randn((B, 1, hq, d), generator=g, device=dev)
    kn = torch.randn((B, 1, hkv, d), generator=g, device=dev)
    vn = torch.randn((B, 1, hkv, d), generator=g, device=dev)
    bt_g, sl_g = torch.from_numpy(bt).to(dev), torch.from_numpy(ctx - 1).to(dev)

    def step():
        return fai.flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=sl_g,
                                           block_table=bt_g, max_context_len=int(ctx.max()))

    for _ in range(args.warmup):
        step()
    warm(torch, [step], min(args.warmup_seconds, 0.5))
    t = launch_avg(torch, step, args.steps)
    nbytes = int(ctx.sum()) * hkv * d * 4 * 2 + 2 * B * hq * d * 4 + 4 * B * hkv * d * 4
    return {"workload": "fp32 paged decode store+attend, 4 seqs, 16 q / 8 kv heads, head_dim 128, "
                        "contexts {17, 64, 200, 511}, block 256, permuted 16-block pool",
            "us_per_step": round(t * 1e6, 2), "bytes_per_step": nbytes,
            "achieved": round(nbytes / t / 1e9, 2), "unit": "GB/s", "ctx": ctx}


# ----------------------------------------------------------------------------
# the same decode through the reference's own slot layout: caches
# [slots, max_seq_len, Hkv, D] picked by cache_batch_idx (model/model.py:233-240)
# ----------------------------------------------------------------------------
def bench_decode_slot(torch, fai, dev, args, lmax=2064):
    # one block (slot) per sequence; the caches allocated apart, as the reference allocates them
    x = make_decode_inputs(torch, dev, args.seed, bs=lmax, layout="separate")
    attend_bytes, step_bytes = decode_bytes(x)
    slots = x["bt_g"][:, 0].contiguous()

    def step():  # the reference's call, store + attend
        return fai.flash_attn_with_kvcache(
            x["q"], x["kc"], x["vc"], k=x["kn"], v=x["vn"], cache_seqlens=x["seqlens_g"],
            cache_batch_idx=slots, causal=False)

    for _ in range(args.warmup):
        step()
    warm(torch, [step], args.warmup_seconds)
    t = launch_avg(torch, step, args.steps)
    ach = step_bytes / t / 1e9
    return {
        "workload": f"paged decode store+attend through flash_attn_with_kvcache(cache_batch_idx=...), "
                    f"the reference's slot caches [256, {lmax}, 8, 128], 256 seqs, 16 q / 8 kv heads, "
                    f"context U[1024,2047], shuffled slots",
        "us_per_step": round(t * 1e6, 2),
        "achieved": round(ach, 2), "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
        "bytes_per_step": step_bytes,
    }


# ----------------------------------------------------------------------------
# long-context GQA-4 decode: 64 seqs x ctx U[16384, 32768], 32/8 heads (split-K)
# ----------------------------------------------------------------------------
def bench_decode_long(torch, fai, dev, args):
    x = make_decode_inputs(torch, dev, args.seed, B=64, hq=32, hkv=8, ctx_lo=16384,
                           ctx_hi=32769)
    attend_bytes, _ = decode_bytes(x)
    maxctx = int(x["ctx"].max())
    q3 = x["q"].view(x["B"], x["hq"], x["d"])
    out3 = torch.empty_like(q3)

    def attend():  # the decode kernel plus the split-K reduction
        return fai.decode_paged(q3, x["kc"], x["vc"], x["bt_g"], x["ctx_g"],
                                max_context_len=maxctx, out=out3)

    for _ in range(args.warmup):
        attend()
    warm(torch, [attend], args.warmup_seconds)
    t = launch_avg(torch, attend, args.steps)
    ach = attend_bytes / t / 1e9
    t_sep, off = separate_caches_time(torch, fai, x, maxctx, args)
    return {
        "workload": "paged decode attend, 64 seqs, 32 q / 8 kv heads (GQA-4), head_dim 128, "
                    "context U[16384,32768], block 256, split-K with log-sum-exp reduction (auto plan)",
        "context_tokens": int(x["ctx"].sum()),
        "cache_layout": CACHE_LAYOUT_NOTE,
        "us_per_call": round(t * 1e6, 2),
        "separate_caches": {"us_per_call": round(t_sep * 1e6, 2), "v_minus_k_mod_1k": off,
                            "frac": round(attend_bytes / t_sep / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "bytes_per_call": attend_bytes,
                     "traffic": measured_traffic(TRAFFIC_DECODE_LONG),
                     "traffic_source": TRAFFIC_DECODE_LONG},
    }


# ----------------------------------------------------------------------------
# KV export / import of one request: Qwen3-0.6B cache (28 layers, 8 KV heads),
# 2048 tokens in 8 blocks of 256 drawn from a 2304-block pool
# ----------------------------------------------------------------------------
def bench_kv_transfer(torch, dev, args):
    from awesome_acceleration_amd import kv_transfer as kt, paged
    L, nb, bs, hkv, d, length = 28, 2304, 256, 8, 128, 2048
    # the engine's cache storage (PagedKVCache): each layer's V cache 512 bytes from its K cache
    st = paged.alloc_kv_storage(L, nb, bs, hkv, d, dtype=torch.bfloat16, device=dev)
    st.view(torch.int16).random_(-30000, 30000, generator=torch.Generator(device=dev).manual_seed(args.seed))
    bt = torch.randperm(nb, device=dev, generator=torch.Generator(device=dev).manual_seed(args.seed))
    bt = bt[:length // bs].to(torch.int32)
    buf = torch.empty((L, 2, length, hkv, d), dtype=torch.bfloat16, device=dev)
    moved = 2 * buf.numel() * buf.element_size()  # read + write

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        warm(torch, [fn], args.warmup_seconds)
        return launch_avg(torch, fn, args.steps)

    t_ex = timed(lambda: kt.kv_export(st, bt, length, out=buf))
    t_im = timed(lambda: kt.kv_import(buf, st, bt, length))
    # a plain device-to-device copy of the same bytes (torch / the HIP runtime's
    # copy kernel): the ceiling a gather of 512 KiB runs can approach
    buf2 = torch.empty_like(buf)
    t_cp = timed(lambda: buf2.copy_(buf))
    del buf2
    t0 = time.perf_counter()
    for _ in range(3):
        kt.export_request_kv(st, bt, length, length)
    t_host = (time.perf_counter() - t0) / 3
    del st
    torch.cuda.empty_cache()
    return {
        "workload": "KV export / import of one 2048-token request, Qwen3-0.6B cache (28 layers, "
                    "8 KV heads, head_dim 128, bf16), 8 blocks of 256 from a 2304-block pool",
        "us_export": round(t_ex * 1e6, 2), "us_import": round(t_im * 1e6, 2),
        "roofline": {"bound": "hbm", "achieved": round(moved / t_ex / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(moved / t_ex / 1e9 / HBM_PEAK_GBS, 4),
                     "bytes_per_call": moved, "traffic": measured_traffic(TRAFFIC_KV_EXPORT),
                     "traffic_source": TRAFFIC_KV_EXPORT},
        "import_GBs": round(moved / t_im / 1e9, 2),
        "copy_GBs": round(moved / t_cp / 1e9, 2),
        "request_to_pinned_host_ms": round(t_host * 1e3, 3),
        "request_to_pinned_host_GBs": round(moved / 2 / t_host / 1e9, 2),
    }


# ----------------------------------------------------------------------------
# prefill: 8 x 1024 causal, 16/8 heads, store in the same call
# ----------------------------------------------------------------------------
def bench_prefill(torch, fai, paged, dev, args, hq=16, hkv=8):
    d, bs = 128, 256
    nseq, L, causal = args.prefill_seqs, args.prefill_len, not args.prefill_noncausal
    N = nseq * L
    nb = -(-L // bs)  # blocks per sequence
    g = torch.Generator(device=dev).manual_seed(args.seed)
    qkv = torch.randn((N, (hq + 2 * hkv) * d), generator=g, device=dev).to(torch.bfloat16)
    q = qkv[:, :hq * d].view(N, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].contiguous().view(N, hkv, d)  # post-RoPE copy
    v = qkv[:, (hq + hkv) * d:].view(N, hkv, d)                      # strided view
    rs = np.random.RandomState(args.seed)
    perm = rs.permutation(nseq * nb).astype(np.int32)
    cu, _, sm = paged.build_prefill_metadata([L] * nseq, perm.reshape(nseq, nb), bs, dev)
    kc = torch.zeros((nseq * nb, bs, hkv, d), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    flops = 4 * hq * d * nseq * (L * (L + 1) // 2 if causal else L * L)

    def step():
        return fai.varlen_prefill_with_kvcache(q, k, v, cu, L, kc, vc, sm, causal=causal)

    def attend():
        return fai.flash_attn_varlen_func(q, k, v, cu, cu, L, L, causal=causal)

    for _ in range(args.warmup):
        step()
        attend()
    warm(torch, [step, attend], args.warmup_seconds)
    t_step = launch_avg(torch, step, args.steps)
    t_att = launch_avg(torch, attend, args.steps)
    return dict(t_step=t_step, t_attend=t_att, flops=flops, tflops=flops / t_att / 1e12,
                sdpa=torch_sdpa_reference(torch, dev, args, nseq, L, hq, hkv, causal, flops))


def torch_sdpa_reference(torch, dev, args, nseq, L, hq, hkv, causal, flops):
    """The platform library's own flash attention on the same shape, for
    reference: torch's scaled_dot_product_attention restricted to its flash
    backend (no fallback to the math path), batch-padded [nseq, hq, L, 128]
    bf16 with the KV heads repeated (equal lengths, so the same work as the
    varlen call).  None when the backend is unavailable."""
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        g = torch.Generator(device=dev).manual_seed(args.seed)
        q = torch.randn((nseq, hq, L, 128), generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn((nseq, hkv, L, 128), generator=g, device=dev).to(torch.bfloat16)
        k = k.repeat_interleave(hq // hkv, dim=1).contiguous()
        v = torch.randn_like(k)

        def f():
            with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)

        for _ in range(3):
            f()
        warm(torch, [f], min(args.warmup_seconds, 0.5))
        t = launch_avg(torch, f, max(5, args.steps // 2))
        del q, k, v
        return {"what": "torch scaled_dot_product_attention, flash backend only, same shape "
                        "batch-padded, KV heads repeated", "us": round(t * 1e6, 2),
                "achieved": round(flops / t / 1e12, 2), "unit": "TFLOP/s"}
    except Exception as e:  # backend missing on this build: report, do not fail the bench
        return {"what": "torch SDPA flash backend", "unavailable": f"{type(e).__name__}: {e}"[:200]}


def bench_prefill_long(torch, fai, dev, args, nseq=8, L=8192, hq=16, hkv=8):
    """The same kernel on long segments (8 x 8192 causal), where the per-item
    start and epilogue costs are small against the tile loop: the kernel's
    steady-state rate."""
    d, N = 128, nseq * L
    g = torch.Generator(device=dev).manual_seed(args.seed)
    qkv = torch.randn((N, (hq + 2 * hkv) * d), generator=g, device=dev).to(torch.bfloat16)
    q = qkv[:, :hq * d].view(N, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].contiguous().view(N, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(N, hkv, d)
    cu = torch.arange(0, N + 1, L, dtype=torch.int32, device=dev)
    flops = 4 * hq * d * nseq * (L * (L + 1) // 2)

    def attend():
        return fai.flash_attn_varlen_func(q, k, v, cu, cu, L, L, causal=True)

    for _ in range(3):
        attend()
    warm(torch, [attend], args.warmup_seconds)
    t = launch_avg(torch, attend, max(5, args.steps // 5))
    ach = flops / t / 1e12
    return {
        "workload": f"varlen causal prefill {nseq} x {L} tokens, {hq}/{hkv} heads, head_dim 128, bf16",
        "us_attend": round(t * 1e6, 2),
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                     "flops_per_launch": flops, "traffic": measured_traffic(TRAFFIC_PREFILL_LONG),
                     "traffic_source": TRAFFIC_PREFILL_LONG},
    }


def bench_prefill_engine(torch, fai, paged, dev, args, nseq=256, L=1024, hq=16, hkv=8):
    """The prefill call the continuous-batching engine makes for 256 fresh
    1024-token requests (llm.py:116-184): one launch over 256 packed causal
    segments with the store into a shuffled paged cache (block 256), about 64
    work items per CU -- the per-item start and epilogue weigh here."""
    d, bs, N = 128, 256, nseq * L
    nb = -(-L // bs)
    g = torch.Generator(device=dev).manual_seed(args.seed)
    qkv = torch.randn((N, (hq + 2 * hkv) * d), generator=g, device=dev).to(torch.bfloat16)
    q = qkv[:, :hq * d].view(N, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].contiguous().view(N, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(N, hkv, d)
    rs = np.random.RandomState(args.seed)
    perm = rs.permutation(nseq * nb).astype(np.int32)
    cu, _, sm = paged.build_prefill_metadata([L] * nseq, perm.reshape(nseq, nb), bs, dev)
    kc = torch.zeros((nseq * nb, bs, hkv, d), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    flops = 4 * hq * d * nseq * (L * (L + 1) // 2)

    def step():
        return fai.varlen_prefill_with_kvcache(q, k, v, cu, L, kc, vc, sm, causal=True)

    def attend():
        return fai.flash_attn_varlen_func(q, k, v, cu, cu, L, L, causal=True)

    for _ in range(3):
        step()
        attend()
    warm(torch, [step, attend], args.warmup_seconds)
    n = max(5, args.steps // 5)
    t_step = launch_avg(torch, step, n)
    t = launch_avg(torch, attend, n)
    ach, ach_s = flops / t / 1e12, flops / t_step / 1e12
    return {
        "workload": f"varlen causal prefill {nseq} x {L} tokens with the KV store into a paged cache "
                    f"(block {bs}, shuffled), {hq}/{hkv} heads, head_dim 128, bf16",
        "us_step_with_store": round(t_step * 1e6, 2),
        "us_attend": round(t * 1e6, 2),
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                     "frac_with_store": round(ach_s / BF16_PEAK_TFLOPS, 4),
                     "flops_per_launch": flops,
                     "traffic": measured_traffic(TRAFFIC_PREFILL_ENGINE),
                     "traffic_with_store": measured_traffic(TRAFFIC_PREFILL_ENGINE,
                                                            "traffic_bytes_per_launch_store"),
                     "traffic_source": TRAFFIC_PREFILL_ENGINE},
    }


def bench_prefill_one_request(torch, fai, dev, args, L=2048, hq=16, hkv=8):
    """One 2048-token request (16/8 heads, causal): 128 work items for 256
    CUs, so each item's key range is split over two workgroups and merged;
    the same call without the split (no workspace) beside it."""
    from awesome_acceleration_amd import _lib
    d = 128
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn((L, hq, d), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((L, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((L, hkv, d), generator=g, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, L], dtype=torch.int32, device=dev)
    flops = 4 * hq * d * (L * (L + 1) // 2)
    out = torch.empty_like(q)
    lib, st = _lib.lib(), torch.cuda.current_stream().cuda_stream

    def split():
        return fai.flash_attn_varlen_func(q, k, v, cu, cu, L, L, causal=True)

    def unsplit():
        lib.aac_prefill_varlen(q.data_ptr(), k.data_ptr(), v.data_ptr(), hq * d, hkv * d, hkv * d,
                               cu.data_ptr(), cu.data_ptr(), 1, L, L, hq, hkv, d, d ** -0.5, 1,
                               out.data_ptr(), hq * d, None, 0, 0, st)

    for _ in range(3):
        split()
        unsplit()
    warm(torch, [split, unsplit], min(args.warmup_seconds, 0.5))
    t = launch_avg(torch, split, args.steps)
    t0 = launch_avg(torch, unsplit, args.steps)
    ws = lib.aac_prefill_workspace_bytes(1, L, L, hq, hkv, d, 1)
    return {"workload": f"varlen causal prefill of one {L}-token request, {hq}/{hkv} heads, "
                        "head_dim 128, bf16: key ranges split over two workgroups and merged",
            "us_attend": round(t * 1e6, 2), "us_unsplit": round(t0 * 1e6, 2),
            "workspace_bytes": int(ws),
            "roofline": {"bound": "mfma", "achieved": round(flops / t / 1e12, 2),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(flops / t / 1e12 / BF16_PEAK_TFLOPS, 4),
                         "flops_per_launch": flops}}


# ----------------------------------------------------------------------------
# end to end: random-init Qwen3-0.6B under the continuous-batching engine
# ----------------------------------------------------------------------------
def bench_e2e(torch, args):
    from awesome_acceleration_amd.llm import LLM
    from awesome_acceleration_amd.qwen3 import Qwen3Config

    B, Lin, Lout = args.e2e_seqs, args.e2e_in, args.e2e_out
    t0 = time.perf_counter()
    llm = LLM(Qwen3Config(), max_num_seqs=B, max_seq_len=Lin + Lout + 16, block_size=256,
              seed=args.seed)
    rs = np.random.RandomState(args.seed)
    prompts = [rs.randint(0, llm.config.vocab_size, Lin).tolist() for _ in range(B)]
    # warm-up request (benchmark_tp.py:357-358) also captures the decode graph of
    # the largest bucket so capture time stays out of the timed region
    llm.generate([prompts[0][:16]] * B, max_tokens=3, ignore_eos=True).result()
    torch.cuda.synchronize()
    t_init = time.perf_counter() - t0
    t0 = time.perf_counter()
    outs = llm.generate(prompts, max_tokens=Lout, ignore_eos=True).result()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    llm.stop()
    gen = sum(o.generated_tokens for o in outs)
    prompt = sum(o.prompt_tokens for o in outs)
    return dict(
        workload=f"Qwen3-0.6B (28 layers, hidden 1024, 16/8 heads, head_dim 128, vocab 151936, "
                 f"random bf16 weights), {B} requests x {Lin} random input tokens, {Lout} greedy "
                 f"output tokens each (ignore_eos), continuous-batching engine, KV block 256",
        output_tok_s=round(gen / el, 1), total_tok_s=round((gen + prompt) / el, 1),
        seconds=round(el, 3), generated_tokens=gen, prompt_tokens=prompt,
        decode_steps=llm.stats["decode_steps"], setup_seconds=round(t_init, 2),
        kv_cache_gib=round(llm.cache.nbytes / 2 ** 30, 1))


# ----------------------------------------------------------------------------
# CPU baselines: the reference's semantics in fp32 torch on the host cores
# (oracle/torch_path.py, oracle/qwen3_ref.py), 3 warm-ups then the median of 5
# ----------------------------------------------------------------------------
def _median_time(fn, warmup=3, reps=5, budget_s=0.0, max_reps=1000):
    """Median of at least ``reps`` timed runs after ``warmup`` untimed ones,
    repeated until ``budget_s`` seconds have been timed (at most ``max_reps``)."""
    for _ in range(warmup):
        fn()
    ts = []
    while len(ts) < reps or (sum(ts) < budget_s and len(ts) < max_reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), ts


def _host_fill(torch, shape, dtype, seed):
    """A host tensor of N(0,1) values (a 4 Mi-value draw repeated; seconds to
    fill gigabytes, and the values do not change the work)."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(1 << 22, generator=g).to(dtype)
    t = torch.empty(shape, dtype=dtype)
    flat = t.view(-1)
    for i in range(0, flat.numel(), base.numel()):
        m = min(base.numel(), flat.numel() - i)
        flat[i:i + m] = base[:m]
    return t


def _paged_tables(ctx, bs, rs):
    need = [int(-(-int(c) // bs)) for c in ctx]
    pool = sum(need)
    perm = rs.permutation(pool)
    bt = np.zeros((len(ctx), max(need)), np.int64)
    k0 = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n
    return bt, pool


def cpu_decode_baseline(torch, ctx, hq, hkv, label, threads, dtype=None, d=128, bs=256, seed=3,
                        budget_s=5.0):
    """Paged decode store+attend (model/model.py:233-241) on the host:
    oracle.torch_path.decode_store_attend in fp32 on bf16-valued caches (or
    ``dtype``), the same contexts, 16/8 or 32/8 heads, block 256."""
    from oracle import torch_path as tp
    dtype = dtype or torch.bfloat16
    rs = np.random.RandomState(seed)
    B = len(ctx)
    bt, pool = _paged_tables(ctx, bs, rs)
    kc = _host_fill(torch, (pool, bs, hkv, d), dtype, seed)
    vc = _host_fill(torch, (pool, bs, hkv, d), dtype, seed + 1)
    q = _host_fill(torch, (B, hq, d), dtype, seed + 2)
    kn = _host_fill(torch, (B, hkv, d), dtype, seed + 3)
    vn = _host_fill(torch, (B, hkv, d), dtype, seed + 4)
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        med, ts = _median_time(lambda: tp.decode_store_attend(q, kn, vn, kc, vc, bt, ctx - 1,
                                                              d ** -0.5), budget_s=budget_s)
    finally:
        torch.set_num_threads(prev)
    esz = torch.tensor([], dtype=dtype).element_size()
    nbytes = int(ctx.sum()) * hkv * d * esz * 2 + 2 * B * hq * d * esz + 4 * B * hkv * d * esz
    return dict(value=round(nbytes / med / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                seconds_per_step=round(med, 4), bytes_per_step=nbytes,
                sample=f"{label}: store+attend of one decode step (oracle.torch_path, fp32 torch "
                       f"on {str(dtype).split('.')[-1]}-valued caches, {threads} host threads), "
                       f"median of {len(ts)} after 3 warm-ups ({sum(ts):.1f} s timed)")


def cpu_prefill_baseline(torch, nseq, L, hq, hkv, threads, d=128, bs=256, seed=4, budget_s=5.0):
    """Varlen causal prefill store+attend (llm.py:171-184) on the host:
    index_copy_ into a shuffled paged cache, then torch SDPA per segment in
    fp32 on bf16-valued q/k/v."""
    from oracle import torch_path as tp
    N = nseq * L
    rs = np.random.RandomState(seed)
    nb = -(-L // bs)
    perm = rs.permutation(nseq * nb)
    pos = np.arange(N) % L
    seg = np.arange(N) // L
    sm = torch.from_numpy(perm.reshape(nseq, nb)[seg, pos // bs] * bs + pos % bs)
    q = _host_fill(torch, (N, hq, d), torch.bfloat16, seed)
    k = _host_fill(torch, (N, hkv, d), torch.bfloat16, seed + 1)
    v = _host_fill(torch, (N, hkv, d), torch.bfloat16, seed + 2)
    kc = torch.zeros((nseq * nb, bs, hkv, d), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    cu = list(range(0, N + 1, L))
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        med, ts = _median_time(lambda: tp.prefill_store_attend(q, k, v, cu, kc, vc, sm,
                                                               d ** -0.5), budget_s=budget_s)
    finally:
        torch.set_num_threads(prev)
    flops = 4 * hq * d * nseq * (L * (L + 1) // 2)
    return dict(value=round(flops / med / 1e12, 4), unit="TFLOP/s", cores=threads, kind="port",
                seconds_per_call=round(med, 4),
                sample=f"varlen causal prefill {nseq} x {L}, {hq}/{hkv} heads: index_copy_ store "
                       f"+ torch SDPA per segment (oracle.torch_path, fp32 on bf16-valued inputs, "
                       f"{threads} host threads), median of {len(ts)} after 3 warm-ups "
                       f"({sum(ts):.1f} s timed)")


def cpu_e2e_small_run(torch, threads, n_req=8, n_in=128, n_out=32, seed=5):
    """A complete small generation run on the host: random-init Qwen3-0.6B
    (oracle.qwen3_ref, fp32 torch, the reference's slot caches, packed varlen
    prefill then batched greedy decode steps), n_req requests x n_in random
    tokens, n_out output tokens each (ignore_eos)."""
    from awesome_acceleration_amd.qwen3 import Qwen3Config
    from oracle.qwen3_ref import Qwen3Ref
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        cfg = Qwen3Config()
        ref = Qwen3Ref.random(cfg, seed=seed, tiled=True)
        rs = np.random.RandomState(seed)
        prompts = [rs.randint(0, cfg.vocab_size, n_in).tolist() for _ in range(n_req)]
        ref.generate(prompts[:2], max_tokens=2, max_seq_len=n_in + n_out + 16)  # warm-up
        t0 = time.perf_counter()
        outs = ref.generate(prompts, max_tokens=n_out, max_seq_len=n_in + n_out + 16)
        el = time.perf_counter() - t0
    finally:
        torch.set_num_threads(prev)
    gen = sum(len(o) for o in outs)
    return dict(value=round(gen / el, 2), unit="output tok/s", cores=threads, kind="port",
                total_tok_s=round((gen + n_req * n_in) / el, 2), seconds=round(el, 3),
                sample=f"complete run of {n_req} requests x {n_in} random input tokens, {n_out} "
                       f"greedy output tokens each, random-init Qwen3-0.6B in fp32 torch "
                       f"(oracle.qwen3_ref: packed prefill + batched decode over slot caches) on "
                       f"{threads} host threads; the full 256 x 1024/1024 workload is not run on "
                       f"the host (hours)")


def oracle_1core(x, reps=12, seed=1):
    """The oracle's store-then-attend over the same decode shape (all 256
    sequences, the same context lengths), single-threaded; the median of
    ``reps`` runs (about 10 s of CPU work)."""
    import oracle
    from threadpoolctl import threadpool_limits

    rng = np.random.default_rng(seed)
    hq, hkv, d, bs = x["hq"], x["hkv"], x["d"], x["bs"]
    ctx = x["ctx"]
    B = ctx.shape[0]
    need = [int(-(-c // bs)) for c in ctx]
    pool = sum(need)
    bt = np.zeros((B, max(need)), np.int32)
    perm = rng.permutation(pool).astype(np.int32)
    k0 = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n

    def bf16(shape):  # bf16 bit patterns of values with |x| in [2^-7, 4), random sign
        n = int(np.prod(shape))
        bits = rng.integers(0x3C00, 0x4080, n, dtype=np.uint16)
        bits |= rng.integers(0, 2, n, dtype=np.uint16) << np.uint16(15)
        return bits.reshape(shape)

    kc, vc = bf16((pool, bs, hkv, d)), bf16((pool, bs, hkv, d))
    q, kn, vn = bf16((B, hq, d)), bf16((B, hkv, d)), bf16((B, hkv, d))
    times = []
    with threadpool_limits(limits=1):
        for _ in range(reps):
            t0 = time.perf_counter()
            oracle.decode_append_attend(q, kc, vc, kn, vn, bt, ctx - 1, bs)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = decode_bytes(dict(ctx=ctx, B=B, hq=hq, hkv=hkv, d=d))[1]
    return dict(value=round(nbytes / med / 1e9, 4), unit="GB/s", cores=1, kind="port",
                sample=f"oracle.decode_append_attend (numpy, float64 math, 1 thread): the full "
                       f"store+attend step over all {B} sequences ({int(ctx.sum())} context "
                       f"tokens), median of {reps} runs ({sum(times):.1f} s of CPU work)",
                seconds_per_step=round(med, 3))


def cpu_e2e_baseline(torch, ctx, threads, reps=3, seed=2, hidden=1024, inter=3072, hq=16, hkv=8,
                     d=128, layers=28, vocab=151936, theta=1e6, eps=1e-6):
    """The end-to-end decode step on the host: one Qwen3 decoder layer
    (model/model.py:202-267: RMSNorm, fused QKV, q/k RMSNorm, RoPE, the K/V
    append into the reference's slot caches, GQA attention over each
    sequence's context, o_proj, residual, RMSNorm, SiLU-gated MLP, residual)
    for all sequences at once in fp32 torch on ``threads`` host threads, the
    median of ``reps`` runs, times the number of layers, plus the tied lm_head
    projection and argmax: output tok/s = sequences / step time."""
    import torch.nn.functional as F
    from awesome_acceleration_amd.qwen3 import rms_norm

    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        g = torch.Generator().manual_seed(seed)
        B, lmax = int(ctx.shape[0]), int(ctx.max())
        rnd = lambda *shape, s=1.0: torch.randn(*shape, generator=g) * s
        w = dict(ln1=1 + rnd(hidden, s=0.1), ln2=1 + rnd(hidden, s=0.1), qn=1 + rnd(d, s=0.1),
                 kn=1 + rnd(d, s=0.1), qkv=rnd((hq + 2 * hkv) * d, hidden, s=0.02),
                 o=rnd(hidden, hq * d, s=0.02), gu=rnd(2 * inter, hidden, s=0.02),
                 down=rnd(hidden, inter, s=0.02))
        base = torch.randn(1 << 22, generator=g).to(torch.bfloat16)

        def filled(*shape):  # random bf16 rows, a 4 Mi-element draw repeated (fast to fill)
            t = torch.empty(*shape, dtype=torch.bfloat16)
            flat = t.view(-1)
            for i in range(0, flat.numel(), base.numel()):
                flat[i:i + base.numel()] = base[:min(base.numel(), flat.numel() - i)]
            return t

        kc = filled(B, lmax, hkv, d)  # slot caches (model/model.py:328-335)
        vc = filled(B, lmax, hkv, d)
        x = rnd(B, hidden)
        pos = torch.from_numpy(ctx.astype(np.int64) - 1)  # the new token's position
        inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        ang = torch.cat((torch.outer(pos.float(), inv),) * 2, dim=-1)
        cos, sin = ang.cos().unsqueeze(1), ang.sin().unsqueeze(1)

        def rope(t):
            t1, t2 = t[..., :d // 2], t[..., d // 2:]
            return t * cos + torch.cat((-t2, t1), dim=-1) * sin

        def layer(x):
            h = rms_norm(x, w["ln1"], eps)
            qkv = F.linear(h, w["qkv"])
            q = rope(rms_norm(qkv[:, :hq * d].view(B, hq, d), w["qn"], eps))
            k = rope(rms_norm(qkv[:, hq * d:(hq + hkv) * d].view(B, hkv, d), w["kn"], eps))
            v = qkv[:, (hq + hkv) * d:].view(B, hkv, d)
            att = torch.empty(B, hq, d)
            for b in range(B):
                n = int(ctx[b])
                kc[b, n - 1], vc[b, n - 1] = k[b].to(torch.bfloat16), v[b].to(torch.bfloat16)
                kb = kc[b, :n].float().permute(1, 2, 0)          # [hkv, d, n]
                vb = vc[b, :n].float().permute(1, 0, 2)          # [hkv, n, d]
                sb = torch.matmul(q[b].view(hkv, hq // hkv, d), kb) * d ** -0.5
                att[b] = torch.matmul(torch.softmax(sb, dim=-1), vb).reshape(hq, d)
            x = x + F.linear(att.reshape(B, hq * d), w["o"])
            gu = F.linear(rms_norm(x, w["ln2"], eps), w["gu"])
            return x + F.linear(F.silu(gu[:, :inter]) * gu[:, inter:], w["down"])

        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            layer(x)
            times.append(time.perf_counter() - t0)
        t_layer = float(np.median(times))
        del kc, vc
        embed = rnd(vocab, hidden, s=0.02)
        t0 = time.perf_counter()
        F.linear(rms_norm(x, w["ln1"], eps), embed).argmax(-1)
        t_head = time.perf_counter() - t0
    finally:
        torch.set_num_threads(prev)
    step = layers * t_layer + t_head
    return dict(value=round(B / step, 2), unit="output tok/s", cores=threads, kind="port",
                sample=f"one decoder layer's decode step for {B} sequences (context "
                       f"{int(ctx.min())}-{int(ctx.max())}, slot caches) in fp32 torch on "
                       f"{threads} host threads, median of {reps} runs ({t_layer:.3f} s), times "
                       f"{layers} layers, plus the lm_head projection and argmax ({t_head:.3f} s)",
                seconds_per_step=round(step, 3))


def device_record(torch, dev):
    """The GPU the line was measured on (the clock and the peak derivation are
    in profiles/device_mi355x.md)."""
    p = torch.cuda.get_device_properties(dev)
    return {"arch": p.gcnArchName.split(":")[0], "compute_units": p.multi_processor_count,
            "memory_gib": round(p.total_memory / 2 ** 30, 1), "properties": DEVICE_PROFILE}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the attention path shards by sequence or KV head with no exchange; "
              "the figure at N GPUs is N independent copies of the N=1 line)", file=sys.stderr)
        sys.exit(2)
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from awesome_acceleration_amd import flash_attn_interface as fai, paged

    dev = torch.device("cuda:0")
    res = {}
    if args.only in (None, "decode"):
        res["decode"] = bench_decode(torch, fai, dev, args)
    if args.only in (None, "decode_fp32_small"):
        res["decode_fp32_small"] = bench_decode_fp32_small(torch, fai, dev, args)
    if args.only in (None, "decode_slot") and not args.no_slot:
        res["decode_slot"] = bench_decode_slot(torch, fai, dev, args)
        torch.cuda.empty_cache()
    if args.only in (None, "decode_long") and not args.no_long:
        res["decode_long"] = bench_decode_long(torch, fai, dev, args)
        torch.cuda.empty_cache()
    if args.only in (None, "tp2_rank") and not args.no_tp2:
        dec2 = bench_decode(torch, fai, dev, args, hq=8, hkv=4)
        pf2 = bench_prefill(torch, fai, paged, dev, args, hq=8, hkv=4)
        res["tp2_rank"] = {
            "workload": "one tensor-parallel rank of TP=2 (8 q / 4 kv heads): the 256-sequence decode "
                        "attention (context U[1024,2047], shuffled pool) and the 8 x 1024 causal prefill",
            "decode": {"us_per_launch": round(dec2["t_attend"] * 1e6, 2),
                       "achieved": round(dec2["achieved"], 2), "unit": "GB/s",
                       "frac": round(dec2["achieved"] / HBM_PEAK_GBS, 4),
                       "bytes_per_launch": dec2["attend_bytes"],
                       "cache_layout": CACHE_LAYOUT_NOTE,
                       "separate_caches": {
                           "us_per_launch": round(dec2["t_attend_separate"][0] * 1e6, 2),
                           "v_minus_k_mod_1k": dec2["t_attend_separate"][1],
                           "frac": round(dec2["attend_bytes"] / dec2["t_attend_separate"][0] / 1e9
                                         / HBM_PEAK_GBS, 4)}},
            "prefill": {"us_attend": round(pf2["t_attend"] * 1e6, 2),
                        "achieved": round(pf2["tflops"], 2), "unit": "TFLOP/s",
                        "frac": round(pf2["tflops"] / BF16_PEAK_TFLOPS, 4),
                        "flops_per_launch": pf2["flops"]},
        }
        del dec2
        torch.cuda.empty_cache()
    if args.only in (None, "kv_transfer") and not args.no_kv:
        res["kv_transfer"] = bench_kv_transfer(torch, dev, args)
    if args.only in (None, "prefill") and not args.no_prefill:
        res["prefill"] = bench_prefill(torch, fai, paged, dev, args)
    if args.only in (None, "prefill_one") and not args.no_prefill:
        res["prefill_one_request"] = bench_prefill_one_request(torch, fai, dev, args)
    if args.only in (None, "prefill_long") and not args.no_prefill_long:
        res["prefill_long"] = bench_prefill_long(torch, fai, dev, args)
        torch.cuda.empty_cache()
    if args.only in (None, "prefill_engine") and not args.no_prefill_engine:
        res["prefill_engine"] = bench_prefill_engine(torch, fai, paged, dev, args)
        torch.cuda.empty_cache()
    if args.only in (None, "e2e") and not args.no_e2e:
        res["e2e"] = bench_e2e(torch, args)
    if args.only is not None:
        # calibration for counter-based traffic: a plain 1 GiB device copy
        # (1 GiB read + 1 GiB written) in the same process
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({k: {kk: vv for kk, vv in v.items() if kk not in ("x", "ctx")}
                          for k, v in res.items()}, default=float))
        return
    dec = res["decode"]
    line = {
        "metric": "decode-attn HBM GB/s + prefill MFMA util; Qwen3-0.6B output tok/s @1 GPU",
        "value": round(dec["step_bytes"] / dec["t_step"] / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_seconds": args.warmup_seconds,
        "ms_per_step": round(dec["t_step"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v and caches, random shuffled block tables; the paged "
                "K/V caches placed as the engine places them, separately allocated caches timed beside)",
        "device": device_record(torch, dev),
        "config": {
            "workload": "paged decode store+attend, 256 seqs, 16 q / 8 kv heads, head_dim 128, "
                        "context U[1024,2047], block 256, shared shuffled pool",
            "seqs": 256, "q_heads": 16, "kv_heads": 8, "head_dim": 128, "block_size": 256,
            "context_tokens": int(dec["x"]["ctx"].sum()),
            "step_bytes": dec["step_bytes"],
        },
        "roofline": {
            "kernel": "decode_paged_kernel (aac_decode_paged; one launch, no split at this shape)",
            "bound": "hbm",
            "achieved": round(dec["achieved"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["achieved"] / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": TRAFFIC_PROFILE,
            "bytes_per_launch": dec["attend_bytes"],
            "us_per_launch": round(dec["t_attend"] * 1e6, 2),
            "cache_layout": CACHE_LAYOUT_NOTE,
            "separate_caches": {
                "us_per_launch": round(dec["t_attend_separate"][0] * 1e6, 2),
                "v_minus_k_mod_1k": dec["t_attend_separate"][1],
                "frac": round(dec["attend_bytes"] / dec["t_attend_separate"][0] / 1e9 / HBM_PEAK_GBS, 4),
            },
        },
    }
    if "prefill" in res:
        pf = res["prefill"]
        line["prefill"] = {
            "workload": f"varlen {'non-causal' if args.prefill_noncausal else 'causal'} prefill "
                        f"{args.prefill_seqs} x {args.prefill_len} tokens, 16/8 heads, head_dim 128, bf16",
            "us_attend": round(pf["t_attend"] * 1e6, 2),
            "us_step_with_store": round(pf["t_step"] * 1e6, 2),
            "roofline": {"bound": "mfma", "achieved": round(pf["tflops"], 2),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(pf["tflops"] / BF16_PEAK_TFLOPS, 4),
                         "flops_per_launch": pf["flops"],
                         "traffic": measured_traffic(TRAFFIC_PREFILL),
                         "traffic_with_store": measured_traffic(TRAFFIC_PREFILL,
                                                                "traffic_bytes_per_launch_store"),
                         "traffic_source": TRAFFIC_PREFILL},
            "torch_sdpa_flash": pf.get("sdpa"),
        }
    if "decode_long" in res:
        line["decode_long"] = res["decode_long"]
    if "decode_slot" in res:
        line["decode_slot"] = res["decode_slot"]
    if "prefill_long" in res:
        line["prefill_long"] = res["prefill_long"]
    if "prefill_engine" in res:
        line["prefill_engine"] = res["prefill_engine"]
    if "prefill_one_request" in res:
        line["prefill_one_request"] = res["prefill_one_request"]
    if "tp2_rank" in res:
        line["tp2_rank"] = res["tp2_rank"]
    if "kv_transfer" in res:
        line["kv_transfer"] = res["kv_transfer"]
    if "e2e" in res:
        line["e2e"] = res["e2e"]
    if "decode_fp32_small" in res:
        line["decode_fp32_small"] = {k: v for k, v in res["decode_fp32_small"].items()
                                     if k != "ctx"}
    if not args.no_cpu:
        from oracle.torch_path import cpu_threads
        n = cpu_threads()
        line["cpu_baseline"] = cpu_decode_baseline(
            torch, dec["x"]["ctx"], 16, 8, f"256 seqs x context U[1024,2047] (the same "
            f"{int(dec['x']['ctx'].sum())} context tokens), 16/8 heads, block 256", n,
            budget_s=10.0)
        line["cpu_baseline"]["host_cpus_visible"] = len(os.sched_getaffinity(0))
        line["cpu_baseline"]["oracle_1core"] = oracle_1core(dec["x"], reps=5)
        if "decode_fp32_small" in res:
            small = cpu_decode_baseline(torch, res["decode_fp32_small"]["ctx"], 16, 8,
                                        "4 seqs x contexts {17, 64, 200, 511}", n,
                                        dtype=torch.float32)
            line["decode_fp32_small"]["cpu_baseline"] = small
            line["decode_fp32_small"]["vs_cpu"] = round(
                small["seconds_per_step"] * 1e6 / line["decode_fp32_small"]["us_per_step"], 1)
        if "prefill" in line:
            line["prefill"]["cpu_baseline"] = cpu_prefill_baseline(
                torch, args.prefill_seqs, args.prefill_len, 16, 8, n)
        if "decode_long" in line:
            ctx_long = np.random.RandomState(args.seed).randint(16384, 32769, 64).astype(np.int32)
            line["decode_long"]["cpu_baseline"] = cpu_decode_baseline(
                torch, ctx_long[:16], 32, 8, "the first 16 of the 64 sequences (context "
                f"{int(ctx_long[:16].sum())} tokens), 32/8 heads, block 256", n)
        if "e2e" in line:
            line["e2e"]["cpu_baseline"] = cpu_e2e_small_run(torch, n)
            # the end-to-end decode step at the workload's batch, extrapolated
            # from one layer (the full run would take hours on the host)
            line["e2e"]["cpu_decode_step_extrapolated"] = cpu_e2e_baseline(
                torch, dec["x"]["ctx"], threads=n)
            line["e2e"]["vs_cpu"] = round(line["e2e"]["output_tok_s"] /
                                          line["e2e"]["cpu_baseline"]["value"], 1)
    print(json.dumps(line))


if __name__ == "__main__":
    main()

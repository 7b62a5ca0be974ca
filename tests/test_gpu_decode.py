"""GPU parity of paged decode (store then attend) against the oracle.

Covers the committed fixtures (fp32 Qwen3-0.6B layer at batch 4, tiny bf16),
the 256-sequence bf16 decode at full size, the long-context GQA-4 decode
(B=64, 16k-32k tokens) on a sample of sequences, the reference's slot layout
through flash_attn_with_kvcache(cache_batch_idx=...), every GQA group, and
the invariants of the split-K plan (partition count, block relabelling).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import flash_attn_interface as fai
from cases import config1_inputs, sha256, tiny_decode_inputs
from gpu_util import bf16_np_to_f64, bytes_of, check_attention, f64, np_of, t_of

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
MANIFEST = json.loads((GOLD / "manifest.json").read_text())


def _abs_v(x):
    """|x| for bf16 bit patterns (sign bit cleared) or float arrays: the V of
    the attention sum_j p_j |v_j| that bounds the effect of rounding the
    probabilities to bf16/fp16 before the PV product."""
    return x & np.uint16(0x7FFF) if x.dtype == np.uint16 else np.abs(x)


def _run_fixture(inp, gpu, dtype):
    q = t_of(inp["q"], gpu, dtype)
    kc = t_of(inp["k_cache"], gpu, dtype)
    vc = t_of(inp["v_cache"], gpu, dtype)
    kn = t_of(inp["k_new"], gpu, dtype)
    vn = t_of(inp["v_new"], gpu, dtype)
    bt = torch.from_numpy(inp["block_tables"]).to(gpu)
    lens = torch.from_numpy(inp["cache_seqlens"]).to(gpu)
    B, hq, d = q.shape
    out = fai.flash_attn_with_kvcache(q.view(B, 1, hq, d), kc, vc, k=kn.view(B, 1, -1, d),
                                      v=vn.view(B, 1, -1, d), cache_seqlens=lens, block_table=bt,
                                      softmax_scale=inp["scale"], causal=False)
    torch.cuda.synchronize()
    return out.view(B, hq, d), kc, vc, lens


def test_config1_fp32_fixture(gpu):
    print("case: config1 fp32 decode fixture", flush=True)
    inp = config1_inputs()
    fx = np.load(GOLD / "config1_decode_fp32.npz")
    out, kc, vc, lens = _run_fixture(inp, gpu, torch.float32)
    man = MANIFEST["config1_decode_fp32"]
    assert sha256(np_of(kc)) == man["digest_k_cache_after"]
    assert sha256(np_of(vc)) == man["digest_v_cache_after"]
    assert np.array_equal(np_of(lens), inp["cache_seqlens"])  # not modified
    check_attention(out, fx["out"], atol=1e-4, what="config1 fp32")


def test_tiny_bf16_fixture(gpu):
    print("case: tiny bf16 decode fixture", flush=True)
    inp = tiny_decode_inputs()
    fx = np.load(GOLD / "tiny_decode_bf16.npz")
    out, kc, vc, _ = _run_fixture(inp, gpu, None)
    man = MANIFEST["tiny_decode_bf16"]
    assert sha256(np_of(kc)) == man["digest_k_cache_after"]
    assert sha256(np_of(vc)) == man["digest_v_cache_after"]
    absv, _ = oracle.decode_append_attend(inp["q"], inp["k_cache"].copy(), _abs_v(inp["v_cache"]),
                                          inp["k_new"], _abs_v(inp["v_new"]), inp["block_tables"],
                                          inp["cache_seqlens"], inp["block_size"], inp["scale"])
    check_attention(out, fx["out"], what="tiny bf16", absv=absv)


def _random_paged(B, hq, hkv, ctx, bs, seed, gpu, dtype=torch.bfloat16, extra_blocks=3):
    """Shared shuffled pool holding exactly the blocks the sequences need."""
    rs = np.random.RandomState(seed)
    need = [int(np.ceil(c / bs)) for c in ctx]
    pool = sum(need) + extra_blocks
    perm = rs.permutation(pool).astype(np.int32)
    width = max(need)
    bt = np.zeros((B, width), np.int32)
    k0 = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n
    g = torch.Generator(device=gpu).manual_seed(seed)
    kc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu, dtype=torch.float32).to(dtype)
    vc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu, dtype=torch.float32).to(dtype)
    q = torch.randn((B, hq, 128), generator=g, device=gpu, dtype=torch.float32).to(dtype)
    kn = torch.randn((B, hkv, 128), generator=g, device=gpu, dtype=torch.float32).to(dtype)
    vn = torch.randn((B, hkv, 128), generator=g, device=gpu, dtype=torch.float32).to(dtype)
    return q, kc, vc, kn, vn, bt


def _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, seqs, scale, abs_v=False):
    out = {}
    for b in seqs:
        ks = oracle.gather_paged(kc_np, bt[b], int(ctx[b]), bs)
        vs = oracle.gather_paged(vc_np, bt[b], int(ctx[b]), bs)
        if ks.dtype == np.uint16:
            ks, vs, qb = bf16_np_to_f64(ks), bf16_np_to_f64(vs), bf16_np_to_f64(q_np[b])
        else:
            ks, vs, qb = ks.astype(np.float64), vs.astype(np.float64), q_np[b].astype(np.float64)
        if abs_v:
            vs = np.abs(vs)
        out[b] = oracle.paged_decode(qb[None], ks[None], vs[None],
                                     np.arange(1, dtype=np.int32)[None], [int(ctx[b])],
                                     block_size=int(ctx[b]), scale=scale)[0]
    return out


def test_decode_256_seqs_full_size(gpu):
    # bf16, 256 sequences, 16/8 heads, D=128, context ~ U[1024, 2047] (after
    # the store), block 256, shuffled shared pool; store one token, attend.
    print("case: decode 256 seqs full size", flush=True)
    B, hq, hkv, bs = 256, 16, 8, 256
    rs = np.random.RandomState(0)
    ctx = rs.randint(1024, 2048, B).astype(np.int32)
    q, kc, vc, kn, vn, bt = _random_paged(B, hq, hkv, ctx, bs, 0, gpu)
    scale = 128 ** -0.5
    lens = torch.from_numpy(ctx - 1).to(gpu)
    bt_g = torch.from_numpy(bt).to(gpu)
    out = fai.flash_attn_with_kvcache(q.view(B, 1, hq, 128), kc, vc, k=kn.view(B, 1, hkv, 128),
                                      v=vn.view(B, 1, hkv, 128), cache_seqlens=lens,
                                      block_table=bt_g, softmax_scale=scale)
    torch.cuda.synchronize()
    kc_np, vc_np, q_np = np_of(kc), np_of(vc), np_of(q)
    # the appended rows are in the cache now (bit-exact store)
    sm = oracle.decode_slot_mapping(bt, ctx - 1, bs)
    assert np.array_equal(kc_np.reshape(-1, hkv, 128)[sm], np_of(kn))
    assert np.array_equal(vc_np.reshape(-1, hkv, 128)[sm], np_of(vn))
    ref = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), scale)
    absv = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), scale, abs_v=True)
    check_attention(out.view(B, hq, 128), np.stack([ref[b] for b in range(B)]),
                    what="decode 256 seqs", absv=np.stack([absv[b] for b in range(B)]))


@pytest.mark.parametrize("hq,hkv", [(6, 3), (12, 3), (10, 5), (16, 2)])
def test_decode_kv_head_counts_odd_and_even(gpu, hq, hkv):
    # The grid's workgroup x attends KV head x ^ 1 when the head count is
    # even (the head's XCD is then of the other parity) and head x when it is
    # odd: every head of every sequence must still be attended exactly once.
    print(f"case: decode {hq}/{hkv} heads", flush=True)
    B, bs = 24, 64
    rs = np.random.RandomState(hq * 16 + hkv)
    ctx = rs.randint(1, 700, B).astype(np.int32)
    q, kc, vc, kn, vn, bt = _random_paged(B, hq, hkv, ctx, bs, 7, gpu)
    scale = 128 ** -0.5
    out = fai.decode_paged(q, kc, vc, torch.from_numpy(bt).to(gpu), torch.from_numpy(ctx).to(gpu),
                           scale)
    torch.cuda.synchronize()
    kc_np, vc_np, q_np = np_of(kc), np_of(vc), np_of(q)
    ref = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), scale)
    absv = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), scale, abs_v=True)
    check_attention(out, np.stack([ref[b] for b in range(B)]), what=f"decode {hq}/{hkv}",
                    absv=np.stack([absv[b] for b in range(B)]))


def test_decode_long_context_gqa4_sampled(gpu):
    # bf16, B=64, 32 query / 8 KV heads, context ~ U[16384, 32768]: split-K
    # with the log-sum-exp reduction.  8 sequences are checked against the
    # oracle; all 64 against the same kernel under other partition sizes.
    print("case: decode long context gqa4", flush=True)
    B, hq, hkv, bs = 64, 32, 8, 256
    rs = np.random.RandomState(1)
    ctx = rs.randint(16384, 32769, B).astype(np.int32)
    q, kc, vc, _, _, bt = _random_paged(B, hq, hkv, ctx, bs, 1, gpu, extra_blocks=0)
    scale = 128 ** -0.5
    bt_g = torch.from_numpy(bt).to(gpu)
    ctx_g = torch.from_numpy(ctx).to(gpu)
    out = fai.decode_paged(q, kc, vc, bt_g, ctx_g, scale, max_context_len=32768)
    alt = [fai.decode_paged(q, kc, vc, bt_g, ctx_g, scale, partition_tokens=p)
           for p in (1024, 4096)]
    torch.cuda.synchronize()
    for a in alt:  # partitioning changes only fp32 summation order
        assert float((a.float() - out.float()).abs().max()) <= 2 ** -8
    sample = [0, 7, 19, 33, 40, 51, 60, 63]
    q_np = np_of(q)
    bt_s = bt[sample]
    used = np.unique(bt_s)
    # copy only the sampled sequences' blocks to the host
    remap = {int(b): i for i, b in enumerate(used)}
    kc_np = np_of(kc[torch.from_numpy(used.astype(np.int64)).to(gpu)])
    vc_np = np_of(vc[torch.from_numpy(used.astype(np.int64)).to(gpu)])
    bt_local = np.vectorize(lambda x: remap[int(x)])(bt_s).astype(np.int32)
    for i, b in enumerate(sample):
        rows = (kc_np, vc_np, q_np[b:b + 1], bt_local[i:i + 1], ctx[b:b + 1], bs, [0], scale)
        check_attention(out[b], _oracle_rows(*rows)[0], what=f"long ctx seq {b}",
                        absv=_oracle_rows(*rows, abs_v=True)[0])


def test_reference_slot_layout_via_cache_batch_idx(gpu):
    # The reference's cache [num_slots, max_seq_len, Hkv, D] with
    # cache_batch_idx picking the slot (model/model.py:233-240); max_seq_len
    # 2064 is not a power of two.
    print("case: slot layout", flush=True)
    S, lmax, B, hq, hkv = 12, 2064, 5, 16, 8
    g = torch.Generator(device=gpu).manual_seed(4)
    kc = torch.randn((S, lmax, hkv, 128), generator=g, device=gpu).to(torch.bfloat16)
    vc = torch.randn((S, lmax, hkv, 128), generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn((B, 1, hq, 128), generator=g, device=gpu).to(torch.bfloat16)
    # k/v as strided views of a fused qkv buffer, like model/model.py:221-222
    qkv = torch.randn((B, 1, (hq + 2 * hkv) * 128), generator=g, device=gpu).to(torch.bfloat16)
    k = qkv[..., hq * 128:(hq + hkv) * 128].view(B, 1, hkv, 128)
    v = qkv[..., (hq + hkv) * 128:].view(B, 1, hkv, 128)
    slots = torch.tensor([7, 0, 11, 3, 5], dtype=torch.int64, device=gpu)
    seqlens = torch.tensor([0, 1000, 2063, 17, 255], dtype=torch.int32, device=gpu)
    kc_before = np_of(kc)
    vc_before = np_of(vc)
    out = fai.flash_attn_with_kvcache(q, kc, vc, k=k, v=v, cache_seqlens=seqlens,
                                      cache_batch_idx=slots.int(), softmax_scale=128 ** -0.5)
    torch.cuda.synchronize()
    # oracle: store then attend, slot layout
    bt = slots.cpu().numpy().astype(np.int32).reshape(B, 1)
    ref, new_lens = oracle.decode_append_attend(
        np_of(q).reshape(B, hq, 128), kc_before, vc_before, np_of(k.contiguous()).reshape(B, hkv, 128),
        np_of(v.contiguous()).reshape(B, hkv, 128), bt, seqlens.cpu().numpy(), lmax, 128 ** -0.5)
    assert np.array_equal(np_of(kc), kc_before)  # oracle stored into kc_before in place
    assert np.array_equal(np_of(vc), vc_before)
    absv, _ = oracle.decode_append_attend(
        np_of(q).reshape(B, hq, 128), kc_before, _abs_v(vc_before),
        np_of(k.contiguous()).reshape(B, hkv, 128), _abs_v(np_of(v.contiguous()).reshape(B, hkv, 128)),
        bt, seqlens.cpu().numpy(), lmax, 128 ** -0.5)
    check_attention(out.view(B, hq, 128), ref, what="slot layout", absv=absv)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_gqa_groups_and_dtypes(gpu, hq, hkv, dtype):
    print(f"case: gqa {hq}/{hkv} {dtype}", flush=True)
    B, bs = 6, 32
    ctx = np.array([1, 31, 32, 33, 300, 777], np.int32)
    q, kc, vc, _, _, bt = _random_paged(B, hq, hkv, ctx, bs, 5, gpu, dtype)
    bt_g, ctx_g = torch.from_numpy(bt).to(gpu), torch.from_numpy(ctx).to(gpu)
    for part in (0, 64, 100):
        out = fai.decode_paged(q, kc, vc, bt_g, ctx_g, 0.1, partition_tokens=part)
        torch.cuda.synchronize()
        kc_np, vc_np = f64(kc), f64(vc)
        q_np = f64(q)
        ref = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), 0.1)
        absv = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), 0.1, abs_v=True)
        check_attention(out, np.stack([ref[b] for b in range(B)]), what=f"gqa part={part}",
                        absv=np.stack([absv[b] for b in range(B)]))


def test_decode_edge_cases_and_block_relabelling(gpu):
    print("case: decode edges", flush=True)
    B, hq, hkv, bs = 4, 16, 8, 64
    ctx = np.array([0, 1, 64, 513], np.int32)
    q, kc, vc, _, _, bt = _random_paged(B, hq, hkv, np.maximum(ctx, 1), bs, 6, gpu)
    bt_g, ctx_g = torch.from_numpy(bt).to(gpu), torch.from_numpy(ctx).to(gpu)
    out = fai.decode_paged(q, kc, vc, bt_g, ctx_g, 128 ** -0.5, partition_tokens=128)
    torch.cuda.synchronize()
    assert not out[0].any()  # empty context -> zeros
    v0 = vc[bt[1, 0], 0]  # [hkv, D]; context 1 returns v0 of the KV head
    assert torch.equal(out[1], v0.repeat_interleave(hq // hkv, 0))
    # relabel the physical blocks: identical bits
    pool = kc.shape[0]
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(7))
    kc2 = torch.empty_like(kc)
    vc2 = torch.empty_like(vc)
    kc2[perm.to(gpu)] = kc
    vc2[perm.to(gpu)] = vc
    bt2 = perm.numpy()[bt].astype(np.int32)
    out2 = fai.decode_paged(q, kc2, vc2, torch.from_numpy(bt2).to(gpu), ctx_g, 128 ** -0.5,
                            partition_tokens=128)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


@pytest.mark.parametrize("B", [700, 1024, 1025])
def test_decode_many_sequences_dispatch_order(gpu, B):
    # Up to 1024 sequences the kernel dispatches them longest-first through a
    # rank -> sequence mapping every workgroup derives on its own; a mapping
    # that is not a bijection would leave some sequence's output unwritten.
    # 1025 sequences take the identity order.
    print(f"case: decode dispatch order B={B}", flush=True)
    rs = np.random.RandomState(B)
    hq, hkv, bs = 8, 2, 16
    ctx = rs.randint(1, 200, B).astype(np.int32)
    ctx[rs.randint(B, size=20)] = 200  # ties in the longest class
    q, kc, vc, _, _, bt = _random_paged(B, hq, hkv, ctx, bs, B, gpu)
    out = torch.full((B, hq, 128), float("nan"), device=gpu, dtype=torch.bfloat16)
    fai.decode_paged(q, kc, vc, torch.from_numpy(bt).to(gpu), torch.from_numpy(ctx).to(gpu), 0.1,
                     max_context_len=200, out=out)
    torch.cuda.synchronize()
    kc_np, vc_np, q_np = f64(kc), f64(vc), f64(q)
    ref = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), 0.1)
    absv = _oracle_rows(kc_np, vc_np, q_np, bt, ctx, bs, range(B), 0.1, abs_v=True)
    check_attention(out, np.stack([ref[b] for b in range(B)]), what=f"B={B}",
                    absv=np.stack([absv[b] for b in range(B)]))


def test_decode_long_context_all_sequences_vs_torch_fp32(gpu):
    """Config 4 at full size: all 64 sequences (32 query / 8 KV heads,
    context U[16384, 32768], block 256, split-K + log-sum-exp reduction)
    against a plain fp32 torch reference of the same op on the GPU
    (softmax(scale q K^T) V per sequence, KV heads repeated for GQA, the
    probabilities' bf16 rounding bounded per element as in check_attention)."""
    print("case: decode long context gqa4, all 64 sequences vs fp32 torch", flush=True)
    B, hq, hkv, bs = 64, 32, 8, 256
    rs = np.random.RandomState(1)
    ctx = rs.randint(16384, 32769, B).astype(np.int32)
    q, kc, vc, _, _, bt = _random_paged(B, hq, hkv, ctx, bs, 1, gpu, extra_blocks=0)
    scale = 128 ** -0.5
    out = fai.decode_paged(q, kc, vc, torch.from_numpy(bt).to(gpu), torch.from_numpy(ctx).to(gpu),
                           scale, max_context_len=32768)
    torch.cuda.synchronize()
    g = hq // hkv
    worst = 0.0
    for b in range(B):
        n = int(ctx[b])
        blocks = torch.from_numpy(bt[b, :-(-n // bs)].astype(np.int64)).to(gpu)
        k = kc[blocks].reshape(-1, hkv, 128)[:n].float()            # [n, hkv, D]
        v = vc[blocks].reshape(-1, hkv, 128)[:n].float()
        qh = q[b].float().view(hkv, g, 128)                         # [hkv, g, D]
        s = torch.matmul(qh, k.permute(1, 2, 0).contiguous()) * scale   # [hkv, g, n]
        p = torch.softmax(s, dim=-1)
        vt = v.permute(1, 0, 2).contiguous()                        # [hkv, n, D]
        ref = torch.matmul(p, vt).reshape(hq, 128)
        absv = torch.matmul(p, vt.abs()).reshape(hq, 128)
        err = (out[b].float() - ref).abs()
        lim = 2.0 ** -8 * (ref.abs() + absv) + 1e-3
        assert bool((err <= lim).all()), f"sequence {b}: {float((err - lim).max()):.3e} over the bound"
        worst = max(worst, float(err.max()))
    assert worst <= 2e-2
    print(f"max-abs error over all 64 sequences {worst:.3e}", flush=True)


@pytest.mark.parametrize("dtype,hq,hkv,part", [
    (torch.bfloat16, 16, 8, 0), (torch.bfloat16, 32, 8, 512), (torch.float16, 16, 8, 256),
    (torch.float32, 16, 8, 0)])
def test_decode_constant_values_return_that_value(gpu, dtype, hq, hkv, part):
    """Every cached V row of KV head h equal to u_h (and the appended one too):
    each query head returns u_h, whatever the scores and the partitioning
    (split-K partials merged by their log-sum-exp).  bf16/fp16: within one
    unit in the last place (the probabilities are rounded before the PV
    product and the row sum is taken over the rounded values); fp32: within
    1e-5 relative, the bound of the other fp32 checks (the PV sum and the row
    sum add the same terms in different orders)."""
    print(f"case: decode constant V {dtype} hq={hq} hkv={hkv} part={part}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(12)
    rs = np.random.RandomState(12)
    B, bs = 24, 64
    ctx = rs.randint(1, 3000, B).astype(np.int32)
    ctx[:3] = [1, bs, bs + 1]
    need = -(-ctx // bs)
    pool = int(need.sum()) + 3
    perm = rs.permutation(pool).astype(np.int32)
    bt = np.zeros((B, int(need.max())), np.int32)
    k0 = 0
    for b in range(B):
        bt[b, :need[b]] = perm[k0:k0 + need[b]]
        k0 += need[b]
    u = torch.randn((hkv, 128), generator=g, device=gpu).to(dtype)
    kc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu).to(dtype)
    vc = u.expand(pool, bs, hkv, 128).contiguous()
    q = (3.0 * torch.randn((B, 1, hq, 128), generator=g, device=gpu)).to(dtype)
    kn = torch.randn((B, 1, hkv, 128), generator=g, device=gpu).to(dtype)
    vn = u.expand(B, 1, hkv, 128).contiguous()
    seqlens = torch.from_numpy(ctx - 1).to(gpu)
    mcl = int(ctx.max())
    out = fai.flash_attn_with_kvcache(q, kc, vc, k=kn, v=vn, cache_seqlens=seqlens,
                                      block_table=torch.from_numpy(bt).to(gpu),
                                      num_splits=(mcl // part if part else 0))
    torch.cuda.synchronize()
    want = u.repeat_interleave(hq // hkv, dim=0).float().expand(B, hq, 128)
    err = (out.view(B, hq, 128).float() - want).abs()
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 1e-5}[dtype]
    bad = err > ulp * want.abs()
    assert not bad.any(), f"{int(bad.sum())} values beyond one ulp (max err {float(err.max()):.3e})"
    print(f"  exact: {bool((err == 0).all())}, max err {float(err.max()):.3e}", flush=True)

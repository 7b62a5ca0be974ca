"""GPU parity of the varlen prefill kernel (and the store in the same call)
against the oracle: committed fixture, the 8 x 1024 Qwen3-0.6B layer at full
size, ragged/empty segments, every GQA group, fp16, non-causal, Lq != Lk,
and the padded flash_attn_func surface."""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import flash_attn_interface as fai, paged
from gpu_util import bytes_of, check_attention, f64, np_of, t_of

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def test_tiny_prefill_fixture(gpu):
    print("case: tiny prefill fixture", flush=True)
    fx = np.load(GOLD / "tiny_prefill_bf16.npz")
    q, k, v = (t_of(fx[n], gpu) for n in ("q", "k", "v"))
    cu = torch.from_numpy(fx["cu_seqlens"]).to(gpu)
    L = int(np.diff(fx["cu_seqlens"]).max())
    out = fai.flash_attn_varlen_func(q, k, v, cu, cu, L, L, softmax_scale=float(fx["scale"]),
                                     causal=True)
    torch.cuda.synchronize()
    absv = oracle.varlen_attention(fx["q"], fx["k"], np.abs(oracle.bf16_bits_to_f32(fx["v"])),
                                   fx["cu_seqlens"], scale=float(fx["scale"]))
    check_attention(out, fx["out"], what="tiny prefill", absv=absv)


def test_prefill_8x1024_with_store_full_size(gpu):
    # Qwen3-0.6B attention shape: 16/8 heads, D=128, 8 packed sequences of
    # 1024 tokens; q/k/v ~ N(0,1) bf16 with v a strided view of the fused qkv
    # buffer; K/V written into a paged cache (block 256, shuffled ids) through
    # slot_mapping in the same call.
    print("case: prefill 8x1024 + store", flush=True)
    N, hq, hkv, d, bs = 8192, 16, 8, 128, 256
    g = torch.Generator(device=gpu).manual_seed(0)
    qkv = torch.randn((N, (hq + 2 * hkv) * d), generator=g, device=gpu).to(torch.bfloat16)
    q = qkv[:, :hq * d].view(N, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(N, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(N, hkv, d)
    rs = np.random.RandomState(0)
    perm = rs.permutation(40).astype(np.int32)  # 32 blocks used out of 40
    bt = perm[:32].reshape(8, 4)
    cu, _, sm = paged.build_prefill_metadata([1024] * 8, bt, bs, gpu)
    kc = torch.randn((40, bs, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    vc = torch.randn((40, bs, hkv, d), generator=g, device=gpu).to(torch.bfloat16)
    kc_ref, vc_ref = np_of(kc).copy(), np_of(vc).copy()
    out = fai.varlen_prefill_with_kvcache(q, k, v, cu, 1024, kc, vc, sm,
                                          softmax_scale=d ** -0.5, causal=True)
    torch.cuda.synchronize()
    sm_np = sm.cpu().numpy()
    oracle.kv_store(kc_ref, np_of(k), sm_np)
    oracle.kv_store(vc_ref, np_of(v), sm_np)
    assert np.array_equal(bytes_of(kc), kc_ref.view(np.uint8))
    assert np.array_equal(bytes_of(vc), vc_ref.view(np.uint8))
    cu_np = cu.cpu().numpy()
    ref = oracle.varlen_attention(f64(q), f64(k), f64(v), cu_np, scale=d ** -0.5)
    absv = oracle.varlen_attention(f64(q), f64(k), np.abs(f64(v)), cu_np, scale=d ** -0.5)
    err = check_attention(out, ref, what="prefill 8x1024", absv=absv)
    print(f"max-abs err {err:.3e}", flush=True)


def _ragged(lens_q, lens_k, hq, hkv, dtype, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    nq, nk = sum(lens_q), sum(lens_k)
    q = torch.randn((nq, hq, 128), generator=g, device=gpu).to(dtype)
    k = torch.randn((nk, hkv, 128), generator=g, device=gpu).to(dtype)
    v = torch.randn((nk, hkv, 128), generator=g, device=gpu).to(dtype)
    cq = torch.tensor(np.concatenate([[0], np.cumsum(lens_q)]), dtype=torch.int32, device=gpu)
    ck = torch.tensor(np.concatenate([[0], np.cumsum(lens_k)]), dtype=torch.int32, device=gpu)
    return q, k, v, cq, ck


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_many_segments_persistent_schedule(gpu, hq, hkv, causal):
    # 200 segments of 0..700 tokens: the persistent grid walks many zigzag
    # rounds with holes in the last one and with q-block ranks that short
    # segments lack (so both the early-loaded candidate and the fallback
    # search pick items).  Every segment against torch SDPA in fp32 (GQA by
    # repeat_interleave), a sample against the oracle.
    print(f"case: many segments {hq}/{hkv} causal={causal}", flush=True)
    rs = np.random.RandomState(7)
    lens = rs.randint(0, 701, 200)
    lens[:4] = [700, 0, 1, 129]
    lens = lens.tolist()
    q, k, v, cq, _ = _ragged(lens, lens, hq, hkv, torch.bfloat16, gpu, 9)
    scale = 128 ** -0.5
    out = fai.flash_attn_varlen_func(q, k, v, cq, cq, max(lens), max(lens), softmax_scale=scale,
                                     causal=causal)
    torch.cuda.synchronize()
    g = hq // hkv
    cu = cq.cpu().numpy()
    sdpa = torch.nn.functional.scaled_dot_product_attention
    worst = 0.0
    for s in range(len(lens)):
        a, b = int(cu[s]), int(cu[s + 1])
        if a == b:
            continue
        qs = q[a:b].float().transpose(0, 1).contiguous()
        ks = k[a:b].float().repeat_interleave(g, 1).transpose(0, 1).contiguous()
        vs = v[a:b].float().repeat_interleave(g, 1).transpose(0, 1).contiguous()
        ref = sdpa(qs, ks, vs, is_causal=causal, scale=scale).transpose(0, 1)
        absv = sdpa(qs, ks, vs.abs(), is_causal=causal, scale=scale).transpose(0, 1)
        err = (out[a:b].float() - ref).abs()
        worst = max(worst, float(err.max()))
        assert bool((err <= 2.0 ** -8 * (ref.abs() + absv) + 1e-3).all()), f"segment {s} (len {b - a})"
    assert worst <= 2e-2, worst
    for s in (0, 3, 17, 99, 150, 199):
        a, b = int(cu[s]), int(cu[s + 1])
        sub = np.array([0, b - a], np.int32)
        ref = oracle.varlen_attention(f64(q[a:b]), f64(k[a:b]), f64(v[a:b]), sub, scale=scale,
                                      causal=causal)
        absv = oracle.varlen_attention(f64(q[a:b]), f64(k[a:b]), np.abs(f64(v[a:b])), sub,
                                       scale=scale, causal=causal)
        check_attention(out[a:b], ref, what=f"segment {s}", absv=absv)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ragged_groups_dtypes(gpu, hq, hkv, dtype, causal):
    print(f"case: ragged {hq}/{hkv} {dtype} causal={causal}", flush=True)
    lens = [1, 5, 31, 32, 33, 0, 127, 128, 129, 300, 64]
    q, k, v, cq, _ = _ragged(lens, lens, hq, hkv, dtype, gpu, 1)
    out = fai.flash_attn_varlen_func(q, k, v, cq, cq, max(lens), max(lens), softmax_scale=0.1,
                                     causal=causal)
    torch.cuda.synchronize()
    ref = oracle.varlen_attention(f64(q), f64(k), f64(v), cq.cpu().numpy(), scale=0.1,
                                  causal=causal)
    absv = oracle.varlen_attention(f64(q), f64(k), np.abs(f64(v)), cq.cpu().numpy(), scale=0.1,
                                   causal=causal)
    check_attention(out, ref, what="ragged", absv=absv)


def test_prefill_bottom_right_causal_lq_ne_lk(gpu):
    # chunked-prefill shape: fewer queries than keys per segment (and one
    # segment with more queries than keys, whose first rows see nothing)
    print("case: lq != lk", flush=True)
    lq, lk = [5, 100, 64, 40], [70, 100, 300, 20]
    q, k, v, cq, ck = _ragged(lq, lk, 16, 8, torch.bfloat16, gpu, 2)
    out = fai.flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), causal=True)
    torch.cuda.synchronize()
    ref = oracle.varlen_attention(f64(q), f64(k), f64(v), cq.cpu().numpy(), ck.cpu().numpy(),
                                  causal=True)
    absv = oracle.varlen_attention(f64(q), f64(k), np.abs(f64(v)), cq.cpu().numpy(),
                                   ck.cpu().numpy(), causal=True)
    check_attention(out, ref, what="lq != lk", absv=absv)
    assert not out[cq[3].item():cq[3].item() + 20].any()  # rows with no visible key


def test_flash_attn_func_padded_batch(gpu):
    print("case: padded flash_attn_func", flush=True)
    g = torch.Generator(device=gpu).manual_seed(3)
    B, T = 3, 200
    q = torch.randn((B, T, 16, 128), generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn((B, T, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn((B, T, 8, 128), generator=g, device=gpu).to(torch.bfloat16)
    out = fai.flash_attn_func(q, k, v, causal=True)
    torch.cuda.synchronize()
    cu = np.arange(0, (B + 1) * T, T, dtype=np.int32)
    qf, kf, vf = (f64(t).reshape(B * T, -1, 128) for t in (q, k, v))
    ref = oracle.varlen_attention(qf, kf, vf, cu)
    absv = oracle.varlen_attention(qf, kf, np.abs(vf), cu)
    check_attention(out.reshape(B * T, 16, 128), ref, what="padded", absv=absv)


def test_decode_equals_last_prefill_row(gpu):
    # invariant: a causal prefill's row i equals a decode over keys 0..i
    print("case: decode == prefill row", flush=True)
    L, hq, hkv, bs = 300, 16, 8, 64
    q, k, v, cq, _ = _ragged([L], [L], hq, hkv, torch.bfloat16, gpu, 4)
    pre = fai.flash_attn_varlen_func(q, k, v, cq, cq, L, L, causal=True)
    nb = (L + bs - 1) // bs
    kc = torch.zeros((nb, bs, hkv, 128), dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    bt = torch.arange(nb, dtype=torch.int32, device=gpu).view(1, nb)
    sm = torch.arange(L, dtype=torch.int64, device=gpu)
    fai.kv_store(k, v, kc, vc, sm)
    rows = [0, 63, 64, 299]
    dec = fai.decode_paged(q[rows].contiguous(), kc, vc, bt.expand(len(rows), nb).contiguous(),
                           torch.tensor([r + 1 for r in rows], dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    diff = (dec.float() - pre[rows].float()).abs().max().item()
    assert diff <= 2 ** -7, diff


def test_empty_sequences_and_understated_max_seqlen_k(gpu):
    print("case: empty sequences, understated max_seqlen_k", flush=True)
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randn((2, 7, 16, 128), generator=g, device=gpu).to(torch.bfloat16)
    none = torch.empty((2, 0, 8, 128), dtype=torch.bfloat16, device=gpu)
    out = fai.flash_attn_func(q, none, none)  # no keys: every row is zero
    torch.cuda.synchronize()
    assert out.shape == q.shape and not out.any()
    assert fai.flash_attn_func(q[:, :0], none, none).shape == (2, 0, 16, 128)
    # A max_seqlen_k below the real key count is a caller error (as in FA2); the
    # kernel clamps every segment to it, so the result is attention over the
    # first max_seqlen_k keys and no read leaves the segment.
    lens_q, lens_k = [40, 9], [300, 120]
    qv, k, v, cq, ck = _ragged(lens_q, lens_k, 16, 8, torch.bfloat16, gpu, 6)
    out = fai.flash_attn_varlen_func(qv, k, v, cq, ck, 40, 100, causal=False)
    torch.cuda.synchronize()
    kk, vv = f64(k), f64(v)
    ckn = ck.cpu().numpy()
    keep = np.concatenate([np.arange(ckn[s], ckn[s] + 100) for s in range(2)])
    ck_t = np.array([0, 100, 200], np.int32)
    ref = oracle.varlen_attention(f64(qv), kk[keep], vv[keep], cq.cpu().numpy(), ck_t, causal=False)
    absv = oracle.varlen_attention(f64(qv), kk[keep], np.abs(vv[keep]), cq.cpu().numpy(), ck_t,
                                   causal=False)
    check_attention(out, ref, what="clamped keys", absv=absv)


@pytest.mark.parametrize("hq,hkv,dtype", [(8, 8, torch.bfloat16), (16, 8, torch.bfloat16),
                                           (32, 8, torch.bfloat16), (64, 8, torch.bfloat16),
                                           (16, 8, torch.float16), (64, 8, torch.float16),
                                           # odd KV head counts (each kernel, each group)
                                           (6, 3, torch.bfloat16), (12, 3, torch.bfloat16),
                                           (24, 3, torch.bfloat16), (5, 5, torch.bfloat16),
                                           (10, 5, torch.float16)])
@pytest.mark.parametrize("causal", [True, False])
def test_store_in_the_attention_kernel_covers_every_token(gpu, hq, hkv, dtype, causal):
    # One cu_seqlens array for queries and keys: the store runs inside the
    # attention kernel, each work item writing its own q-block's K/V rows.
    # Tokens before cu[0] and after cu[n], empty segments, padding slots (-1)
    # and a max_seqlen below the longest segment (q-blocks no work item owns)
    # must still be stored exactly as index_copy_ would.
    print(f"case: store in the attention kernel hq={hq} hkv={hkv} {dtype} causal={causal}", flush=True)
    lens, lead, tail = [0, 37, 300, 1, 129, 0, 64], 3, 5
    cu_np = (np.concatenate([[0], np.cumsum(lens)]) + lead).astype(np.int32)
    N, d = lead + sum(lens) + tail, 128
    g = torch.Generator(device=gpu).manual_seed(7)
    qkv = torch.randn((N, (hq + 2 * hkv) * d), generator=g, device=gpu).to(dtype)
    q = qkv[:, :hq * d].view(N, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].contiguous().view(N, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(N, hkv, d)
    cu = torch.from_numpy(cu_np).to(gpu)
    rows = N + 40
    rs = np.random.RandomState(hq + int(causal))
    for max_len in (300, 100):
        sm_np = rs.permutation(rows)[:N].astype(np.int64)
        sm_np[rs.rand(N) < 0.1] = -1
        kc = torch.randn((rows, hkv, d), generator=g, device=gpu).to(dtype)
        vc = torch.randn((rows, hkv, d), generator=g, device=gpu).to(dtype)
        kc_ref, vc_ref = np_of(kc).copy(), np_of(vc).copy()
        out = fai.varlen_prefill_with_kvcache(q, k, v, cu, max_len, kc, vc,
                                              torch.from_numpy(sm_np).to(gpu), causal=causal)
        torch.cuda.synchronize()
        oracle.kv_store(kc_ref, np_of(k), sm_np)
        oracle.kv_store(vc_ref, np_of(v), sm_np)
        assert np.array_equal(bytes_of(kc), kc_ref.view(np.uint8)), f"k cache, max_seqlen {max_len}"
        assert np.array_equal(bytes_of(vc), vc_ref.view(np.uint8)), f"v cache, max_seqlen {max_len}"
        if max_len >= max(lens):
            a, b = int(cu_np[0]), int(cu_np[-1])
            ref = oracle.varlen_attention(f64(q), f64(k), f64(v), cu_np, causal=causal)[a:b]
            absv = oracle.varlen_attention(f64(q), f64(k), np.abs(f64(v)), cu_np, causal=causal)[a:b]
            check_attention(out[a:b], ref, what="attention beside the store", absv=absv)


def _unsplit(q, k, v, cq, ck, Lq, Lk, causal, scale):
    """aac_prefill_varlen without a workspace: the same kernel, never split."""
    from awesome_acceleration_amd import _lib
    out = torch.empty_like(q)
    rc = _lib.lib().aac_prefill_varlen(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0), v.stride(0),
        cq.data_ptr(), ck.data_ptr(), cq.shape[0] - 1, Lq, Lk, q.shape[1], k.shape[1], 128, scale,
        int(causal), out.data_ptr(), out.stride(0), None, 0, _lib.AAC_DTYPE[q.dtype],
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.lib().aac_strerror(rc)
    return out


@pytest.mark.parametrize("lens_q,lens_k,hq,hkv,causal,dtype", [
    ([1024], [1024], 16, 8, True, torch.bfloat16),        # one request: 64 items for 256 CUs
    ([2048] * 2, [2048] * 2, 8, 4, True, torch.bfloat16),  # a TP=2 rank's heads, 2 requests
    ([300, 1000], [300, 1000], 16, 8, True, torch.bfloat16),
    ([512], [2048], 32, 8, False, torch.bfloat16),          # non-causal, Lq != Lk
    ([1500], [1500], 8, 8, True, torch.float16),
    ([200, 5, 600], [260, 5, 1200], 16, 4, True, torch.bfloat16),  # Lq < Lk, bottom-right
    ([4096], [4096], 8, 1, True, torch.bfloat16),          # group 8: one 32-query slot, 8 heads
])
def test_split_keys_match_unsplit_and_oracle(gpu, lens_q, lens_k, hq, hkv, causal, dtype):
    """Few work items: the key range of every item is split over several
    workgroups and merged (log-sum-exp) by the last piece to finish.  The
    result matches the oracle to the same bound as the unsplit kernel, is
    close to it, and is the same on every call (fixed merge order; the
    per-item counters are back at zero after each call)."""
    print(f"case: split prefill q={lens_q} k={lens_k} {hq}/{hkv} causal={causal} {dtype}",
          flush=True)
    from awesome_acceleration_amd import _lib
    q, k, v, cq, ck = _ragged(lens_q, lens_k, hq, hkv, dtype, gpu, seed=31)
    Lq, Lk = max(lens_q), max(lens_k)
    ws = _lib.lib().aac_prefill_workspace_bytes(len(lens_q), Lq, Lk, hq, hkv, 128, int(causal))
    assert ws > 0, "the plan should split this shape"
    scale = 128 ** -0.5
    outs = [fai.flash_attn_varlen_func(q, k, v, cq, ck, Lq, Lk, causal=causal) for _ in range(3)]
    base = _unsplit(q, k, v, cq, ck, Lq, Lk, causal, scale)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    cq_np, ck_np = cq.cpu().numpy(), ck.cpu().numpy()
    ref = oracle.varlen_attention(f64(q), f64(k), f64(v), cq_np, ck_np, scale=scale, causal=causal)
    absv = oracle.varlen_attention(f64(q), f64(k), np.abs(f64(v)), cq_np, ck_np, scale=scale,
                                   causal=causal)
    check_attention(outs[0], ref, what="split", absv=absv)
    check_attention(base, ref, what="unsplit", absv=absv)
    assert float((outs[0].float() - base.float()).abs().max()) <= 2 ** -6


def test_split_workspace_reused_by_a_call_with_more_items(gpu):
    """Regression: a split call with few items leaves partial results in the
    shared workspace; a later split call with more items keeps its item
    counters in the same fixed region at the start, which no partial result
    ever overwrites, so every row of the later call is written."""
    print("case: split workspace reuse, few then many items", flush=True)
    from awesome_acceleration_amd import _lib
    small = _ragged([1024], [1024], 16, 8, torch.bfloat16, gpu, seed=41)      # 64 items, split
    big = _ragged([2048] * 2, [2048] * 2, 8, 4, torch.bfloat16, gpu, seed=42)  # 128 items, split
    assert _lib.lib().aac_prefill_workspace_bytes(1, 1024, 1024, 16, 8, 128, 1) > 0
    assert _lib.lib().aac_prefill_workspace_bytes(2, 2048, 2048, 8, 4, 128, 1) > 0
    for (q, k, v, cq, ck) in (small, big, small, big):
        L = int((cq[1:] - cq[:-1]).max())
        out = torch.full_like(q, float("nan"))
        out.copy_(fai.flash_attn_varlen_func(q, k, v, cq, ck, L, L, causal=True))
        base = _unsplit(q, k, v, cq, ck, L, L, True, 128 ** -0.5)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        assert float((out.float() - base.float()).abs().max()) <= 2 ** -6


@pytest.mark.parametrize("hq,hkv,dtype,causal,lens", [
    (16, 8, torch.bfloat16, True, [1024] * 8),             # the 8 x 1024 layer
    (32, 8, torch.bfloat16, True, [3000, 17, 700]),         # GQA-4, ragged
    (16, 8, torch.float16, False, [300, 1500]),            # fp16, non-causal
    (16, 8, torch.bfloat16, True, [2048]),                  # one request: split key ranges
])
def test_constant_values_return_that_value(gpu, hq, hkv, dtype, causal, lens):
    """Every V row of KV head h equal to one vector u_h: every query row returns
    u_h (its softmax weights sum to one), whatever the scores.  The kernel
    normalises by the row sum of the very probabilities it rounds for the PV
    product, so the result is u_h to the last bit; a dropped, doubled or
    misplaced key, tile or split piece, or a row sum taken over other
    probabilities, moves it."""
    print(f"case: constant V hq={hq} hkv={hkv} {dtype} causal={causal} lens={lens}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(11)
    N = sum(lens)
    q = (3.0 * torch.randn((N, hq, 128), generator=g, device=gpu)).to(dtype)
    k = torch.randn((N, hkv, 128), generator=g, device=gpu).to(dtype)
    u = torch.randn((hkv, 128), generator=g, device=gpu).to(dtype)
    v = u.expand(N, hkv, 128).contiguous()
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    want = u.repeat_interleave(hq // hkv, dim=0).expand(N, hq, 128)
    outs = {"varlen": fai.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=causal)}
    if causal:
        kc = torch.zeros((N, hkv, 128), dtype=dtype, device=gpu)
        vc = torch.zeros_like(kc)
        slots = torch.randperm(N, generator=g, device=gpu)
        outs["with store"] = fai.varlen_prefill_with_kvcache(q, k, v, cu, max(lens), kc, vc, slots)
    torch.cuda.synchronize()
    for name, out in outs.items():
        assert torch.equal(out, want), \
            f"{name}: max |out - u| = {float((out.float() - want.float()).abs().max()):.3e}"


def test_split_prefills_on_two_streams_keep_their_own_workspaces(gpu):
    """Two split-key prefills launched on two streams with nothing ordering
    them: each stream has its own workspace (per-item counters and partial
    results), so each result equals the same call made alone, bit for bit."""
    print("case: split prefills on two streams", flush=True)
    from awesome_acceleration_amd import _lib
    a = _ragged([2048], [2048], 16, 8, torch.bfloat16, gpu, seed=51)
    b = _ragged([1536], [1536], 16, 8, torch.bfloat16, gpu, seed=52)
    assert _lib.lib().aac_prefill_workspace_bytes(1, 2048, 2048, 16, 8, 128, 1) > 0
    assert _lib.lib().aac_prefill_workspace_bytes(1, 1536, 1536, 16, 8, 128, 1) > 0

    def call(x):
        q, k, v, cq, ck = x
        L = int((cq[1:] - cq[:-1]).max())
        return fai.flash_attn_varlen_func(q, k, v, cq, ck, L, L, causal=True)

    alone = (call(a), call(b))
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=gpu), torch.cuda.Stream(device=gpu)
    for rnd in range(4):
        s1.wait_stream(torch.cuda.current_stream(gpu))
        s2.wait_stream(torch.cuda.current_stream(gpu))
        with torch.cuda.stream(s1):
            o1 = call(a)
        with torch.cuda.stream(s2):
            o2 = call(b)
        torch.cuda.synchronize()
        assert torch.equal(o1, alone[0]), f"stream 1, round {rnd}"
        assert torch.equal(o2, alone[1]), f"stream 2, round {rnd}"
    keys = {k for k in fai._pf_ws if k[0] == gpu.index or gpu.index is None}
    assert {s1.cuda_stream, s2.cuda_stream} <= {k[1] for k in keys}

"""Seeded random sweeps of the three kernels against the oracle, mixing what
the targeted tests vary one at a time: segment lengths (empty, Lq != Lk),
token strides, GQA group, dtype, softmax scale, causal or not (prefill);
batch, context length, block size (power of two or not), partitioning,
dtype, append (decode); slot mappings with padding and repeated rounds (KV store).
Long segments (split key ranges) and the store inside the attention kernel
are checked against a float64 torch restatement on the GPU, at shapes the
numpy oracle would take minutes over.

Every case prints its parameters before the GPU call; the seeds are fixed, so
a failure names a reproducible case.  ``AAC_RANDOM_SEEDS=N`` widens each sweep
to seeds ``0..N-1`` (default 12; the KV-store sweep runs half as many); a
1000-seed run of all five sweeps (4500 cases) takes about four minutes on one
MI355X."""
import os

import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import _lib
from awesome_acceleration_amd import flash_attn_interface as fai
from gpu_util import bytes_of, check_attention, f64, np_of

pytestmark = pytest.mark.gpu

_SEEDS = max(1, int(os.environ.get("AAC_RANDOM_SEEDS", "12")))

_DT = {0: torch.bfloat16, 1: torch.float16, 2: torch.float32}


def _abs64(a: np.ndarray) -> np.ndarray:
    """|a| in float64 (uint16 arrays are bf16 bit patterns)."""
    return np.abs(oracle.bf16_bits_to_f32(a) if a.dtype == np.uint16 else a).astype(np.float64)


def _same_bytes(t: torch.Tensor, a: np.ndarray) -> bool:
    return np.array_equal(bytes_of(t).reshape(-1), np.ascontiguousarray(a).view(np.uint8).reshape(-1))


def _strided(n, h, extra, g, dtype, gpu):
    """[n, h, 128] view with a token stride of (h + extra) * 128 elements."""
    buf = torch.randn((n, (h + extra) * 128), generator=g, device=gpu).to(dtype)
    return buf[:, :h * 128].view(n, h, 128) if extra else buf.view(n, h, 128)


@pytest.mark.parametrize("seed", range(_SEEDS))
def test_prefill_random(gpu, seed):
    rs = np.random.RandomState(1000 + seed)
    hkv = int(rs.choice([1, 2, 4, 8]))
    grp = int(rs.choice([1, 2, 4, 8]))
    hq = hkv * grp
    nseg = int(rs.randint(1, 7))
    lq = [int(x) for x in rs.randint(0, 260, nseg)]
    lq[int(rs.randint(nseg))] = int(rs.choice([0, 1, 31, 32, 33, 129]))
    causal = bool(rs.randint(2))
    # keys: Lk >= Lq for the causal cases (bottom-right alignment), anything otherwise
    lk = [q_ + int(rs.randint(0, 70)) if causal else int(rs.randint(0, 300)) for q_ in lq]
    dtype = _DT[int(rs.randint(2))]
    scale = float(rs.uniform(0.05, 0.2))
    ex = [int(rs.choice([0, 0, 3])) for _ in range(3)]
    print(f"case: prefill seed={seed} hq={hq} hkv={hkv} lq={lq} lk={lk} causal={causal} "
          f"{dtype} scale={scale:.3f} extra={ex}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(seed)
    q = _strided(sum(lq), hq, ex[0], g, dtype, gpu)
    k = _strided(sum(lk), hkv, ex[1], g, dtype, gpu)
    v = _strided(sum(lk), hkv, ex[2], g, dtype, gpu)
    cq = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32, device=gpu)
    ck = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32, device=gpu)
    out = fai.flash_attn_varlen_func(q, k, v, cq, ck, max(lq), max(lk), softmax_scale=scale,
                                     causal=causal)
    torch.cuda.synchronize()
    cqn, ckn = cq.cpu().numpy(), ck.cpu().numpy()
    ref = oracle.varlen_attention(f64(q), f64(k), f64(v), cqn, ckn, scale=scale, causal=causal)
    absv = oracle.varlen_attention(f64(q), f64(k), np.abs(f64(v)), cqn, ckn, scale=scale,
                                   causal=causal)
    check_attention(out, ref, what=f"prefill seed {seed}", absv=absv)


def _paged(rs, ctx, bs, hkv, dtype, g, gpu, spare=2):
    need = [max(1, -(-int(c) // bs)) for c in ctx]
    pool = sum(need) + spare
    perm = rs.permutation(pool).astype(np.int32)
    bt = np.zeros((len(ctx), max(need) + int(rs.randint(0, 3))), np.int32)
    k0 = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n
    kc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu).to(dtype)
    vc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu).to(dtype)
    return kc, vc, bt


@pytest.mark.parametrize("seed", range(_SEEDS))
def test_decode_random(gpu, seed):
    rs = np.random.RandomState(2000 + seed)
    hkv = int(rs.choice([1, 2, 4, 8]))
    hq = hkv * int(rs.choice([1, 2, 4, 8]))
    B = int(rs.randint(1, 41))
    bs = int(rs.choice([16, 32, 64, 100, 128, 256]))
    ctx = rs.randint(1, 2500, B).astype(np.int32)
    ctx[int(rs.randint(B))] = int(rs.choice([1, bs - 1, bs, bs + 1]))
    dtype = _DT[int(rs.randint(3))]
    part = int(rs.choice([0, 0, 64, 256, 1000]))
    append = bool(rs.randint(2))
    scale = float(rs.uniform(0.05, 0.2))
    print(f"case: decode seed={seed} B={B} hq={hq} hkv={hkv} bs={bs} {dtype} part={part} "
          f"append={append} ctx_max={int(ctx.max())}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(100 + seed)
    kc, vc, bt = _paged(rs, ctx, bs, hkv, dtype, g, gpu)
    q = torch.randn((B, hq, 128), generator=g, device=gpu).to(dtype)
    bt_g = torch.from_numpy(bt).to(gpu)
    kc0, vc0 = np_of(kc), np_of(vc)
    if append:
        kn = torch.randn((B, 1, hkv, 128), generator=g, device=gpu).to(dtype)
        vn = torch.randn((B, 1, hkv, 128), generator=g, device=gpu).to(dtype)
        seqlens = torch.from_numpy(ctx - 1).to(gpu)
        out = fai.flash_attn_with_kvcache(q.view(B, 1, hq, 128), kc, vc, k=kn, v=vn,
                                          cache_seqlens=seqlens, block_table=bt_g,
                                          softmax_scale=scale,
                                          num_splits=(int(ctx.max()) // part if part else 0))
        torch.cuda.synchronize()
        kce, vce = kc0.copy(), vc0.copy()
        ref, _ = oracle.decode_append_attend(np_of(q), kce, vce, np_of(kn).reshape(B, hkv, 128),
                                             np_of(vn).reshape(B, hkv, 128), bt, ctx - 1, bs,
                                             scale)
        assert np.array_equal(np_of(kc), kce) and np.array_equal(np_of(vc), vce), "appended cache"
        absv = oracle.paged_decode(np_of(q), kce, _abs64(vce), bt, ctx, bs, scale)
        out = out.view(B, hq, 128)
    else:
        ctx_g = torch.from_numpy(ctx).to(gpu)
        out = fai.decode_paged(q, kc, vc, bt_g, ctx_g, scale, partition_tokens=part)
        torch.cuda.synchronize()
        ref = oracle.paged_decode(np_of(q), kc0, vc0, bt, ctx, bs, scale)
        absv = oracle.paged_decode(np_of(q), kc0, _abs64(vc0), bt, ctx, bs, scale)
    check_attention(out, ref, what=f"decode seed {seed}", absv=absv)


@pytest.mark.parametrize("seed", range(max(1, _SEEDS // 2)))
def test_kv_store_random(gpu, seed):
    rs = np.random.RandomState(3000 + seed)
    hkv = int(rs.choice([1, 2, 8]))
    dtype = _DT[int(rs.randint(3))]
    rows = int(rs.randint(50, 3000))
    print(f"case: kv store seed={seed} hkv={hkv} {dtype} rows={rows}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(200 + seed)
    kc = torch.randn((rows, hkv, 128), generator=g, device=gpu).to(dtype)
    vc = torch.randn((rows, hkv, 128), generator=g, device=gpu).to(dtype)
    ke, ve = np_of(kc).copy(), np_of(vc).copy()
    for rnd in range(3):  # later rounds overwrite rows written earlier
        n = int(rs.randint(0, rows))
        sm = rs.permutation(rows)[:n].astype(np.int64)
        sm[rs.rand(n) < 0.1] = -1  # padding tokens
        k = torch.randn((n, hkv, 128), generator=g, device=gpu).to(dtype)
        v = torch.randn((n, hkv, 128), generator=g, device=gpu).to(dtype)
        fai.kv_store(k, v, kc, vc, torch.from_numpy(sm).to(gpu))
        torch.cuda.synchronize()
        oracle.kv_store(ke, np_of(k), sm)
        oracle.kv_store(ve, np_of(v), sm)
        assert _same_bytes(kc, ke), f"k cache round {rnd}"
        assert _same_bytes(vc, ve), f"v cache round {rnd}"


def _torch_reference(q, k, v, lq, lk, scale, causal):
    """Float64 restatement on the GPU of the oracle's varlen attention (the
    same bottom-right causal mask and GQA head mapping), for shapes the numpy
    oracle would take minutes over; returns the attention and the same with
    |V| (the rounding-bound term of check_attention)."""
    G = q.shape[1] // k.shape[1]
    outs, absvs = [], []
    oq = ok = 0
    for a, b in zip(lq, lk):
        Q = q[oq:oq + a].double().permute(1, 0, 2).contiguous()
        K = k[ok:ok + b].double().repeat_interleave(G, dim=1).permute(1, 2, 0).contiguous()
        V = v[ok:ok + b].double().repeat_interleave(G, dim=1).permute(1, 0, 2).contiguous()
        s = torch.bmm(Q, K) * scale
        if causal:
            i = torch.arange(a, device=q.device).view(a, 1)
            j = torch.arange(b, device=q.device).view(1, b)
            s = s.masked_fill(j > i + (b - a), float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)  # no visible key: zeros
        outs.append(torch.bmm(p, V).permute(1, 0, 2))
        absvs.append(torch.bmm(p, V.abs()).permute(1, 0, 2))
        oq += a
        ok += b
    return torch.cat(outs).cpu().numpy(), torch.cat(absvs).cpu().numpy()


def _unsplit(q, k, v, cq, ck, mq, mk, scale, causal):
    """aac_prefill_varlen without a workspace: the key ranges are never split."""
    out = torch.empty_like(q)
    rc = _lib.lib().aac_prefill_varlen(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0), v.stride(0),
        cq.data_ptr(), ck.data_ptr(), cq.shape[0] - 1, mq, mk, q.shape[1], k.shape[1], 128, scale,
        int(causal), out.data_ptr(), out.stride(0), None, 0, 0 if q.dtype == torch.bfloat16 else 1,
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "aac_prefill_varlen")
    return out


@pytest.mark.parametrize("seed", range(_SEEDS))
def test_prefill_split_random(gpu, seed):
    """Few long segments (the shapes whose key ranges are split over two
    workgroups when the plan asks for it): the split result equals itself on a
    second call and both it and the unsplit kernel meet the parity bound."""
    rs = np.random.RandomState(7000 + seed)
    hkv = int(rs.choice([1, 2, 4, 8]))
    hq = hkv * int(rs.choice([1, 2, 4, 8]))
    nseg = int(rs.randint(1, 4))
    lq = [int(x) for x in rs.randint(700, 4200, nseg)]
    if nseg > 1 and rs.randint(3) == 0:
        lq[int(rs.randint(nseg))] = int(rs.choice([0, 1, 63, 300]))
    causal = bool(rs.randint(3))
    lk = [x + int(rs.randint(0, 300)) if causal else int(rs.randint(1, 4200)) for x in lq]
    dtype = _DT[int(rs.randint(2))]
    scale = float(rs.uniform(0.05, 0.2))
    mq, mk = max(lq), max(lk)
    ws = _lib.lib().aac_prefill_workspace_bytes(nseg, mq, mk, hq, hkv, 128, int(causal))
    print(f"case: split prefill seed={seed} hq={hq} hkv={hkv} lq={lq} lk={lk} causal={causal} "
          f"{dtype} workspace={ws}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(seed)
    q = torch.randn((sum(lq), hq, 128), generator=g, device=gpu).to(dtype)
    k = torch.randn((sum(lk), hkv, 128), generator=g, device=gpu).to(dtype)
    v = torch.randn((sum(lk), hkv, 128), generator=g, device=gpu).to(dtype)
    cq = torch.tensor(np.concatenate([[0], np.cumsum(lq)]), dtype=torch.int32, device=gpu)
    ck = torch.tensor(np.concatenate([[0], np.cumsum(lk)]), dtype=torch.int32, device=gpu)
    out = fai.flash_attn_varlen_func(q, k, v, cq, ck, mq, mk, softmax_scale=scale, causal=causal)
    again = fai.flash_attn_varlen_func(q, k, v, cq, ck, mq, mk, softmax_scale=scale, causal=causal)
    whole = _unsplit(q, k, v, cq, ck, mq, mk, scale, causal)
    torch.cuda.synchronize()
    assert torch.equal(out, again), "split result differs between two calls"
    ref, absv = _torch_reference(q, k, v, lq, lk, scale, causal)
    check_attention(out, ref, what=f"split prefill seed {seed}", absv=absv)
    check_attention(whole, ref, what=f"unsplit prefill seed {seed}", absv=absv)


@pytest.mark.parametrize("seed", range(_SEEDS))
def test_prefill_store_random(gpu, seed):
    """The store inside the causal self-attention kernel at random segment
    lengths, GQA groups, tokens before cu[0] and after cu[n], padding slots and
    (in some cases) an understated max_seqlen: the caches equal the oracle's
    store byte for byte, and the attention equals the attention kernel's."""
    rs = np.random.RandomState(8000 + seed)
    hkv = int(rs.choice([1, 2, 4, 8]))
    hq = hkv * int(rs.choice([1, 2, 4, 8]))
    nseg = int(rs.randint(1, 7))
    lens = [int(x) for x in rs.randint(1, 1500, nseg)]
    if rs.randint(3) == 0:
        lens[int(rs.randint(nseg))] = int(rs.choice([1, 2, 255, 256, 257]))
    N = sum(lens)
    lead, tail = int(rs.choice([0, 0, 5])), int(rs.choice([0, 0, 7]))
    mseq = max(1, max(lens) - (int(rs.randint(1, 200)) if rs.randint(4) == 0 else 0))
    dtype = _DT[int(rs.randint(2))]
    scale = float(rs.uniform(0.05, 0.2))
    rows = N + lead + tail + int(rs.randint(0, 500))
    T = N + lead + tail
    print(f"case: prefill store seed={seed} hq={hq} hkv={hkv} lens={lens} lead={lead} tail={tail} "
          f"max_seqlen={mseq} rows={rows} {dtype}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(300 + seed)
    q = torch.randn((T, hq, 128), generator=g, device=gpu).to(dtype)
    k = torch.randn((T, hkv, 128), generator=g, device=gpu).to(dtype)
    v = torch.randn((T, hkv, 128), generator=g, device=gpu).to(dtype)
    cu = torch.tensor(lead + np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=gpu)
    sm = rs.permutation(rows)[:T].astype(np.int64)
    sm[rs.rand(T) < 0.05] = -1  # padding tokens
    kc = torch.randn((rows, hkv, 128), generator=g, device=gpu).to(dtype)
    vc = torch.randn((rows, hkv, 128), generator=g, device=gpu).to(dtype)
    ke, ve = np_of(kc).copy(), np_of(vc).copy()
    out = fai.varlen_prefill_with_kvcache(q, k, v, cu, mseq, kc, vc, torch.from_numpy(sm).to(gpu),
                                          softmax_scale=scale, causal=True)
    torch.cuda.synchronize()
    oracle.kv_store(ke, np_of(k), sm)
    oracle.kv_store(ve, np_of(v), sm)
    assert _same_bytes(kc, ke), "k cache"
    assert _same_bytes(vc, ve), "v cache"
    if mseq == max(lens):  # an understated max_seqlen leaves uncovered rows unwritten
        seg = slice(lead, lead + N)
        whole = _unsplit(q, k, v, cu, cu, mseq, mseq, scale, True)
        torch.cuda.synchronize()
        assert torch.equal(out[seg].view(torch.int16), whole[seg].view(torch.int16)), \
            "store variant attention != attention kernel"
        ref, absv = _torch_reference(q[seg], k[seg], v[seg], lens, lens, scale, True)
        check_attention(out[seg], ref, what=f"prefill store seed {seed}", absv=absv)

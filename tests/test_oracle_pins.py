"""Pins for the oracle: each check is independent of the oracle's own formula.

* torch.Tensor.index_copy_ (the reference's KV-store op, llm.py:171-174) and
  torch.nn.functional.scaled_dot_product_attention (a library attention) run
  on CPU as independent implementations;
* closed forms whose value the mathematics fixes (q = 0 gives a causal prefix
  mean; a dominant one-hot score selects one value row; single-key rows
  return v);
* invariants (block-id permutation, segment independence, decode == last
  prefill row).
Each check is chosen so a plausible mistake -- a causal off-by-one, a wrong
GQA head map, a transposed operand, a dropped scale -- fails it.
"""
import numpy as np
import pytest
import torch

import oracle
from cases import config1_inputs, ragged_block_tables


def _sdpa_segments(q, k, v, cu, scale, causal=True):
    g = q.shape[1] // k.shape[1]
    out = np.zeros(q.shape)
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        qt = torch.from_numpy(q[a:b]).double().permute(1, 0, 2)
        kt = torch.from_numpy(k[a:b]).double().permute(1, 0, 2).repeat_interleave(g, 0)
        vt = torch.from_numpy(v[a:b]).double().permute(1, 0, 2).repeat_interleave(g, 0)
        o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=causal,
                                                             scale=scale)
        out[a:b] = o.permute(1, 0, 2).numpy()
    return out


# ------------------------------------------------------------------ bf16
def test_bf16_round_matches_torch():
    rs = np.random.RandomState(3)
    x = np.concatenate([
        rs.standard_normal(4096).astype(np.float32) * 10.0 ** rs.randint(-8, 8, 4096),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.0 + 2 ** -8,
                  1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9], dtype=np.float32),
    ]).astype(np.float32)
    ours = oracle.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    back = oracle.bf16_bits_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    assert np.isnan(oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.float32([np.nan])))).all()


# ------------------------------------------------------------------ KV store
@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
def test_kv_store_matches_index_copy(dtype):
    rs = np.random.RandomState(4)
    rows, hkv, d, n = 300, 4, 16, 77
    if dtype == np.uint16:
        cache = rs.randint(0, 2 ** 16, (rows // 10, 10, hkv, d)).astype(np.uint16)
        x = rs.randint(0, 2 ** 16, (n, hkv, d)).astype(np.uint16)
        tconv = lambda a: torch.from_numpy(a.view(np.int16))  # noqa: E731
    else:
        cache = rs.standard_normal((rows // 10, 10, hkv, d)).astype(np.float32)
        x = rs.standard_normal((n, hkv, d)).astype(np.float32)
        tconv = torch.from_numpy
    slots = rs.permutation(rows)[:n].astype(np.int64)
    ours = cache.copy()
    oracle.kv_store(ours, x, slots)
    ref = tconv(cache.copy())
    ref.view(-1, hkv, d).index_copy_(0, torch.from_numpy(slots), tconv(x))
    assert np.array_equal(ours.view(np.uint8), ref.numpy().view(np.uint8))


def test_kv_store_skip_and_range():
    cache = np.zeros((4, 2, 3), np.float32)
    x = np.ones((3, 2, 3), np.float32)
    oracle.kv_store(cache, x, np.array([-1, 2, -5]))
    assert cache[2].sum() == 6 and cache.sum() == 6
    with pytest.raises(IndexError):
        oracle.kv_store(cache, x, np.array([0, 1, 4]))
    with pytest.raises(IndexError):  # index_copy_ rejects the same index
        torch.zeros(4, 2, 3).index_copy_(0, torch.tensor([0, 1, 4]), torch.ones(3, 2, 3))


# ------------------------------------------------------------------ metadata
def test_prefill_metadata_matches_torch_evaluation():
    seq_lens, slots, lmax = [5, 1, 9, 3], [3, 0, 7, 2], 16
    cu, pos, sc = oracle.prefill_metadata(seq_lens, slots, lmax)
    # llm.py:129-140 evaluated with torch
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    tcu = torch.zeros(len(seq_lens) + 1, dtype=torch.int32)
    tcu[1:] = sl.cumsum(0)
    tpos = torch.cat([torch.arange(L) for L in seq_lens])
    tsc = torch.repeat_interleave(torch.tensor(slots) * lmax, sl.long()) + tpos
    assert np.array_equal(cu, tcu.numpy()) and cu.dtype == np.int32
    assert np.array_equal(pos, tpos.numpy())
    assert np.array_equal(sc, tsc.numpy())


def test_paged_mapping_reduces_to_slot_layout():
    seq_lens, slots, lmax = [5, 1, 9, 3], [3, 0, 7, 2], 16
    _, _, sc = oracle.prefill_metadata(seq_lens, slots, lmax)
    bt = np.asarray(slots, np.int32).reshape(-1, 1)
    assert np.array_equal(oracle.paged_slot_mapping(bt, seq_lens, lmax), sc)
    # decode append: position cache_seqlens[b] of slot b
    sl = np.array([4, 0, 8, 2])
    assert np.array_equal(oracle.decode_slot_mapping(bt, sl, lmax),
                          np.asarray(slots) * lmax + sl)


def test_paged_mapping_is_bijective_over_a_permuted_pool():
    rs = np.random.RandomState(5)
    bs, lens = 8, [13, 8, 1, 30]
    perm = rs.permutation(16)
    bt = ragged_block_tables(lens, bs, perm)
    sm = oracle.paged_slot_mapping(bt, lens, bs)
    assert len(set(sm.tolist())) == sum(lens)
    assert set((sm // bs).tolist()) <= set(perm[:sum(-(-L // bs) for L in lens)].tolist())
    # offsets within a block run 0..bs-1 in order
    assert np.array_equal(sm[:8] % bs, np.arange(8))


# ------------------------------------------------------------------ prefill
@pytest.mark.parametrize("hq,hkv", [(4, 4), (4, 2), (8, 2), (8, 1)])
def test_varlen_matches_sdpa(hq, hkv):
    rs = np.random.RandomState(6)
    lens = [1, 7, 33, 16]
    n, d = sum(lens), 32
    q = rs.standard_normal((n, hq, d))
    k = rs.standard_normal((n, hkv, d))
    v = rs.standard_normal((n, hkv, d))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    for causal in (True, False):
        ours = oracle.varlen_attention(q, k, v, cu, scale=0.3, causal=causal)
        ref = _sdpa_segments(q, k, v, cu, 0.3, causal)
        assert np.abs(ours - ref).max() < 1e-12


def test_varlen_zero_query_is_causal_prefix_mean_per_kv_head():
    # q = 0 -> uniform weights over the visible keys: out[i] = mean(v[0..i]) of
    # the KV head h // g.  A mask off-by-one or wrong GQA map changes it.
    rs = np.random.RandomState(7)
    lens, hq, hkv, d = [6, 11], 8, 2, 16
    n = sum(lens)
    q = np.zeros((n, hq, d))
    k = rs.standard_normal((n, hkv, d))
    v = rs.standard_normal((n, hkv, d)) + np.arange(hkv)[None, :, None] * 100.0
    cu = np.array([0, 6, 17], np.int32)
    out = oracle.varlen_attention(q, k, v, cu)
    for s in range(2):
        seg = v[cu[s]:cu[s + 1]]
        cm = np.cumsum(seg, axis=0) / np.arange(1, len(seg) + 1)[:, None, None]
        for h in range(hq):
            assert np.allclose(out[cu[s]:cu[s + 1], h], cm[:, h // (hq // hkv)], atol=1e-12)


def test_varlen_single_key_rows_and_one_hot_selection():
    rs = np.random.RandomState(8)
    d = 16
    # single-token segments return v exactly
    q = rs.standard_normal((3, 2, d))
    k = rs.standard_normal((3, 1, d))
    v = rs.standard_normal((3, 1, d))
    out = oracle.varlen_attention(q, k, v, np.array([0, 1, 2, 3], np.int32))
    assert np.allclose(out, np.repeat(v, 2, axis=1), atol=1e-15)
    # dominant score: query 5 aligned with key 2 (scale huge) selects v[2]
    L = 8
    k = np.eye(L, d)[:, None, :]
    q = np.zeros((L, 1, d))
    q[5, 0, 2] = 1.0
    v = rs.standard_normal((L, 1, d))
    out = oracle.varlen_attention(q, k, v, np.array([0, L], np.int32), scale=1e4)
    assert np.allclose(out[5, 0], v[2, 0], atol=1e-12)
    # key 7 is in the future of query 5: aligning with it must NOT select it
    q[5, 0] = 0
    q[5, 0, 7] = 1.0
    out = oracle.varlen_attention(q, k, v, np.array([0, L], np.int32), scale=1e4)
    assert np.allclose(out[5, 0], v[:6, 0].mean(0), atol=1e-12)


def test_varlen_segments_are_independent():
    rs = np.random.RandomState(9)
    lens, d = [4, 9, 2], 8
    n = sum(lens)
    q, k, v = (rs.standard_normal((n, 2, d)) for _ in range(3))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    whole = oracle.varlen_attention(q, k, v, cu)
    for s in range(3):
        a, b = cu[s], cu[s + 1]
        part = oracle.varlen_attention(q[a:b], k[a:b], v[a:b], np.array([0, b - a], np.int32))
        assert np.array_equal(whole[a:b], part)


def test_varlen_bottom_right_causal_alignment():
    # Lq < Lk: the last query row sees every key (FA2 >= 2.1)
    rs = np.random.RandomState(10)
    d = 8
    q = rs.standard_normal((2, 1, d))
    k = rs.standard_normal((5, 1, d))
    v = rs.standard_normal((5, 1, d))
    out = oracle.varlen_attention(q, k, v, np.array([0, 2], np.int32), np.array([0, 5], np.int32))
    full = oracle.varlen_attention(q[1:], k, v, np.array([0, 1], np.int32),
                                   np.array([0, 5], np.int32), causal=False)
    assert np.allclose(out[1], full[0], atol=1e-15)
    first = oracle.varlen_attention(q[:1], k[:4], v[:4], np.array([0, 1], np.int32),
                                    np.array([0, 4], np.int32), causal=False)
    assert np.allclose(out[0], first[0], atol=1e-15)


# ------------------------------------------------------------------ decode
def test_decode_is_last_prefill_row():
    rs = np.random.RandomState(11)
    hq, hkv, d, L, bs = 4, 2, 16, 21, 4
    q = rs.standard_normal((L, hq, d))
    k = rs.standard_normal((L, hkv, d))
    v = rs.standard_normal((L, hkv, d))
    pre = oracle.varlen_attention(q, k, v, np.array([0, L], np.int32))
    pool = 8
    perm = rs.permutation(pool)
    bt = ragged_block_tables([L], bs, perm)
    kc = np.zeros((pool, bs, hkv, d))
    vc = np.zeros((pool, bs, hkv, d))
    sm = oracle.paged_slot_mapping(bt, [L], bs)
    oracle.kv_store(kc, k, sm)
    oracle.kv_store(vc, v, sm)
    for i in (0, 5, L - 1):
        dec = oracle.paged_decode(q[i:i + 1], kc, vc, bt, [i + 1], bs)
        assert np.allclose(dec[0], pre[i], atol=1e-13)


def test_decode_block_permutation_invariance_and_context_one():
    inp = config1_inputs()
    kc, vc = inp["k_cache"], inp["v_cache"]
    ctx = inp["context_lens"]
    out = oracle.paged_decode(inp["q"], kc, vc, inp["block_tables"], ctx, 256)
    # relabel physical blocks: move block p to position perm[p]
    rs = np.random.RandomState(12)
    perm = rs.permutation(kc.shape[0])
    kc2 = np.empty_like(kc)
    vc2 = np.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    bt2 = np.where(inp["block_tables"] >= 0, perm[np.maximum(inp["block_tables"], 0)], -1)
    out2 = oracle.paged_decode(inp["q"], kc2, vc2, bt2, ctx, 256)
    assert np.array_equal(out, out2)
    one = oracle.paged_decode(inp["q"], kc, vc, inp["block_tables"], [1, 1, 1, 1], 256)
    for b in range(4):
        v0 = vc[inp["block_tables"][b, 0], 0]
        assert np.allclose(one[b], np.repeat(v0, 2, axis=0), atol=1e-15)
    zero = oracle.paged_decode(inp["q"], kc, vc, inp["block_tables"], [0, 0, 0, 0], 256)
    assert not zero.any()


def test_decode_lse_splits_recombine():
    # split-K identity: combining two halves by log-sum-exp reproduces the whole
    inp = config1_inputs()
    b = 3
    kc, vc, bt = inp["k_cache"], inp["v_cache"], inp["block_tables"][b:b + 1]
    q = inp["q"][b:b + 1]
    n = int(inp["context_lens"][b])
    whole = oracle.paged_decode(q, kc, vc, bt, [n], 256)
    o1, l1 = oracle.paged_decode(q, kc, vc, bt, [256], 256, return_lse=True)
    ks = oracle.gather_paged(kc, bt[0], n, 256)[256:]
    vs = oracle.gather_paged(vc, bt[0], n, 256)[256:]
    o2 = oracle.varlen_attention(q, ks, vs, np.array([0, 1]), np.array([0, n - 256]),
                                 causal=False)
    g = 2
    s = np.einsum("hd,khd->hk", q[0].astype(np.float64),
                  np.repeat(ks, g, axis=1).astype(np.float64)) * 128 ** -0.5
    l2 = np.log(np.exp(s - s.max(1, keepdims=True)).sum(1)) + s.max(1)
    m = np.maximum(l1[0], l2)
    w1, w2 = np.exp(l1[0] - m), np.exp(l2 - m)
    comb = (w1[:, None] * o1[0] + w2[:, None] * o2[0]) / (w1 + w2)[:, None]
    assert np.allclose(comb, whole[0], atol=1e-12)


def test_kv_export_import_reduce_to_reference_slot_slices():
    # Slot layout (block_size = max_seq_len, block_table = [slot]): the export
    # is the reference's k_cache[slot, :length] / v_cache[slot, :length] per
    # layer (model/model.py:162-163) and the import its
    # k_cache[slot, :length].copy_(k[:length]) (:174-175), evaluated with torch.
    rs = np.random.RandomState(21)
    L, S, lmax, hkv, d = 3, 4, 40, 2, 8
    storage = rs.randint(0, 1 << 16, (L, 2, S, lmax, hkv, d)).astype(np.uint16)
    slot, length = 2, 29
    exp = oracle.kv_export(storage, [slot], length)
    for layer in range(L):
        for c in range(2):
            ref = torch.from_numpy(storage[layer, c].view(np.int16))[slot, :length]
            assert np.array_equal(exp[layer, c].view(np.int16), ref.numpy())
    src = rs.randint(0, 1 << 16, (L, 2, length + 5, hkv, d)).astype(np.uint16)
    got = oracle.kv_import(src, storage.copy(), [slot], length)
    want = torch.from_numpy(storage.view(np.int16).copy())
    for layer in range(L):
        for c in range(2):
            want[layer, c][slot, :length].copy_(torch.from_numpy(src[layer, c].view(np.int16))[:length])
    assert np.array_equal(got.view(np.int16), want.numpy())


def test_kv_export_import_round_trip_and_relabelling_over_a_permuted_pool():
    rs = np.random.RandomState(22)
    L, nb, bs, hkv, d, length = 2, 12, 4, 2, 4, 18
    storage = rs.standard_normal((L, 2, nb, bs, hkv, d)).astype(np.float32)
    bt = rs.permutation(nb)[:5].astype(np.int32)  # 5 blocks hold 18 tokens
    exp = oracle.kv_export(storage, bt, length)
    # rows of the export are the sequence's tokens in order
    p = 13
    assert np.array_equal(exp[1, 1, p], storage[1, 1, bt[p // bs], p % bs])
    # import into a sentinel pool with another table, export again: the payload
    sentinel = np.full_like(storage, 7.0)
    bt2 = rs.permutation(nb)[:5].astype(np.int32)
    back = oracle.kv_import(exp, sentinel.copy(), bt2, length)
    assert np.array_equal(oracle.kv_export(back, bt2, length), exp)
    touched = np.zeros((nb, bs), bool)
    q = np.arange(length)
    touched[bt2[q // bs], q % bs] = True
    assert (back[:, :, ~touched] == 7.0).all()  # nothing else written
    # relabelling the physical blocks commutes with the export
    perm = rs.permutation(nb)
    moved = np.empty_like(storage)
    moved[:, :, perm] = storage
    assert np.array_equal(oracle.kv_export(moved, perm[bt], length), exp)
    # an invalid block id exports zeros and is skipped by the import
    bad = bt.copy()
    bad[2] = -1
    e2 = oracle.kv_export(storage, bad, length)
    assert not e2[:, :, 8:12].any() and np.array_equal(e2[:, :, :8], exp[:, :, :8])
    s2 = sentinel.copy()
    oracle.kv_import(exp, s2, bad, length)
    assert (s2[:, :, bt[2]] == 7.0).all()  # the skipped block keeps its bytes

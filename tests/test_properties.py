"""Property tests on the CPU (hypothesis, derandomized so every run checks the
same examples): the oracle's varlen attention against a brute-force float64
triple loop on tiny shapes; the block allocator against a set model under
random allocate/free sequences; the prefill and decode slot mappings against
each other over random block tables."""
import math

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

import oracle
from awesome_acceleration_amd import paged

SETTINGS = settings(max_examples=60, deadline=None, derandomize=True)


def _naive_attention(q, k, v, lq, lk, scale, causal):
    """One segment, explicit loops: out[i, h] = sum_j p_ij v[j, h // g]."""
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    out = np.zeros(q.shape, dtype=np.float64)
    for i in range(lq):
        for h in range(hq):
            keys = [j for j in range(lk) if not causal or j <= i + (lk - lq)]
            if not keys:
                continue  # a row that sees no key is zero
            s = [scale * float(np.dot(q[i, h], k[j, h // g])) for j in keys]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            tot = sum(w)
            for wj, j in zip(w, keys):
                out[i, h] += (wj / tot) * v[j, h // g]
    return out


@SETTINGS
@given(
    segs=st.lists(st.tuples(st.integers(0, 9), st.integers(0, 9)), min_size=1, max_size=3),
    hkv=st.sampled_from([1, 2]),
    g=st.sampled_from([1, 2, 4]),
    d=st.sampled_from([2, 5, 8]),
    causal=st.booleans(),
    seed=st.integers(0, 2**16),
)
def test_oracle_varlen_equals_brute_force(segs, hkv, g, d, causal, seed):
    rs = np.random.RandomState(seed)
    lq = [a for a, _ in segs]
    lk = [max(a, b) if causal else b for a, b in segs]  # bottom-right causal needs Lk >= Lq
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = rs.standard_normal((cq[-1], hkv * g, d))
    k = rs.standard_normal((ck[-1], hkv, d))
    v = rs.standard_normal((ck[-1], hkv, d))
    scale = 0.7
    got = oracle.varlen_attention(q, k, v, cq, ck, scale=scale, causal=causal)
    for s in range(len(segs)):
        want = _naive_attention(q[cq[s]:cq[s + 1]], k[ck[s]:ck[s + 1]], v[ck[s]:ck[s + 1]],
                                lq[s], lk[s], scale, causal)
        np.testing.assert_allclose(got[cq[s]:cq[s + 1]], want, rtol=1e-12, atol=1e-12)


@SETTINGS
@given(ops=st.lists(st.tuples(st.booleans(), st.integers(0, 7)), max_size=40),
       num_blocks=st.integers(1, 24))
def test_block_allocator_matches_a_set_model(ops, num_blocks):
    a = paged.BlockAllocator(num_blocks)
    free = set(range(num_blocks))
    held: list[list[int]] = []
    for is_alloc, n in ops:
        if is_alloc:
            if n > len(free):
                with pytest.raises(RuntimeError):
                    a.allocate(n)
            else:
                got = a.allocate(n)
                assert got == sorted(free)[:n]  # lowest free ids first
                free -= set(got)
                held.append(got)
        elif held:
            blocks = held.pop(n % len(held))
            a.free(blocks + blocks)  # a repeated id is ignored the second time
            free |= set(blocks)
        assert a.num_free == len(free)


@SETTINGS
@given(lens=st.lists(st.integers(0, 40), min_size=1, max_size=5),
       block_size=st.sampled_from([1, 4, 16]), seed=st.integers(0, 2**16))
def test_prefill_and_decode_slot_mappings_agree(lens, block_size, seed):
    rs = np.random.RandomState(seed)
    need = [paged.blocks_needed(L + 1, block_size) for L in lens]
    perm = rs.permutation(sum(need) + 3).astype(np.int32)
    tables, k = [], 0
    for n in need:
        tables.append(list(perm[k:k + n]))
        k += n
    bt = paged.pad_block_tables(tables)
    pre = paged.prefill_slot_mapping(bt, lens, block_size)
    # every prefill token lands in a distinct row of its own sequence's blocks
    assert len(set(pre.tolist())) == pre.shape[0] == sum(lens)
    off = 0
    for b, L in enumerate(lens):
        rows = pre[off:off + L]
        assert set((rows // block_size).tolist()) <= set(tables[b])
        # the decode append at position p writes where a prefill of p+1 tokens put token p
        for p in range(L):
            assert paged.decode_slot_mapping(bt[b:b + 1], [p], block_size)[0] == rows[p]
        off += L
    # appending the next token never collides with a prefilled row
    nxt = paged.decode_slot_mapping(bt, lens, block_size)
    assert not set(nxt.tolist()) & set(pre.tolist())


@SETTINGS
@given(
    segs=st.lists(st.tuples(st.integers(1, 9), st.integers(0, 9)), min_size=1, max_size=3),
    hkv=st.sampled_from([1, 2]),
    g=st.sampled_from([1, 2, 4]),
    causal=st.booleans(),
    seed=st.integers(0, 2**16),
)
def test_oracle_constant_values_return_that_value(segs, hkv, g, causal, seed):
    """Every V row of KV head h equal to one vector u_h: each query row that
    sees a key returns u_h (the softmax weights sum to one), in the varlen
    attention and in the paged decode, whatever the scores."""
    rs = np.random.RandomState(seed)
    d = 8
    lq = [a for a, _ in segs]
    lk = [max(a, b) if causal else max(b, 1) for a, b in segs]  # every row sees a key
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    u = rs.standard_normal((hkv, d))
    q = 3.0 * rs.standard_normal((cq[-1], hkv * g, d))
    k = rs.standard_normal((ck[-1], hkv, d))
    v = np.broadcast_to(u, (ck[-1], hkv, d)).copy()
    got = oracle.varlen_attention(q, k, v, cq, ck, scale=0.9, causal=causal)
    np.testing.assert_allclose(got, np.repeat(u, g, axis=0)[None].repeat(cq[-1], 0),
                               rtol=1e-12, atol=1e-12)
    # paged decode over the same keys of segment 0, scattered over shuffled blocks
    bs = 4
    n = lk[0]
    nb = -(-n // bs)
    perm = rs.permutation(nb + 2)
    kc = rs.standard_normal((nb + 2, bs, hkv, d))
    vc = rs.standard_normal((nb + 2, bs, hkv, d))
    for t in range(n):
        kc[perm[t // bs], t % bs] = k[t]
        vc[perm[t // bs], t % bs] = u
    qd = rs.standard_normal((1, hkv * g, d))
    got_d = oracle.paged_decode(qd, kc, vc, perm[None, :nb].astype(np.int32), np.array([n]), bs, 0.9)
    np.testing.assert_allclose(got_d[0], np.repeat(u, g, axis=0), rtol=1e-12, atol=1e-12)

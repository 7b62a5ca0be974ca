"""KV export / import (the PD migration payload, model/model.py:156-177 and
:386-401) on the GPU against the oracle: the export is bit-exact with the
oracle's gather, the import writes exactly the sequence's token rows (every
other cache byte untouched), and the reference's payload format round-trips
through export_request_kv / import_request_kv."""
import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import kv_transfer as kt
from awesome_acceleration_amd.qwen3 import PagedKVCache, Qwen3Config
from gpu_util import np_of

pytestmark = pytest.mark.gpu


def _storage(L, nb, bs, hkv, d, dtype, gpu, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return torch.randn((L, 2, nb, bs, hkv, d), generator=g, device=gpu).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_export_matches_oracle_and_import_touches_only_the_sequence(gpu, dtype):
    print(f"case: kv export/import {dtype}", flush=True)
    L, nb, bs, hkv, d, length = 5, 40, 16, 8, 128, 203
    st = _storage(L, nb, bs, hkv, d, dtype, gpu, 0)
    rs = np.random.RandomState(3)
    bt = rs.permutation(nb)[:13].astype(np.int32)  # 13 blocks of 16 hold 203 tokens
    bt[5] = -1  # an invalid entry exports zeros
    out = kt.kv_export(st, torch.from_numpy(bt).to(gpu), length)
    torch.cuda.synchronize()
    assert np.array_equal(np_of(out), oracle.kv_export(np_of(st), bt, length))
    # import into a sentinel pool through another table; export again
    dst = torch.full_like(st, 3.0)
    bt2 = rs.permutation(nb)[:13].astype(np.int32)
    bt2[7] = nb + 4  # out of range: skipped
    kt.kv_import(out, dst, torch.from_numpy(bt2).to(gpu), length)
    torch.cuda.synchronize()
    want = oracle.kv_import(np_of(out), np_of(torch.full_like(st, 3.0)), bt2, length)
    assert np.array_equal(np_of(dst), want)  # whole pool, untouched rows included


def test_reference_payload_round_trip_through_the_cache(gpu):
    print("case: kv request payload round trip", flush=True)
    cfg = Qwen3Config(num_hidden_layers=4, num_key_value_heads=8, head_dim=128)
    src = PagedKVCache(cfg, num_blocks=20, block_size=64, device=gpu, dtype=torch.bfloat16)
    src.storage.copy_(_storage(4, 20, 64, 8, 128, torch.bfloat16, gpu, 1))
    blocks, length = [17, 3, 9, 12], 230
    payload = src.export_request_kv(blocks, length, seqlen=length)
    layers = payload["layers"]
    assert len(layers) == 4
    for i, lp in enumerate(layers):
        assert lp["k"].device.type == "cpu" and lp["k"].dtype == torch.bfloat16
        assert tuple(lp["k"].shape) == (length, 8, 128) and lp["seqlen"] == length
        # the reference's slice of the same sequence
        ref_k = oracle.gather_paged(np_of(src.storage[i, 0]), blocks, length, 64)
        assert np.array_equal(np_of(lp["k"]), ref_k)
        ref_v = oracle.gather_paged(np_of(src.storage[i, 1]), blocks, length, 64)
        assert np.array_equal(np_of(lp["v"]), ref_v)
    dst = PagedKVCache(cfg, num_blocks=20, block_size=64, device=gpu, dtype=torch.bfloat16)
    assert dst.import_request_kv([0, 5, 19, 2], payload, length) == length
    back = dst.export_request_kv([0, 5, 19, 2], length, seqlen=length)
    for a, b in zip(layers, back["layers"]):
        assert torch.equal(a["k"], b["k"]) and torch.equal(a["v"], b["v"])
    with pytest.raises(ValueError):
        dst.import_request_kv([0], {"layers": layers[:3]}, 10)


def test_export_rejects_bad_shapes(gpu):
    print("case: kv export rejections", flush=True)
    st = _storage(2, 4, 16, 8, 128, torch.bfloat16, gpu, 2)
    with pytest.raises(RuntimeError):
        kt.kv_export(st, [0, 1], 40)  # 2 blocks of 16 cannot hold 40 tokens
    with pytest.raises(RuntimeError):
        kt.kv_export(st[..., ::2], [0], 8)  # a cache whose rows are not contiguous
    # the first two blocks of every cache: strided, each cache contiguous; exports
    # the same rows as a contiguous copy of them
    part = st[:, :, :2]
    got = kt.kv_export(part, [1, 0], 20)
    torch.cuda.synchronize()
    assert torch.equal(got, kt.kv_export(part.contiguous(), [1, 0], 20))


def test_export_import_on_the_engine_cache_placement(gpu):
    """The engine's storage (each layer's V cache 512 bytes past its K cache,
    modulo 1 KiB) exports and imports like a contiguous one."""
    print("case: kv export/import, engine cache placement", flush=True)
    from awesome_acceleration_amd import paged
    L, nb, bs, hkv, d, length = 3, 24, 32, 8, 128, 300
    st = paged.alloc_kv_storage(L, nb, bs, hkv, d, dtype=torch.bfloat16, device=gpu)
    st.copy_(_storage(L, nb, bs, hkv, d, torch.bfloat16, gpu, 5))
    rs = np.random.RandomState(9)
    bt = rs.permutation(nb)[:10].astype(np.int32)  # 10 blocks of 32 hold 300 tokens
    out = kt.kv_export(st, torch.from_numpy(bt).to(gpu), length)
    torch.cuda.synchronize()
    assert np.array_equal(np_of(out), oracle.kv_export(np_of(st), bt, length))
    dst = paged.alloc_kv_storage(L, nb, bs, hkv, d, dtype=torch.bfloat16, device=gpu)
    dst.fill_(2.0)
    kt.kv_import(out, dst, torch.from_numpy(bt).to(gpu), length)
    torch.cuda.synchronize()
    want = oracle.kv_import(np_of(out), np_of(torch.full_like(st, 2.0)), bt, length)
    assert np.array_equal(np_of(dst), want)

"""GPU parity of the KV-store kernels (bit-exact against the oracle's
index_copy_ restatement, llm.py:171-174, including every untouched row)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import _lib, flash_attn_interface as fai, paged
from gpu_util import bytes_of, np_of

pytestmark = pytest.mark.gpu


def _sentinel_cache(shape, dtype, device, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(device)


def test_store_prefill_shape_strided_v_bitexact(gpu):
    # 8 sequences x 1024 tokens, Hkv=8, D=128, bf16; v is a view of the fused
    # qkv buffer (token stride 4096 elements) as at llm.py:156; shuffled pool
    # of 32 blocks x 256 pre-filled with sentinel values.
    print("case: store 8x1024 bf16 strided-v", flush=True)
    N, hkv, d, bs = 8192, 8, 128, 256
    g = torch.Generator(device="cpu").manual_seed(0)
    qkv = torch.randn(N, 4096, generator=g).to(torch.bfloat16)
    perm = torch.randperm(32, generator=g).to(torch.int32).numpy()
    bt = perm.reshape(8, 4)
    sm = paged.prefill_slot_mapping(bt, [1024] * 8, bs)
    kc = _sentinel_cache((32, bs, hkv, d), torch.bfloat16, "cpu", 1)
    vc = _sentinel_cache((32, bs, hkv, d), torch.bfloat16, "cpu", 2)
    k_ref, v_ref = np_of(kc).copy(), np_of(vc).copy()
    k_np = np_of(qkv[:, 2048:3072].reshape(N, hkv, d))
    v_np = np_of(qkv[:, 3072:].reshape(N, hkv, d))
    oracle.kv_store(k_ref, k_np, sm)
    oracle.kv_store(v_ref, v_np, sm)

    qkv_g = qkv.to(gpu)
    k_g = qkv_g[:, 2048:3072].contiguous().view(N, hkv, d)
    v_g = qkv_g[:, 3072:].view(N, hkv, d)
    assert v_g.stride(0) == 4096
    kc_g, vc_g = kc.to(gpu), vc.to(gpu)
    fai.kv_store(k_g, v_g, kc_g, vc_g, torch.from_numpy(sm).to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(bytes_of(kc_g), k_ref.view(np.uint8))
    assert np.array_equal(bytes_of(vc_g), v_ref.view(np.uint8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("tok_pad", [0, 1, 3])
def test_store_dtypes_alignment_and_skips(gpu, dtype, tok_pad):
    # token strides that break 16-B alignment exercise the 8/4/2-byte paths;
    # negative slots are skipped, out-of-range slots are never written.
    print(f"case: store dtype={dtype} pad={tok_pad}", flush=True)
    n, hkv, d, rows = 37, 2, 128, 64
    g = torch.Generator(device="cpu").manual_seed(3)
    src = torch.randn(n, hkv * d + tok_pad, generator=g).to(dtype)
    k = src[:, :hkv * d].reshape(n, hkv, d) if tok_pad == 0 else None
    kc = _sentinel_cache((rows // 8, 8, hkv, d), dtype, "cpu", 4)
    vc = _sentinel_cache((rows // 8, 8, hkv, d), dtype, "cpu", 5)
    rs = np.random.RandomState(6)
    sm = rs.permutation(rows)[:n].astype(np.int64)
    sm[[3, 10]] = -1
    sm[20] = -7
    sm_dev = sm.copy()
    sm_dev[25] = rows + 5  # out of range on the device: skipped
    sm_ref = sm.copy()
    sm_ref[25] = -1
    k_np = np_of(src[:, :hkv * d].contiguous().view(n, hkv, d))
    k_ref, v_ref = np_of(kc).copy(), np_of(vc).copy()
    oracle.kv_store(k_ref, k_np, sm_ref)
    oracle.kv_store(v_ref, k_np, sm_ref)
    src_g = src.to(gpu)
    kv_g = src_g[:, :hkv * d].view(n, hkv, d) if tok_pad == 0 else \
        src_g.as_strided((n, hkv, d), (hkv * d + tok_pad, d, 1))
    kc_g, vc_g = kc.to(gpu), vc.to(gpu)
    fai.kv_store(kv_g, kv_g, kc_g, vc_g, torch.from_numpy(sm_dev).to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(bytes_of(kc_g), k_ref.view(np.uint8))
    assert np.array_equal(bytes_of(vc_g), v_ref.view(np.uint8))


def test_store_empty_is_noop(gpu):
    kc = torch.zeros(2, 4, 8, 128, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(0, 8, 128, dtype=torch.bfloat16, device=gpu)
    fai.kv_store(k, k, kc, kc.clone(), torch.zeros(0, dtype=torch.int64, device=gpu))
    torch.cuda.synchronize()
    assert not kc.any()


def test_append_paged_through_c_abi(gpu):
    # aac_kv_append_paged: token b lands at position cache_seqlens[b] of its
    # block table (the k=/v= half of flash_attn_with_kvcache).
    print("case: append paged", flush=True)
    B, hkv, d, bs, pool = 9, 8, 128, 16, 40
    rs = np.random.RandomState(7)
    perm = rs.permutation(pool).astype(np.int32)
    lens = rs.randint(0, 60, B).astype(np.int32)
    lens[0], lens[1] = 0, 15
    need = [int(np.ceil((L + 1) / bs)) for L in lens]
    width = 5
    bt = np.full((B, width), -1, np.int32)
    k0 = 0
    for b, nb in enumerate(need):
        bt[b, :nb] = perm[k0:k0 + nb]
        k0 += nb
    lens_dev = lens.copy()
    lens_dev[2] = width * bs  # beyond table capacity: skipped
    kc = _sentinel_cache((pool, bs, hkv, d), torch.bfloat16, "cpu", 8)
    vc = _sentinel_cache((pool, bs, hkv, d), torch.bfloat16, "cpu", 9)
    kn = _sentinel_cache((B, hkv, d), torch.bfloat16, "cpu", 10)
    vn = _sentinel_cache((B, hkv, d), torch.bfloat16, "cpu", 11)
    k_ref, v_ref = np_of(kc).copy(), np_of(vc).copy()
    sm = oracle.decode_slot_mapping(bt, lens, bs)
    sm[2] = -1
    oracle.kv_store(k_ref, np_of(kn), sm)
    oracle.kv_store(v_ref, np_of(vn), sm)
    kc_g, vc_g, kn_g, vn_g = (t.to(gpu) for t in (kc, vc, kn, vn))
    bt_g = torch.from_numpy(bt).to(gpu)
    lens_g = torch.from_numpy(lens_dev).to(gpu)
    stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.lib().aac_kv_append_paged(kn_g.data_ptr(), vn_g.data_ptr(), hkv * d, hkv * d,
                                        kc_g.data_ptr(), vc_g.data_ptr(), pool, bs,
                                        bt_g.data_ptr(), width, lens_g.data_ptr(), B, hkv, d, 0,
                                        stream)
    assert rc == 0, _lib.lib().aac_strerror(rc)
    torch.cuda.synchronize()
    assert np.array_equal(bytes_of(kc_g), k_ref.view(np.uint8))
    assert np.array_equal(bytes_of(vc_g), v_ref.view(np.uint8))


def test_check_mode_raises_index_error_like_index_copy(gpu, monkeypatch):
    """With AAC_CHECK the store raises IndexError for every slot index_copy_
    rejects (negative or >= rows), before anything is written; by default it
    skips them (the padding convention), leaving those rows untouched."""
    print("case: store error contract (AAC_CHECK on / off)", flush=True)
    n, hkv, d, rows = 6, 2, 128, 16
    kc = _sentinel_cache((rows // 4, 4, hkv, d), torch.bfloat16, gpu, 12)
    before = kc.clone()
    k = torch.ones(n, hkv, d, dtype=torch.bfloat16, device=gpu)
    monkeypatch.setattr(fai, "_CHECK", True)
    for bad in (-1, rows, rows + 40):
        sm = torch.tensor([0, 1, 2, bad, 4, 5], dtype=torch.int64, device=gpu)
        with pytest.raises(IndexError, match="out of bounds"):
            fai.kv_store(k, k, kc, kc.clone(), sm)
        cu = torch.tensor([0, n], dtype=torch.int32, device=gpu)
        q = torch.ones(n, 4, d, dtype=torch.bfloat16, device=gpu)
        with pytest.raises(IndexError, match="out of bounds"):
            fai.varlen_prefill_with_kvcache(q, k, k, cu, n, kc, kc.clone(), sm)
    torch.cuda.synchronize()
    assert torch.equal(kc, before)  # nothing was launched
    monkeypatch.setattr(fai, "_CHECK", False)
    sm = torch.tensor([0, -1, 2, rows, 4, -3], dtype=torch.int64, device=gpu)
    fai.kv_store(k, k, kc, kc.clone(), sm)
    torch.cuda.synchronize()
    flat, ref = kc.view(rows, hkv, d), before.view(rows, hkv, d)
    for r in range(rows):
        want = torch.ones_like(flat[r]) if r in (0, 2, 4) else ref[r]
        assert torch.equal(flat[r], want), r


def test_padded_branch_store_is_one_kv_store(gpu):
    """The padded prefill branch's per-slot copies (model/model.py:244-250)
    as one kv_store through paged.padded_prefill_slot_mapping: bit-exact
    against the copies made by torch slicing, untouched rows included."""
    print("case: padded-branch store", flush=True)
    B, T, hkv, d, lmax, nslot = 4, 300, 8, 128, 2064, 6
    g = torch.Generator(device="cpu").manual_seed(13)
    qkv = torch.randn(B, T, (16 + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(gpu)
    k = qkv[..., 16 * d:(16 + hkv) * d].contiguous().view(B, T, hkv, d)
    v = qkv[..., (16 + hkv) * d:].view(B, T, hkv, d)  # strided view, as model/model.py:222
    slots, lens = [5, 0, 3, 2], [300, 17, 0, 256]
    kc = _sentinel_cache((nslot, lmax, hkv, d), torch.bfloat16, gpu, 14)
    vc = _sentinel_cache((nslot, lmax, hkv, d), torch.bfloat16, gpu, 15)
    kr, vr = kc.clone(), vc.clone()
    for i, s in enumerate(slots):
        kr[s, :lens[i]] = k[i, :lens[i]]
        vr[s, :lens[i]] = v[i, :lens[i]]
    sm = torch.from_numpy(paged.padded_prefill_slot_mapping(slots, lens, T, lmax)).to(gpu)
    fai.kv_store(k.reshape(B * T, hkv, d), v.reshape(B * T, hkv, d), kc, vc, sm)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), kr.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vr.view(torch.int16))

"""Host logic: block/slot allocators, metadata builders and the Python
wrappers' argument checks (CPU only; nothing here launches a kernel)."""
import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import flash_attn_interface as fai
from awesome_acceleration_amd import paged


def test_slot_manager_mirrors_reference():
    m = paged.SlotCacheManager(3)
    assert [m.allocate_slot() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(RuntimeError, match="No free slots"):
        m.allocate_slot()
    m.free_slot(1)
    m.free_slot(1)  # unknown slot ignored
    m.free_slot(0)
    assert m.allocate_slot() == 0
    m.reset()
    assert m.free_slots == [0, 1, 2]


def test_block_allocator_lowest_first_and_exhaustion():
    a = paged.BlockAllocator(6)
    assert a.allocate(2) == [0, 1]
    assert a.allocate(3) == [2, 3, 4]
    with pytest.raises(RuntimeError, match="No free blocks"):
        a.allocate(2)
    assert a.num_free == 1  # failed request leaves the pool unchanged
    a.free([3, 0])
    assert a.allocate(2) == [0, 3]
    a.free([42])
    assert a.num_free == 1


def test_metadata_matches_oracle_and_slot_layout():
    seq_lens, slots, lmax = [5, 1, 9], [2, 0, 1], 12
    bt = paged.slot_block_tables(slots)
    cu, pos, sm = paged.build_prefill_metadata(seq_lens, bt, lmax, "cpu")
    ocu, opos, osc = oracle.prefill_metadata(seq_lens, slots, lmax)
    assert np.array_equal(cu.numpy(), ocu) and cu.dtype == torch.int32
    assert np.array_equal(pos.numpy(), opos) and pos.dtype == torch.int64
    assert np.array_equal(sm.numpy(), osc) and sm.dtype == torch.int64
    bt2 = paged.pad_block_tables([[7, 3], [5], [1, 2, 4]])
    assert bt2.shape == (3, 3) and bt2.dtype == np.int32
    assert np.array_equal(paged.prefill_slot_mapping(bt2, [6, 2, 9], 4),
                          oracle.paged_slot_mapping(bt2, [6, 2, 9], 4))
    assert np.array_equal(paged.decode_slot_mapping(bt2, [5, 1, 8], 4),
                          oracle.decode_slot_mapping(bt2, [5, 1, 8], 4))
    assert paged.blocks_needed(257, 256) == 2 and paged.blocks_needed(0, 256) == 0


def test_wrappers_refuse_cpu_tensors_and_unsupported_features():
    q = torch.zeros(4, 16, 128, dtype=torch.bfloat16)
    k = torch.zeros(4, 8, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        fai.flash_attn_varlen_func(q, k, k, cu, cu, 4, 4, causal=True)
    with pytest.raises(NotImplementedError):
        fai.flash_attn_varlen_func(q, k, k, cu, cu, 4, 4, dropout_p=0.1)
    with pytest.raises(NotImplementedError):
        fai.flash_attn_varlen_func(q, k, k, cu, cu, 4, 4, window_size=(8, 0))
    with pytest.raises(RuntimeError, match="GPU"):
        fai.kv_store(k, k, torch.zeros(2, 4, 8, 128, dtype=torch.bfloat16),
                     torch.zeros(2, 4, 8, 128, dtype=torch.bfloat16),
                     torch.arange(4, dtype=torch.int64))
    with pytest.raises(NotImplementedError):
        fai.flash_attn_with_kvcache(q.view(4, 1, 16, 128), k, k, cache_seqlens=1,
                                    rotary_cos=torch.zeros(1))

"""CPU oracle for the attention hot path (test infrastructure only).

This package is the test oracle, not the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the library under ``awesome_acceleration_amd`` never does, and its
HIP entry points fail loudly when the compiled extension is missing.

Contents (each function cites the reference file:line it restates):

* ``kv_store``            -- ``cache.view(-1,Hkv,D).index_copy_(0, idx, x)``
                             (llm.py:171-174), byte-exact, negative index = skip.
* ``prefill_metadata``    -- cu_seqlens / positions / scatter indices
                             (llm.py:127-140).
* ``paged_slot_mapping``  -- block_table[b][p // bs] * bs + p % bs, the paged
                             generalisation of llm.py:139-140.
* ``varlen_attention``    -- flash_attn_varlen_func(causal=True) semantics
                             (llm.py:178-184), float64 math.
* ``paged_decode``        -- flash_attn_with_kvcache attend half
                             (model/model.py:233-240), float64 math.
* ``decode_append_attend``-- store-then-attend, followed by the caller's
                             ``cache_seqlens += 1`` (model/model.py:233-241).
* bf16 helpers            -- round-to-nearest-even fp32 <-> bf16 bit casts.

How each function is pinned is documented in ``oracle/attention.py``'s module
docstring; none is "parity unpinned".
"""
from .attention import *  # noqa: F401,F403

# The fp32 Qwen3 model / engine-loop restatement (oracle/qwen3_ref.py) is
# imported on demand: ``from oracle.qwen3_ref import Qwen3Ref``.

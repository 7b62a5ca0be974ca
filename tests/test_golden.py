"""The oracle against the committed fixtures (tests/golden/, written by
make_golden.py after cross-checking the oracle with torch SDPA/index_copy_)."""
import json
from pathlib import Path

import numpy as np

import oracle
from cases import config1_inputs, sha256, tiny_decode_inputs, tiny_prefill_inputs

G = Path(__file__).resolve().parent / "golden"
MANIFEST = json.loads((G / "manifest.json").read_text())


def _decode_check(inp, fx, man):
    assert sha256(inp["q"], inp["k_new"], inp["v_new"], inp["k_cache"], inp["v_cache"],
                  inp["block_tables"], inp["cache_seqlens"]) == man["digest_inputs"]
    kc, vc = inp["k_cache"].copy(), inp["v_cache"].copy()
    out, lens = oracle.decode_append_attend(inp["q"], kc, vc, inp["k_new"], inp["v_new"],
                                            inp["block_tables"], inp["cache_seqlens"],
                                            inp["block_size"], inp["scale"])
    assert sha256(kc) == man["digest_k_cache_after"]
    assert sha256(vc) == man["digest_v_cache_after"]
    assert np.array_equal(lens, fx["new_lens"])
    assert np.array_equal(oracle.decode_slot_mapping(inp["block_tables"], inp["cache_seqlens"],
                                                     inp["block_size"]), fx["slot_mapping"])
    assert np.abs(out - fx["out"]).max() < 1e-12


def test_config1_decode_fixture():
    _decode_check(config1_inputs(), np.load(G / "config1_decode_fp32.npz"),
                  MANIFEST["config1_decode_fp32"])


def test_tiny_decode_fixture():
    fx = np.load(G / "tiny_decode_bf16.npz")
    inp = tiny_decode_inputs()
    for k in ("q", "k_new", "v_new", "k_cache", "v_cache", "block_tables", "cache_seqlens"):
        assert np.array_equal(inp[k], fx[k]), k
    _decode_check(inp, fx, MANIFEST["tiny_decode_bf16"])


def test_tiny_prefill_fixture():
    fx = np.load(G / "tiny_prefill_bf16.npz")
    inp = tiny_prefill_inputs()
    assert sha256(inp["q"], inp["k"], inp["v"], inp["cu_seqlens"]) == \
        MANIFEST["tiny_prefill_bf16"]["digest_inputs"]
    out = oracle.varlen_attention(fx["q"], fx["k"], fx["v"], fx["cu_seqlens"],
                                  scale=float(fx["scale"]))
    assert np.abs(out - fx["out"]).max() < 1e-12

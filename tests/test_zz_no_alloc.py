"""aac_decode_paged_noalloc -- the split-K paged decode with the library's
static scratch instead of a caller workspace -- against aac_decode_paged with
a workspace, through the C ABI: bit-identical outputs on two calls in a row
(the second with a smaller input), both checked against the oracle on a
sample of sequences; a plan larger than the scratch is refused before
anything is enqueued."""

import numpy as np
import pytest
import torch

import oracle
from awesome_acceleration_amd import _lib, flash_attn_interface as fai
from gpu_util import check_attention, np_of

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # AAC_DECODE_SCRATCH_BYTES


def _case(gpu, B, hq, hkv, lo, hi, seed, bs=256):
    rs = np.random.RandomState(seed)
    ctx = rs.randint(lo, hi, B).astype(np.int32)
    need = [-(-int(c) // bs) for c in ctx]
    pool = sum(need)
    perm = rs.permutation(pool).astype(np.int32)
    bt = np.zeros((B, max(need)), np.int32)
    k0 = 0
    for b, n in enumerate(need):
        bt[b, :n] = perm[k0:k0 + n]
        k0 += n
    g = torch.Generator(device=gpu).manual_seed(seed)
    kc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu).to(torch.bfloat16)
    vc = torch.randn((pool, bs, hkv, 128), generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn((B, hq, 128), generator=g, device=gpu).to(torch.bfloat16)
    return dict(q=q, kc=kc, vc=vc, bt=bt, ctx=ctx, bs=bs, bt_g=torch.from_numpy(bt).to(gpu),
                ctx_g=torch.from_numpy(ctx).to(gpu), max_ctx=int(ctx.max()))


def _noalloc(x, out):
    q, kc = x["q"], x["kc"]
    B, hq, d = q.shape
    rc = _lib.lib().aac_decode_paged_noalloc(
        q.data_ptr(), q.stride(0), kc.data_ptr(), x["vc"].data_ptr(), kc.shape[0], x["bs"],
        x["bt_g"].data_ptr(), x["bt"].shape[1], x["ctx_g"].data_ptr(), B, x["max_ctx"], hq,
        kc.shape[2], d, d ** -0.5, out.data_ptr(), out.stride(0), 0, 0,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.lib().aac_strerror(rc)


def _oracle_sample(x, seqs):
    """Oracle output of a few sequences (only their blocks copied to the host)."""
    used = np.unique(x["bt"][seqs])
    remap = {int(b): i for i, b in enumerate(used)}
    idx = torch.from_numpy(used.astype(np.int64)).to(x["kc"].device)
    kc, vc = np_of(x["kc"][idx]), np_of(x["vc"][idx])
    bt = np.vectorize(lambda v: remap[int(v)])(x["bt"][seqs]).astype(np.int32)
    q = np_of(x["q"])[seqs]
    ref = oracle.paged_decode(q, kc, vc, bt, x["ctx"][seqs], x["bs"], 128 ** -0.5)
    # sum_j p_j |v_j|: the rounding bound of the bf16 probabilities in P.V
    absv = oracle.paged_decode(q, kc, vc & np.uint16(0x7FFF), bt, x["ctx"][seqs], x["bs"],
                               128 ** -0.5)
    return ref, absv


def test_noalloc_matches_the_workspace_entry_point_twice(gpu):
    L = _lib.lib()
    cases = [("GQA-4, 16 seqs x 16k-24k", (16, 32, 8, 16384, 24577, 21)),
             ("GQA-2, 6 seqs x 3k-9k (smaller)", (6, 16, 8, 3000, 9001, 22))]
    for name, args in cases:
        print(f"case: decode_paged_noalloc {name}", flush=True)
        x = _case(gpu, *args)
        B, hq, _ = x["q"].shape
        ws = L.aac_decode_workspace_bytes(B, hq, x["kc"].shape[2], 128, x["bs"], x["bt"].shape[1],
                                          x["max_ctx"], 0)
        assert 0 < ws <= SCRATCH_BYTES, ws  # a split plan that uses the scratch
        ref = fai.decode_paged(x["q"], x["kc"], x["vc"], x["bt_g"], x["ctx_g"],
                               max_context_len=x["max_ctx"])
        out = torch.full_like(x["q"], float("nan"))
        _noalloc(x, out)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), name
        seqs = [0, B // 2, B - 1]
        o_ref, absv = _oracle_sample(x, seqs)
        check_attention(out[seqs], o_ref, what=f"noalloc {name}", absv=absv)


def test_noalloc_refuses_a_plan_beyond_the_scratch(gpu):
    # 1024 sequences x 32 query heads, 64k-token tables split in 256-token
    # partitions: a 4.3 GB plan.  Refused on the host; the placeholder
    # pointers are never passed to a kernel.
    L = _lib.lib()
    need = L.aac_decode_workspace_bytes(1024, 32, 8, 128, 256, 256, 0, 256)
    assert need > SCRATCH_BYTES
    p = 1 << 12
    rc = L.aac_decode_paged_noalloc(p, 4096, p, p, 1 << 16, 256, p, 256, p, 1024, 0, 32, 8, 128,
                                    0.088, p, 4096, 256, 0, None)
    assert rc == -6 and b"scratch" in L.aac_strerror(rc)


_CAPTURE_CHILD = r"""
import sys
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2]]
from awesome_acceleration_amd import flash_attn_interface as fai
import test_zz_no_alloc as t

gpu = torch.device("cuda:0")
x = t._case(gpu, 16, 32, 8, 16384, 24577, 21)

def eager():
    return fai.decode_paged(x["q"], x["kc"], x["vc"], x["bt_g"], x["ctx_g"],
                            max_context_len=x["max_ctx"])

ref = eager()
out = torch.full_like(x["q"], float("nan"))
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):  # the process's first aac_decode_paged_noalloc call
    t._noalloc(x, out)
torch.cuda.synchronize()
for i in range(3):
    out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
    again = eager()  # eager work between the replays
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), ref.view(torch.int16))
print("capture ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(gpu):
    """A fresh process whose first no-alloc call is made under HIP graph
    capture (the scratch address is looked up then): the captured graph,
    replayed three times with eager calls in between, gives the eager
    workspace entry point's result bit for bit."""
    import os
    import subprocess
    import sys
    print("case: decode_paged_noalloc first called under graph capture (child process)", flush=True)
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root, here], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0 and "capture ok" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])

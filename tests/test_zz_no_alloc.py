"""fam_attention_noalloc (key-split attention with the split partials in the library's static
device scratch) against fam_attention + fam_attention_combine with caller-provided partial
buffers, through the C ABI: bit-identical outputs on two calls in a row, the second smaller
(the scratch keeps the first call's contents), and oversized calls rejected before launch."""
import ctypes as C
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _desc(q, k, v, o, H, splits, part_o=None, part_ml=None, mask=None):
    from fam import _capi
    B, Sq, A = q.shape
    Dh = A // H
    d = _capi.AttnDesc()
    d.q, d.q_bs, d.q_rs, d.q_hs = q.data_ptr(), q.stride(0), q.stride(1), Dh
    d.k0, d.k0_bs, d.k0_rs, d.k0_hs = k.data_ptr(), (k.stride(0) if k.shape[0] == B else 0), k.stride(1), Dh
    d.v0, d.v0_bs, d.v0_rs, d.v0_hs = v.data_ptr(), (v.stride(0) if v.shape[0] == B else 0), v.stride(1), Dh
    d.o, d.o_bs, d.o_rs, d.o_hs = o.data_ptr(), o.stride(0), o.stride(1), Dh
    d.batch, d.heads, d.sq, d.sk0, d.sk1, d.head_dim = B, H, Sq, k.shape[1], 0, Dh
    d.scale = 1.0 / math.sqrt(Dh)
    d.mask_kind = _capi.FAM_MASK_NONE
    if mask is not None:
        d.mask, d.mask_kind, d.mask_bs, d.mask_hs, d.mask_qs = mask.data_ptr(), _capi.FAM_MASK_BOOL, 0, 0, mask.stride(0)
    d.num_splits = splits
    if part_o is not None:
        d.part_o, d.part_ml = part_o.data_ptr(), part_ml.data_ptr()
    return d


def _reference(lib, q, k, v, H, splits, mask=None):
    B, Sq, A = q.shape
    nq = B * H * Sq
    part_o = torch.empty(splits * nq * (A // H), dtype=torch.float32, device="cuda")
    part_ml = torch.empty(splits * nq * 2, dtype=torch.float32, device="cuda")
    o = torch.empty_like(q)
    d = _desc(q, k, v, o, H, splits, part_o, part_ml, mask)
    s = torch.cuda.current_stream().cuda_stream
    assert lib.fam_attention(C.byref(d), s) == 0
    assert lib.fam_attention_combine(C.byref(d), s) == 0
    return o


def _noalloc(lib, q, k, v, H, splits, mask=None):
    o = torch.full_like(q, float("nan"))
    d = _desc(q, k, v, o, H, splits, mask=mask)
    rc = lib.fam_attention_noalloc(C.byref(d), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.fam_last_error().decode()
    return o


def _inputs(seed, B, Sq, Sk, H, Dh, ctx_batch):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Sq, H * Dh, generator=g).to(BF).cuda()
    k = torch.randn(ctx_batch, Sk, H * Dh, generator=g).to(BF).cuda()
    v = torch.randn(ctx_batch, Sk, H * Dh, generator=g).to(BF).cuda()
    return q, k, v


def test_noalloc_first_call_under_graph_capture():
    """The set-up call resolves the scratch address; the first fam_attention_noalloc of the process
    (when this file runs alone) is then made under torch.cuda.graph capture.  Each replay, with new
    inputs copied into the captured buffers and eager library work and synchronisations between
    replays, is bit-identical to fam_attention + fam_attention_combine on caller buffers."""
    from fam import _capi
    lib = _capi.load()
    assert lib.fam_attention_noalloc_max_bytes() == 8 << 20   # set-up, before any capture
    B, Sq, Sk, H, Dh, splits = 1, 32, 1560, 16, 64, 13
    q, k, v = _inputs(200, B, Sq, Sk, H, Dh, 1)
    o = torch.full_like(q, float("nan"))
    d = _desc(q, k, v, o, H, splits)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.fam_attention_noalloc(C.byref(d), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.fam_last_error().decode()
    for rep in range(3):
        q2, k2, v2 = _inputs(300 + rep, B, Sq, Sk, H, Dh, 1)
        q.copy_(q2), k.copy_(k2), v.copy_(v2)
        o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        # eager library work between replays, on other inputs, through the same scratch
        _noalloc(lib, *_inputs(400 + rep, 1, 17, 600, 8, 128, 1), 8, 5)
        ref = _reference(lib, q, k, v, H, splits)
        torch.cuda.synchronize()
        print(f"graph replay {rep}: bit-identical {torch.equal(o, ref)}", flush=True)
        assert torch.equal(o, ref)


def test_noalloc_matches_caller_buffers_on_two_calls():
    from fam import _capi
    lib = _capi.load()
    assert lib.fam_attention_noalloc_max_bytes() == 8 << 20
    # call 1: the config-1 cross attention (32 action tokens x 1560 context keys, 16 x 64 heads,
    # 13 key splits); call 2: smaller (fewer queries, heads and splits), so a stale tail of the
    # first call's partials stays in the scratch
    cases = [(1, 32, 1560, 16, 64, 13, 1), (1, 17, 600, 8, 128, 5, 1)]
    outs = []
    for (B, Sq, Sk, H, Dh, splits, cb) in cases:
        q, k, v = _inputs(100 + Sq, B, Sq, Sk, H, Dh, cb)
        ref = _reference(lib, q, k, v, H, splits)
        got = _noalloc(lib, q, k, v, H, splits)
        torch.cuda.synchronize()
        print(f"noalloc B={B} Sq={Sq} Sk={Sk} H={H} Dh={Dh} splits={splits}: bit-identical {torch.equal(got, ref)}",
              flush=True)
        assert torch.equal(got, ref)
        outs.append(got)
    # the scratch now holds the second call's partials over a stale tail of the first's: a third
    # call with mostly empty key splits (40 keys over 8 splits) and the first call again must read
    # only partials they wrote themselves
    for (B, Sq, Sk, H, Dh, splits, cb) in [(1, 32, 40, 16, 64, 8, 1), cases[0]]:
        q, k, v = _inputs(500 + Sk, B, Sq, Sk, H, Dh, cb)
        ref = _reference(lib, q, k, v, H, splits)
        got = _noalloc(lib, q, k, v, H, splits)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (Sk, splits)


def test_noalloc_masked_batched_rows():
    """Two batch rows over a shared context with a bool mask (a fully masked query row gives 0)."""
    from fam import _capi
    lib = _capi.load()
    q, k, v = _inputs(7, 2, 32, 300, 16, 64, 1)
    mask = torch.rand(32, 300, generator=torch.Generator().manual_seed(8)) > 0.4
    mask[3] = False
    mask = mask.cuda()
    ref = _reference(lib, q, k, v, 16, 4, mask)
    got = _noalloc(lib, q, k, v, 16, 4, mask)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.count_nonzero(got[:, 3]) == 0


def test_noalloc_rejects_oversize_and_bad_splits():
    from fam import _capi
    lib = _capi.load()
    s = torch.cuda.current_stream().cuda_stream
    # 32 rows x 16 heads x 32 queries x 64 splits x (64 + 2) x 4 bytes = 138 MB > 8 MiB
    q, k, v = _inputs(9, 32, 32, 2048, 16, 64, 1)
    o = torch.empty_like(q)
    d = _desc(q, k, v, o, 16, 64)
    assert lib.fam_attention_noalloc(C.byref(d), s) == _capi.FAM_ERR_UNSUPPORTED
    assert "scratch" in lib.fam_last_error().decode()
    d.num_splits = 1
    assert lib.fam_attention_noalloc(C.byref(d), s) == _capi.FAM_ERR_INVALID_ARG

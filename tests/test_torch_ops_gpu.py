"""GPU parity of the torch.library operator layer against the oracle: the reference's fastwam::
operator forms (fam.fastwam_ops) and the fam:: drop-ins under torch.compile(fullgraph=True).
Bar: normwise max relative error <= 2e-2 against the fp32 oracle on bf16-valued inputs."""
import math

import pytest
import torch

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _rel(y, ref):
    y, ref = y.float().cpu(), ref.float().cpu()
    return ((y - ref).abs().max() / ref.abs().max()).item()


def _rand(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(BF)


@pytest.fixture(scope="module")
def fw():
    from fam import fastwam_ops
    return fastwam_ops


@pytest.mark.parametrize("mask_kind", [None, "bool", "add_f32", "add_bf16"])
@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
def test_short_attn(fw, layout, mask_kind):
    g = torch.Generator().manual_seed(3)
    B, H, Sq, Sk, D = 1, 24, 32, 130, 128
    q, k, v = _rand(g, B, H, Sq, D), _rand(g, B, H, Sk, D), _rand(g, B, H, Sk, D)
    keep = torch.rand(Sq, Sk, generator=g) > 0.3
    keep[:, 0] = True
    mask = None
    if mask_kind == "bool":
        mask = keep
    elif mask_kind is not None:
        mask = torch.zeros(Sq, Sk).masked_fill(~keep, float("-inf")).to(torch.float32 if mask_kind == "add_f32" else BF)
    ref = O.attention(q.float(), k.float(), v.float(), keep if mask_kind else None)
    dm = mask.cuda() if mask is not None else None
    if layout == "bhsd":
        o = torch.ops.fastwam.short_attn.default(q.cuda(), k.cuda(), v.cuda(), dm, H)
        assert o.shape == (B, H, Sq, D)
        assert _rel(o, ref) <= 2e-2
        o2 = torch.ops.fastwam.short_attn_bsd.default(q.cuda(), k.cuda(), v.cuda(), dm, H)
        assert o2.shape == (B, Sq, H * D)
        assert _rel(o2, ref.transpose(1, 2).reshape(B, Sq, H * D)) <= 2e-2
    else:
        f = lambda t: t.transpose(1, 2).reshape(B, t.shape[2], H * D).contiguous().cuda()  # noqa: E731
        o = torch.ops.fastwam.short_attn.default(f(q), f(k), f(v), dm, H)
        assert _rel(o, ref.transpose(1, 2).reshape(B, Sq, H * D)) <= 2e-2


def test_qrms_attn(fw):
    g = torch.Generator().manual_seed(4)
    Sq, Sk, H, D = 32, 129, 24, 128
    qraw, k, v = _rand(g, 1, Sq, H * D), _rand(g, 1, Sk, H * D), _rand(g, 1, Sk, H * D)
    wq = (1 + 0.2 * torch.randn(H * D, generator=g)).to(BF)
    o = torch.ops.fastwam.qrms_attn.default(qraw.cuda(), wq.cuda(), k.cuda(), v.cuda(), None, H, 1e-6)
    ref = O.flash_attention(O.rms_norm(qraw, wq, 1e-6).float(), k.float(), v.float(), H)
    assert _rel(o, ref) <= 2e-2


def _packed(freqs):
    """The reference's packed real table [S, Dh] = cat(cos, sin) (FG/wan_video_dit.py:173-177)."""
    f = freqs.reshape(freqs.shape[0], -1)
    return torch.cat([f.real, f.imag], -1).float().contiguous()


@pytest.mark.parametrize("S,Sv,N,head", [(32, 98, 3072, 128), (8, 6, 1024, 64)])
def test_qkv_post_and_qk_post(fw, S, Sv, N, head):
    """q returned; RMSNorm+RoPE'd k and raw v land in rows [Sv, Sv + S) of the joint cache;
    the video rows stay untouched.  qk_post returns the same q and k."""
    g = torch.Generator().manual_seed(5)
    qkv = _rand(g, S, 3 * N)
    wqk = (1 + 0.2 * torch.randn(2, N, generator=g)).to(BF)
    fr = O.action_freqs(head, S)
    kbuf = _rand(g, 1, Sv + S, N).cuda()
    vbuf = _rand(g, 1, Sv + S, N).cuda()
    kv0, vv0 = kbuf[:, :Sv].clone(), vbuf[:, :Sv].clone()
    sgn = torch.tensor([-1.0, 1.0], device="cuda")
    nh = N // head
    q = torch.ops.fastwam.qkv_post.default(qkv.cuda(), wqk.cuda(), _packed(fr).cuda(), sgn, kbuf, vbuf, Sv, head, 1e-6)
    x = qkv.float().reshape(1, S, 3 * N)
    rq = O.rope_apply(O.rms_norm(x[..., :N].to(BF), wqk[0], 1e-6).float(), fr, nh)
    rk = O.rope_apply(O.rms_norm(x[..., N:2 * N].to(BF), wqk[1], 1e-6).float(), fr, nh)
    assert q.shape == (1, S, N)
    assert _rel(q, rq) <= 2e-2
    assert _rel(kbuf[:, Sv:], rk) <= 2e-2
    assert torch.equal(vbuf[:, Sv:].cpu(), qkv[:, 2 * N:].reshape(1, S, N))
    assert torch.equal(kbuf[:, :Sv], kv0) and torch.equal(vbuf[:, :Sv], vv0)
    q2, k2 = torch.ops.fastwam.qk_post.default(qkv.cuda(), wqk.cuda(), _packed(fr).cuda(), sgn, head, 1e-6)
    assert torch.equal(q2, q) and torch.equal(k2, kbuf[:, Sv:])


@pytest.mark.parametrize("M,N,K", [(32, 1024, 3072), (32, 4096, 1024), (98, 3072, 3072)])
def test_skmm(fw, M, N, K):
    g = torch.Generator().manual_seed(6)
    x, w = _rand(g, 1, M, K), _rand(g, N, K, scale=0.02)
    y = torch.ops.fastwam.skmm.default(x.cuda(), w.cuda())
    assert y.shape == (1, M, N)
    assert _rel(y, x.float() @ w.float().t()) <= 2e-2


@pytest.mark.parametrize("mode", ["ln_affine_gate", "adaln_gate", "adaln_nogate", "ln_fp32_x"])
def test_skpost(fw, mode):
    """Split-K product + bias + gate*y + residual + LayerNorm / AdaLN (FG/mot.py:1315-1348),
    against the reference block's eager order (FB/wan_video_dit.py:271-285)."""
    g = torch.Generator().manual_seed(7)
    M, N, K = 32, 1024, 3072
    a, w = _rand(g, 1, M, K), _rand(g, N, K, scale=0.02)
    bias, res = _rand(g, N, scale=0.02), _rand(g, 1, M, N)
    modg, moda, tmod = _rand(g, 1, 6, N, scale=0.1), _rand(g, 1, 6, N, scale=0.1), _rand(g, 1, 6, N, scale=0.1)
    lnw, lnb = (1 + 0.2 * torch.randn(N, generator=g)).to(BF), (0.2 * torch.randn(N, generator=g)).to(BF)
    affine = mode.startswith("ln")
    gi, si, hi = (2 if mode != "adaln_nogate" else -1), 4, 3
    xdt = 1 if mode == "ln_fp32_x" else 0
    d = lambda t: t.cuda() if t is not None else None  # noqa: E731
    xo, yo = torch.ops.fastwam.skpost.default(d(a), d(w), d(bias), d(res), d(modg), d(moda), d(tmod),
                                              d(lnw) if affine else None, d(lnb) if affine else None,
                                              gi, si, hi, 1e-6, xdt)
    assert xo.dtype == (torch.float32 if xdt else BF) and yo.dtype == BF
    y = O.linear(a.float(), w.float(), bias.float())
    if gi >= 0:
        y = (modg[0, gi] + tmod[0, gi]).float() * y
    x = res.float() + y
    if affine:
        o = O.layer_norm(x, lnw.float(), lnb.float(), 1e-6)
    else:
        o = O.adaln(x, (moda[0, hi] + tmod[0, hi]).float(), (moda[0, si] + tmod[0, si]).float(), 1e-6)
    assert _rel(xo, x) <= 2e-2
    assert _rel(yo, o) <= 2e-2


@pytest.mark.parametrize("xdt,affine", [(0, True), (0, False), (1, True), (1, False)])
def test_skpost_follows_the_eager_rounding(fw, xdt, affine):
    """fastwam::skpost pinned to the eager block it stands in for (FB/wan_video_dit.py:271-285), far
    inside the 2e-2 bar: the gate is the bf16 sum modulation + t_mod (the eager chunk), the
    residual add rounds once to bf16 and the norm reads that bf16 row.  (The GEAK Triton op,
    FG/mot.py:1283-1313, sums the gate in fp32 and normalises the unrounded fp32 x instead: a
    different rounding order, about one bf16 ulp apart.)  With xdt = 1 the stored x is the fp32
    res + gate * (a w^T + bias)."""
    g = torch.Generator().manual_seed(17)
    M, N, K = 32, 1024, 3072
    a, w = _rand(g, 1, M, K), _rand(g, N, K, scale=0.02)
    bias, res = _rand(g, N, scale=0.02), _rand(g, 1, M, N)
    modg, moda, tmod = _rand(g, 1, 6, N, scale=0.1), _rand(g, 1, 6, N, scale=0.1), _rand(g, 1, 6, N, scale=0.1)
    lnw, lnb = (1 + 0.2 * torch.randn(N, generator=g)).to(BF), (0.2 * torch.randn(N, generator=g)).to(BF)
    gi, si, hi = 2, 4, 3
    d = lambda t: t.cuda() if t is not None else None  # noqa: E731
    xo, yo = torch.ops.fastwam.skpost.default(d(a), d(w), d(bias), d(res), d(modg), d(moda), d(tmod),
                                              d(lnw) if affine else None, d(lnb) if affine else None,
                                              gi, si, hi, 1e-6, xdt)
    # eager bf16 composition: chunks of (modulation + t_mod) in bf16, nn.Linear output in bf16,
    # x = x + gate * y in bf16, then the norm of the bf16 x
    chunks, chunks_a = (modg + tmod)[0], (moda + tmod)[0]         # bf16 sums
    y32 = a[0].double() @ w.double().t() + bias.double()
    gate = chunks[gi].double()
    x_e = (res[0].double() + gate * y32.to(BF).double()).to(BF)
    xf = x_e.double()
    ln = (xf - xf.mean(-1, keepdim=True)) / torch.sqrt(xf.var(-1, unbiased=False, keepdim=True) + 1e-6)
    if affine:
        o_e = ln * lnw.double() + lnb.double()
    else:
        o_e = ln * (1 + chunks_a[si].double()) + chunks_a[hi].double()
    xo, yo = xo[0].cpu().double(), yo[0].cpu().double()
    if xdt:
        x32 = res[0].double() + gate * y32
        assert ((xo - x32).abs().max() / x32.abs().max()).item() <= 1e-5
    else:
        # one bf16 rounding of x apart at most (the eager form rounds y and gate * y as well)
        ulp = torch.finfo(BF).eps
        assert ((xo - xf).abs() <= ulp * (xf.abs() + (gate * y32).abs()) + 1e-6).all()
    assert ((yo - o_e).abs().max() / o_e.abs().max()).item() <= 8e-3
    # a swapped scale / shift or a dropped gate moves the result far past these bounds
    if not affine:
        swapped = ln * (1 + chunks_a[hi].double()) + chunks_a[si].double()
        assert ((yo - swapped).abs().max() / o_e.abs().max()).item() > 5e-2


def test_fam_ops_under_torch_compile_match_eager():
    """A block-shaped module calling the fam:: drop-ins, compiled with fullgraph=True
    (aot_eager: no generated kernels around them), gives the eager result bit for bit."""
    from fam import ops

    class Blk(torch.nn.Module):
        def __init__(self, g, D=1024, H=16):
            super().__init__()
            self.H = H
            self.norm = torch.nn.LayerNorm(D, elementwise_affine=False, eps=1e-6)
            self.wq = torch.nn.Parameter(_rand(g, D, D, scale=0.02).cuda(), requires_grad=False)
            self.bq = torch.nn.Parameter(_rand(g, D, scale=0.02).cuda(), requires_grad=False)
            self.nq = torch.nn.Parameter((1 + 0.2 * torch.randn(D, generator=g)).to(BF).cuda(), requires_grad=False)

        def forward(self, x, shift, scale, freqs, delta, ctx):
            h = ops.adaln_forward(x, self.norm, shift, scale)
            q = ops.rms_norm_rope(ops.linear(h, self.wq, self.bq), self.nq, 1e-6, freqs, self.H, "complex")
            o = ops.flash_attention(q, ctx, ctx, self.H)
            o = ops.layer_norm(o, None, None, 1e-6)
            return ops.WanContinuousFlowMatchScheduler.step(o, delta, x)

    g = torch.Generator().manual_seed(8)
    m = Blk(g)
    x, sh, sc = _rand(g, 1, 32, 1024).cuda(), _rand(g, 1, 1, 1024, scale=0.1).cuda(), _rand(g, 1, 1, 1024,
                                                                                           scale=0.1).cuda()
    ctx = _rand(g, 1, 1560, 1024).cuda()
    fr = O.action_freqs(64, 32).cuda()
    delta = torch.tensor(-0.0625, dtype=BF, device="cuda")
    with torch.no_grad():
        e = m(x, sh, sc, fr, delta, ctx)
        c = torch.compile(m, fullgraph=True, backend="aot_eager")(x, sh, sc, fr, delta, ctx)
    torch.cuda.synchronize()
    assert torch.equal(e, c)
    # and the eager result against the oracle
    p = {"w": m.wq.float().cpu(), "b": m.bq.float().cpu(), "n": m.nq.float().cpu()}
    h = O.adaln(x.float().cpu(), sh.float().cpu(), sc.float().cpu(), 1e-6).to(BF).float()
    q = O.rope_apply(O.rms_norm(O.linear(h, p["w"], p["b"]).to(BF), p["n"].to(BF), 1e-6).float(), fr.cpu(), 16)
    o = O.layer_norm(O.flash_attention(q, ctx.float().cpu(), ctx.float().cpu(), 16), None, None, 1e-6)
    ref = x.float().cpu() + o * -0.0625
    assert (e.float().cpu() - ref).abs().max().item() <= 0.0625 * 0.1 + 2e-2


@pytest.mark.parametrize("layout", ["cat", "interleaved"])
def test_rope_real_device_tables_match_complex(layout):
    """rope_apply with FG's packed table and rope_apply_cae with CA's interleaved table, both fp32
    device tables used in place, give the rotation of the complex table; each rejects the other."""
    from fam import ops
    g = torch.Generator().manual_seed(9)
    x = _rand(g, 1, 64, 1024).cuda()
    fr = O.action_freqs(64, 64)
    cat = _packed(fr).reshape(64, 1, 64)
    ref = O.rope_apply(x.float().cpu(), fr, 16)
    if layout == "cat":
        y = ops.rope_apply(x, cat.cuda(), 16)
        with pytest.raises(ValueError):
            ops.rope_apply_cae(x, cat.cuda(), 16)
    else:
        inter = torch.stack([cat[..., :32], cat[..., 32:]], -1).reshape(64, 1, 64).contiguous()
        y = ops.rope_apply_cae(x, inter.cuda(), 16)
        with pytest.raises(ValueError):
            ops.rope_apply(x, inter.cuda(), 16)
    assert _rel(y, ref) <= 2e-2
    assert torch.equal(y, ops.rope_apply(x, fr.cuda(), 16))

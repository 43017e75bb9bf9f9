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


# --------------------------------------------------------------------------- GEAK prefill / CAE operators
def test_geak_prefill_ops(fw):
    """pf_mm, pf_mm_gelu and the residual + LayerNorm / AdaLN operators of the GEAK prefill at its
    shape (98 tokens, hidden 3072, per-token t_mod [S, 6N]) against the oracle's restatement of the
    reference kernel (FG/mot.py:1693-1899)."""
    g = torch.Generator().manual_seed(91)
    S, N, K, eps = 98, 3072, 512, 1e-6
    x, w, b = _rand(g, 1, S, K), _rand(g, N, K, scale=0.05), _rand(g, N, scale=0.1)
    assert _rel(fw.pf_mm(x.cuda(), w.cuda(), b.cuda()), O.linear(x.float(), w.float(), b.float())) <= 2e-2
    assert _rel(fw.pf_mm_gelu(x.cuda(), w.cuda(), b.cuda()),
                O.gelu_tanh(O.linear(x.float(), w.float(), b.float()))) <= 2e-2
    xr, o1, o2 = _rand(g, 1, S, N), _rand(g, 1, S, N), _rand(g, 1, S, N)
    mb, mb2, tm = _rand(g, 6 * N, scale=0.3), _rand(g, 6 * N, scale=0.3), _rand(g, S, 6 * N, scale=0.3)
    wn, bn = (1 + 0.2 * torch.randn(N, generator=g)).to(BF), _rand(g, N, scale=0.2)
    f = lambda t: t.float()  # noqa: E731

    def ch(m, off):
        return f(m).reshape(-1)[off:off + N][None, :] + f(tm)[:, off:off + N]
    dev = [t.cuda() for t in (xr, o1, o2, mb, mb2, tm, wn, bn)]
    xd, o1d, o2d, mbd, mb2d, tmd, wnd, bnd = dev
    y1 = fw.res_ln1(xd, o1d, mbd, tmd, wnd, bnd, 2 * N, eps)
    _, r1 = O.geak_res_ln(f(xr)[0], [f(o1)[0]], ch(mb, 2 * N), eps, ln=(f(wn), f(bn)))
    x2, y2 = fw.res_ln2(xd, o1d, o2d, mbd, mb2d, tmd, 2 * N, 3 * N, 4 * N, eps)
    t2, r2 = O.geak_res_ln(f(xr)[0], [f(o1)[0], f(o2)[0]], ch(mb, 2 * N), eps, ada=(ch(mb2, 3 * N), ch(mb2, 4 * N)))
    x3, y3 = fw.res_ln_tail(xd, o1d, mbd, mb2d, tmd, 5 * N, 0, N, eps)
    t3, r3 = O.geak_res_ln(f(xr)[0], [f(o1)[0]], ch(mb, 5 * N), eps, ada=(ch(mb2, 0), ch(mb2, N)))
    errs = [_rel(y1[0], r1), _rel(x2[0], t2), _rel(y2[0], r2), _rel(x3[0], t3), _rel(y3[0], r3)]
    print("res_ln1 / res_ln2 (x, norm) / res_ln_tail (x, norm):", " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) <= 2e-2



def test_geak_prefill_split_planes(fw):
    """pf_skmm / pf_skmm_big and their consumers res_ln1_sk, res_ln2_sk, res_ln_tail_sk and
    pf_qcomb at the prefill's shape (FG/mot.py:2017-2329).  The consumers get planes made the way
    the reference's producer makes them (the K-chunks of a product in the first sk planes, other
    values past sk) and are held to the oracle's restatement of the reference kernels; the
    producers' planes summed over any leading count give the product."""
    g = torch.Generator().manual_seed(93)
    S, N, K, sk, eps = 98, 3072, 512, 4, 1e-6
    f = lambda t: t.float()  # noqa: E731
    a, w, bi = _rand(g, 1, S, K), _rand(g, N, K, scale=0.05), _rand(g, N, scale=0.1)
    prod = O.linear(f(a)[0], f(w), None)
    for op, skmax in ((fw.pf_skmm, 8), (fw.pf_skmm_big, 16)):
        pl = op(a.cuda(), w.cuda())
        assert pl.shape == (skmax, S, N) and pl.dtype == torch.float32
        for n in (1, sk, skmax):
            assert _rel(pl[:n].sum(0), prod) <= 2e-2
    planes = torch.randn(8, S, N, generator=g) * 5.0   # past sk: values the consumer must not read
    for i in range(sk):
        c = slice(i * K // sk, (i + 1) * K // sk)
        planes[i] = f(a)[0, :, c] @ f(w)[:, c].T
    o_ref = O.geak_split_combine(planes, f(bi), sk)
    xr, o1 = _rand(g, 1, S, N), _rand(g, 1, S, N)
    mb, mb2, tm = _rand(g, 6 * N, scale=0.3), _rand(g, 6 * N, scale=0.3), _rand(g, S, 6 * N, scale=0.3)
    wn, bn = (1 + 0.2 * torch.randn(N, generator=g)).to(BF), _rand(g, N, scale=0.2)
    wq = (1 + 0.2 * torch.randn(N, generator=g)).to(BF)

    def ch(m, off):
        return f(m).reshape(-1)[off:off + N][None, :] + f(tm)[:, off:off + N]
    pd, bid, xd, o1d, mbd, mb2d, tmd = (t.cuda() for t in (planes, bi, xr, o1, mb, mb2, tm))
    y1, o = fw.res_ln1_sk(xd, pd, bid, mbd, tmd, wn.cuda(), bn.cuda(), 2 * N, eps, sk)
    _, r1 = O.geak_res_ln(f(xr)[0], [o_ref], ch(mb, 2 * N), eps, ln=(f(wn), f(bn)))
    x2, y2 = fw.res_ln2_sk(xd, o1d, pd, bid, mbd, mb2d, tmd, 2 * N, 3 * N, 4 * N, eps, sk)
    t2, r2 = O.geak_res_ln(f(xr)[0], [f(o1)[0], o_ref], ch(mb, 2 * N), eps, ada=(ch(mb2, 3 * N), ch(mb2, 4 * N)))
    x3, y3 = fw.res_ln_tail_sk(xd, pd, bid, mbd, mb2d, tmd, 5 * N, 0, N, eps, sk)
    t3, r3 = O.geak_res_ln(f(xr)[0], [o_ref], ch(mb, 5 * N), eps, ada=(ch(mb2, 0), ch(mb2, N)))
    qn = fw.pf_qcomb(pd, bid, wq.cuda(), eps, sk)
    rq = O.geak_qcomb(planes, f(bi), f(wq), eps, sk)
    errs = [_rel(o[0], o_ref), _rel(y1[0], r1), _rel(x2[0], t2), _rel(y2[0], r2), _rel(x3[0], t3),
            _rel(y3[0], r3), _rel(qn[0], rq)]
    print("combine / res_ln1_sk / res_ln2_sk (x, norm) / res_ln_tail_sk (x, norm) / pf_qcomb:",
          " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) <= 2e-2
    assert _rel(O.geak_split_combine(planes, f(bi), sk + 1), o_ref) > 0.5   # a plane past sk would show
    # the producer feeding the consumer: the o-projection through pf_skmm into res_ln1_sk
    y1c, oc = fw.res_ln1_sk(xd, fw.pf_skmm(a.cuda(), w.cuda()), bid, mbd, tmd, wn.cuda(), bn.cuda(), 2 * N, eps, sk)
    assert _rel(oc[0], O.linear(f(a)[0], f(w), f(bi))) <= 2e-2 and _rel(y1c[0], r1) <= 2e-2
    with pytest.raises(ValueError):
        fw.pf_qcomb(pd, bid, wq.cuda(), eps, 9)


def test_cae_ops(fw):
    """The CAE action expert's operators at its shape (8 tokens, hidden 32, 24 x 128 heads, 98 + 8
    joint keys, 129 context keys, 30 layers' context K) against the oracle's restatements of the
    reference kernels (CA/mot.py:1369-1456, 2119-2142, 2240-2343, 2485-2521; CA/action_dit.py:127-187)."""
    g = torch.Generator().manual_seed(92)
    M, H, hd, Sv, Lc, eps = 8, 24, 128, 98, 129, 1e-6
    D = H * hd
    f = lambda t: t.float()  # noqa: E731
    # q/k post-processing into the head-major joint K/V cache
    qkv = _rand(g, 1, M, 3 * D)
    qw, kw = (1 + 0.2 * torch.randn(D, generator=g)).to(BF), (1 + 0.2 * torch.randn(D, generator=g)).to(BF)
    ang = torch.arange(M, dtype=torch.float64)[:, None] * (10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    freqs = torch.stack([ang.cos(), ang.sin()], -1).reshape(M, hd).float()
    kbuf, vbuf = _rand(g, 1, H, Sv + M, hd), _rand(g, 1, H, Sv + M, hd)
    kb, vb = kbuf.cuda(), vbuf.cuda()
    q = fw.mot_qkv_post(qkv.cuda(), qw.cuda(), kw.cuda(), freqs.cuda(), kb, vb, Sv, eps)
    rq, rk, rv = O.cae_qkv_post(f(qkv[0]), f(qw), f(kw), freqs.double().float(), H, eps)
    errs = {"qkv_post q": _rel(q[0], rq), "k rows": _rel(kb[0, :, Sv:], rk), "v rows": _rel(vb[0, :, Sv:], rv)}
    assert torch.equal(kb[0, :, :Sv].cpu(), kbuf[0, :, :Sv]) and torch.equal(vb[0, :, :Sv].cpu(), vbuf[0, :, :Sv])
    # joint attention, head-major and row layouts, with a keep mask
    keep = torch.rand(M, Sv + M, generator=g) > 0.25
    keep[:, Sv:] = True
    oa = fw.mot_attn(q, kb, vb, keep.to(torch.uint8).cuda(), H, hd, True)
    ra = O.attention(f(q.cpu()), f(kb.cpu()), f(vb.cpu()), keep[None, None])[0].transpose(0, 1).reshape(M, D)
    errs["mot_attn"] = _rel(oa[0], ra)
    qb = q[0].transpose(0, 1).reshape(1, M, D).contiguous()
    kr = kb[0].transpose(0, 1).reshape(1, Sv + M, D).contiguous()
    vr = vb[0].transpose(0, 1).reshape(1, Sv + M, D).contiguous()
    errs["mot_attn rows"] = _rel(fw.mot_attn(qb, kr, vr, keep.cuda(), H, hd, False)[0], ra)
    # cross attention with the whole-row query norm
    qr, kc, vc = _rand(g, 1, M, D), _rand(g, 1, Lc, D), _rand(g, 1, Lc, D)
    ck = torch.ones(M, Lc, dtype=torch.bool)
    ck[:, Lc - 20:] = False
    ox = fw.xattn_qn(qr.cuda(), qw.cuda(), kc.cuda(), vc.cuda(), ck.cuda(), H, hd, eps)
    errs["xattn_qn"] = _rel(ox[0], O.cae_xattn_qn(f(qr[0]), f(qw), f(kc[0]), f(vc[0]), ck, H, eps))
    # every layer's context keys
    nl = 30
    gk, nkw = _rand(g, Lc, 2 * nl * D), (1 + 0.2 * torch.randn(nl, D, generator=g)).to(BF)
    kn = fw.ctx_kv_norm(gk.cuda(), nkw.cuda(), nl, D, eps)
    assert kn.shape == (1, nl, 1, Lc, D)
    errs["ctx_kv_norm"] = _rel(kn[0, :, 0], O.cae_ctx_kv_norm(f(gk), f(nkw), nl, D, eps))
    # o projection, FFN, time MLP + action encoder
    wo, bo = _rand(g, 32, D, scale=0.02), _rand(g, 32, scale=0.1)
    errs["mot_oproj"] = _rel(fw.mot_oproj(ox, wo.cuda(), bo.cuda())[0], O.linear(f(ox[0].cpu()), f(wo), f(bo)))
    xa = _rand(g, 1, M, 32)
    w1, b1, w2, b2 = _rand(g, 256, 32, scale=0.2), _rand(g, 256, scale=0.1), _rand(g, 32, 256, scale=0.06), _rand(g, 32, scale=0.1)
    errs["mot_ffn"] = _rel(fw.mot_ffn(xa.cuda(), w1.cuda(), b1.cuda(), w2.cuda(), b2.cuda())[0],
                           O.cae_ffn(f(xa[0]), f(w1), f(b1), f(w2), f(b2)))
    w0, b0 = _rand(g, 32, 256, scale=0.06), _rand(g, 32, scale=0.1)
    wt1, bt1, wt2, bt2 = _rand(g, 32, 32, scale=0.2), _rand(g, 32, scale=0.1), _rand(g, 192, 32, scale=0.2), _rand(g, 192, scale=0.1)
    atok, aw, ab = _rand(g, 1, M, 16), _rand(g, 32, 16, scale=0.25), _rand(g, 32, scale=0.1)
    inv = (10000.0 ** (-torch.arange(128, dtype=torch.float64) / 128)).cuda()
    ts = torch.tensor([640.0])
    t, tmod, tk = fw.adit_tmod(ts.cuda(), inv, w0.cuda(), b0.cuda(), wt1.cuda(), bt1.cuda(), wt2.cuda(), bt2.cuda(),
                               atok.cuda(), aw.cuda(), ab.cuda(), 1)
    rt, rtm, rtk = O.cae_adit_tmod(ts, f(w0), f(b0), f(wt1), f(bt1), f(wt2), f(bt2), f(atok), f(aw), f(ab))
    errs["adit_tmod t"], errs["t_mod"], errs["tokens"] = _rel(t, rt), _rel(tmod, rtm), _rel(tk, rtk)
    print("CAE operators:", ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert max(errs.values()) <= 2e-2, errs


def test_cae_fused_lever_ops(fw):
    """The CAE tree's fused operators at the action expert's shape (8 tokens, hidden 32, 24 x 128
    attention, 98 + 8 joint keys, 129 context keys, FFN 256) against the oracle's restatements of
    the reference kernels (CA/mot.py:1369-1680, 2015-2077, 2119-2210, 2346-2780, 2830-3565,
    3621-3750): the accumulating o-projections add their term to what acc held, the *_z forms
    clear rows [0, M) of their accumulators, and the bias planes of mask_bias drive the same
    attention as the keep masks they encode."""
    g = torch.Generator().manual_seed(94)
    M, D, H, hd, Sv, Lc, Fd, eps = 8, 32, 24, 128, 98, 129, 256, 1e-6
    NQ, SK = H * hd, Sv + M
    f = lambda t: t.float().cpu()  # noqa: E731
    cu = lambda *ts: [t.cuda() for t in ts]  # noqa: E731
    errs = {}
    # norm3 + cross q (+ its whole-row norm), and the cross attention with its o-projection
    res, so = _rand(g, 1, M, D), torch.randn(M, D, generator=g) * 0.5
    mod, tmod = _rand(g, 6 * D, scale=0.3), _rand(g, 1, 6 * D, scale=0.3)
    lnw, lnb = (1 + 0.2 * torch.randn(D, generator=g)).to(BF), _rand(g, D, scale=0.2)
    qw, qb = _rand(g, NQ, D, scale=D ** -0.5), _rand(g, NQ, scale=0.1)
    qnw, gram = (1 + 0.2 * torch.randn(NQ, generator=g)).to(BF), torch.zeros(D * D + D + 1)
    dres, dso, dmod, dtmod, dlnw, dlnb, dqw, dqb, dqnw, dgram = cu(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram)
    x, cq = fw.mod_n3q(dres, dso, dmod, dtmod, dlnw, dlnb, dqw, dqb, eps)
    rx, rcq = O.cae_mod_n3q(f(res)[0], so, f(mod), f(tmod), f(lnw), f(lnb), f(qw), f(qb), eps)
    errs["mod_n3q x"], errs["mod_n3q cq"] = _rel(x[0], rx), _rel(cq[0], rcq)
    _, cqn = fw.mod_n3q_qn(dres, dso, dmod, dtmod, dlnw, dlnb, dqw, dqb, dqnw, dgram, eps, eps)
    errs["mod_n3q_qn"] = _rel(cqn[0], O.cae_mod_n3q(f(res)[0], so, f(mod), f(tmod), f(lnw), f(lnb), f(qw), f(qb), eps,
                                                    qn=(f(qnw), eps))[1])
    ckv = _rand(g, 1, Lc, 2 * NQ)                          # keys and values interleaved per row: strided
    dckv = ckv.cuda()
    ck, cv = dckv[..., :NQ], dckv[..., NQ:]
    cm = torch.ones(1, Lc, dtype=torch.bool)
    cm[0, Lc - 20:] = False
    wo, bo = _rand(g, D, NQ, scale=NQ ** -0.5), _rand(g, D, scale=0.1)
    dwo, dbo = cu(wo, bo)
    acc0 = torch.randn(M, D, generator=g)
    acc = acc0.cuda()
    xr = fw.n3q_xoproj(dres, dso, dmod, dtmod, dlnw, dlnb, dqw, dqb, dqnw, dgram, ck, cv,
                       cm.expand(M, Lc)[None].cuda(), dwo, dbo, acc, H, eps, eps)
    rxx, term = O.cae_n3q_xoproj(f(res)[0], so, f(mod), f(tmod), f(lnw), f(lnb), f(qw), f(qb), f(qnw), f(ckv)[0, :, :NQ],
                                 f(ckv)[0, :, NQ:], cm.expand(M, Lc), f(wo), f(bo), H, eps, eps)
    errs["n3q_xoproj x"], errs["n3q_xoproj acc"] = _rel(xr[0], rxx), _rel(acc.cpu() - acc0, term)
    # the additive planes, and the same cross attention through them
    am = torch.rand(M, SK, generator=g) > 0.25
    am[:, Sv:] = True
    mp, skp, ncp = 16, 128, 256
    sb, xb = fw.mask_bias(am.cuda(), cm.cuda(), mp, skp, ncp)
    rsb, rxb = O.cae_mask_bias(am, cm, mp, skp, ncp)
    assert torch.equal(sb.cpu(), rsb) and torch.equal(xb.cpu(), rxb)
    acc_b = acc0.cuda()
    fw.n3q_xoproj(dres, dso, dmod, dtmod, dlnw, dlnb, dqw, dqb, dqnw, dgram, ck, cv, xb, dwo, dbo, acc_b, H, eps, eps)
    errs["n3q_xoproj via mask_bias"] = _rel(acc_b.cpu() - acc0, term)
    # self attention + o-projection into the accumulator, keep plane and bias plane
    q, kb, vb = _rand(g, 1, H, M, hd), _rand(g, 1, H, SK, hd), _rand(g, 1, H, SK, hd)
    rterm = O.cae_attn_oproj(f(q)[0], f(kb)[0], f(vb)[0], am, f(wo), f(bo))
    for name, mk in (("keep", am.to(torch.uint8).cuda()), ("bias", sb)):
        acc_s = acc0.cuda()
        fw.mot_attn_oproj(*cu(q, kb, vb), mk, dwo, dbo, acc_s, H, hd)
        errs["mot_attn_oproj " + name] = _rel(acc_s.cpu() - acc0, rterm)
    # FFN fold (+ the next block's AdaLN1), and the fused FFN + next layer's q / k / v
    xa, oacc = _rand(g, 1, M, D), torch.randn(M, D, generator=g) * 0.5
    modn = _rand(g, 6 * D, scale=0.3)
    w1, b1, w2, b2 = _rand(g, Fd, D, scale=D ** -0.5), _rand(g, Fd, scale=0.1), _rand(g, D, Fd, scale=Fd ** -0.5), \
        _rand(g, D, scale=0.1)
    dxa, doacc, dmodn, dw1, db1, dw2, db2 = cu(xa, oacc, modn, w1, b1, w2, b2)
    xo, ai = fw.mot_ffn_fold(dxa, doacc, dmod, dmodn, dtmod, dw1, db1, dw2, db2, eps, eps, 1)
    rxo, rai = O.cae_ffn_fold(f(xa)[0], oacc, f(mod), f(modn), f(tmod), f(w1), f(b1), f(w2), f(b2), eps, eps)
    errs["ffn_fold x"], errs["ffn_fold next"] = _rel(xo[0], rxo), _rel(ai[0], rai)
    xo0, _ = fw.mot_ffn_fold(dxa, doacc, dmod, dmodn, dtmod, dw1, db1, dw2, db2, eps, eps, 0)
    assert torch.equal(xo0, xo)
    # q / k / v post-processing variants, each against cae_qkv_post of the same projection
    ang = torch.arange(M, dtype=torch.float64)[:, None] * (10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    freqs = torch.stack([ang.cos(), ang.sin()], -1).reshape(M, hd).float()
    nqw, nkw = (1 + 0.2 * torch.randn(NQ, generator=g)).to(BF), (1 + 0.2 * torch.randn(NQ, generator=g)).to(BF)
    wqkv, bqkv = _rand(g, 3 * NQ, D, scale=D ** -0.5), _rand(g, 3 * NQ, scale=0.1)
    kv0 = _rand(g, 1, H, SK, hd)
    dfreqs, dnqw, dnkw, dwqkv, dbqkv = cu(freqs, nqw, nkw, wqkv, bqkv)
    qgr = torch.zeros(D * D + D + 1).cuda()

    def post_ref(rows):
        return O.cae_qkv_post(rows, f(nqw), f(nkw), freqs, H, eps)

    def chk(name, qo, kbuf, vbuf, rows, head_major=True, sv=Sv):
        rq, rk, rv = post_ref(rows)
        qh = qo[0] if head_major else qo[0].view(M, H, hd).transpose(0, 1)
        errs[name + " q"] = _rel(qh, rq)
        errs[name + " k"] = _rel(kbuf[0, :, sv:sv + M], rk)
        errs[name + " v"] = _rel(vbuf[0, :, sv:sv + M], rv)
        if sv:
            assert torch.equal(kbuf[0, :, :sv].cpu(), kv0[0, :, :sv])
    zn = 64
    za, zb = torch.ones(M + 2, zn).cuda(), torch.ones(M + 2, zn).cuda()

    def zeroed(z):
        return bool((z[:M] == 0).all()) and bool((z[M:] == 1).all())
    xin = _rand(g, 1, M, D)
    rows = O.linear(f(xin)[0], f(wqkv), f(bqkv))
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    qo = fw.mot_sa_qkv(xin.cuda(), dwqkv, dbqkv, qgr, qgr, dnqw, dnkw, dfreqs, kbuf, vbuf, za, zb, Sv, eps)
    chk("sa_qkv", qo, kbuf, vbuf, rows)
    assert zeroed(za) and zeroed(zb)
    za.fill_(1), zb.fill_(1)
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    qo = fw.mot_qkv_gemm_post_z(xin.cuda(), wqkv.t().contiguous().cuda(), dbqkv, dnqw, dnkw, dfreqs, kbuf, vbuf, za,
                                zb, Sv, eps)
    chk("qkv_gemm_post_z", qo, kbuf, vbuf, rows)
    assert zeroed(za) and zeroed(zb)
    za.fill_(1), zb.fill_(1)
    qkv = _rand(g, 1, M, 3 * NQ)
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    qo = fw.mot_qkv_post_z(qkv.cuda(), dnqw, dnkw, dfreqs, kbuf, vbuf, za, zb, Sv, eps)
    chk("qkv_post_z", qo, kbuf, vbuf, f(qkv)[0])
    assert zeroed(za) and zeroed(zb)
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    qs, ks, vs = (qkv[..., i * NQ:(i + 1) * NQ].contiguous().cuda() for i in range(3))
    qo = fw.mot_l0_qkv_rope(qs, ks, vs, dnqw, dnkw, dfreqs, kbuf, vbuf, Sv, eps)
    assert qo.shape == (1, M, NQ)
    chk("l0_qkv_rope", qo, kbuf, vbuf, f(qkv)[0], head_major=False)
    oz = torch.ones(M + 1, D).cuda()
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    qz = fw.mot_l0_qkv_rope_z(qs, ks, vs, dnqw, dnkw, dfreqs, kbuf, vbuf, oz, Sv, eps)
    assert torch.equal(qz, qo) and bool((oz[:M] == 0).all()) and bool((oz[M:] == 1).all())
    za.fill_(1), zb.fill_(1)
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    xs, qf = fw.mot_ffn_sa_qkv(dxa, doacc, dmod, dmodn, dtmod, dw1, db1, dw2, db2, dwqkv, dbqkv, qgr, qgr, dnqw, dnkw,
                               dfreqs, kbuf, vbuf, za, zb, Sv, eps, eps, eps)
    errs["ffn_sa_qkv x"] = _rel(xs[0], rxo)
    chk("ffn_sa_qkv", qf, kbuf, vbuf, O.linear(rai.to(BF).float(), f(wqkv), f(bqkv)))
    assert zeroed(za) and zeroed(zb)
    # the video prefill's post: token-major q / k / v, head-major caches from row 0, rows past M cleared
    kbuf, vbuf = kv0.cuda(), kv0.cuda()
    out = fw.vqkv_post(qkv.cuda(), dnqw, dnkw, dfreqs, kbuf, vbuf, eps)
    assert out.shape == (3, 1, M, NQ)
    rq, rk, rv = post_ref(f(qkv)[0])
    errs["vqkv_post q"] = _rel(out[0, 0].view(M, H, hd).transpose(0, 1), rq)
    errs["vqkv_post k"] = _rel(out[1, 0].view(M, H, hd).transpose(0, 1), rk)
    assert torch.equal(out[2, 0].cpu(), qkv[0, :, 2 * NQ:])
    errs["vqkv_post kbuf"] = _rel(kbuf[0, :, :M], rk)
    assert bool((kbuf[0, :, M:] == 0).all()) and bool((vbuf[0, :, M:] == 0).all())
    # every layer's context K / V into one buffer, from g and from the embedding
    nl, C = 30, 64
    e, wc, bc = _rand(g, Lc, C), _rand(g, 2 * nl * D, C, scale=C ** -0.5), _rand(g, 2 * nl * D, scale=0.1)
    nkwc = (1 + 0.2 * torch.randn(nl, D, generator=g)).to(BF)
    gg = O.linear(f(e), f(wc), f(bc))
    kv_out = torch.empty(2, nl, 1, Lc, D, dtype=BF).cuda()
    fw.ctx_kv_gemm_norm_into(*cu(e, wc, bc, nkwc), kv_out, nl, D, eps, True)
    errs["ctx_kv_gemm_norm_into k"] = _rel(kv_out[0, :, 0], O.cae_ctx_kv_norm(gg, f(nkwc), nl, D, eps))
    errs["ctx_kv_gemm_norm_into v"] = _rel(kv_out[1, :, 0], gg[:, nl * D:].reshape(Lc, nl, D).transpose(0, 1))
    gb = gg.to(BF)
    kv2 = torch.empty(2, nl, 1, Lc, D, dtype=BF).cuda()
    fw.ctx_kv_norm_into(gb.cuda(), nkwc.cuda(), kv2, nl, D, eps)
    assert torch.equal(kv2[1].cpu(), gb[:, nl * D:].reshape(Lc, nl, D).transpose(0, 1)[:, None])
    errs["ctx_kv_norm_into k"] = _rel(kv2[0, :, 0], O.cae_ctx_kv_norm(gb.float(), f(nkwc), nl, D, eps))
    print("CAE fused operators:", ", ".join(f"{k} {v:.2e}" for k, v in errs.items()))
    assert max(errs.values()) <= 2e-2, errs


@pytest.mark.parametrize("D", [3072, 14336, 4096])
def test_vfp8_row_ops(fw, D):
    """row_q8, gelu_q8, ln_mod_q8 and add_ln_mod_q8 at the video prefill's row widths (hidden 3072,
    FFN 14336, text 4096) against the oracle (CA/mot.py:3763-3980): the scales agree to fp32
    rounding, the fp8 codes are identical for the plain rows and, where the row operation's fp32
    arithmetic may move a value across a rounding boundary, at most one e4m3 step apart in a
    handful of entries; the dequantised rows match the oracle's rows at e4m3's precision."""
    g = torch.Generator().manual_seed(95 + D)
    M, eps = 98, 1e-6
    x = (torch.randn(M, D, generator=g) * torch.logspace(-2, 1, M)[:, None]).to(BF)
    sh, sc = _rand(g, D, scale=0.3), _rand(g, D, scale=0.3)
    x2 = _rand(g, M, D)

    def cmp(name, got, ref, exact=False):
        (q, s), (rq, rs) = got, ref
        assert q.dtype == torch.float8_e4m3fn and q.shape == (M, D) and s.shape == (M, 1)
        q, s = q.cpu().float(), s.cpu()
        rqf = rq.float()
        assert torch.allclose(s, rs, rtol=2e-6 if exact else 1e-2), name
        diff = (q != rqf).float().mean().item()
        step = (q - rqf).abs() <= rqf.abs() * 2 ** -3 + 2 ** -9 * 1.0001
        print(f"{name} D={D}: codes differing {diff:.2e}")
        if exact:
            assert diff == 0, name
        else:
            assert step.all() and diff <= 1e-3, name
    cmp("row_q8", fw.row_q8(x.cuda()), O.vfp8_row_q8(x.float()), exact=True)
    cmp("gelu_q8", fw.gelu_q8(x.cuda()), O.vfp8_gelu_q8(x.float()))
    cmp("ln_mod_q8", fw.ln_mod_q8(x.cuda(), sh.cuda(), sc.cuda(), eps), O.vfp8_ln_mod_q8(x.float(), sh, sc, eps))
    xo, q, s = fw.add_ln_mod_q8(x.cuda(), x2.cuda(), sh.cuda(), sc.cuda(), eps)
    rxo, rq, rs = O.vfp8_add_ln_mod_q8(x.float(), x2.float(), sh, sc, eps)
    assert xo.dtype == BF and torch.equal(xo.cpu().float(), rxo)
    cmp("add_ln_mod_q8", (q, s), (rq, rs))

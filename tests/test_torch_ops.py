"""CPU checks of the torch.library operator layer: the drop-ins trace as single graph nodes under
torch.compile(fullgraph=True) (their fake implementations run; nothing launches), and the RoPE
table cache / layout checks of fam.ops.rope_tables."""
import pytest
import torch

from fam import ops


def _compile_graph(module, *args):
    graphs = []

    def backend(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    with torch.no_grad():
        y = torch.compile(module, fullgraph=True, backend=backend)(*args)
        y2 = torch.compile(module, fullgraph=True, backend="aot_eager")(*args)
    targets = [str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"]
    return y, y2, targets


def _meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="meta")


class _Block(torch.nn.Module):
    """The reference block's call pattern: adaln_forward -> linear -> RMSNorm+RoPE / rope_apply ->
    flash_attention -> layer_norm -> scheduler step."""

    def __init__(self, D=64, H=4):
        super().__init__()
        self.H = H
        self.norm = torch.nn.LayerNorm(D, elementwise_affine=False, eps=1e-6)
        self.wq = torch.nn.Parameter(_meta(D, D), requires_grad=False)
        self.bq = torch.nn.Parameter(_meta(D), requires_grad=False)
        self.nq = torch.nn.Parameter(_meta(D), requires_grad=False)

    def forward(self, x, shift, scale, freqs, delta, mask):
        h = ops.adaln_forward(x, self.norm, shift, scale)
        q = ops.rms_norm_rope(ops.linear(h, self.wq, self.bq), self.nq, 1e-6, freqs, self.H, "cat")
        k = ops.rope_apply(ops.linear(h, self.wq), freqs, self.H)
        o = ops.flash_attention(q, k, h, self.H, ctx_mask=mask)
        o = ops.layer_norm(o, None, None, 1e-6) + ops.rms_norm(o, self.nq, 1e-6)
        return ops.WanContinuousFlowMatchScheduler.step(o, delta, x)


def test_fam_ops_trace_as_single_nodes():
    m = _Block()
    x = _meta(2, 8, 64)
    y, y2, targets = _compile_graph(m, x, _meta(2, 1, 64), _meta(2, 1, 64), _meta(8, 1, 16, dtype=torch.float32),
                                    _meta((), dtype=torch.bfloat16), _meta(8, 8, dtype=torch.bool))
    assert y.shape == x.shape and y.dtype == torch.bfloat16 and y2.shape == x.shape
    for op in ("fam.adaln", "fam.linear", "fam.rope", "fam.attention", "fam.euler_step"):
        assert any(t.startswith(op) for t in targets), (op, targets)
    # one node per drop-in call, nothing decomposed into aten kernels around them
    assert sum(t.startswith("fam.rope") for t in targets) == 3
    assert sum(t.startswith("fam.adaln") for t in targets) == 2


def test_fam_ops_fake_shapes_and_checks():
    q = _meta(1, 32, 1024)
    assert torch.ops.fam.attention(q, _meta(1, 1560, 1024), _meta(1, 1560, 1024), None, 16, None, None, None,
                                   1).shape == (1, 32, 1024)
    assert torch.ops.fam.linear(q, _meta(3072, 1024), None).shape == (1, 32, 3072)
    with pytest.raises(ValueError):
        torch.ops.fam.linear(q, _meta(3072, 512), None)
    with pytest.raises(TypeError):
        torch.ops.fam.adaln(_meta(1, 4, 64, dtype=torch.float16), None, None, None, None, 1e-6)
    with pytest.raises(ValueError):
        torch.ops.fam.rope(q, _meta(16, 1, 32, dtype=torch.float32), 16, "cat", None, 0.0)   # 16 < 32 positions


def test_fastwam_ops_trace_with_mutation():
    from fam import fastwam_ops  # noqa: F401  (defines torch.ops.fastwam.*)

    class M(torch.nn.Module):
        def forward(self, qkv, wqk, freqs, sgn, kbuf, vbuf, vk, vv, x, w, bias, res, mod, tmod, lnw, lnb):
            q = torch.ops.fastwam.qkv_post.default(qkv, wqk, freqs, sgn, kbuf, vbuf, 6, 16, 1e-6)
            qh = q.view(1, 8, 4, 16).transpose(1, 2)
            kh = kbuf.view(1, 14, 4, 16).transpose(1, 2)
            vh = vbuf.view(1, 14, 4, 16).transpose(1, 2)
            o4 = torch.ops.fastwam.short_attn.default(qh, kh, vh, None, 4)
            o3 = torch.ops.fastwam.short_attn_bsd.default(qh, kh, vh, None, 4)
            oq = torch.ops.fastwam.qrms_attn.default(q, wqk[0], vk, vv, None, 4, 1e-6)
            qq, kk = torch.ops.fastwam.qk_post.default(qkv, wqk, freqs, sgn, 16, 1e-6)
            y = torch.ops.fastwam.skmm.default(o3 + oq + qq + kk, w)
            xo, yo = torch.ops.fastwam.skpost.default(y, w, bias, res, mod, mod, tmod, lnw, lnb, 2, -1, -1, 1e-6, 0)
            return o4, xo, yo

    args = (_meta(8, 192), _meta(2, 64), _meta(8, 16, dtype=torch.float32), _meta(2, dtype=torch.float32),
            _meta(1, 14, 64), _meta(1, 14, 64), _meta(1, 20, 64), _meta(1, 20, 64), None, _meta(64, 64), _meta(64),
            _meta(1, 8, 64), _meta(1, 6, 64), _meta(1, 6, 64), _meta(64), _meta(64))
    (o4, xo, yo), _, targets = _compile_graph(M(), *args)
    assert o4.shape == (1, 4, 8, 16) and xo.shape == (1, 8, 64) and yo.shape == (1, 8, 64)
    for op in ("fastwam.qkv_post", "fastwam.short_attn", "fastwam.short_attn_bsd", "fastwam.qrms_attn",
               "fastwam.qk_post", "fastwam.skmm", "fastwam.skpost"):
        assert any(t.startswith(op) for t in targets), (op, targets)


def test_geak_prefill_and_cae_ops_trace():
    """The GEAK prefill's and the CAE tree's fastwam:: operators trace as single nodes (fake
    kernels give the reference's output shapes)."""
    from fam import fastwam_ops  # noqa: F401

    class M(torch.nn.Module):
        def forward(self, x, w, b, mb, tm, wn, qkv, qw, kw, freqs, kbuf, vbuf, msk, k, v, g, nkw, a, w1, b1, w2, b2,
                    te, inv, w0, b0, w1t, b1t, w2t, b2t, atok, aw, ab):
            y = torch.ops.fastwam.pf_mm.default(x, w, b)
            yg = torch.ops.fastwam.pf_mm_gelu.default(x, w, b)
            h3 = torch.ops.fastwam.res_ln1.default(x, y, mb, tm, wn, b, 128, 1e-6)
            x1, n1 = torch.ops.fastwam.res_ln2.default(x, y, yg, mb, mb, tm, 128, 192, 256, 1e-6)
            x2, n2 = torch.ops.fastwam.res_ln_tail.default(x1, y, mb, mb, tm, 320, 0, 64, 1e-6)
            q = torch.ops.fastwam.mot_qkv_post.default(qkv, qw, kw, freqs, kbuf, vbuf, 5, 1e-6)
            oa = torch.ops.fastwam.mot_attn.default(q, kbuf, vbuf, msk, 2, 16, True)
            ox = torch.ops.fastwam.xattn_qn.default(oa, qw, k, v, msk, 2, 16, 1e-6)
            kv = torch.ops.fastwam.ctx_kv_norm.default(g, nkw, 3, 32, 1e-6)
            op = torch.ops.fastwam.mot_oproj.default(ox, w1, b1)
            f = torch.ops.fastwam.mot_ffn.default(a, w1t, b1t, w2t, b2t)
            t, tmod, tk = torch.ops.fastwam.adit_tmod.default(te, inv, w0, b0, w2, b2, w1, b1, atok, aw, ab, 1)
            return h3, n1, x2, n2, oa, kv, op, f, t, tmod, tk

    args = (_meta(1, 6, 64), _meta(64, 64), _meta(64), _meta(384), _meta(6, 384), _meta(64),
            _meta(1, 4, 96), _meta(32), _meta(32), _meta(4, 16, dtype=torch.float32), _meta(1, 2, 9, 16),
            _meta(1, 2, 9, 16), _meta(4, 9, dtype=torch.bool), _meta(1, 9, 32), _meta(1, 9, 32),
            _meta(9, 192), _meta(3, 32), _meta(1, 4, 32), _meta(32, 32), _meta(32), _meta(32, 32), _meta(32),
            _meta(1, dtype=torch.float32), _meta(16, dtype=torch.float64), _meta(32, 32), _meta(32), _meta(64, 32),
            _meta(64), _meta(32, 64), _meta(32), _meta(1, 4, 16), _meta(32, 16), _meta(32))
    outs, _, targets = _compile_graph(M(), *args)
    h3, n1, x2, n2, oa, kv, op, f, t, tmod, tk = outs
    assert h3.shape == n1.shape == x2.shape == n2.shape == (1, 6, 64)
    assert oa.shape == (1, 4, 32) and kv.shape == (1, 3, 1, 9, 32) and op.shape == (1, 4, 32)
    assert f.shape == (1, 4, 32) and t.shape == (1, 32) and tmod.shape == (1, 32) and tk.shape == (1, 4, 32)
    for op_ in ("pf_mm", "pf_mm_gelu", "res_ln1", "res_ln2", "res_ln_tail", "mot_qkv_post", "mot_attn",
                "xattn_qn", "ctx_kv_norm", "mot_oproj", "mot_ffn", "adit_tmod"):
        assert any(t_.startswith("fastwam." + op_ + ".") for t_ in targets), (op_, targets)



def test_geak_split_plane_ops_trace():
    """pf_skmm / pf_skmm_big give fp32 planes [8 | 16, M, N] whatever the split count, and the
    consumers res_ln1_sk, res_ln2_sk, res_ln_tail_sk and pf_qcomb trace as single nodes of the
    reference's output shapes (FG/mot.py:2045-2074, :2170-2244, :2331-2333)."""
    from fam import fastwam_ops  # noqa: F401

    class M(torch.nn.Module):
        def forward(self, x, a, w, bi, mb, tm, wn, bn, o1, h, w2):
            p1 = torch.ops.fastwam.pf_skmm.default(a, w)
            h3, o = torch.ops.fastwam.res_ln1_sk.default(x, p1, bi, mb, tm, wn, bn, 128, 1e-6, 4)
            q = torch.ops.fastwam.pf_qcomb.default(torch.ops.fastwam.pf_skmm.default(h3, w), bi, wn, 1e-6, 4)
            x1, n1 = torch.ops.fastwam.res_ln2_sk.default(x, o, p1, bi, mb, mb, tm, 128, 192, 256, 1e-6, 4)
            p3 = torch.ops.fastwam.pf_skmm_big.default(h, w2)
            x2, n2 = torch.ops.fastwam.res_ln_tail_sk.default(x1, p3, bi, mb, mb, tm, 320, 0, 64, 1e-6, 8)
            return p1, p3, h3, o, q, x1, n1, x2, n2

    args = (_meta(1, 6, 64), _meta(1, 6, 64), _meta(64, 64), _meta(64), _meta(384), _meta(6, 384), _meta(64),
            _meta(64), _meta(1, 6, 64), _meta(1, 6, 256), _meta(64, 256))
    outs, _, targets = _compile_graph(M(), *args)
    p1, p3, *rest = outs
    assert p1.shape == (8, 6, 64) and p3.shape == (16, 6, 64) and p1.dtype == p3.dtype == torch.float32
    assert all(t_.shape == (1, 6, 64) and t_.dtype == torch.bfloat16 for t_ in rest)
    for op_ in ("pf_skmm", "pf_skmm_big", "res_ln1_sk", "res_ln2_sk", "res_ln_tail_sk", "pf_qcomb"):
        assert any(t_.startswith("fastwam." + op_ + ".") for t_ in targets), (op_, targets)



def test_cae_fused_and_fp8_ops_trace():
    """The CAE tree's fused operators (mutating acc / kbuf / vbuf / za / zb / out as the reference
    declares) and the fp8 row operators trace under torch.compile(fullgraph=True) with the
    reference's output shapes (CA/mot.py:2830-3980)."""
    from fam import fastwam_ops  # noqa: F401
    M, D, H, hd, SK, NS, F_ = 4, 32, 2, 16, 9, 7, 64
    NQ = H * hd
    f32 = torch.float32

    class Mod(torch.nn.Module):
        def forward(self, res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, ck, cv, cmsk, wo, bo, acc, q, k, v, am, cm,
                    w1, b1, w2, b2, wqkv, bqkv, gr, freqs, kbuf, vbuf, za, zb, qkv, g, nkw, kvo, e, wc, bc, vx, vsh):
            x, cq = torch.ops.fastwam.mod_n3q.default(res, so, mod, tmod, lnw, lnb, qw, qb, 1e-6)
            x2, cqn = torch.ops.fastwam.mod_n3q_qn.default(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, 1e-6, 1e-6)
            x3 = torch.ops.fastwam.n3q_xoproj.default(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, ck, cv, cmsk, wo,
                                                      bo, acc, H, 1e-6, 1e-6)
            sb, xb = torch.ops.fastwam.mask_bias.default(am, cm, 16, 16, 8)
            torch.ops.fastwam.mot_attn_oproj.default(q, k, v, sb, wo, bo, acc, H, hd)
            xo, ai = torch.ops.fastwam.mot_ffn_fold.default(x, so, mod, mod, tmod, w1, b1, w2, b2, 1e-6, 1e-6, 1)
            qa = torch.ops.fastwam.mot_sa_qkv.default(ai, wqkv, bqkv, gr, gr, qnw, qnw, freqs, kbuf, vbuf, za, zb, 5, 1e-6)
            xs, qs = torch.ops.fastwam.mot_ffn_sa_qkv.default(x, so, mod, mod, tmod, w1, b1, w2, b2, wqkv, bqkv, gr, gr,
                                                              qnw, qnw, freqs, kbuf, vbuf, za, zb, 5, 1e-6, 1e-6, 1e-6)
            qz = torch.ops.fastwam.mot_qkv_post_z.default(qkv, qnw, qnw, freqs, kbuf, vbuf, za, zb, 5, 1e-6)
            qg = torch.ops.fastwam.mot_qkv_gemm_post_z.default(ai, wqkv.t(), bqkv, qnw, qnw, freqs, kbuf, vbuf, za, zb,
                                                               5, 1e-6)
            q0 = torch.ops.fastwam.mot_l0_qkv_rope.default(cq, cq, cq, qnw, qnw, freqs, kbuf, vbuf, 5, 1e-6)
            q1 = torch.ops.fastwam.mot_l0_qkv_rope_z.default(cq, cq, cq, qnw, qnw, freqs, kbuf, vbuf, acc, 5, 1e-6)
            torch.ops.fastwam.ctx_kv_norm_into.default(g, nkw, kvo, 3, D, 1e-6)
            torch.ops.fastwam.ctx_kv_gemm_norm_into.default(e, wc, bc, nkw, kvo, 3, D, 1e-6, True)
            vq = torch.ops.fastwam.vqkv_post.default(qkv, qnw, qnw, freqs, kbuf, vbuf, 1e-6)
            r8, rs = torch.ops.fastwam.row_q8.default(vx)
            g8, gs = torch.ops.fastwam.gelu_q8.default(vx)
            l8, ls = torch.ops.fastwam.ln_mod_q8.default(vx, vsh, vsh, 1e-6)
            ao, a8, as_ = torch.ops.fastwam.add_ln_mod_q8.default(vx, vx, vsh, vsh, 1e-6)
            return x, cq, cqn, x3, sb, xb, xo, ai, qa, xs, qs, qz, qg, q0, q1, vq, r8, rs, g8, l8, ao, a8, as_

    args = (_meta(1, M, D), _meta(M, D, dtype=f32), _meta(6 * D), _meta(1, 6 * D), _meta(D), _meta(D), _meta(NQ, D),
            _meta(NQ), _meta(NQ), _meta(D * D + D + 1, dtype=f32), _meta(1, NS, NQ), _meta(1, NS, NQ),
            _meta(1, M, NS, dtype=torch.bool), _meta(D, NQ), _meta(D), _meta(M, D, dtype=f32), _meta(1, H, M, hd),
            _meta(1, H, SK, hd), _meta(1, H, SK, hd), _meta(M, SK, dtype=torch.bool), _meta(1, NS, dtype=torch.bool),
            _meta(F_, D), _meta(F_), _meta(D, F_), _meta(D), _meta(3 * NQ, D), _meta(3 * NQ), _meta(D * D + D + 1),
            _meta(M, hd, dtype=f32), _meta(1, H, SK, hd), _meta(1, H, SK, hd), _meta(M, 16, dtype=f32),
            _meta(M, 16, dtype=f32), _meta(1, M, 3 * NQ), _meta(NS, 6 * D), _meta(3, D), _meta(2, 3, 1, NS, D),
            _meta(NS, 24), _meta(6 * D, 24), _meta(6 * D), _meta(1, 6, 64), _meta(64))
    outs, _, targets = _compile_graph(Mod(), *args)
    x, cq, cqn, x3, sb, xb, xo, ai, qa, xs, qs, qz, qg, q0, q1, vq, r8, rs, g8, l8, ao, a8, as_ = outs
    assert x.shape == x3.shape == xo.shape == ai.shape == xs.shape == (1, M, D)
    assert cq.shape == cqn.shape == q0.shape == q1.shape == (1, M, NQ)
    assert sb.shape == (16, 16) and xb.shape == (16, 8) and sb.dtype == f32
    assert qa.shape == qs.shape == qz.shape == qg.shape == (1, H, M, hd) and vq.shape == (3, 1, M, NQ)
    assert r8.shape == g8.shape == l8.shape == a8.shape == (6, 64) and r8.dtype == torch.float8_e4m3fn
    assert rs.shape == as_.shape == (6, 1) and ao.shape == (1, 6, 64)
    for op_ in ("mod_n3q", "mod_n3q_qn", "n3q_xoproj", "mask_bias", "mot_attn_oproj", "mot_ffn_fold", "mot_sa_qkv",
                "mot_ffn_sa_qkv", "mot_qkv_post_z", "mot_qkv_gemm_post_z", "mot_l0_qkv_rope", "mot_l0_qkv_rope_z",
                "ctx_kv_norm_into", "ctx_kv_gemm_norm_into", "vqkv_post", "row_q8", "gelu_q8", "ln_mod_q8",
                "add_ln_mod_q8"):
        assert any(t_.startswith("fastwam." + op_ + ".") for t_ in targets), (op_, targets)



# every operator name the reference's GEAK trees register in the fastwam namespace
# (src/fastwam-geak/fastwam/models/wan22/{mot,wan_video_dit}.py, src/cae-fastwam/fastwam/models/wan22/
# {mot,action_dit}.py: the torch.library.custom_op("fastwam::...") definitions)
_REFERENCE_FASTWAM_OPS = (
    "add_ln_mod_q8", "adit_tmod", "ctx_kv_gemm_norm_into", "ctx_kv_norm", "ctx_kv_norm_into", "gelu_q8", "ln_mod_q8",
    "mask_bias", "mod_n3q", "mod_n3q_qn", "mot_attn", "mot_attn_oproj", "mot_ffn", "mot_ffn_fold", "mot_ffn_sa_qkv",
    "mot_l0_qkv_rope", "mot_l0_qkv_rope_z", "mot_oproj", "mot_qkv_gemm_post_z", "mot_qkv_post", "mot_qkv_post_z",
    "mot_sa_qkv", "n3q_xoproj", "pf_mm", "pf_mm_gelu", "pf_qcomb", "pf_skmm", "pf_skmm_big", "qk_post", "qkv_post",
    "qrms_attn", "res_ln1", "res_ln1_sk", "res_ln2", "res_ln2_sk", "res_ln_tail", "res_ln_tail_sk", "row_q8",
    "short_attn", "short_attn_bsd", "skmm", "skpost", "vqkv_post", "xattn_qn")


def test_every_reference_fastwam_op_is_defined():
    """Importing fam.fastwam_ops defines each of the reference trees' 44 fastwam:: operators."""
    from fam import fastwam_ops  # noqa: F401
    assert len(_REFERENCE_FASTWAM_OPS) == 44
    missing = [n for n in _REFERENCE_FASTWAM_OPS if not hasattr(torch.ops.fastwam, n)]
    assert not missing, missing


# --------------------------------------------------------------------------- RoPE tables
def _cat_table(S, Dh, offset=0.0):
    ang = (torch.arange(S, dtype=torch.float64)[:, None] + offset) * \
        (1.0 / 10000 ** (torch.arange(0, Dh, 2, dtype=torch.float64) / Dh))[None, :]
    return torch.cat([ang.cos(), ang.sin()], -1).float().reshape(S, 1, Dh)


def _interleaved(cat):
    S, _, Dh = cat.shape
    c, s = cat[..., : Dh // 2], cat[..., Dh // 2:]
    return torch.stack([c, s], -1).reshape(S, 1, Dh)


def test_rope_tables_cache_never_returns_a_freed_tables_values():
    """A cached conversion keeps its source alive, so a new same-shape table with other values
    (the reference builds a fresh freqs every pre_dit call) is never served the old entry."""
    dev = torch.device("cpu")
    seen = []
    for i in range(6):
        t = _cat_table(16, 32, offset=float(i)).double()       # fp64 -> converted and cached
        cos, sin, trs, tes = ops.rope_tables(t, "cat", dev)
        assert torch.equal(cos[:, :16], t.reshape(16, 32)[:, :16].float())
        seen.append(cos.data_ptr())
        del t
    assert len(ops._TABLES) >= 6
    t = _cat_table(16, 32, offset=3.0).double()
    t.mul_(1.0)                                               # in-place change bumps the version
    cos, _, _, _ = ops.rope_tables(t, "cat", dev)
    assert torch.equal(cos[:, :16], t.reshape(16, 32)[:, :16].float())


def test_rope_tables_fp32_device_table_used_in_place():
    t = _cat_table(8, 16)
    cos, sin, trs, tes = ops.rope_tables(t, "cat", torch.device("cpu"))
    assert cos.data_ptr() == t.data_ptr() and sin.data_ptr() == t.data_ptr() + 4 * 8 and (trs, tes) == (16, 1)
    ti = _interleaved(t).contiguous()
    cos, sin, trs, tes = ops.rope_tables(ti, "interleaved", torch.device("cpu"))
    assert cos.data_ptr() == ti.data_ptr() and sin.data_ptr() == ti.data_ptr() + 4 and (trs, tes) == (16, 2)


def test_rope_tables_reject_the_other_packing():
    """FG's cat(cos, sin) and CA's interleaved tables have the same shape; each entry point
    rejects the other's table instead of rotating the wrong pairs."""
    cat = _cat_table(8, 16, offset=2.0)
    inter = _interleaved(cat).contiguous()
    with pytest.raises(ValueError, match="rope_apply_cae"):
        ops.rope_tables(inter, "cat", torch.device("cpu"))
    with pytest.raises(ValueError, match="rope_apply "):
        ops.rope_tables(cat, "interleaved", torch.device("cpu"))
    with pytest.raises(ValueError):
        ops.rope_tables(cat, "complex", torch.device("cpu"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_tables_accept_a_half_precision_table_in_the_right_packing(dtype):
    """A table packed right but stored in bf16 / fp16 (FG's pack_rope_real takes a dtype) has
    pairs off unit modulus by its own rounding: it is accepted (and converted to fp32), while the
    same table in the other packing is still refused."""
    cat = _cat_table(64, 128, offset=0.0).to(dtype)
    inter = _interleaved(cat).contiguous()
    cos, sin, trs, tes = ops.rope_tables(cat, "cat", torch.device("cpu"))
    assert cos.dtype == torch.float32 and torch.equal(cos[:, :64], cat.reshape(64, 128)[:, :64].float())
    ops.rope_tables(inter, "interleaved", torch.device("cpu"))
    with pytest.raises(ValueError, match="rope_apply_cae"):
        ops.rope_tables(inter, "cat", torch.device("cpu"))
    with pytest.raises(ValueError, match="rope_apply "):
        ops.rope_tables(cat, "interleaved", torch.device("cpu"))

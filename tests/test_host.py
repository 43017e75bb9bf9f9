"""CPU checks of the host-side logic of the package against the oracle."""
import torch

from oracle import fam_oracle as O
from fam import action_dit as AD


def test_synthetic_params_match_oracle_init():
    cfg = AD.ActionDiTConfig(num_layers=2, hidden_dim=64, ffn_dim=128, text_dim=48, freq_dim=32, num_heads=4,
                             attn_head_dim=16)
    a = AD.synthetic_params(cfg, 77)
    b = O.init_action_dit_params(O.ActionDiTConfig(**cfg.to_dict()), 77)
    assert sorted(a) == sorted(b)
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_param_shapes_match_oracle():
    cfg = AD.ActionDiTConfig()
    assert AD.param_shapes(cfg) == O.action_dit_param_shapes(O.ActionDiTConfig(**cfg.to_dict()))


def test_schedule_matches_oracle():
    for n, s in ((10, 5.0), (4, 5.0), (2, 1.0)):
        ts, ds = AD.schedule(n, s)
        ots, ods = O.build_inference_schedule(n, s, torch.bfloat16)
        assert torch.equal(ts, ots) and torch.equal(ds, ods)


def test_rope_tables_match_oracle():
    cos, sin = AD.rope_1d_tables(64, 32)
    oc, os_ = O.rope_tables_real(O.action_freqs(64, 32))
    assert torch.equal(cos, oc) and torch.equal(sin, os_)


def test_fused_plan_builds_on_host():
    """The launch plan of the fused loop is assembled (descriptors validated by shape only,
    nothing launched) for B=1 and for B*S above the 64-row partial limit."""
    cfg = AD.ActionDiTConfig(num_layers=2, hidden_dim=64, ffn_dim=128, text_dim=48, freq_dim=32, num_heads=4,
                             attn_head_dim=16)
    params = AD.synthetic_params(cfg, 3)
    for batch in (1, 4):
        m = AD.FusedActionDiT(cfg, params, batch=batch, seq_len=32, ctx_len=200, num_steps=3, device="cpu")
        kinds = [d["kernel"] for d in m.plan.meta]
        # prologue: copy, sinusoid, 3 time GEMMs, modulation, 3 context GEMMs, the K-norm of every layer
        pro = 10
        # per step: encoder row + per block (6 projections x 2 + self-attn + cross-attn + combine) + head x 2;
        # at M <= 64 the FFN-up projection is one whole-K kernel with its epilogue (and, when the
        # attention width allows the on-load q/k norm, so are the q/k/v and cross-q projections)
        small = batch * 32 <= 64
        fused_qk = small and cfg.attn_dim % 1024 == 0
        per_block = 15 - (0 if m.kv_splits > 1 else 1) - (1 if small else 0) - (2 if fused_qk else 0)
        assert m.num_launches == pro + 3 * (1 + cfg.num_layers * per_block + 2)
        assert kinds.count("attention") == 3 * 2 * cfg.num_layers
        if batch * 32 > 64:
            assert "gemm_partial" not in kinds
        else:
            assert kinds.count("gemm_partial") == 3 * (5 * cfg.num_layers + 1)
            assert kinds.count("gemm_final") == 3 * cfg.num_layers
    # attention width 1024: q/k norms move into the attention kernels
    cfg2 = AD.ActionDiTConfig(num_layers=1, hidden_dim=64, ffn_dim=128, text_dim=48, freq_dim=32, num_heads=16,
                              attn_head_dim=64)
    m3 = AD.FusedActionDiT(cfg2, AD.synthetic_params(cfg2, 3), batch=1, seq_len=32, ctx_len=200, num_steps=2,
                           device="cpu")
    kinds3 = [d["kernel"] for d in m3.plan.meta]
    assert kinds3.count("gemm_final") == 2 * 3 and kinds3.count("gemm_partial") == 2 * (3 + 1)
    assert kinds3.count("attention") == 2 * 2
    fwd = AD.FusedActionDiT(cfg, params, batch=1, seq_len=32, ctx_len=200, num_steps=1, device="cpu", mode="forward")
    assert fwd.plan.meta[-1]["kernel"] == "rowop"


def test_fused_plan_mot_mode_on_host():
    """MoT mode: the self-attention of every block becomes a two-segment joint attention over
    the cached video K/V; the caches copy into static buffers."""
    cfg = AD.ActionDiTConfig(num_layers=2, hidden_dim=64, ffn_dim=128, text_dim=48, freq_dim=32, num_heads=4,
                             attn_head_dim=16)
    params = AD.synthetic_params(cfg, 3)
    m = AD.FusedActionDiT(cfg, params, batch=1, seq_len=32, ctx_len=129, num_steps=2, device="cpu", video_len=98)
    names = m.plan.names
    assert sum(n.endswith(".joint_attn") for n in names) == 2 * cfg.num_layers
    assert not any(n.endswith(".self_attn") for n in names)
    k = [torch.full((98, cfg.attn_dim), float(i + 1)) for i in range(cfg.num_layers)]
    m.set_video_kv(k, k)
    assert float(m.video_k[1].float().mean()) == 2.0


def test_tiny_expert_plan_and_gram_on_host():
    """Hidden 32 selects fam_tiny_expert: two launches per block step plus the final phase after
    the prologue (no noise copy: phase 0 reads it).  The packed Gram parts reproduce the whole-row
    sums of squares the RMSNorm needs, sum_j q_j^2 = h G h + 2 h.c + |b|^2 (fp64 here): with the
    lo part dropped, or c not doubled, the identity fails."""
    cfg = AD.ActionDiTConfig(num_layers=3, hidden_dim=32, action_dim=16, ffn_dim=256, text_dim=64, freq_dim=32,
                             num_heads=24, attn_head_dim=128)
    params = AD.synthetic_params(cfg, 9)
    m = AD.FusedActionDiT(cfg, params, batch=1, seq_len=8, ctx_len=129, num_steps=4, device="cpu", video_len=98)
    assert m.tiny is not None and m.tiny["G"] == 24
    kinds = [d["kernel"] for d in m.plan.meta]
    assert kinds.count("tiny_self") == kinds.count("tiny_cross") == 3 * 4 and kinds[-1] == "tiny_final"
    # 128-wide slices: the keys' factors in one launch replace the context K/V GEMM and key norm
    assert m.tiny["folded"] and kinds.count("tiny_context") == 1 and "rmsnorm_rope" not in kinds
    assert "copy" not in kinds and m.num_launches == 8 + 2 * 3 * 4 + 1
    g = torch.Generator().manual_seed(1)
    h = torch.randn(5, 32, generator=g, dtype=torch.float64)
    A = cfg.attn_dim
    gram, gc, gb = m.tiny["gram"].double(), m.tiny["gram_c"].double(), m.tiny["gram_b"].double()
    for l in range(3):
        for j, (w, b) in enumerate(((m.tiny["qkv_w"][l, :A], m.tiny["qkv_b"][l, :A]),
                                    (m.tiny["qkv_w"][l, A:2 * A], m.tiny["qkv_b"][l, A:2 * A]),
                                    (m.tiny["cq_w"][l], m.tiny["cq_b"][l]),
                                    (m.tiny["ck_wt"][l].t(), m.tiny["ck_b"][l]))):
            q = h @ w.double().t() + b.double()
            direct = (q * q).sum(1)
            G = gram[l, j, 0] + gram[l, j, 1]
            form = ((h @ G) * h).sum(1) + 2 * h @ gc[l, j] + gb[l, j]
            assert torch.allclose(form, direct, rtol=2e-5), (l, j)
            assert not torch.allclose(((h @ gram[l, j, 0]) * h).sum(1) + 2 * h @ gc[l, j] + gb[l, j], direct, rtol=2e-5)
            assert not torch.allclose(form - h @ gc[l, j], direct, rtol=2e-5)
    # the generic plan stays available, and hidden 64 never takes the tiny path
    assert AD.FusedActionDiT(cfg, params, batch=1, seq_len=8, ctx_len=129, num_steps=4, device="cpu", video_len=98,
                             tiny=False).tiny is None
    # 32-wide slices keep the context K/V
    c32 = AD.ActionDiTConfig(num_layers=3, hidden_dim=32, action_dim=16, ffn_dim=256, text_dim=64, freq_dim=32,
                             num_heads=4, attn_head_dim=32)
    m32 = AD.FusedActionDiT(c32, AD.synthetic_params(c32, 9), batch=1, seq_len=8, ctx_len=129, num_steps=4,
                            device="cpu", video_len=98, tiny_slice=32)
    k32 = [d["kernel"] for d in m32.plan.meta]
    assert not m32.tiny["folded"] and "tiny_context" not in k32 and m32.num_launches == 9 + 2 * 3 * 4 + 1


def test_tiny_folded_context_attention_identity():
    """The wide-slice cross attention of fam_tiny_expert works in the 32-wide space of the context
    rows h with the packed host weights: for a head's query q (already RMS-normalised) the
    reference's score q . norm_k(W_k h + b_k) equals r (h . W_k^T (q * w_k) + b_k . (q * w_k)), r the
    key's RMS factor from the Gram form, and its output sum p v / l equals W_v (sum p h / l) + b_v
    (fp64 here).  A folded query without the bias term, without w_k, or with the Gram's lo part
    dropped misses the explicit scores."""
    cfg = AD.ActionDiTConfig(num_layers=2, hidden_dim=32, action_dim=16, ffn_dim=256, text_dim=64, freq_dim=32,
                             num_heads=4, attn_head_dim=32)
    params = AD.synthetic_params(cfg, 11)
    # unit-scale key weights and biases so that every term matters
    g = torch.Generator().manual_seed(12)
    for l in range(2):
        params[f"blocks.{l}.cross_attn.k.weight"] = (torch.randn(128, 32, generator=g) / 32 ** 0.5).to(torch.bfloat16)
        params[f"blocks.{l}.cross_attn.k.bias"] = (0.5 * torch.randn(128, generator=g)).to(torch.bfloat16)
        params[f"blocks.{l}.cross_attn.norm_k.weight"] = (1 + 0.3 * torch.randn(128, generator=g)).to(torch.bfloat16)
        params[f"blocks.{l}.cross_attn.v.bias"] = (0.5 * torch.randn(128, generator=g)).to(torch.bfloat16)
    m = AD.FusedActionDiT(cfg, params, batch=1, seq_len=8, ctx_len=40, num_steps=2, device="cpu")
    tw, A, eps = m.tiny, cfg.attn_dim, float(cfg.eps)
    assert tw["folded"] and tw["G"] == 1
    h = torch.randn(40, 32, generator=g, dtype=torch.float64)
    q = torch.randn(3, 32, generator=g, dtype=torch.float64)      # 3 queries of head 1 (dims 32..63)
    p = torch.rand(3, 40, generator=g, dtype=torch.float64)
    for l in range(2):
        wk, bk = tw["ck_wt"][l].double().t(), tw["ck_b"][l].double()
        wn = tw["nk_stack"][l].double()
        wv, bv = tw["cv_w"][l].double(), tw["cv_b"][l].double()
        k = h @ wk.t() + bk
        kn = k * torch.rsqrt((k * k).mean(1, keepdim=True) + eps) * wn
        qf = torch.zeros(3, A, dtype=torch.float64)
        qf[:, 32:64] = q
        explicit = qf @ kn.t()
        G = tw["gram"][l, 3].double()
        ss = ((h @ (G[0] + G[1])) * h).sum(1) + 2 * h @ tw["gram_c"][l, 3].double() + tw["gram_b"][l, 3].double()
        r = torch.rsqrt(ss / A + eps)
        qw = qf * wn
        folded = r * (h @ (wk.t() @ qw.t())).t() + r * (qw @ bk)[:, None]
        assert torch.allclose(folded, explicit, rtol=1e-4, atol=1e-4 * explicit.abs().max().item())
        bad = {"no bias term": r * (h @ (wk.t() @ qw.t())).t(),
               "no w_k": r * (h @ (wk.t() @ qf.t())).t() + r * (qf @ bk)[:, None]}
        ss_hi = ((h @ G[0]) * h).sum(1) + 2 * h @ tw["gram_c"][l, 3].double() + tw["gram_b"][l, 3].double()
        bad["Gram lo dropped"] = torch.rsqrt(ss_hi / A + eps) * (h @ (wk.t() @ qw.t())).t() + \
            torch.rsqrt(ss_hi / A + eps) * (qw @ bk)[:, None]
        for name, v in bad.items():
            assert not torch.allclose(v, explicit, rtol=1e-4, atol=1e-4 * explicit.abs().max().item()), name
        v = h @ wv.t() + bv
        out_explicit = (p @ v) / p.sum(1, keepdim=True)
        z = (p @ h) / p.sum(1, keepdim=True)
        assert torch.allclose(z @ wv.t() + bv, out_explicit, rtol=1e-10, atol=1e-10)


def test_video_rope_table_matches_oracle():
    from fam.video_dit import video_freqs_3d
    for dh, (f, h, w) in ((128, (2, 30, 26)), (64, (1, 4, 5))):
        assert torch.equal(video_freqs_3d(dh, f, h, w), O.video_freqs(O.precompute_freqs_cis_3d(dh), f, h, w))


def test_fold_layernorm_identity_fp64():
    """fold_layernorm's (w', bias', colsum) reproduce LN -> affine -> AdaLN -> linear through
    rstd * (x w'^T - mean * colsum) + bias' (evaluated here in fp64 on the CPU); a dropped
    (1 + scale), a shift folded without the weight, or a wrong colsum fails it."""
    import torch.nn.functional as F
    from fam import ops
    g = torch.Generator().manual_seed(5)
    M, K, N = 7, 48, 24
    x = (torch.randn(M, K, generator=g) * 2 + torch.randn(M, 1, generator=g) * 5).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    lw, lb = torch.randn(K, generator=g) * 0.3 + 1, torch.randn(K, generator=g) * 0.3
    sc, sh = torch.randn(K, generator=g) * 0.2, torch.randn(K, generator=g) * 0.2
    eps = 1e-5
    x64 = x.double()
    z = F.layer_norm(x64, (K,), eps=eps) * lw.double() + lb.double()
    z = z * (1 + sc.double()) + sh.double()
    ref = z @ w.double().t() + b.double()
    w2, b2, cs = ops.fold_layernorm(w, b, ln_weight=lw, ln_bias=lb, scale=sc, shift=sh)
    assert w2.dtype == torch.bfloat16 and b2.dtype == torch.bfloat16 and cs.dtype == torch.float32
    mu = x64.mean(1, keepdim=True)
    rstd = 1.0 / torch.sqrt(x64.var(1, unbiased=False, keepdim=True) + eps)
    y = rstd * (x64 @ w2.double().t() - mu * cs.double()[None, :]) + b2.double()
    err = ((y - ref).abs().max() / ref.abs().max()).item()
    assert err < 1e-2, err          # bf16 rounding of w' and bias' only
    # plain LayerNorm: w' is w itself, bias' is bias itself
    w3, b3, cs3 = ops.fold_layernorm(w, b)
    assert torch.equal(w3, w) and torch.equal(b3, b)
    assert torch.allclose(cs3.double(), w.double().sum(1), rtol=1e-6, atol=1e-6)


def test_d4d_param_shapes_and_init_match_oracle():
    from fam import dit4dit as D4
    for kw in ({}, {"state_dim": 0}, {"num_layers": 3, "heads": 2, "head_dim": 16, "cross_dim": 24, "state_dim": 16}):
        a, b = D4.DiT4DiTHeadConfig(**kw), O.DiT4DiTHeadConfig(**kw)
        assert D4.param_shapes(a) == O.d4d_param_shapes(b)
    small = {"num_layers": 2, "heads": 2, "head_dim": 16, "cross_dim": 24, "output_dim": 40, "hidden_size": 40,
             "state_dim": 16}
    pa = D4.synthetic_params(D4.DiT4DiTHeadConfig(**small), 9)
    pb = O.init_d4d_params(O.DiT4DiTHeadConfig(**small), 9)
    assert sorted(pa) == sorted(pb) and all(torch.equal(pa[k], pb[k]) for k in pa)


def test_cosmos_shapes_and_rope_tables_match_oracle():
    """fam.cosmos's parameter layout and host fp32 RoPE tables equal the oracle's restatement."""
    from fam import cosmos
    cfg = cosmos.CosmosConfig(num_layers=3)
    ocfg = O.CosmosConfig(num_layers=3)
    assert cosmos.param_shapes(cfg) == O.cosmos_param_shapes(ocfg)
    for fps in (None, 16.0):
        c1, s1 = cosmos.cosmos_rope_tables(cfg, 2, 32, 32, fps, "cpu")
        c2, s2 = O.cosmos_rope_tables(ocfg, 2, 32, 32, fps)
        assert torch.equal(c1, c2) and torch.equal(s1, s2)

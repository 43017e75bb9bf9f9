"""Parity of the MoT video K/V prefill (FB/mot.py:262-376) built from the library's kernels
(fam.video_dit.FusedVideoPrefill) against the oracle's mot_prefill_video_cache, which the
reference's own prefill pins (tests/golden/mot_prefill_tiny.safetensors): every layer's cached
k (RMSNorm + RoPE) and v, normwise relative error <= 2e-2 (bf16 kernels vs fp32 oracle on
bf16-valued weights and inputs).  Cases: a first-frame-causal mask over two latent frames
(the masked attention path), the single-frame inference call (no mask: the long-sequence
kernel), video layer drafting, a ragged text mask and no context at all."""
import pytest
import torch

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu


def _relerr(y, ref):
    return ((y.float() - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.parametrize("frames,tpf,Lc,num_run,ragged,nh", [(2, 49, 40, 0, True, 4), (1, 98, 40, 0, False, 4),
                                                             (2, 24, 24, 2, True, 4), (1, 48, 0, 0, False, 4),
                                                             (2, 49, 40, 0, True, 8), (1, 48, 0, 0, False, 8)])
def test_video_prefill_kv_matches_oracle(frames, tpf, Lc, num_run, ragged, nh):
    """Every layer's K/V against the oracle's prefill.  Each block's q|k|v row is finished by
    one row launch when the head width A = nh * 128 tiles it (nh=8: A=1024), segment by
    segment otherwise; the o row carries norm3 (or, without context, the FFN's AdaLN) and the
    cross-o row the FFN's AdaLN."""
    from fam.video_dit import FusedVideoPrefill
    Sv, H, Dh, F, L = frames * tpf, 512, 128, 1024, 3
    ocfg = O.ActionDiTConfig(hidden_dim=H, action_dim=7, ffn_dim=F, text_dim=H, freq_dim=256, num_heads=nh,
                             attn_head_dim=Dh, num_layers=L)
    p = {k: v.to(torch.bfloat16) for k, v in O.init_action_dit_params(ocfg, 41).items()}
    g = torch.Generator().manual_seed(42)
    x = torch.randn(1, Sv, H, generator=g).to(torch.bfloat16)
    tm = (torch.randn(1, Sv, 6, H, generator=g) * 0.2).to(torch.bfloat16)
    ctx = torch.randn(1, Lc, H, generator=g).to(torch.bfloat16) if Lc else None
    cmask = None
    if Lc and ragged:
        cmask = torch.ones(1, Sv, Lc, dtype=torch.bool)
        cmask[:, :, Lc - 7:] = False
    vmask = O.mot_joint_mask(Sv, 0, tpf) if frames > 1 else None
    freqs = O.action_freqs(Dh, Sv)
    pf = FusedVideoPrefill(p, num_layers=L, hidden=H, num_heads=nh, head_dim=Dh, ffn_dim=F, batch=1, video_len=Sv,
                           ctx_len=Lc, freqs=freqs, video_mask=vmask, ctx_mask=cmask, num_run=num_run)
    kv = pf.prefill(x.cuda(), tm.cuda(), ctx.cuda() if ctx is not None else None)
    p32 = {k: v.float() for k, v in p.items()}
    ref = O.mot_prefill_video_cache(p32, ocfg, x.float(), freqs, tm.float(), None if ctx is None else ctx.float(),
                                    vmask if vmask is not None else torch.ones(Sv, Sv, dtype=torch.bool), cmask,
                                    num_run)
    assert len(kv) == L
    worst = 0.0
    for i, ((k, v), (rk, rv)) in enumerate(zip(kv, ref)):
        ek, ev = _relerr(k.cpu(), rk), _relerr(v.cpu(), rv)
        worst = max(worst, ek, ev)
        assert ek <= 2e-2 and ev <= 2e-2, (i, ek, ev)
    print(f"prefill frames={frames} tpf={tpf} Lc={Lc} num_run={num_run} heads={nh}: {pf.num_launches} launches, "
          f"worst relerr {worst:.3e}")
    # graph replay: the same bits
    first = [(k.clone(), v.clone()) for k, v in kv]
    pf.capture()
    kv2 = pf.prefill(x.cuda(), tm.cuda(), ctx.cuda() if ctx is not None else None)
    assert all(torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) for a, b in zip(first, kv2))


def test_video_prefill_context_kv_split_k():
    """129 context rows: the stacked context K/V of the 11 cross-attending blocks
    (129 x 16896 x 768) on the streaming split-K kernel with 9 m-tiles in one split, which
    stores the bf16 rows with their bias itself (fam_gemm; no plane, no row launch), instead of
    the large-M GEMM; every layer's K/V against the oracle."""
    from fam import _capi
    from fam.video_dit import FusedVideoPrefill
    Sv, H, nh, Dh, F, L, Lc = 98, 768, 6, 128, 1536, 12, 129
    assert _capi.lib().fam_gemm_partial_splits(Lc, (L - 1) * 2 * nh * Dh, H) == 1
    ocfg = O.ActionDiTConfig(hidden_dim=H, action_dim=7, ffn_dim=F, text_dim=H, freq_dim=256, num_heads=nh,
                             attn_head_dim=Dh, num_layers=L)
    p = {k: v.to(torch.bfloat16) for k, v in O.init_action_dit_params(ocfg, 71).items()}
    g = torch.Generator().manual_seed(72)
    x = torch.randn(1, Sv, H, generator=g).to(torch.bfloat16)
    tm = (torch.randn(1, Sv, 6, H, generator=g) * 0.2).to(torch.bfloat16)
    ctx = torch.randn(1, Lc, H, generator=g).to(torch.bfloat16)
    freqs = O.action_freqs(Dh, Sv)
    pf = FusedVideoPrefill(p, num_layers=L, hidden=H, num_heads=nh, head_dim=Dh, ffn_dim=F, batch=1, video_len=Sv,
                           ctx_len=Lc, freqs=freqs)
    assert [m["name"] for m in pf.meta[:2]] == ["ctx_kv_all", "cross_k_norm_all"]
    kv = pf.prefill(x.cuda(), tm.cuda(), ctx.cuda())
    p32 = {k: v.float() for k, v in p.items()}
    ref = O.mot_prefill_video_cache(p32, ocfg, x.float(), freqs, tm.float(), ctx.float(),
                                    torch.ones(Sv, Sv, dtype=torch.bool))
    worst = 0.0
    for i, ((k, v), (rk, rv)) in enumerate(zip(kv, ref)):
        ek, ev = _relerr(k.cpu(), rk), _relerr(v.cpu(), rv)
        worst = max(worst, ek, ev)
        assert ek <= 2e-2 and ev <= 2e-2, (i, ek, ev)
    print(f"prefill, 129 context rows on split-K: {pf.num_launches} launches, worst relerr {worst:.3e}")


def test_video_prefill_broadcast_modulation():
    """Per-batch t_mod ([B, 6, H], per_token_mod=False): the chained blocks read their
    modulation from one [B, blocks, 6H] buffer with a zero row stride; against the oracle fed
    the same t_mod for every token."""
    from fam.video_dit import FusedVideoPrefill
    Sv, H, nh, Dh, F, L, Lc = 98, 512, 8, 128, 1024, 3, 40
    ocfg = O.ActionDiTConfig(hidden_dim=H, action_dim=7, ffn_dim=F, text_dim=H, freq_dim=256, num_heads=nh,
                             attn_head_dim=Dh, num_layers=L)
    p = {k: v.to(torch.bfloat16) for k, v in O.init_action_dit_params(ocfg, 61).items()}
    g = torch.Generator().manual_seed(62)
    x = torch.randn(1, Sv, H, generator=g).to(torch.bfloat16)
    tm = (torch.randn(1, 6, H, generator=g) * 0.2).to(torch.bfloat16)
    ctx = torch.randn(1, Lc, H, generator=g).to(torch.bfloat16)
    freqs = O.action_freqs(Dh, Sv)
    pf = FusedVideoPrefill(p, num_layers=L, hidden=H, num_heads=nh, head_dim=Dh, ffn_dim=F, batch=1, video_len=Sv,
                           ctx_len=Lc, freqs=freqs, per_token_mod=False)
    kv = pf.prefill(x.cuda(), tm.cuda(), ctx.cuda())
    p32 = {k: v.float() for k, v in p.items()}
    ref = O.mot_prefill_video_cache(p32, ocfg, x.float(), freqs, tm.float()[:, None].expand(1, Sv, 6, H), ctx.float(),
                                    torch.ones(Sv, Sv, dtype=torch.bool))
    worst = 0.0
    for i, ((k, v), (rk, rv)) in enumerate(zip(kv, ref)):
        ek, ev = _relerr(k.cpu(), rk), _relerr(v.cpu(), rv)
        worst = max(worst, ek, ev)
        assert ek <= 2e-2 and ev <= 2e-2, (i, ek, ev)
    print(f"prefill with per-batch t_mod: {pf.num_launches} launches, worst relerr {worst:.3e}")


def test_video_prefill_feeds_the_mot_action_loop():
    """The inference call's video half feeding its action half: GPU prefill of a single-frame
    video (98 tokens, 2 layers, hidden 768) -> FusedActionDiT in MoT mode (set_video_kv from the
    prefill's cache views) -> 3 Euler steps, against oracle prefill -> oracle MoT loop: the final
    action chunk within 1e-2 abs."""
    from fam.action_dit import ActionDiTConfig, FusedActionDiT
    from fam.video_dit import FusedVideoPrefill
    S, Sv, Lc, steps, L = 32, 98, 129, 3, 2
    acfg = ActionDiTConfig(hidden_dim=512, action_dim=7, ffn_dim=1024, text_dim=256, freq_dim=256, num_heads=12,
                           attn_head_dim=64, num_layers=L)
    vcfg = O.ActionDiTConfig(hidden_dim=768, action_dim=7, ffn_dim=1536, text_dim=768, freq_dim=256, num_heads=12,
                             attn_head_dim=64, num_layers=L)
    pa = {k: v.to(torch.bfloat16) for k, v in O.init_action_dit_params(O.ActionDiTConfig(**acfg.to_dict()), 51).items()}
    pv = {k: v.to(torch.bfloat16) for k, v in O.init_action_dit_params(vcfg, 52).items()}
    g = torch.Generator().manual_seed(53)
    noise = torch.randn(1, S, 7, generator=g).to(torch.bfloat16)
    ctx = torch.randn(1, Lc, 256, generator=g).to(torch.bfloat16)
    xv = torch.randn(1, Sv, 768, generator=g).to(torch.bfloat16)
    tmv = (torch.randn(1, Sv, 6, 768, generator=g) * 0.2).to(torch.bfloat16)
    ctxv = torch.randn(1, Lc, 768, generator=g).to(torch.bfloat16)
    fv = O.action_freqs(64, Sv)
    pf = FusedVideoPrefill(pv, num_layers=L, hidden=768, num_heads=12, head_dim=64, ffn_dim=1536, batch=1,
                           video_len=Sv, ctx_len=Lc, freqs=fv)
    kv = pf.prefill(xv.cuda(), tmv.cuda(), ctxv.cuda())
    m = FusedActionDiT(acfg, pa, batch=1, seq_len=S, ctx_len=Lc, num_steps=steps, shift=5.0, video_len=Sv)
    m.set_video_kv([k for k, _ in kv], [v for _, v in kv])
    y = m.infer(noise.cuda(), ctx.cuda()).float().cpu()

    pa32 = {k: v.float() for k, v in pa.items()}
    pv32 = {k: v.float() for k, v in pv.items()}
    vkv = O.mot_prefill_video_cache(pv32, vcfg, xv.float(), fv, tmv.float(), ctxv.float(),
                                    torch.ones(Sv, Sv, dtype=torch.bool))
    ocfg = O.ActionDiTConfig(**acfg.to_dict())
    joint = O.mot_joint_mask(Sv, S, Sv)
    ts, ds = O.build_inference_schedule(steps, 5.0, torch.bfloat16)
    ctx_emb = O.text_embedding(pa32, ctx.float())
    freqs = O.action_freqs(64, S)
    x_lat = noise.float()
    for t, d in zip(ts.float(), ds.float()):
        _, t_mod = O.time_mlp(pa32, ocfg, t.reshape(1))
        x = O.linear(x_lat, pa32["action_encoder.weight"], pa32["action_encoder.bias"])
        x = O.mot_action_forward(pa32, ocfg, x, freqs, t_mod, ctx_emb, vkv, joint, Sv)
        x_lat = x_lat + O.linear(x, pa32["head.weight"], pa32["head.bias"]) * d
    dd = (y - x_lat).abs()
    print(f"prefill -> MoT loop: max|d| {dd.max().item():.3e} mean|d| {dd.mean().item():.3e}")
    assert dd.max().item() <= 1e-2

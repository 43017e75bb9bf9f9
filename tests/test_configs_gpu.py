"""Every BASELINE configuration at its own shape on the GPU, against the oracle (fp32 arithmetic
on bf16-valued weights and inputs), plus a model built from a reference-layout checkpoint
payload.  Bars: the denoised chunk within 1e-2 absolute after the full loop; single forwards
within 2e-2 normwise relative.

  config 1 at B=32   12 blocks, hidden 1024, 16 x 64 heads, FFN 4096, 10 steps, 1560 context
  config 2           one Wan2.2-5B-style video block: 1560 tokens (2 x 30 x 26, 3-D RoPE),
                     hidden 3072, 24 x 128 heads, FFN 14336, 512 text tokens, per-token t_mod
  config 3 at B=256  compact expert (hidden 32, 4 x 8 heads, 8 blocks, 8 x 16 latent, 4 steps)
                     over 1560 context tokens, then the action-VAE decoder to 32 x 7
  config 4 head      DiT4DiT action head at hidden 1024 (16 x 64 heads) on a 16 x 29 chunk
                     (16 action rows: M = 16 split-K products), 4 steps, 2048 VLM tokens x 2048
"""
import os

import pytest
import torch

from block_checks import BAR, gpu_block_errors
from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _p(cfg, seed):
    return {k: v.to(BF) for k, v in O.init_action_dit_params(cfg, seed).items()}


def _oracle_loop(p32, ocfg, noise, ctx, steps, shift):
    ts, ds = O.build_inference_schedule(steps, shift, BF)
    ctx_emb = O.text_embedding(p32, ctx)
    x = noise
    for t, d in zip(ts.float(), ds.float()):
        x = x + O.action_dit_forward(p32, ocfg, x, t.reshape(1), ctx, context_emb=ctx_emb) * d
    return x


def test_config1_b32_full_loop():
    """The throughput point: 32 chunks (M = 1024 rows through the large-M GEMM and the row
    kernels), one shared context.  Rows 0, 17 and 31 against the oracle."""
    from fam.action_dit import ActionDiTConfig, FusedActionDiT
    cfg = ActionDiTConfig()
    ocfg = O.ActionDiTConfig(**cfg.to_dict())
    p = _p(ocfg, 101)
    g = torch.Generator().manual_seed(102)
    noise = torch.randn(32, 32, 7, generator=g).to(BF)
    ctx = torch.randn(1, 1560, 1024, generator=g).to(BF)
    m = FusedActionDiT(cfg, p, batch=32, seq_len=32, ctx_len=1560, num_steps=10, shift=5.0)
    y = m.infer(noise.cuda(), ctx.cuda()).float().cpu()
    rows = [0, 17, 31]
    p32 = {k: v.float() for k, v in p.items()}
    ref = _oracle_loop(p32, ocfg, noise[rows].float(), ctx.float().expand(len(rows), -1, -1), 10, 5.0)
    d = (y[rows] - ref).abs()
    print(f"config1 B=32: rows {rows} max|d| {d.max().item():.3e} mean|d| {d.mean().item():.3e}")
    assert d.max().item() <= 1e-2
    assert torch.isfinite(y).all()


def test_config2_video_block_full_shape():
    """One backbone block at config 2's shape with per-token modulation (FB/wan_video_dit.py:267-286,
    t_mod per token as at :555-568) against the oracle's dit_block."""
    from fam.video_dit import FusedVideoDiTBlock
    f, hh, ww = 2, 30, 26
    S, H, nh, Dh, F, Lc = f * hh * ww, 3072, 24, 128, 14336, 512
    ocfg = O.ActionDiTConfig(hidden_dim=H, action_dim=7, ffn_dim=F, text_dim=H, freq_dim=256, num_heads=nh,
                             attn_head_dim=Dh, num_layers=1)
    p = _p(ocfg, 103)
    g = torch.Generator().manual_seed(104)
    x = torch.randn(1, S, H, generator=g).to(BF)
    ctx = torch.randn(1, Lc, H, generator=g).to(BF)
    tm = (torch.randn(1, S, 6, H, generator=g) * 0.2).to(BF)
    freqs = O.video_freqs(O.precompute_freqs_cis_3d(Dh), f, hh, ww)
    blk = FusedVideoDiTBlock(p, 0, hidden=H, num_heads=nh, head_dim=Dh, ffn_dim=F, batch=1, seq_len=S, ctx_len=Lc,
                             freqs=freqs, per_token_mod=True)
    y = blk.forward(x.cuda(), tm.cuda(), ctx.cuda()).float().cpu()
    p32 = {k: v.float() for k, v in p.items()}
    tr = {}
    ref = O.dit_block(p32, 0, x.float(), ctx.float(), tm.float(), freqs, nh, 1e-6, trace=tr)
    err = ((y - ref).abs().max() / ref.abs().max()).item()
    # the output is dominated by the residual stream: the branch metrics are the ones a dropped
    # or transposed RoPE or a zeroed self-attention moves past the bar
    # (tests/test_oracle.py::test_block_branch_metrics_catch_planted_slips, same seeds and shape)
    errs = gpu_block_errors(blk, x, tm, ctx, tr, y, ref)
    print(f"config2 block (1560 x 3072, 24 x 128, FFN 14336, 512 text): normwise rel err {err:.3e}; branches "
          + ", ".join(f"{k} {v:.3e}" for k, v in errs.items()))
    assert err <= BAR
    assert all(v <= BAR for v in errs.values()), errs


def test_config3_b256_loop_and_decoder():
    from fam.action_dit import ActionDiTConfig, FusedActionDiT
    from fam.cae import CaeDecoder
    cfg = ActionDiTConfig(hidden_dim=32, action_dim=16, ffn_dim=256, text_dim=1024, freq_dim=256, num_heads=4,
                          attn_head_dim=8, num_layers=8)
    ocfg = O.ActionDiTConfig(**cfg.to_dict())
    p = _p(ocfg, 105)
    g = torch.Generator().manual_seed(106)
    B = 256
    noise = torch.randn(B, 8, 16, generator=g).to(BF)
    ctx = torch.randn(1, 1560, 1024, generator=g).to(BF)
    m = FusedActionDiT(cfg, p, batch=B, seq_len=8, ctx_len=1560, num_steps=4, shift=5.0)
    lat = m.infer(noise.cuda(), ctx.cuda())
    dcfg = O.CaeDecoderConfig()
    dp = O.init_cae_decoder_params(dcfg, 107)
    dec = CaeDecoder(dp, latent_dim=16, num_tokens=8, action_horizon=32, action_dim=7, decoder_hidden=128, batch=B)
    y = dec.decode(lat).cpu()
    p32 = {k: v.float() for k, v in p.items()}
    ref_lat = _oracle_loop(p32, ocfg, noise.float(), ctx.float(), 4, 5.0)
    dl = (lat.float().cpu() - ref_lat).abs().max().item()
    ref = O.cae_decode(dp, dcfg, ref_lat)
    dd = (y - ref).abs().max().item()
    print(f"config3 B=256: latent max|d| {dl:.3e}, decoded max|d| {dd:.3e}")
    assert dl <= 1e-2
    assert dd <= 2e-2 * max(1.0, ref.abs().max().item())


def test_config4_dit4dit_head_shape():
    """The DiT4DiT head at BASELINE config 4's action side: hidden 1024 (16 x 64 heads), a 16 x 29
    chunk with no state token (16 rows per product), 4 steps, 2048 VLM tokens of width 2048."""
    from fam.dit4dit import FusedDiT4DiTHead
    cfg = O.DiT4DiTHeadConfig(heads=16, head_dim=64, action_dim=29, horizon=16, num_steps=4, cross_dim=2048)
    p = {k: v.to(BF) for k, v in O.init_d4d_params(cfg, 108).items()}
    g = torch.Generator().manual_seed(109)
    vl = torch.randn(1, 2048, 2048, generator=g).to(BF)
    noise = torch.randn(1, 16, 29, generator=g).to(BF)
    head = FusedDiT4DiTHead(cfg, p, batch=1, vl_len=2048, device=torch.device("cuda:0"), state_len=0)
    out = head.predict_action(vl.cuda(), noise.cuda()).float().cpu()
    ref = O.d4d_predict_action({k: v.float() for k, v in p.items()}, cfg, vl.float(), noise.float(), None)
    err = ((out - ref).abs().max() / ref.abs().max()).item()
    print(f"config4 DiT4DiT head (1024 wide, 16 x 29, 2048 VLM tokens): relerr {err:.3e}, "
          f"max|d| {(out - ref).abs().max().item():.3e}")
    assert err <= 3e-2


def _fused_layout(sd, layers, prefix):
    """The reference's saved layout: fused self-attention q|k|v and cross-attention k|v row blocks
    (FB/fused_qkv.py:141-199) under the MoT prefix (FB/mot.py:22-31)."""
    out = {}
    for k, v in sd.items():
        out[prefix + k] = v
    for i in range(layers):
        for leaf in ("weight", "bias"):
            b = f"{prefix}blocks.{i}.self_attn."
            out[b + "qkv." + leaf] = torch.cat([out.pop(b + n + "." + leaf) for n in "qkv"], 0)
            b = f"{prefix}blocks.{i}.cross_attn."
            out[b + "kv." + leaf] = torch.cat([out.pop(b + n + "." + leaf) for n in "kv"], 0)
    return out


def test_model_from_reference_checkpoint_payload(tmp_path):
    """A FastWAM-style payload ({"mot": state dict, "step", "torch_dtype"}, FB/fastwam.py:1113-1123)
    in the fused attention layout is written with torch.save, read back with fam.checkpoint
    (weights_only) and run: the action expert's denoise loop and the video expert's K/V prefill
    built from it match the oracle on the original weights."""
    from fam import checkpoint as CK
    from fam.action_dit import ActionDiTConfig, FusedActionDiT
    from fam.video_dit import FusedVideoPrefill
    acfg = ActionDiTConfig(num_layers=2, hidden_dim=1024, ffn_dim=4096, text_dim=1024, num_heads=16, attn_head_dim=64)
    vcfg = O.ActionDiTConfig(hidden_dim=512, action_dim=7, ffn_dim=1024, text_dim=512, freq_dim=256, num_heads=8,
                             attn_head_dim=128, num_layers=2)
    pa, pv = _p(O.ActionDiTConfig(**acfg.to_dict()), 110), _p(vcfg, 111)
    mot = {**_fused_layout(pa, 2, "mixtures.action."), **_fused_layout(pv, 2, "mixtures.video.")}
    path = os.path.join(tmp_path, "fastwam_step100.pt")
    torch.save({"mot": mot, "step": 100, "torch_dtype": "bfloat16"}, path)
    experts = CK.expert_state_dicts(CK.load_checkpoint(path))
    assert set(experts) == {"action", "video"}

    g = torch.Generator().manual_seed(112)
    noise = torch.randn(1, 32, 7, generator=g).to(BF)
    ctx = torch.randn(1, 300, 1024, generator=g).to(BF)
    m = FusedActionDiT(acfg, experts["action"], batch=1, seq_len=32, ctx_len=300, num_steps=4, shift=5.0)
    y = m.infer(noise.cuda(), ctx.cuda()).float().cpu()
    ref = _oracle_loop({k: v.float() for k, v in pa.items()}, O.ActionDiTConfig(**acfg.to_dict()), noise.float(),
                       ctx.float(), 4, 5.0)
    d = (y - ref).abs().max().item()
    print(f"action expert from the payload: max|d| {d:.3e}")
    assert d <= 1e-2

    Sv, Lc = 98, 40
    x = torch.randn(1, Sv, 512, generator=g).to(BF)
    tm = (torch.randn(1, Sv, 6, 512, generator=g) * 0.2).to(BF)
    vctx = torch.randn(1, Lc, 512, generator=g).to(BF)
    freqs = O.action_freqs(128, Sv)
    pf = FusedVideoPrefill(experts["video"], num_layers=2, hidden=512, num_heads=8, head_dim=128, ffn_dim=1024,
                           batch=1, video_len=Sv, ctx_len=Lc, freqs=freqs)
    kv = pf.prefill(x.cuda(), tm.cuda(), vctx.cuda())
    rkv = O.mot_prefill_video_cache({k: v.float() for k, v in pv.items()}, vcfg, x.float(), freqs, tm.float(),
                                    vctx.float(), torch.ones(Sv, Sv, dtype=torch.bool))
    for i, ((k, v), (rk, rv)) in enumerate(zip(kv, rkv)):
        for a, b in ((k, rk), (v, rv)):
            err = ((a.float().cpu() - b).abs().max() / b.abs().max()).item()
            assert err <= 2e-2, (i, err)

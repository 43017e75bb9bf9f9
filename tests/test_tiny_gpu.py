"""fam_tiny_expert (the hidden-32 action experts in two launches per block step) against the
oracle and against the generic launch plan of FusedActionDiT.

Oracle side as in tests/test_model_gpu.py: bf16-valued weights and inputs, fp32 arithmetic, the
bf16 schedule.  Bar: the denoised chunk within 1% of its motion (max |chunk - noise|) of the
oracle after the loop, where dropping the context or the video values moves it by more than 3%;
weights are unit-scale so that every branch reaches the chunk.  The shapes cover
one attention slice (every head in one workgroup, direct sums of squares) and several slices
(the Gram-matrix normaliser), video prefixes whose last 32-key block is ragged, the MoT joint
mask, a batch of several chunks, an action dim that is not a multiple of 8, and FFN widths
below 256.
"""
import pytest
import torch

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu


def _cls():
    from fam.action_dit import ActionDiTConfig, FusedActionDiT
    return ActionDiTConfig, FusedActionDiT


def _params(cfg, seed):
    """Unit-scale weights: each linear N(0, 1 / fan_in), biases N(0, 0.1^2) (the reference's
    N(0, 0.02) init leaves a hidden-32 expert's attention branches almost without effect on
    the chunk, so a test on it could not tell a dropped branch); modulation and norm affines as
    the oracle's init."""
    p = O.init_action_dit_params(O.ActionDiTConfig(**cfg.to_dict()), seed, std=1.0)
    out = {}
    for k, v in p.items():
        if k.endswith(".weight") and v.dim() == 2:
            v = v / v.shape[1] ** 0.5
        elif k.endswith(".bias") and "norm" not in k:
            v = v * 0.1
        out[k] = v.to(torch.bfloat16)
    return out


def _oracle_mot_loop(p, cfg, noise, ctx, vks, vvs, joint, steps, shift=5.0):
    p32 = {k: v.float() for k, v in p.items()}
    ocfg = O.ActionDiTConfig(**cfg.to_dict())
    ts, ds = O.build_inference_schedule(steps, shift, torch.bfloat16)
    ctx_emb = O.text_embedding(p32, ctx.float())
    S = noise.shape[1]
    freqs = O.action_freqs(cfg.attn_head_dim, S)
    x_lat = noise.float()
    Sv = vks[0].shape[1] if vks else 0
    for t, d in zip(ts.float(), ds.float()):
        _, t_mod = O.time_mlp(p32, ocfg, t.reshape(1))
        x = O.linear(x_lat, p32["action_encoder.weight"], p32["action_encoder.bias"])
        if Sv:
            vkv = [(k.float(), v.float()) for k, v in zip(vks, vvs)]
            x = O.mot_action_forward(p32, ocfg, x, freqs, t_mod, ctx_emb, vkv, joint, Sv)
        else:
            for i in range(cfg.num_layers):
                x = O.dit_block(p32, i, x, ctx_emb, t_mod, freqs, cfg.num_heads, cfg.eps)
        x_lat = x_lat + O.linear(x, p32["head.weight"], p32["head.bias"]) * d
    return x_lat


@pytest.mark.parametrize(
    "B,S,heads,dh,ffn,Sv,Lc,layers,steps,slice_,masked,da",
    [
        (1, 8, 4, 32, 256, 40, 33, 2, 3, 32, False, 16),     # 4 slices: Gram normaliser; ragged video block
        (1, 8, 4, 32, 256, 40, 33, 2, 3, 0, True, 16),      # one slice (A = 128), joint mask
        (3, 8, 2, 64, 128, 98, 129, 2, 2, 64, False, 16),   # batch of 3, 2 slices of one 64-dim head
        (2, 6, 24, 128, 256, 98, 60, 2, 2, 0, False, 7),    # the CAE heads, 6 tokens, action dim 7
        (1, 16, 2, 16, 64, 0, 20, 2, 3, 0, False, 7),       # no video prefix, 16 tokens, 2 x 16 heads
        (1, 8, 4, 8, 64, 0, 300, 2, 3, 0, False, 16),       # config 3's heads: the context over 3 splits
        (2, 8, 4, 8, 64, 40, 1560, 2, 2, 0, True, 16),      # 7 splits of 1560 keys, joint mask, 2 rows
    ])
def test_tiny_expert_matches_oracle_and_generic_plan(B, S, heads, dh, ffn, Sv, Lc, layers, steps, slice_, masked,
                                                     da):
    Cfg, Model = _cls()
    cfg = Cfg(hidden_dim=32, action_dim=da, ffn_dim=ffn, text_dim=64, freq_dim=32, num_heads=heads,
              attn_head_dim=dh, num_layers=layers)
    A = heads * dh
    p = _params(cfg, 101 + heads + S)
    g = torch.Generator().manual_seed(202 + B)
    noise = torch.randn(B, S, da, generator=g).to(torch.bfloat16)
    ctx = torch.randn(1, Lc, 64, generator=g).to(torch.bfloat16)
    vks = [torch.randn(B, Sv, A, generator=g).to(torch.bfloat16) for _ in range(layers)] if Sv else []
    vvs = [torch.randn(B, Sv, A, generator=g).to(torch.bfloat16) for _ in range(layers)] if Sv else []
    joint = torch.ones(Sv + S, Sv + S, dtype=torch.bool)
    if masked:
        joint = torch.rand(Sv + S, Sv + S, generator=g) > 0.3
        joint[:, Sv:] = True          # every action row keeps its own keys (no empty rows)
    kw = dict(batch=B, seq_len=S, ctx_len=Lc, num_steps=steps, shift=5.0, video_len=Sv,
              video_mask=joint[Sv:, :] if (Sv and masked) else None)
    m = Model(cfg, p, tiny=True, tiny_slice=slice_, **kw)
    assert m.tiny is not None and m.num_launches < 2 * layers * steps + 16
    if heads * dh == 32 and Lc >= 128:
        assert m.tiny["KS"] > 1   # the cross phases split the context over workgroups
    if Sv:
        m.set_video_kv([k.cuda() for k in vks], [v.cuda() for v in vvs])
    y = m.infer(noise.cuda(), ctx.cuda()).float().cpu()
    ref = _oracle_mot_loop(p, cfg, noise, ctx, vks, vvs, joint, steps)
    d_or = (y - ref).abs().max().item()
    gen = Model(cfg, p, tiny=False, **kw)
    if Sv:
        gen.set_video_kv([k.cuda() for k in vks], [v.cuda() for v in vvs])
    yg = gen.infer(noise.cuda(), ctx.cuda()).float().cpu()
    d_gen = (y - yg).abs().max().item()
    motion = (ref - noise.float()).abs().max().item()
    # the metric can fail: an oracle whose video values (or context) are zeroed moves the chunk by
    # far more than the bar, so a kernel that dropped the joint attention's video keys or the
    # cross attention would not pass
    slips = {"no context": _oracle_mot_loop(p, cfg, noise, torch.zeros_like(ctx), vks, vvs, joint, steps)}
    if Sv:
        slips["video values zeroed"] = _oracle_mot_loop(p, cfg, noise, ctx, vks, [v * 0 for v in vvs], joint, steps)
    print(f"tiny expert B={B} S={S} {heads}x{dh} slice={slice_ or 'auto'} Sv={Sv} Lc={Lc}: max|d| vs oracle "
          f"{d_or:.3e} (chunk motion {motion:.3e}), vs the generic plan {d_gen:.3e} ({m.num_launches} against "
          f"{gen.num_launches} launches); planted slips move it " +
          ", ".join(f"{k} {(v - ref).abs().max().item():.3e}" for k, v in slips.items()))
    bar = 1e-2 * motion
    assert d_or <= bar
    assert d_gen <= bar
    for k, v in slips.items():
        assert (v - ref).abs().max().item() > 3 * bar, k


def test_tiny_expert_graph_replay_and_rerun():
    """The tiny path replays from a captured graph bit-identically to eager launches, twice in a
    row (every phase rewrites the state it reads: nothing carries over between calls), and a
    second call with other noise gives that noise's result."""
    Cfg, Model = _cls()
    cfg = Cfg(hidden_dim=32, action_dim=16, ffn_dim=256, text_dim=64, freq_dim=32, num_heads=24, attn_head_dim=128,
              num_layers=3)
    p = _params(cfg, 303)
    g = torch.Generator().manual_seed(304)
    A = cfg.attn_dim
    n1, n2 = (torch.randn(1, 8, 16, generator=g).to(torch.bfloat16) for _ in range(2))
    ctx = torch.randn(1, 129, 64, generator=g).to(torch.bfloat16)
    vk = [torch.randn(1, 98, A, generator=g).to(torch.bfloat16).cuda() for _ in range(3)]
    vv = [torch.randn(1, 98, A, generator=g).to(torch.bfloat16).cuda() for _ in range(3)]
    m = Model(cfg, p, batch=1, seq_len=8, ctx_len=129, num_steps=4, video_len=98, video_kv=list(zip(vk, vv)))
    assert m.tiny is not None
    e1 = m.infer(n1.cuda(), ctx.cuda())
    e2 = m.infer(n2.cuda(), ctx.cuda())
    m.capture()
    for _ in range(2):
        r1 = m.infer(n1.cuda(), ctx.cuda())
        torch.cuda.synchronize()
        assert torch.equal(r1, e1)
        r2 = m.infer(n2.cuda(), ctx.cuda())
        torch.cuda.synchronize()
        assert torch.equal(r2, e2)
    assert not torch.equal(e1, e2)

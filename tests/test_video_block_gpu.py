"""Parity of the long-sequence DiT block (the video backbone's block, FB/wan_video_dit.py:267-286)
built from the library's kernels, against the oracle's dit_block: per-token AdaLN modulation,
3-D RoPE over an (f, h, w) grid, self-attention over all video tokens, cross-attention to the
text tokens.  Bar: 2e-2 normwise relative (bf16 kernels vs fp32 oracle on bf16-valued weights
and inputs) on the block output, on what the block adds (output minus input), on the rotated
q / k and the v, and on each attention's output before its o projection (tests/block_checks.py).
"""
import pytest
import torch

from block_checks import BAR, gpu_block_errors
from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_token", [True, False])
def test_video_dit_block(per_token):
    from fam.video_dit import FusedVideoDiTBlock
    f, hh, ww = 2, 6, 8
    S, H, nh, Dh, F, Lc = f * hh * ww, 1024, 8, 128, 2048, 64
    ocfg = O.ActionDiTConfig(hidden_dim=H, action_dim=7, ffn_dim=F, text_dim=H, freq_dim=256, num_heads=nh,
                             attn_head_dim=Dh, num_layers=1)
    p = {k: v.to(torch.bfloat16) for k, v in O.init_action_dit_params(ocfg, 31).items()}
    g = torch.Generator().manual_seed(32)
    x = torch.randn(1, S, H, generator=g).to(torch.bfloat16)
    ctx = torch.randn(1, Lc, H, generator=g).to(torch.bfloat16)
    tm = (torch.randn(1, S, 6, H, generator=g) * 0.2) if per_token else (torch.randn(1, 6, H, generator=g) * 0.2)
    tm = tm.to(torch.bfloat16)
    freqs = O.video_freqs(O.precompute_freqs_cis_3d(Dh), f, hh, ww)
    blk = FusedVideoDiTBlock(p, 0, hidden=H, num_heads=nh, head_dim=Dh, ffn_dim=F, batch=1, seq_len=S, ctx_len=Lc,
                             freqs=freqs, per_token_mod=per_token)
    y = blk.forward(x.cuda(), tm.cuda(), ctx.cuda()).float().cpu()
    p32 = {k: v.float() for k, v in p.items()}
    tr = {}
    ref = O.dit_block(p32, 0, x.float(), ctx.float(), tm.float(), freqs, nh, 1e-6, trace=tr)
    err = ((y - ref).abs().max() / ref.abs().max()).item()
    errs = gpu_block_errors(blk, x, tm, ctx, tr, y, ref)
    print(f"video block (per_token={per_token}): normwise rel err {err:.3e}; branches "
          + ", ".join(f"{k} {v:.3e}" for k, v in errs.items()))
    assert err <= BAR
    assert all(v <= BAR for v in errs.values()), errs
    # graph replay gives the same bits
    blk.capture()
    y2 = blk.forward(x.cuda(), tm.cuda(), ctx.cuda()).float().cpu()
    assert torch.equal(y, y2)

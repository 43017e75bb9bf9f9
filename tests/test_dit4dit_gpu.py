"""DiT4DiT flow-matching head on the library vs the oracle's restatement of
FlowmatchingActionHead.predict_action (fp32 oracle on bf16-rounded weights and inputs).

The oracle's head composition follows diffusers semantics that no reference fixture pins here
(diffusers is absent), so these tests pin the GPU path to the oracle; the oracle's own pins are
the closed forms and structural checks in tests/test_oracle.py."""
import pytest
import torch

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu


def _params(cfg, seed):
    return {k: v.to(torch.bfloat16) for k, v in O.init_d4d_params(cfg, seed).items()}


def _run(cfg, B, L, seed, capture=False):
    from fam.dit4dit import FusedDiT4DiTHead
    p = _params(cfg, seed)
    g = torch.Generator().manual_seed(seed + 1)
    vl = torch.randn(B, L, cfg.cross_dim, generator=g).to(torch.bfloat16)
    noise = torch.randn(B, cfg.horizon, cfg.action_dim, generator=g).to(torch.bfloat16)
    head = FusedDiT4DiTHead(cfg, p, batch=B, vl_len=L, device=torch.device("cuda:0"))
    out = head.predict_action(vl.cuda(), noise.cuda())
    ref = O.d4d_predict_action({k: v.float() for k, v in p.items()}, cfg, vl.float(), noise.float())
    return head, vl, noise, out.float().cpu(), ref


def _relerr(y, ref):
    return ((y - ref).abs().max() / ref.abs().max()).item()


def test_d4d_head_tiny_config():
    cfg = O.DiT4DiTHeadConfig(num_layers=4, heads=2, head_dim=16, cross_dim=24, output_dim=40, hidden_size=40,
                              action_dim=5, horizon=6)
    _, _, _, out, ref = _run(cfg, 2, 40, 11)
    err = _relerr(out, ref)
    print(f"tiny DiT4DiT head: relerr {err:.3e}, max|d| {(out - ref).abs().max().item():.3e}")
    assert err <= 3e-2


def test_d4d_head_dit_b_config_and_graph_replay():
    """DiT-B head of the reference config (12 x 64 heads, 16 interleaved blocks, VLM width
    2048, decoder 2560, 16 x 32 actions), 256 VLM tokens; a captured replay is bit-identical."""
    cfg = O.DiT4DiTHeadConfig()
    head, vl, noise, out, ref = _run(cfg, 1, 256, 21)
    err = _relerr(out, ref)
    print(f"DiT-B head: relerr {err:.3e}, max|d| {(out - ref).abs().max().item():.3e}")
    assert err <= 3e-2
    head.capture()
    again = head.predict_action(vl.cuda(), noise.cuda()).float().cpu()
    assert torch.equal(again, out)

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


def _run(cfg, B, L, seed, state_len, fold_norms=True):
    """state_len 0 is the reference's state=None call; 1 is what the eval clients pass."""
    from fam.dit4dit import FusedDiT4DiTHead
    p = _params(cfg, seed)
    g = torch.Generator().manual_seed(seed + 1)
    vl = torch.randn(B, L, cfg.cross_dim, generator=g).to(torch.bfloat16)
    noise = torch.randn(B, cfg.horizon, cfg.action_dim, generator=g).to(torch.bfloat16)
    state = torch.randn(B, state_len, cfg.state_dim, generator=g).to(torch.bfloat16) if state_len else None
    head = FusedDiT4DiTHead(cfg, p, batch=B, vl_len=L, device=torch.device("cuda:0"), state_len=state_len,
                            fold_norms=fold_norms)
    out = head.predict_action(vl.cuda(), noise.cuda(), None if state is None else state.cuda())
    ref = O.d4d_predict_action({k: v.float() for k, v in p.items()}, cfg, vl.float(), noise.float(),
                               None if state is None else state.float())
    return head, (vl, noise, state), out.float().cpu(), ref


def _relerr(y, ref):
    return ((y - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.parametrize("B,state_len,fold", [(2, 1, True), (3, 0, True), (2, 2, True), (2, 1, False), (10, 1, True)])
def test_d4d_head_tiny_config(B, state_len, fold):
    """fold: LayerNorm / AdaLN folded into the projections (<= 64 rows; B=10 has 70 rows and
    takes the normalising prologue) or applied in the GEMM prologue."""
    cfg = O.DiT4DiTHeadConfig(num_layers=4, heads=2, head_dim=16, cross_dim=24, output_dim=40, hidden_size=40,
                              action_dim=5, horizon=6, state_dim=16)
    head, _, out, ref = _run(cfg, B, 40, 11, state_len, fold)
    assert head.fold == (fold and B * (6 + state_len) <= 64)
    err = _relerr(out, ref)
    print(f"tiny DiT4DiT head B={B} state_len={state_len} fold={head.fold}: relerr {err:.3e}, "
          f"max|d| {(out - ref).abs().max().item():.3e}")
    assert err <= 3e-2


def test_d4d_head_dit_b_config_and_graph_replay():
    """DiT-B head of the reference config (12 x 64 heads, 16 interleaved blocks, VLM width
    2048, decoder 2560, 16 x 32 actions, one 64-wide state token), 256 VLM tokens; a captured
    replay is bit-identical."""
    cfg = O.DiT4DiTHeadConfig()
    head, (vl, noise, state), out, ref = _run(cfg, 1, 256, 21, 1)
    err = _relerr(out, ref)
    print(f"DiT-B head: relerr {err:.3e}, max|d| {(out - ref).abs().max().item():.3e}")
    assert err <= 3e-2
    head.capture()
    for _ in range(2):
        again = head.predict_action(vl.cuda(), noise.cuda(), state.cuda()).float().cpu()
        assert torch.equal(again, out)


def test_d4d_head_robocasa_shape():
    """The DiT-B head at the RoboCasa-GR1 policy's shape: 588 VLM tokens (the backbone's 3 x 14 x 14
    video tokens at extract_layer), one 64-wide state token, a 16 x 32 chunk, 4 steps."""
    cfg = O.DiT4DiTHeadConfig()
    head, (vl, noise, state), out, ref = _run(cfg, 1, 588, 23, 1)
    err = _relerr(out, ref)
    print(f"DiT-B head over 588 tokens: relerr {err:.3e}, max|d| {(out - ref).abs().max().item():.3e}")
    assert err <= 3e-2


def test_d4d_head_rejects_state_mismatch():
    from fam.dit4dit import FusedDiT4DiTHead
    cfg = O.DiT4DiTHeadConfig(num_layers=2, heads=2, head_dim=16, cross_dim=24, output_dim=40, hidden_size=40,
                              action_dim=5, horizon=6, state_dim=16)
    p = _params(cfg, 3)
    dev = torch.device("cuda:0")
    vl = torch.zeros(1, 8, 24, dtype=torch.bfloat16, device=dev)
    noise = torch.zeros(1, 6, 5, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        FusedDiT4DiTHead(cfg, p, batch=1, vl_len=8, device=dev, state_len=1).predict_action(vl, noise)
    with pytest.raises(ValueError):
        FusedDiT4DiTHead(cfg, p, batch=1, vl_len=8, device=dev, state_len=0).predict_action(
            vl, noise, torch.zeros(1, 1, 16, dtype=torch.bfloat16, device=dev))

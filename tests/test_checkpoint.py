"""Checkpoint / state-dict loading (fam.checkpoint) on the CPU: the reference's payload layout
(FB/fastwam.py:1113-1131), its MoT key prefixes (FB/mot.py:22-31) and its fused attention layout
(FB/fused_qkv.py:141-199) into the expert keys the fused modules take."""
import pytest
import torch

from fam import action_dit as AD
from fam import checkpoint as CK

CFG = AD.ActionDiTConfig(num_layers=2, hidden_dim=64, ffn_dim=128, text_dim=48, freq_dim=32, num_heads=4,
                         attn_head_dim=16)


def _fused(sd):
    """The reference's fused layout built by hand: q|k|v row blocks of self-attention, k|v of
    cross-attention (cat along the output dimension)."""
    out = dict(sd)
    for i in range(CFG.num_layers):
        for leaf in ("weight", "bias"):
            p = f"blocks.{i}.self_attn."
            out[p + "qkv." + leaf] = torch.cat([out.pop(p + n + "." + leaf) for n in "qkv"], 0)
            p = f"blocks.{i}.cross_attn."
            out[p + "kv." + leaf] = torch.cat([out.pop(p + n + "." + leaf) for n in "kv"], 0)
    return out


def _equal(a, b):
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_unfuse_splits_in_reference_order():
    """Row blocks tagged 1/2/3 (q/k/v) and 4/5 (k/v) come back under the right names."""
    A, H = CFG.attn_dim, CFG.hidden_dim
    sd = {"blocks.0.self_attn.qkv.weight": torch.cat([torch.full((A, H), float(v)) for v in (1, 2, 3)]),
          "blocks.0.self_attn.qkv.bias": torch.cat([torch.full((A,), float(v)) for v in (1, 2, 3)]),
          "blocks.0.cross_attn.kv.weight": torch.cat([torch.full((A, H), float(v)) for v in (4, 5)]),
          "blocks.0.cross_attn.q.weight": torch.full((A, H), 6.0),
          "blocks.0.ffn.0.weight": torch.full((8, H), 7.0)}
    out = CK.unfuse_attention(sd)
    for key, v in (("self_attn.q.weight", 1), ("self_attn.k.weight", 2), ("self_attn.v.weight", 3),
                   ("self_attn.q.bias", 1), ("self_attn.v.bias", 3), ("cross_attn.k.weight", 4),
                   ("cross_attn.v.weight", 5), ("cross_attn.q.weight", 6), ("ffn.0.weight", 7)):
        t = out["blocks.0." + key]
        assert torch.all(t == v), key
    assert out["blocks.0.self_attn.q.weight"].shape == (A, H)
    assert "blocks.0.self_attn.qkv.weight" not in out and "blocks.0.cross_attn.kv.weight" not in out
    # a split-layout dict comes back unchanged
    plain = AD.synthetic_params(CFG, 1)
    _equal(CK.unfuse_attention(plain), plain)
    with pytest.raises(ValueError):
        CK.unfuse_attention({"blocks.0.self_attn.qkv.weight": torch.zeros(10, 4)})


@pytest.mark.parametrize("fused", [False, True])
def test_reference_payload_round_trip(tmp_path, fused):
    """A `FastWAM.save_checkpoint`-style payload ({"mot": MoT state dict, "step", "torch_dtype"})
    loads (weights only) into both experts' dicts, equal to what was saved; the action expert's
    dict builds the fused denoise loop and the video expert's the fused prefill (host plans)."""
    video, action = AD.synthetic_params(CFG, 2), AD.synthetic_params(CFG, 3)
    lay = _fused if fused else (lambda d: d)
    mot = {**{f"mixtures.video.{k}": v for k, v in lay(video).items()},
           **{f"mixtures.action.{k}": v for k, v in lay(action).items()}}
    path = str(tmp_path / "ckpt.pt")
    torch.save({"mot": mot, "step": 7, "torch_dtype": "torch.bfloat16"}, path)
    payload = CK.load_checkpoint(path)
    assert payload["step"] == 7
    experts = CK.expert_state_dicts(payload)
    _equal(experts["video"], video)
    _equal(experts["action"], action)
    m = AD.FusedActionDiT(CFG, experts["action"], batch=1, seq_len=32, ctx_len=20, num_steps=2, device="cpu")
    assert m.num_launches > 0
    from fam.video_dit import FusedVideoPrefill
    from oracle import fam_oracle as O
    pf = FusedVideoPrefill(experts["video"], num_layers=CFG.num_layers, hidden=CFG.hidden_dim,
                           num_heads=CFG.num_heads, head_dim=CFG.attn_head_dim, ffn_dim=CFG.ffn_dim, batch=1,
                           video_len=20, ctx_len=8, freqs=O.action_freqs(CFG.attn_head_dim, 20), device="cpu")
    assert pf.num_launches > 0


def test_safetensors_full_model_keys_and_legacy_dit(tmp_path):
    """A full FastWAM state dict (`mot.mixtures.*` keys) in a .safetensors file, and a legacy
    {"dit": video state dict} payload."""
    from safetensors.torch import save_file
    video, action = AD.synthetic_params(CFG, 4), AD.synthetic_params(CFG, 5)
    sd = {**{f"mot.mixtures.video.{k}": v.contiguous() for k, v in _fused(video).items()},
          **{f"mot.mixtures.action.{k}": v.contiguous() for k, v in action.items()},
          "proprio_encoder.weight": torch.zeros(4, 4)}
    path = str(tmp_path / "model.safetensors")
    save_file(sd, path)
    experts = CK.expert_state_dicts(CK.load_checkpoint(path))
    _equal(experts["video"], video)
    _equal(experts["action"], action)
    legacy = str(tmp_path / "legacy.pt")
    torch.save({"dit": _fused(video)}, legacy)
    experts = CK.expert_state_dicts(CK.load_checkpoint(legacy))
    assert list(experts) == ["video"]
    _equal(experts["video"], video)


def test_rejects_foreign_files(tmp_path):
    path = str(tmp_path / "other.pt")
    torch.save({"model": {}}, path)
    with pytest.raises(ValueError):
        CK.load_checkpoint(path)
    with pytest.raises(ValueError):
        CK.expert_state_dicts({"mot": {"foo.weight": torch.zeros(1)}})
    with pytest.raises(FileNotFoundError):
        CK.load_checkpoint(str(tmp_path / "missing.pt"))

"""Pins of the CPU oracle: closed forms, library routines, brute force and the golden
vectors written from the reference modules (tests/golden/make_golden.py)."""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import load_file

from oracle import fam_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "action_dit_tiny.safetensors")
TINY = O.ActionDiTConfig(hidden_dim=32, action_dim=7, ffn_dim=64, text_dim=24, freq_dim=16,
                         eps=1e-6, num_heads=2, attn_head_dim=16, num_layers=2)


# --------------------------------------------------------------------------- sinusoid
def test_sinusoid_closed_forms():
    pos = torch.tensor([0.0, 1.0, 250.0, 999.5], dtype=torch.float64)
    e = O.sinusoidal_embedding_1d(256, pos)
    assert e.shape == (4, 256) and e.dtype == torch.float64
    # position 0: cos = 1, sin = 0
    assert torch.all(e[0, :128] == 1) and torch.all(e[0, 128:] == 0)
    # first frequency is 1: column 0 is cos(p), column 128 is sin(p)
    assert torch.allclose(e[:, 0], torch.cos(pos)) and torch.allclose(e[:, 128], torch.sin(pos))
    # last frequency is 10000^(-127/128)
    f_last = 10000.0 ** (-127.0 / 128.0)
    assert torch.allclose(e[:, 127], torch.cos(pos * f_last)) and torch.allclose(e[:, 255], torch.sin(pos * f_last))
    # every (cos, sin) pair is a unit vector
    assert torch.allclose(e[:, :128] ** 2 + e[:, 128:] ** 2, torch.ones(4, 128, dtype=torch.float64))
    # cast to the dtype of the positions (bf16 timesteps -> bf16 embedding)
    assert O.sinusoidal_embedding_1d(16, pos.to(torch.bfloat16)).dtype == torch.bfloat16


# --------------------------------------------------------------------------- rope
def test_rope_tables():
    f = O.precompute_freqs_cis(64, 1024)
    assert f.shape == (1024, 32) and f.dtype == torch.complex128
    assert torch.allclose(f.abs(), torch.ones_like(f.abs()))
    # angle(pos, j) = pos * 10000^(-2j/64); checked where the angle is below pi
    pos, j = 3, 5
    assert math.isclose(torch.angle(f[pos, j]).item(), pos * 10000.0 ** (-2 * j / 64), rel_tol=1e-12)
    ff, fh, fw = O.precompute_freqs_cis_3d(128)
    assert (ff.shape[1], fh.shape[1], fw.shape[1]) == (22, 21, 21)  # 44/42/42 dims
    vf = O.video_freqs((ff, fh, fw), 2, 3, 4)
    assert vf.shape == (24, 1, 64)
    # token (f=1, h=2, w=3) -> row 1*12 + 2*4 + 3
    r = vf[1 * 12 + 2 * 4 + 3, 0]
    assert torch.equal(r[:22], ff[1]) and torch.equal(r[22:43], fh[2]) and torch.equal(r[43:], fw[3])


def test_rope_apply_invariants():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 6, 4 * 16, generator=g, dtype=torch.float64)
    fr = O.action_freqs(16, 6)
    y = O.rope_apply(x, fr, 4)
    # position 0 is the identity
    assert torch.allclose(y[:, 0], x[:, 0])
    # pairwise norms preserved
    xp = x.reshape(2, 6, 4, 8, 2)
    yp = y.reshape(2, 6, 4, 8, 2)
    assert torch.allclose(xp.norm(dim=-1), yp.norm(dim=-1))
    # rotating back by the conjugate recovers x
    assert torch.allclose(O.rope_apply(y, fr.conj(), 4), x)
    # brute force: a 2x2 rotation matrix per pair
    c, s = fr.real[:, 0, :], fr.imag[:, 0, :]
    for t in range(6):
        for i in range(8):
            a, b = x[1, t, 2 * 16 + 2 * i], x[1, t, 2 * 16 + 2 * i + 1]
            exp0 = a * c[t, i] - b * s[t, i]
            exp1 = a * s[t, i] + b * c[t, i]
            assert math.isclose(y[1, t, 32 + 2 * i].item(), exp0.item(), abs_tol=1e-12)
            assert math.isclose(y[1, t, 32 + 2 * i + 1].item(), exp1.item(), abs_tol=1e-12)


# --------------------------------------------------------------------------- norms
def test_norms():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 5, 48, generator=g) * 3 + 0.5
    ones = torch.ones(48)
    r = O.rms_norm(x, ones, 1e-6)
    assert torch.allclose(r.pow(2).mean(-1), torch.ones(3, 5), atol=1e-5)
    assert torch.allclose(O.rms_norm(7.0 * x, ones, 1e-6), r, atol=1e-5)   # scale invariant
    ln = O.layer_norm(x, None, None, 1e-6)
    assert torch.allclose(ln.mean(-1), torch.zeros(3, 5), atol=1e-5)
    assert torch.allclose(ln.var(-1, unbiased=False), torch.ones(3, 5), atol=1e-4)
    w, b = torch.randn(48, generator=g), torch.randn(48, generator=g)
    assert torch.allclose(O.layer_norm(x, w, b, 1e-6), F.layer_norm(x, (48,), w, b, 1e-6), atol=1e-5)
    z = torch.zeros(3, 1, 48)
    assert torch.allclose(O.adaln(x, z, z, 1e-6), F.layer_norm(x, (48,), eps=1e-6), atol=1e-5)
    # bf16: the rounding point before the weight multiply (FB/wan_video_dit.py:166-167)
    xb = x.to(torch.bfloat16)
    wb = torch.full((48,), 1.5, dtype=torch.bfloat16)
    exp = (xb.float() * torch.rsqrt(xb.float().pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * wb
    assert torch.equal(O.rms_norm(xb, wb, 1e-6), exp)


def test_gelu_silu_library():
    x = torch.linspace(-6, 6, 1001)
    assert torch.allclose(O.gelu_tanh(x), F.gelu(x, approximate="tanh"), atol=1e-6)
    assert torch.allclose(O.silu(x), F.silu(x), atol=1e-6)


# --------------------------------------------------------------------------- attention
def _brute_attention(q, k, v, mask):
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    out = np.zeros((B, H, Sq, D))
    qn, kn, vn = q.double().numpy(), k.double().numpy(), v.double().numpy()
    for b in range(B):
        for h in range(H):
            for i in range(Sq):
                sc = []
                for j in range(Sk):
                    if mask is not None and not bool(mask[i, j]):
                        continue
                    sc.append((j, float(np.dot(qn[b, h, i], kn[b, h, j]) / math.sqrt(D))))
                if not sc:
                    continue
                m = max(s for _, s in sc)
                den = sum(math.exp(s - m) for _, s in sc)
                for j, s in sc:
                    out[b, h, i] += math.exp(s - m) / den * vn[b, h, j]
    return torch.from_numpy(out)


@pytest.mark.parametrize("sq,sk", [(3, 5), (4, 1), (6, 9)])
def test_attention_bruteforce_and_sdpa(sq, sk):
    g = torch.Generator().manual_seed(sq * 10 + sk)
    q = torch.randn(2, 2, sq, 8, generator=g)
    k = torch.randn(2, 2, sk, 8, generator=g)
    v = torch.randn(2, 2, sk, 8, generator=g)
    mask = torch.rand(sq, sk, generator=g) > 0.3
    mask[0] = False                     # a fully masked row -> zeros
    if sk > 1:
        mask[1, :] = True
    o = O.attention(q, k, v, mask)
    assert torch.allclose(o.double(), _brute_attention(q, k, v, mask), atol=1e-5)
    assert torch.allclose(o, F.scaled_dot_product_attention(q, k, v, attn_mask=mask), atol=1e-5)
    assert torch.allclose(O.attention(q, k, v), F.scaled_dot_product_attention(q, k, v), atol=1e-5)
    # additive masks are added to the scores
    add = torch.where(mask, 0.0, float("-inf"))
    assert torch.allclose(O.attention(q, k, v, add)[:, :, 1:], o[:, :, 1:], atol=1e-6)


def test_attention_invariants():
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, 3, 5, 16, generator=g)
    k = torch.randn(1, 3, 7, 16, generator=g)
    v = torch.randn(1, 3, 7, 16, generator=g)
    perm = torch.randperm(7, generator=g)
    assert torch.allclose(O.attention(q, k, v), O.attention(q, k[:, :, perm], v[:, :, perm]), atol=1e-6)
    assert torch.allclose(O.attention(q, k[:, :, :1], v[:, :, :1]), v[:, :, :1].expand(1, 3, 5, 16), atol=1e-6)
    o = O.attention(q, k, v)
    assert torch.all(o.amax(2) <= v.amax(2) + 1e-5) and torch.all(o.amin(2) >= v.amin(2) - 1e-5)


# --------------------------------------------------------------------------- scheduler
def test_schedule_known_answers():
    t, d = O.build_inference_schedule(10, 5.0)
    exp_t = [1000, 978.261, 952.381, 921.053, 882.353, 833.333, 769.231, 681.818, 555.556, 357.143]
    exp_d = [-0.021739, -0.025880, -0.031328, -0.038700, -0.049020, -0.064103, -0.087413,
             -0.126263, -0.198413, -0.357143]
    assert np.allclose(t.numpy(), exp_t, atol=2e-3)
    assert np.allclose(d.numpy(), exp_d, atol=2e-6)
    assert math.isclose(d.sum().item(), -1.0, abs_tol=1e-6)
    tb, _ = O.build_inference_schedule(10, 5.0, torch.bfloat16)
    assert tb.float().tolist() == [1000, 980, 952, 920, 884, 832, 768, 680, 556, 358]
    t4, d4 = O.build_inference_schedule(4, 5.0)
    assert np.allclose(t4.numpy(), [1000, 937.5, 833.333, 625], atol=2e-3)
    assert np.allclose(d4.numpy(), [-0.0625, -0.104167, -0.208333, -0.625], atol=2e-6)
    _, d1 = O.build_inference_schedule(8, 1.0)
    assert np.allclose(d1.numpy(), -1.0 / 8, atol=1e-7)
    with pytest.raises(ValueError):
        O.build_inference_schedule(0, 5.0)
    x = torch.ones(2, 3)
    assert torch.equal(O.scheduler_step(torch.full((2, 3), 2.0), torch.tensor(-0.25), x), torch.full((2, 3), 0.5))


# --------------------------------------------------------------------------- goldens
@pytest.fixture(scope="module")
def golden():
    return load_file(GOLDEN)


@pytest.fixture(scope="module")
def tiny_params(golden):
    p = O.init_action_dit_params(TINY, int(golden["meta.seed"][0]), std=float(golden["meta.std"][0]))
    acc = torch.zeros((), dtype=torch.float64)
    for i, k in enumerate(sorted(p)):
        acc = acc + (i + 1) * p[k].double().sum()
    assert math.isclose(float(acc), float(golden["meta.param_checksum"][0]), rel_tol=0, abs_tol=1e-9)
    return p


def _tol(name):
    return (2e-5, 2e-5) if name == "fp32" else (3e-2, 3e-2)


@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_block(golden, tiny_params, name, dt):
    p = O.cast_params(tiny_params, dt)
    S = golden["block.in.x"].shape[1]
    cm = golden["in.context_mask"].bool().unsqueeze(1).expand(-1, S, -1)
    y = O.dit_block(p, 0, golden["block.in.x"].to(dt), golden["block.in.context"].to(dt),
                    golden["block.in.t_mod"].to(dt), O.action_freqs(TINY.attn_head_dim, S),
                    TINY.num_heads, TINY.eps, cm)
    rt, at = _tol(name)
    assert torch.allclose(y.float(), golden[f"block.out.{name}"], rtol=rt, atol=at)


@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_action_dit(golden, tiny_params, name, dt):
    p = O.cast_params(tiny_params, dt)
    y = O.action_dit_forward(p, TINY, golden["in.actions"].to(dt), golden["in.timestep"].to(dt),
                             golden["in.context"].to(dt), golden["in.context_mask"].bool())
    rt, at = _tol(name)
    assert torch.allclose(y.float(), golden[f"action_dit.out.{name}"], rtol=rt, atol=at)


@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_loop(golden, tiny_params, name, dt):
    p = O.cast_params(tiny_params, dt)
    ts, ds = O.build_inference_schedule(3, 5.0, dt)
    assert torch.equal(ts.float(), golden[f"loop.timesteps.{name}"])
    assert torch.equal(ds.float(), golden[f"loop.deltas.{name}"])
    y = O.denoise_loop(p, TINY, golden["loop.in.noise"].to(dt), golden["in.context"][:1].to(dt), 3, 5.0)
    rt, at = _tol(name)
    assert torch.allclose(y.float(), golden[f"loop.out.{name}"], rtol=rt, atol=at)


@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_mot(golden, tiny_params, name, dt):
    p = O.cast_params(tiny_params, dt)
    S = golden["mot.in.x"].shape[1]
    kv = [(golden[f"mot.in.k{i}"].to(dt), golden[f"mot.in.v{i}"].to(dt)) for i in range(TINY.num_layers)]
    Sv = kv[0][0].shape[1]
    y = O.mot_action_forward(p, TINY, golden["mot.in.x"].to(dt), O.action_freqs(TINY.attn_head_dim, S),
                             golden["mot.in.t_mod"].to(dt), golden["mot.in.context"].to(dt), kv,
                             golden["mot.in.joint_mask"].bool(), Sv)
    rt, at = _tol(name)
    assert torch.allclose(y.float(), golden[f"mot.out.{name}"], rtol=rt, atol=at)


@pytest.fixture(scope="module")
def prefill_golden():
    return load_file(os.path.join(os.path.dirname(__file__), "golden", "mot_prefill_tiny.safetensors"))


def _prefill(g, p, dt, num_run):
    fr = torch.view_as_complex(g["in.freqs_real"].double().contiguous())
    return O.mot_prefill_video_cache(p, TINY, g["in.x"].to(dt), fr, g["in.t_mod"].to(dt), g["in.context"].to(dt),
                                     g["in.video_mask"].bool(), g["in.context_mask"].bool(), num_run)


@pytest.mark.parametrize("tag,num_run", [("all", 0), ("draft1", 1)])
@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_mot_prefill(prefill_golden, tiny_params, tag, num_run, name, dt):
    """The oracle's video K/V prefill against MoT.prefill_video_cache of the reference: every
    layer's k (normalised, rotated) and v, first-frame-causal video mask, per-token t_mod,
    ragged text mask; drafted (one layer run, its K/V reused) and full."""
    g = prefill_golden
    kv = _prefill(g, O.cast_params(tiny_params, dt), dt, num_run)
    rt, at = _tol(name)
    assert len(kv) == TINY.num_layers
    for i, (k, v) in enumerate(kv):
        assert torch.allclose(k.float(), g[f"out.{tag}.{name}.k{i}"], rtol=rt, atol=at), (tag, i, "k")
        assert torch.allclose(v.float(), g[f"out.{tag}.{name}.v{i}"], rtol=rt, atol=at), (tag, i, "v")


def test_golden_mot_prefill_detects_planted_mistakes(prefill_golden, tiny_params):
    """Plausible slips fail the prefill golden: the video mask ignored (bidirectional), or the
    cached key taken before RoPE."""
    g = prefill_golden
    p = O.cast_params(tiny_params, torch.float32)
    fr = torch.view_as_complex(g["in.freqs_real"].double().contiguous())
    args = (g["in.x"], fr, g["in.t_mod"], g["in.context"])
    kv = O.mot_prefill_video_cache(p, TINY, *args, torch.ones_like(g["in.video_mask"].bool()),
                                   g["in.context_mask"].bool())
    assert not torch.allclose(kv[1][0], g["out.all.fp32.k1"], rtol=2e-5, atol=2e-5)
    no_rope = O.mot_prefill_video_cache(p, TINY, g["in.x"], torch.ones_like(fr), g["in.t_mod"], g["in.context"],
                                        g["in.video_mask"].bool(), g["in.context_mask"].bool())
    assert not torch.allclose(no_rope[0][0], g["out.all.fp32.k0"], rtol=2e-5, atol=2e-5)


def test_golden_detects_planted_mistake(golden, tiny_params):
    """A dropped term in the block (no cross-attention) must fail the golden comparison."""
    p = O.cast_params(tiny_params, torch.float32)
    for k in list(p):
        if ".cross_attn.o." in k:
            p[k] = torch.zeros_like(p[k])
    S = golden["block.in.x"].shape[1]
    cm = golden["in.context_mask"].bool().unsqueeze(1).expand(-1, S, -1)
    y = O.dit_block(p, 0, golden["block.in.x"], golden["block.in.context"], golden["block.in.t_mod"],
                    O.action_freqs(TINY.attn_head_dim, S), TINY.num_heads, TINY.eps, cm)
    assert not torch.allclose(y, golden["block.out.fp32"], rtol=2e-5, atol=2e-5)


def _swap_norm_qk(p, att):
    q = p
    for k in list(q):
        if f".{att}.norm_q." in k:
            kk = k.replace(".norm_q.", ".norm_k.")
            q[k], q[kk] = q[kk], q[k]
    return q


@pytest.mark.parametrize("slip", ["swap_self_qk", "drop_cross_norm_q", "drop_norm3_bias", "norm3_weight_of_next_layer"])
def test_golden_detects_planted_norm_affine_mistakes(golden, tiny_params, slip):
    """With non-identity norm affines in the golden run, a swapped self-attention q/k RMSNorm
    weight, a dropped cross-attention query norm weight, a dropped norm3 bias or a norm weight
    taken from the wrong layer must each fail the reference goldens.  (Swapping the
    cross-attention q/k norm weights is an exact symmetry: without RoPE the score is
    sum_d q_d w_q[d] k_d w_k[d], so no output can detect it.)"""
    p = O.cast_params(tiny_params, torch.float32)
    if slip == "swap_self_qk":
        _swap_norm_qk(p, "self_attn")
    elif slip == "drop_cross_norm_q":
        for k in list(p):
            if ".cross_attn.norm_q." in k:
                p[k] = torch.ones_like(p[k])
    elif slip == "drop_norm3_bias":
        for k in list(p):
            if k.endswith("norm3.bias"):
                p[k] = torch.zeros_like(p[k])
    else:
        p["blocks.0.norm3.weight"] = p["blocks.1.norm3.weight"].clone()
    S = golden["block.in.x"].shape[1]
    cm = golden["in.context_mask"].bool().unsqueeze(1).expand(-1, S, -1)
    y = O.dit_block(p, 0, golden["block.in.x"], golden["block.in.context"], golden["block.in.t_mod"],
                    O.action_freqs(TINY.attn_head_dim, S), TINY.num_heads, TINY.eps, cm)
    assert not torch.allclose(y, golden["block.out.fp32"], rtol=2e-5, atol=2e-5)
    y = O.action_dit_forward(p, TINY, golden["in.actions"], golden["in.timestep"], golden["in.context"],
                             golden["in.context_mask"].bool())
    assert not torch.allclose(y, golden["action_dit.out.fp32"], rtol=2e-5, atol=2e-5)


def test_golden_norm_affines_are_not_identity(tiny_params):
    """The golden weights carry non-trivial norm affines (otherwise the tests above pin nothing)."""
    for k, v in tiny_params.items():
        if ".norm_q." in k or ".norm_k." in k or k.endswith("norm3.weight"):
            assert (v - 1).abs().max() > 0.1, k
        if k.endswith("norm3.bias"):
            assert v.abs().max() > 0.1, k


# --------------------------------------------------------------------------- CAE action decoder
CAE_CASES = {"base": (16, 8, 32, 7, 128, 0, 41), "two_stage_suite": (8, 4, 32, 7, 64, 3, 42),
             "stride3_pad": (6, 3, 10, 5, 32, 0, 43)}


def _checksum(p) -> float:
    acc = torch.zeros((), dtype=torch.float64)
    for i, k in enumerate(sorted(p)):
        acc = acc + (i + 1) * p[k].double().sum()
    return float(acc)


@pytest.fixture(scope="module")
def cae_golden():
    from safetensors.torch import load_file
    return load_file(os.path.join(os.path.dirname(__file__), "golden", "cae_decoder.safetensors"))


def _cae(name):
    L, T0, hz, A, C, ns, seed = CAE_CASES[name]
    cfg = O.CaeDecoderConfig(latent_dim=L, num_tokens=T0, action_horizon=hz, action_dim=A, decoder_hidden=C)
    return cfg, O.init_cae_decoder_params(cfg, seed)


@pytest.mark.parametrize("name", sorted(CAE_CASES))
def test_cae_decoder_golden(cae_golden, name):
    """The oracle's ActionDecoder restatement against the reference module's own outputs."""
    cfg, p = _cae(name)
    assert abs(cae_golden[f"{name}.checksum"].item() - _checksum(p)) < 1e-9
    suite = cae_golden.get(f"{name}.suite_rows")
    y = O.cae_decode(p, cfg, cae_golden[f"{name}.z"], suite)
    torch.testing.assert_close(y, cae_golden[f"{name}.out"], rtol=1e-5, atol=1e-5)


def test_cae_decoder_detects_planted_mistake(cae_golden):
    cfg, p = _cae("base")
    q = dict(p)
    q["decoder.up.3.net.4.weight"] = -q["decoder.up.3.net.4.weight"]   # residual branch sign
    y = O.cae_decode(q, cfg, cae_golden["base.z"])
    assert (y - cae_golden["base.out"]).abs().max() > 1e-2
    assert O.cae_strides(4) == [4] and O.cae_strides(8) == [4, 2] and O.cae_strides(12) == [4, 3]


# --------------------------------------------------------------------------- DiT4DiT head
def test_d4d_embeddings_closed_forms():
    """The two sinusoidal embeddings of the DiT4DiT head (action_encoder.py:21-37, diffusers
    Timesteps as configured at cross_attention_dit.py:34) at closed-form points."""
    D = 768
    t = torch.tensor([0.0, 750.0])
    tau = O.d4d_tau_encoding(t, D)
    assert tau.shape == (2, D)
    assert torch.equal(tau[0, :D // 2], torch.zeros(D // 2)) and torch.equal(tau[0, D // 2:], torch.ones(D // 2))
    # first frequency is 1, last is 10000^(-(half-1)/half); (sin, cos) order
    assert math.isclose(tau[1, 0].item(), math.sin(750.0), abs_tol=1e-5)
    assert math.isclose(tau[1, D // 2].item(), math.cos(750.0), abs_tol=1e-5)
    fl = 10000.0 ** (-(D // 2 - 1) / (D // 2))
    assert math.isclose(tau[1, D // 2 - 1].item(), math.sin(750.0 * fl), abs_tol=1e-6)
    assert torch.allclose(tau[1, :D // 2] ** 2 + tau[1, D // 2:] ** 2, torch.ones(D // 2), atol=1e-6)
    pr = O.d4d_timestep_proj(torch.tensor([0, 250]), 256)
    assert pr.shape == (2, 256)
    assert torch.equal(pr[0, :128], torch.ones(128)) and torch.equal(pr[0, 128:], torch.zeros(128))
    # flip_sin_to_cos: cos first; downscale_freq_shift = 1 makes the last frequency exactly 1/10000
    assert math.isclose(pr[1, 0].item(), math.cos(250.0), abs_tol=1e-5)
    assert math.isclose(pr[1, 128].item(), math.sin(250.0), abs_tol=1e-5)
    assert math.isclose(pr[1, 127].item(), math.cos(0.025), abs_tol=1e-7)
    assert math.isclose(pr[1, 255].item(), math.sin(0.025), abs_tol=1e-7)


def test_d4d_schedule_and_block_structure():
    """Timesteps 1000, 750, 500, 250 and dt = 0.25 (the DiT4DiT 4-step schedule's known answer); interleaved
    blocks (odd = self attention); a block with zero AdaLN / attention / FFN weights is the
    identity on the residual stream, and a head whose decoder outputs zero leaves the noise."""
    cfg = O.DiT4DiTHeadConfig(num_layers=4, heads=2, head_dim=16, cross_dim=24, output_dim=40, hidden_size=40,
                              action_dim=5, horizon=6)
    assert O.d4d_timesteps(O.DiT4DiTHeadConfig()) == [1000, 750, 500, 250]
    assert [cfg.is_cross(i) for i in range(4)] == [True, False, True, False]
    p = O.init_d4d_params(cfg, 3)
    x, ctx = torch.randn(2, 6, cfg.dim), torch.randn(2, 9, cfg.cross_dim)
    temb = torch.randn(2, cfg.dim)
    z = dict(p)
    b = "model.transformer_blocks.1."
    for n in ("attn1.to_out.0.weight", "attn1.to_out.0.bias", "ff.net.2.weight", "ff.net.2.bias"):
        z[b + n] = torch.zeros_like(p[b + n])
    assert torch.equal(O.d4d_block(z, cfg, 1, x, ctx, temb), x)
    # cross blocks read the context, self blocks do not
    y1 = O.d4d_block(p, cfg, 0, x, ctx, temb)
    assert not torch.equal(y1, O.d4d_block(p, cfg, 0, x, ctx * 2, temb))
    assert torch.equal(O.d4d_block(p, cfg, 1, x, ctx, temb), O.d4d_block(p, cfg, 1, x, ctx * 2, temb))
    zd = dict(p)
    zd["action_decoder.layer2.weight"] = torch.zeros_like(p["action_decoder.layer2.weight"])
    zd["action_decoder.layer2.bias"] = torch.zeros_like(p["action_decoder.layer2.bias"])
    noise = torch.randn(2, 6, 5)
    assert torch.equal(O.d4d_predict_action(zd, cfg, ctx, noise), noise)
    # with a constant velocity c the N Euler steps move the noise by exactly -c
    zc = dict(zd)
    zc["action_decoder.layer2.bias"] = torch.full_like(p["action_decoder.layer2.bias"], 0.5)
    assert torch.allclose(O.d4d_predict_action(zc, cfg, ctx, noise), noise - 0.5, atol=1e-6)


def _d4d_tiny():
    cfg = O.DiT4DiTHeadConfig(num_layers=2, heads=2, head_dim=8, cross_dim=12, output_dim=16, hidden_size=16,
                              action_dim=5, horizon=6, state_dim=0)
    g = torch.Generator().manual_seed(41)
    x = torch.randn(2, 6, cfg.dim, generator=g, dtype=torch.float64)
    x[1, 2] = 0.3 + 1e-3 * x[1, 2]          # a row of variance ~1e-6: its LayerNorm output depends on eps
    ctx = torch.randn(2, 7, cfg.cross_dim, generator=g, dtype=torch.float64)
    temb = torch.randn(2, cfg.dim, generator=g, dtype=torch.float64)
    p = {k: v.double() for k, v in O.init_d4d_params(cfg, 42).items()}
    return cfg, g, x, ctx, temb, p


def _ln(x, eps):
    """LayerNorm without affine, written out: (x - mean) / sqrt(biased var + eps)."""
    mu = x.mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(((x - mu) ** 2).mean(-1, keepdim=True) + eps)


def test_d4d_block_adaln_closed_form():
    """AdaLayerNorm of a DiT4DiT head block (DB/.../flow_matching_head/cross_attention_dit.py:59-67:
    (scale, shift) = chunk(linear(SiLU(temb)), 2), LN without affine at eps 1e-5) through a self
    block whose attention is a plain token mean: zero to_q / to_k (a uniform softmax), identity
    to_v / to_out and a zero FFN give x + mean_tokens(LN(x)(1 + scale) + shift).  With the linear's
    weight zero its bias is the (scale, shift) pair: a swapped pair or another eps fails."""
    cfg, g, x, ctx, temb, p = _d4d_tiny()
    D, b = cfg.dim, "model.transformer_blocks.1."       # block 1: self attention (interleaved)
    assert not cfg.is_cross(1)
    I = torch.eye(D, dtype=torch.float64)
    scale, shift = torch.randn(D, generator=g, dtype=torch.float64), torch.randn(D, generator=g, dtype=torch.float64)
    q = dict(p)
    q[b + "norm1.linear.weight"] = torch.zeros(2 * D, D, dtype=torch.float64)
    q[b + "norm1.linear.bias"] = torch.cat([scale, shift])
    for n in ("to_q", "to_k"):
        q[b + f"attn1.{n}.weight"], q[b + f"attn1.{n}.bias"] = torch.zeros(D, D, dtype=torch.float64), torch.zeros(D, dtype=torch.float64)
    for n in ("to_v", "to_out.0"):
        q[b + f"attn1.{n}.weight"], q[b + f"attn1.{n}.bias"] = I.clone(), torch.zeros(D, dtype=torch.float64)
    q[b + "ff.net.2.weight"], q[b + "ff.net.2.bias"] = torch.zeros(D, 4 * D, dtype=torch.float64), torch.zeros(D, dtype=torch.float64)
    y = O.d4d_block(q, cfg, 1, x, ctx, temb)

    def expect(sc, sh, eps):
        return x + (_ln(x, eps) * (1 + sc) + sh).mean(1, keepdim=True)
    assert torch.allclose(y, expect(scale, shift, 1e-5), atol=1e-9)
    assert (y - expect(shift, scale, 1e-5)).abs().max() > 0.1          # (shift, scale) order: fails
    assert (y - expect(scale, shift, 1e-6)).abs().max() > 1e-2         # eps 1e-6: fails


def test_d4d_block_norm3_and_ffn_closed_form():
    """norm3 is a LayerNorm without affine at eps 1e-5 (cross_attention_dit.py:136, 207-208 with
    DiT's norm_elementwise_affine False) and the FeedForward is net.2(GELU_tanh(net.0.proj(h)))
    added to x: with the attention branch zero and identity-embedding FFN weights ([I; 0] up,
    [I, 0] down) a cross block gives x + GELU_tanh(LN(x)) -- independent of the AdaLN
    modulation (norm3 does not take it) and of the context."""
    cfg, g, x, ctx, temb, p = _d4d_tiny()
    D, b = cfg.dim, "model.transformer_blocks.0."
    assert cfg.is_cross(0)
    q = dict(p)
    q[b + "attn1.to_out.0.weight"], q[b + "attn1.to_out.0.bias"] = torch.zeros(D, D, dtype=torch.float64), torch.zeros(D, dtype=torch.float64)
    q[b + "ff.net.0.proj.weight"] = torch.cat([torch.eye(D, dtype=torch.float64), torch.zeros(3 * D, D, dtype=torch.float64)])
    q[b + "ff.net.0.proj.bias"] = torch.zeros(4 * D, dtype=torch.float64)
    q[b + "ff.net.2.weight"] = torch.cat([torch.eye(D, dtype=torch.float64), torch.zeros(D, 3 * D, dtype=torch.float64)], 1)
    q[b + "ff.net.2.bias"] = torch.zeros(D, dtype=torch.float64)
    y = O.d4d_block(q, cfg, 0, x, ctx, temb)

    def gelu(u):
        return 0.5 * u * (1 + torch.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
    assert torch.allclose(y, x + gelu(_ln(x, 1e-5)), atol=1e-9)
    assert (y - (x + gelu(_ln(x, 1e-6)))).abs().max() > 1e-2
    assert (y - (x + torch.nn.functional.gelu(_ln(x, 1e-5)))).abs().max() > 1e-5   # erf GELU differs
    assert torch.equal(y, O.d4d_block(q, cfg, 0, x, ctx * 3, temb * 2))


def test_d4d_output_stage_closed_form():
    """DiT.forward's output stage (cross_attention_dit.py:302-304): (shift, scale) =
    chunk(proj_out_1(SiLU(temb)), 2) -- the opposite order of the blocks' AdaLayerNorm --
    LN without affine at eps 1e-6 (norm_out, :253), then proj_out_2.  Blocks that are the
    identity (zero attention output and FFN) and an identity proj_out_2 leave
    LN_1e-6(x)(1 + scale) + shift; a swapped pair or eps 1e-5 fails."""
    cfg, g, x, ctx, temb, p = _d4d_tiny()
    D = cfg.dim
    q = dict(p)
    for i in range(cfg.num_layers):
        b = f"model.transformer_blocks.{i}."
        for n in ("attn1.to_out.0", "ff.net.2"):
            q[b + n + ".weight"] = torch.zeros_like(p[b + n + ".weight"])
            q[b + n + ".bias"] = torch.zeros_like(p[b + n + ".bias"])
    shift, scale = torch.randn(D, generator=g, dtype=torch.float64), torch.randn(D, generator=g, dtype=torch.float64)
    q["model.proj_out_1.weight"] = torch.zeros(2 * D, D, dtype=torch.float64)
    q["model.proj_out_1.bias"] = torch.cat([shift, scale])
    q["model.proj_out_2.weight"] = torch.eye(cfg.output_dim, D, dtype=torch.float64)
    q["model.proj_out_2.bias"] = torch.zeros(cfg.output_dim, dtype=torch.float64)
    y = O.d4d_dit_forward(q, cfg, x, ctx, torch.tensor([1000, 250]))
    assert torch.allclose(y, _ln(x, 1e-6) * (1 + scale) + shift, atol=1e-9)
    assert (y - (_ln(x, 1e-6) * (1 + shift) + scale)).abs().max() > 0.1
    assert (y - (_ln(x, 1e-5) * (1 + scale) + shift)).abs().max() > 1e-2


def test_d4d_action_encoder_closed_form():
    """ActionEncoder (DB/modules/action_model/ActionDiT.py:74-98): layer2 reads cat(layer1(a), tau)
    in that order, swish, layer3.  With layer2 = [0 | I] (it keeps only the tau half), layer3 = I
    and zero biases the output is swish(tau(t)) for every token, whatever the actions; with
    layer2 = [I | 0] it is swish(layer1(a)).  Reading (tau, a) instead fails both."""
    cfg, g, _, _, _, p = _d4d_tiny()
    D = cfg.dim
    acts = torch.randn(2, 6, cfg.action_dim, generator=g, dtype=torch.float64)
    t = torch.tensor([1000, 250])
    q = dict(p)
    I, Z = torch.eye(D, dtype=torch.float64), torch.zeros(D, D, dtype=torch.float64)
    q["action_encoder.layer2.bias"] = torch.zeros(D, dtype=torch.float64)
    q["action_encoder.layer3.weight"], q["action_encoder.layer3.bias"] = I.clone(), torch.zeros(D, dtype=torch.float64)
    swish = lambda u: u * torch.sigmoid(u)  # noqa: E731
    q["action_encoder.layer2.weight"] = torch.cat([Z, I], 1)
    tau = O.d4d_tau_encoding(t[:, None].expand(2, 6), D).double()
    assert torch.allclose(O.d4d_action_encoder(q, acts, t), swish(tau), atol=1e-9)
    q["action_encoder.layer2.weight"] = torch.cat([I, Z], 1)
    a = acts @ p["action_encoder.layer1.weight"].t() + p["action_encoder.layer1.bias"]
    assert torch.allclose(O.d4d_action_encoder(q, acts, t), swish(a), atol=1e-9)


# --------------------------------------------------------------------------- WanVideoDiT pre_dit / forward
WAN_TINY = O.WanVideoConfig(hidden_dim=32, in_dim=4, ffn_dim=64, out_dim=4, text_dim=24, freq_dim=16, eps=1e-6,
                            patch_size=(1, 2, 2), num_heads=2, attn_head_dim=24, num_layers=2)


@pytest.fixture(scope="module")
def wan_golden():
    return load_file(os.path.join(os.path.dirname(__file__), "golden", "wan_video_tiny.safetensors"))


@pytest.fixture(scope="module")
def wan_params(wan_golden):
    p = O.init_wan_params(WAN_TINY, int(wan_golden["meta.seed"][0]), std=float(wan_golden["meta.std"][0]))
    assert math.isclose(_checksum(p), float(wan_golden["meta.param_checksum"][0]), rel_tol=0, abs_tol=1e-9)
    return p


def _wan_in(g, dt):
    return g["in.x"].to(dt), g["in.timestep"].to(dt), g["in.context"].to(dt), g["in.context_mask"].bool()


@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_wan_pre_dit(wan_golden, wan_params, name, dt):
    """The oracle's pre_dit against WanVideoDiT.pre_dit: tokens of the patch embedding, per-token
    t and t_mod (first latent frame at timestep 0), the text embedding, the broadcast context mask
    and the 3-D RoPE table of the (f, h, w) grid."""
    g = wan_golden
    pre = O.wan_pre_dit(O.cast_params(wan_params, dt), WAN_TINY, *_wan_in(g, dt))
    rt, at = _tol(name)
    for k in ("tokens", "t", "t_mod", "context"):
        assert torch.allclose(pre[k].float(), g[f"pre.{k}.{name}"], rtol=rt, atol=at), k
    assert torch.equal(pre["context_mask"].to(torch.uint8), g["pre.context_mask"])
    assert torch.equal(torch.view_as_real(pre["freqs"].to(torch.complex128)).float(), g["pre.freqs_real"])
    assert pre["grid"] == (2, 2, 3) and pre["tokens_per_frame"] == 6


@pytest.mark.parametrize("name,dt", [("fp32", torch.float32), ("bf16", torch.bfloat16)])
def test_golden_wan_forward(wan_golden, wan_params, name, dt):
    """pre_dit -> 2 blocks under the first-frame-causal video mask -> head -> unpatchify, against
    WanVideoDiT.forward."""
    g = wan_golden
    x, t, c, cm = _wan_in(g, dt)
    S = 12
    vmask = O.mot_joint_mask(S, 0, 6)
    y = O.wan_forward(O.cast_params(wan_params, dt), WAN_TINY, x, t, c, cm, vmask)
    rt, at = _tol(name)
    assert y.shape == (2, 4, 2, 4, 6)
    assert torch.allclose(y.float(), g[f"forward.{name}"], rtol=rt, atol=at)


def test_golden_wan_detects_planted_mistakes(wan_golden, wan_params):
    """Plausible slips fail the goldens: every token at the shared timestep (the first frame's
    zero dropped), the un-patchify's channel taken slowest instead of fastest, and the head's
    shift and scale swapped."""
    g = wan_golden
    p = O.cast_params(wan_params, torch.float32)
    x, t, c, cm = _wan_in(g, torch.float32)
    pre = O.wan_pre_dit(p, WAN_TINY, x, t, c, cm)
    # (1) no first-frame zero: recompute t as if every token carried the sample's timestep
    emb = O.sinusoidal_embedding_1d(16, t.repeat_interleave(12))
    t_all = O.linear(O.silu(O.linear(emb, p["time_embedding.0.weight"], p["time_embedding.0.bias"])),
                     p["time_embedding.2.weight"], p["time_embedding.2.bias"]).reshape(2, 12, 32)
    assert not torch.allclose(t_all, g["pre.t.fp32"], rtol=2e-5, atol=2e-5)
    assert torch.allclose(pre["t"], g["pre.t.fp32"], rtol=2e-5, atol=2e-5)
    # (2) un-patchify with (c x y z) feature order
    y_tok = torch.randn(2, 12, 16, generator=torch.Generator().manual_seed(1))
    good = O.wan_unpatchify(y_tok, (2, 2, 3), (1, 2, 2), 4)
    bad = y_tok.reshape(2, 2, 2, 3, 4, 1, 2, 2).permute(0, 4, 1, 5, 2, 6, 3, 7).reshape(2, 4, 2, 4, 6)
    assert not torch.equal(good, bad)
    # (3) head shift / scale swapped
    m = p["head.modulation"]
    p2 = dict(p)
    p2["head.modulation"] = m.flip(1).contiguous()
    vmask = O.mot_joint_mask(12, 0, 6)
    y = O.wan_forward(p2, WAN_TINY, x, t, c, cm, vmask)
    assert not torch.allclose(y, g["forward.fp32"], rtol=2e-5, atol=2e-5)


# --------------------------------------------------------------------------- Wan2.2 VAE encoder
VAE_TINY = O.WanVaeConfig(dim=16, z_dim=8)


@pytest.fixture(scope="module")
def vae_golden():
    return load_file(os.path.join(os.path.dirname(__file__), "golden", "wan_vae_tiny.safetensors"))


@pytest.fixture(scope="module")
def vae_params(vae_golden):
    p = O.init_wan_vae_params(VAE_TINY, int(vae_golden["meta.seed"][0]))
    assert math.isclose(_checksum(p), float(vae_golden["meta.param_checksum"][0]), rel_tol=0, abs_tol=1e-9)
    return p


def _vae(g, p, name, **kw):
    return O.wan_vae_encode_first_frame(p, VAE_TINY, g[f"in.image.{name}"], g["in.mean"], g["in.std"], **kw)


@pytest.mark.parametrize("name", ["a", "b"])
def test_golden_wan_vae_encode_first_frame(vae_golden, vae_params, name):
    """The oracle's first-frame encode against VideoVAE38_.encode (64 x 128 and 48 x 80 images)."""
    y = _vae(vae_golden, vae_params, name)
    ref = vae_golden[f"out.mu.{name}"]
    assert y.shape == ref.shape
    assert torch.allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_golden_wan_vae_detects_planted_mistakes(vae_golden, vae_params, monkeypatch):
    """Plausible slips fail the goldens: the patchify's sub-pixel order transposed (c q r instead
    of c r q), the AvgDown3D shortcut without its zero frame, the two RMS_norm gammas of a
    residual block swapped, and the attention's k and q swapped."""
    g, p = vae_golden, vae_params
    ref = g["out.mu.a"]
    close = lambda y: torch.allclose(y, ref, rtol=1e-4, atol=1e-4)   # noqa: E731
    assert close(_vae(g, p, "a"))

    def patch_cqr(x, patch=2):
        b, c, h, w = x.shape
        x = x.reshape(b, c, h // patch, patch, w // patch, patch)
        return x.permute(0, 1, 3, 5, 2, 4).reshape(b, c * patch * patch, h // patch, w // patch)
    with monkeypatch.context() as m:
        m.setattr(O, "vae_patchify", patch_cqr)
        assert not close(_vae(g, p, "a"))

    real_avg = O.vae_avg_down

    def avg_no_zero_frame(x, out_channels, factor_t, factor_s):
        return real_avg(x, out_channels, 1, factor_s) if factor_t == 1 else \
            real_avg(torch.cat([x, x], 1), out_channels, 1, factor_s)
    with monkeypatch.context() as m:
        m.setattr(O, "vae_avg_down", avg_no_zero_frame)
        assert not close(_vae(g, p, "a"))

    p2 = dict(p)
    pre = "encoder.downsamples.0.downsamples.1."
    p2[pre + "residual.0.gamma"], p2[pre + "residual.3.gamma"] = p[pre + "residual.3.gamma"], p[pre + "residual.0.gamma"]
    assert not close(_vae(g, p2, "a"))

    real_att = O.attention

    def att_kq(q, k, v, mask=None, scale=None):
        return real_att(k, q, v, mask, scale)
    with monkeypatch.context() as m:
        m.setattr(O, "attention", att_kq)
        assert not close(_vae(g, p, "a"))


def test_wan_vae_avg_down_closed_forms():
    """AvgDown3D on one frame: factor_t 1 / factor_s 2 with out = in channels is a 2x2 average
    pool; factor_t 2 doubles the channels, even outputs averaging the zero frame (0), odd
    outputs the 2x2 pool of channel o // 2; factor 1 is the identity."""
    x = torch.randn(1, 6, 4, 8, generator=torch.Generator().manual_seed(3))
    pool = F.avg_pool2d(x, 2)
    assert torch.allclose(O.vae_avg_down(x, 6, 1, 2), pool, atol=1e-6)
    y = O.vae_avg_down(x, 12, 2, 2)
    assert torch.equal(y[:, 0::2], torch.zeros_like(y[:, 0::2]))
    assert torch.allclose(y[:, 1::2], pool, atol=1e-6)
    assert torch.equal(O.vae_avg_down(x, 6, 1, 1), x)


# --------------------------------------------------------------------------- branch metrics' power
def test_block_branch_metrics_catch_planted_slips(monkeypatch):
    """The config-2 block test (tests/test_configs_gpu.py::test_config2_video_block_full_shape, same
    seeds and shape: 1560 tokens on a 2 x 30 x 26 grid, hidden 3072, 24 x 128 heads, FFN 14336,
    512 text tokens) asserts its branch metrics at 2e-2.  Each slip planted here in the oracle moves
    at least one of them past that bar, while the block's output alone moves less than the bar for
    the first two (measured 1.8e-2 and 2.0e-2): RoPE dropped, the (h, w) grid of the 3-D table
    transposed, the self-attention zeroed, and V read one head off (a mis-strided head)."""
    from block_checks import BAR, rel, trace_errors
    f, hh, ww = 2, 30, 26
    S, H, nh, Dh, F_, Lc = f * hh * ww, 3072, 24, 128, 14336, 512
    ocfg = O.ActionDiTConfig(hidden_dim=H, action_dim=7, ffn_dim=F_, text_dim=H, freq_dim=256, num_heads=nh,
                             attn_head_dim=Dh, num_layers=1)
    p = {k: v.to(torch.bfloat16).float() for k, v in O.init_action_dit_params(ocfg, 103).items()}
    g = torch.Generator().manual_seed(104)
    x = torch.randn(1, S, H, generator=g).to(torch.bfloat16).float()
    ctx = torch.randn(1, Lc, H, generator=g).to(torch.bfloat16).float()
    tm = (torch.randn(1, S, 6, H, generator=g) * 0.2).to(torch.bfloat16).float()
    tab = O.precompute_freqs_cis_3d(Dh)
    freqs = O.video_freqs(tab, f, hh, ww)
    tr = {}
    ref = O.dit_block(p, 0, x, ctx, tm, freqs, nh, 1e-6, trace=tr)

    def planted(params=p, fr=freqs):
        t = {}
        y = O.dit_block(params, 0, x, ctx, tm, fr, nh, 1e-6, trace=t)
        return trace_errors(t, tr, x, y, ref), rel(y, ref)

    zeroed = dict(p)
    for n in ("o.weight", "o.bias"):
        zeroed["blocks.0.self_attn." + n] = torch.zeros_like(p["blocks.0.self_attn." + n])
    cases = {"rope dropped": planted(fr=torch.ones_like(freqs)),
             "(h, w) transposed": planted(fr=O.video_freqs(tab, f, ww, hh)),
             "self-attention zeroed": planted(params=zeroed)}
    attn = O.flash_attention
    monkeypatch.setattr(O, "flash_attention",
                        lambda q, k, v, n, mask=None: attn(q, k, v.roll(v.shape[-1] // n, dims=-1), n, mask))
    cases["V one head off"] = planted()
    monkeypatch.undo()
    for name, (errs, out_err) in cases.items():
        print(f"{name}: output {out_err:.3e}, " + ", ".join(f"{k} {v:.3e}" for k, v in errs.items()))
        assert max(errs.values()) > BAR, (name, errs)
    assert cases["rope dropped"][1] < BAR and cases["(h, w) transposed"][1] < BAR
    assert cases["rope dropped"][0]["self_attn"] > 10 * BAR and cases["(h, w) transposed"][0]["self_attn"] > 10 * BAR
    assert cases["self-attention zeroed"][0]["delta"] > BAR


# --------------------------------------------------------------------------- Cosmos backbone (config 4)
def test_cosmos_rope_table_closed_form():
    """CosmosRotaryPosEmbed (CP = src/dit4dit-geak/patches/diffusers-3996788-transformer_cosmos-geak.patch
    :1953-1976): head dims 128 split 44 / 42 / 42 over (t, h, w); angle of dim j of the t part =
    t_pos * theta_t^(-2j/44) with theta_t = 1e4 * s_t^(44/42) (NTK), likewise h and w; the second
    half repeats the first; temporal positions scale by base_fps / fps."""
    cfg = O.CosmosConfig()
    T, H, W = 3, 5, 7
    cos, sin = O.cosmos_rope_tables(cfg, T, H, W)
    assert cos.shape == (T * H * W, 128) and cos.dtype == torch.float32
    assert torch.equal(cos[:, :64], cos[:, 64:]) and torch.equal(sin[:, :64], sin[:, 64:])

    def angle(pos, j, dim, s):
        theta = 1e4 * s ** (dim / (dim - 2))
        return pos * theta ** (-2.0 * j / dim)
    st, sh, sw = cfg.rope_scale
    for (ti, hi, wi) in [(0, 0, 0), (2, 4, 6), (1, 3, 0)]:
        r = (ti * H + hi) * W + wi
        want = [angle(ti, j, 44, st) for j in range(22)] + [angle(hi, j, 42, sh) for j in range(21)] + \
               [angle(wi, j, 42, sw) for j in range(21)]
        got = torch.atan2(sin[r, :64].double(), cos[r, :64].double())
        want = torch.tensor(want, dtype=torch.float64)
        assert torch.allclose(torch.cos(got - want), torch.ones(64, dtype=torch.float64), atol=1e-6), (ti, hi, wi)
    c2, s2 = O.cosmos_rope_tables(cfg, T, H, W, fps=12.0)       # t positions doubled (24 / 12)
    r = (2 * H + 0) * W + 0
    assert math.isclose(math.atan2(s2[r, 1].item(), c2[r, 1].item()), angle(4, 1, 44, st), abs_tol=1e-5)


def test_cosmos_rope_and_head_norm_closed_forms():
    """apply_rotary_emb(use_real=True, use_real_unbind_dim=-2) rotates the pairs (d, d + D/2) of each
    head: a 2x2 rotation brute force, pair norms kept; the per-head RMSNorm gives every head unit
    RMS (weight ones) and one head's scale does not reach the others."""
    g = torch.Generator().manual_seed(5)
    B, S, nh, D = 1, 6, 3, 16
    x = torch.randn(B, S, nh * D, generator=g, dtype=torch.float64)
    ang = torch.rand(S, D // 2, generator=g, dtype=torch.float64) * 6
    cos, sin = torch.cat([ang.cos()] * 2, -1), torch.cat([ang.sin()] * 2, -1)
    y = O.cosmos_apply_rope(x, cos, sin, nh)
    xh, yh = x.reshape(S, nh, D), y.reshape(S, nh, D)
    for s_ in range(S):
        for hh in range(nh):
            for d in range(D // 2):
                c, s = ang[s_, d].cos(), ang[s_, d].sin()
                a, b = xh[s_, hh, d], xh[s_, hh, d + D // 2]
                assert torch.allclose(yh[s_, hh, d], a * c - b * s) and torch.allclose(yh[s_, hh, d + D // 2], b * c + a * s)
    assert torch.allclose(xh[..., :D // 2] ** 2 + xh[..., D // 2:] ** 2, yh[..., :D // 2] ** 2 + yh[..., D // 2:] ** 2)
    n = O.cosmos_head_rms_norm(x, torch.ones(D, dtype=torch.float64), nh, 1e-12).reshape(S, nh, D)
    assert torch.allclose(n.pow(2).mean(-1), torch.ones(S, nh, dtype=torch.float64))
    x2 = x.clone().reshape(S, nh, D)
    x2[:, 1] *= 7.0
    n2 = O.cosmos_head_rms_norm(x2.reshape(B, S, nh * D), torch.ones(D, dtype=torch.float64), nh, 1e-12).reshape(S, nh, D)
    assert torch.allclose(n2, n)


def _cosmos_tiny():
    cfg = O.CosmosConfig(hidden=32, num_heads=2, head_dim=16, num_layers=1, in_channels=4, text_dim=12,
                         adaln_lora_dim=8)
    p = {k: v.double() for k, v in O.init_cosmos_params(cfg, 61).items()}
    g = torch.Generator().manual_seed(62)
    S, C = 6, cfg.hidden
    x = torch.randn(1, S, C, generator=g, dtype=torch.float64)
    ctx = torch.randn(1, 5, cfg.text_dim, generator=g, dtype=torch.float64)
    et = torch.randn(1, S, C, generator=g, dtype=torch.float64)
    temb = torch.randn(1, S, 3 * C, generator=g, dtype=torch.float64)
    cos, sin = O.cosmos_rope_tables(cfg, 1, 2, 3)
    return cfg, p, g, x, ctx, et, temb, cos.double(), sin.double()


def _zero(p, *names):
    q = dict(p)
    for n in names:
        q[n] = torch.zeros_like(p[n])
    return q


def test_cosmos_block_self_attention_subblock_closed_form():
    """The first sub-block of a Cosmos block (CP:1851-1879): with the LoRA up-projection of norm1 zero
    its modulation is temb, chunked (shift, scale, gate); zero to_q / to_k make the softmax uniform
    (the per-head RMSNorm of zero is zero), identity to_v / to_out leave the token mean, and zero
    output projections of the other two sub-blocks make them the identity:
    y = x + gate * mean_tokens(LN_1e-6(x) (1 + scale) + shift).  Another chunk order fails."""
    cfg, p, g, x, ctx, et, temb, cos, sin = _cosmos_tiny()
    C, b = cfg.hidden, "transformer_blocks.0."
    q = _zero(p, b + "norm1.linear_2.weight", b + "attn1.to_q.weight", b + "attn1.to_k.weight",
              b + "attn2.to_out.0.weight", b + "ff.net.2.weight")
    q[b + "attn1.to_v.weight"] = torch.eye(C, dtype=torch.float64)
    q[b + "attn1.to_out.0.weight"] = torch.eye(C, dtype=torch.float64)
    y = O.cosmos_block(q, cfg, 0, x, ctx, et, temb, cos, sin)
    c0, c1, c2 = temb[..., :C], temb[..., C:2 * C], temb[..., 2 * C:]

    def expect(shift, scale, gate):
        h = _ln(x, 1e-6) * (1 + scale) + shift
        return x + gate * h.mean(1, keepdim=True)
    assert torch.allclose(y, expect(c0, c1, c2), atol=1e-9)
    for order in [(c1, c0, c2), (c0, c2, c1), (c2, c1, c0)]:
        assert (y - expect(*order)).abs().max() > 0.1


def test_cosmos_block_ffn_subblock_and_lora_closed_form():
    """The FFN sub-block: x + gate3 * net.2(GELU_erf(net.0.proj(LN(x) (1 + scale3) + shift3))) with
    identity-embedding FFN weights and both attention outputs zero; the modulation is the LoRA
    linear_2(linear_1(SiLU(e))) + temb (CP:2091): with linear_1 = [I 0] and linear_2 = [I; 0]-like
    embeddings, the shift picks up SiLU(e)."""
    cfg, p, g, x, ctx, et, temb, cos, sin = _cosmos_tiny()
    C, L, b = cfg.hidden, cfg.adaln_lora_dim, "transformer_blocks.0."
    q = _zero(p, b + "attn1.to_out.0.weight", b + "attn2.to_out.0.weight")
    q[b + "ff.net.0.proj.weight"] = torch.cat([torch.eye(C, dtype=torch.float64),
                                               torch.zeros(3 * C, C, dtype=torch.float64)])
    q[b + "ff.net.2.weight"] = torch.cat([torch.eye(C, dtype=torch.float64),
                                          torch.zeros(C, 3 * C, dtype=torch.float64)], 1)
    l1 = torch.zeros(L, C, dtype=torch.float64)
    l1[:, :L] = torch.eye(L, dtype=torch.float64)            # the first L channels of SiLU(e)
    l2 = torch.zeros(3 * C, L, dtype=torch.float64)
    l2[:L, :] = torch.eye(L, dtype=torch.float64)            # into the first L channels of the shift
    q[b + "norm3.linear_1.weight"], q[b + "norm3.linear_2.weight"] = l1, l2
    y = O.cosmos_block(q, cfg, 0, x, ctx, et, temb, cos, sin)
    silu_e = et * torch.sigmoid(et)
    shift = temb[..., :C].clone()
    shift[..., :L] += silu_e[..., :L]
    scale, gate = temb[..., C:2 * C], temb[..., 2 * C:]
    h = _ln(x, 1e-6) * (1 + scale) + shift
    gelu = 0.5 * h * (1 + torch.erf(h / math.sqrt(2)))
    assert torch.allclose(y, x + gate * gelu, atol=1e-9)
    tanh_gelu = 0.5 * h * (1 + torch.tanh(math.sqrt(2 / math.pi) * (h + 0.044715 * h ** 3)))
    assert (y - (x + gate * tanh_gelu)).abs().max() > 1e-5
    shift_nosilu = temb[..., :C].clone()
    shift_nosilu[..., :L] += et[..., :L]
    h2 = _ln(x, 1e-6) * (1 + scale) + shift_nosilu
    assert (y - (x + gate * 0.5 * h2 * (1 + torch.erf(h2 / math.sqrt(2))))).abs().max() > 1e-3


def test_cosmos_time_embedding_closed_form():
    """CosmosEmbedding's Timesteps(C, flip_sin_to_cos=True, downscale_freq_shift=0): cat(cos, sin) with
    f_i = 10000^(-i / (C/2)) (shift 0: the last frequency is 10000^(-(C/2 - 1)/(C/2)), unlike the DiT4DiT
    head's shift 1); t = 0 gives (1, 0); embedded_timestep = RMSNorm(proj) has unit RMS with weight 1."""
    C = 64
    pr = O.cosmos_timestep_proj(torch.tensor([0.0, 500.0]), C)
    assert torch.equal(pr[0, :32], torch.ones(32)) and torch.equal(pr[0, 32:], torch.zeros(32))
    f_last = 10000.0 ** (-(31 / 32))
    assert math.isclose(pr[1, 31].item(), math.cos(500.0 * f_last), abs_tol=1e-5)
    assert math.isclose(pr[1, 63].item(), math.sin(500.0 * f_last), abs_tol=1e-5)
    assert math.isclose(pr[1, 1].item(), math.cos(500.0 * 10000.0 ** (-1 / 32)), abs_tol=1e-4)
    cfg = O.CosmosConfig(hidden=C, num_heads=2, head_dim=32, num_layers=1)
    p = {"time_embed.t_embedder.linear_1.weight": torch.randn(C, C), "time_embed.t_embedder.linear_2.weight":
         torch.randn(3 * C, C), "time_embed.norm.weight": torch.ones(C)}
    temb, et = O.cosmos_time_embed(p, cfg, torch.tensor([0.0, 500.0]))
    assert temb.shape == (2, 3 * C) and torch.allclose(et.pow(2).mean(-1), torch.ones(2), atol=1e-5)


def test_geak_operator_restatements_pinned():
    """The GEAK trees' fused operators in the oracle reduce to the pinned primitives: the prefill's
    residual + LayerNorm / AdaLN (F.layer_norm, adaln), the CAE q/k post-processing (RMSNorm then
    rope_apply with the interleaved table as a complex one), the CAE cross attention with its
    whole-row query norm (attention), the context-key norm, the FFN and the time MLP (the
    golden-pinned ffn / time_mlp); a planted slip in each fails."""
    g = torch.Generator().manual_seed(77)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    S, N, eps = 5, 48, 1e-6
    x, o1, o2, gate, w, b, sh, sc = r(S, N), r(S, N), r(S, N), r(S, N), r(N), r(N), r(S, N), r(S, N)
    t, y = O.geak_res_ln(x, [o1], gate, eps, ln=(w, b))
    assert torch.allclose(y, F.layer_norm(x + gate * o1, (N,), w, b, eps))
    t2, y2 = O.geak_res_ln(x, [o1, o2], gate, eps, ada=(sh, sc))
    assert torch.allclose(t2, x + gate * o1 + o2) and torch.allclose(y2, O.adaln(t2, sh, sc, eps))
    assert (O.geak_res_ln(x, [o1, o2 * gate], gate, eps, ada=(sh, sc))[1] - y2).abs().max() > 1e-2  # gate on o2
    # CAE q/k post-processing
    H, hd, M = 3, 16, 6
    D = H * hd
    qkv, qw, kw = r(M, 3 * D), r(D), r(D)
    ang = torch.arange(M, dtype=torch.float64)[:, None] * (10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    inter = torch.stack([ang.cos(), ang.sin()], -1).reshape(M, hd)            # cos at 2p, sin at 2p + 1
    q, k, v = O.cae_qkv_post(qkv, qw, kw, inter, H, eps)
    fc = torch.polar(torch.ones_like(ang), ang).reshape(M, 1, hd // 2)

    def rms(u, wt):
        return u * torch.rsqrt((u * u).mean(-1, keepdim=True) + eps) * wt
    qref = O.rope_apply(rms(qkv[:, :D], qw)[None], fc, H)[0].reshape(M, H, hd).transpose(0, 1)
    kref = O.rope_apply(rms(qkv[:, D:2 * D], kw)[None], fc, H)[0].reshape(M, H, hd).transpose(0, 1)
    assert torch.allclose(q, qref) and torch.allclose(k, kref)
    assert torch.equal(v, qkv[:, 2 * D:].reshape(M, H, hd).transpose(0, 1))
    swapped = torch.stack([ang.sin(), ang.cos()], -1).reshape(M, hd)
    assert (O.cae_qkv_post(qkv, qw, kw, swapped, H, eps)[0] - qref).abs().max() > 1e-2
    # CAE cross attention, whole-row query RMSNorm
    Nk = 7
    qr, kc, vc = r(M, D), r(Nk, D), r(Nk, D)
    keep = torch.rand(M, Nk, generator=g) > 0.3
    keep[:, 0] = True
    ox = O.cae_xattn_qn(qr, qw, kc, vc, keep, H, eps)
    assert torch.allclose(ox, O.attention(rms(qr, qw).reshape(M, H, hd).transpose(0, 1)[None],
                                          kc.reshape(Nk, H, hd).transpose(0, 1)[None],
                                          vc.reshape(Nk, H, hd).transpose(0, 1)[None], keep[None, None])[0]
                          .transpose(0, 1).reshape(M, D))
    per_head = torch.cat([rms(qr[:, i * hd:(i + 1) * hd], qw[i * hd:(i + 1) * hd]) for i in range(H)], 1)
    assert (O.flash_attention(per_head[None], kc[None], vc[None], H, keep[None, None])[0] - ox).abs().max() > 1e-2
    # context keys of every layer
    nl, ahd = 3, 16
    gk, nkw = r(S, 2 * nl * ahd), r(nl, ahd)
    kn = O.cae_ctx_kv_norm(gk, nkw, nl, ahd, eps)
    for l in range(nl):
        assert torch.allclose(kn[l], rms(gk[:, l * ahd:(l + 1) * ahd], nkw[l]))
    assert (rms(gk[:, (nl + 1) * ahd:(nl + 2) * ahd], nkw[1]) - kn[1]).abs().max() > 1e-2   # a V slice
    # FFN and time MLP (golden-pinned ffn / time_mlp)
    cfg = O.ActionDiTConfig(hidden_dim=32, action_dim=16, ffn_dim=64, text_dim=24, freq_dim=32, num_heads=2,
                            attn_head_dim=16, num_layers=1)
    p = {k_: v_.double() for k_, v_ in O.init_action_dit_params(cfg, 5, std=0.2).items()}
    xa = r(1, 8, 32)
    assert torch.allclose(O.cae_ffn(xa, p["blocks.0.ffn.0.weight"], p["blocks.0.ffn.0.bias"], p["blocks.0.ffn.2.weight"],
                                    p["blocks.0.ffn.2.bias"]), O.ffn(p, "blocks.0.", xa))
    ts = torch.tensor([640.0], dtype=torch.float64)
    atok = r(1, 8, 16)
    tt, tm, tk = O.cae_adit_tmod(ts, p["time_embedding.0.weight"], p["time_embedding.0.bias"],
                                 p["time_embedding.2.weight"], p["time_embedding.2.bias"],
                                 p["time_projection.1.weight"], p["time_projection.1.bias"], atok,
                                 p["action_encoder.weight"], p["action_encoder.bias"])
    t_ref, tm_ref = O.time_mlp(p, cfg, ts)
    assert torch.allclose(tt, t_ref) and torch.allclose(tm, tm_ref.reshape(1, -1))
    assert torch.allclose(tk, O.linear(atok, p["action_encoder.weight"], p["action_encoder.bias"]))


def test_geak_split_combine_and_qcomb_pinned():
    """The prefill's split-K combine: planes holding the K-chunks of a product sum (first sk in
    plane order) to the whole matmul plus bias, rounded to bf16 once; planes past sk are not read.
    qcomb's output has unit RMS before the weight.  Dropping a plane, the bias, or rounding before
    the weight each fails."""
    g = torch.Generator().manual_seed(78)
    M, K, N, sk, eps = 6, 64, 40, 4, 1e-6
    x, w = torch.randn(M, K, generator=g), torch.randn(N, K, generator=g)
    bias = torch.randn(N, generator=g)
    planes = torch.full((8, M, N), 1e3)            # planes past sk carry garbage
    for i in range(sk):
        c = slice(i * K // sk, (i + 1) * K // sk)
        planes[i] = x[:, c] @ w[:, c].T
    y = O.geak_split_combine(planes, bias, sk)
    want = (x.double() @ w.double().T + bias.double()).float()
    assert ((y - want).abs() <= 2 ** -7 * want.abs() + 1e-4).all()              # one bf16 rounding
    assert torch.equal(y, y.to(torch.bfloat16).float())
    assert (O.geak_split_combine(planes, bias, sk - 1) - want).abs().max() > 1.0   # a plane dropped
    assert (O.geak_split_combine(planes, bias * 0, sk) - want).abs().max() > 0.5   # the bias dropped
    with pytest.raises(ValueError):
        O.geak_split_combine(planes, bias, 9)
    wq = 1 + 0.3 * torch.randn(N, generator=g)
    q = O.geak_qcomb(planes, bias, wq, eps, sk)
    unit = q / wq
    assert torch.allclose(unit.pow(2).mean(-1), torch.ones(M), atol=1e-4)
    assert torch.allclose(unit * y.pow(2).mean(-1, keepdim=True).add(eps).sqrt(), y, rtol=1e-4, atol=1e-4)
    assert (O.rms_norm(y.to(torch.bfloat16), wq, eps).float() - q).abs().max() > 0  # eager order rounds first


def test_cae_fused_operator_restatements_pinned():
    """The CAE tree's fused operators in the oracle against library routines and closed forms:
    mod_n3q's gate is chunk 2 (a zero gate leaves the residual, a unit gate adds so), its norm is
    F.layer_norm with the affine, the whole-row query norm leaves unit RMS and its sum of squares
    equals the Gram form the reference reads; attn_oproj per head through
    F.scaled_dot_product_attention and F.linear; ffn_fold's gate is chunk 5 (zero gate: xn = x +
    oacc) and its next-block input is adaln of xn; mask_bias's planes reproduce the keep mask under
    a softmax; the fp8 rows dequantise to within e4m3's step and put the row's largest entry at 448."""
    g = torch.Generator().manual_seed(79)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    M, D, N, eps = 5, 32, 48, 1e-6
    res, so, lnw, lnb, qw, qb, qnw = bf(r(M, D)), bf(r(M, D)), bf(1 + 0.2 * r(D)), bf(0.2 * r(D)), bf(r(N, D) / 6), \
        bf(0.1 * r(N)), bf(1 + 0.2 * r(N))
    mod, tmod = bf(r(6 * D)), bf(r(6 * D))
    z = mod.clone()
    z[2 * D:3 * D] = 0
    x0, _ = O.cae_mod_n3q(res, so, z, torch.zeros(6 * D), lnw, lnb, qw, qb, eps)
    assert torch.equal(x0, res)
    z[2 * D:3 * D] = 1
    x1, cq1 = O.cae_mod_n3q(res, so, z, torch.zeros(6 * D), lnw, lnb, qw, qb, eps)
    assert torch.equal(x1, bf(res + so))
    assert torch.allclose(cq1, F.linear(F.layer_norm(x1, (D,), lnw, lnb, eps), qw, qb), atol=0.05, rtol=0.02)
    assert (O.cae_mod_n3q(res, so, mod, tmod, lnw, lnb, qw, qb, eps)[0] - x1).abs().max() > 0.1
    n = bf(F.layer_norm(x1, (D,), lnw, lnb, eps))
    raw = F.linear(n, qw, qb)
    gram_ss = ((n @ (qw.T @ qw)) * n).sum(-1) + 2 * (n * (qw.T @ qb)).sum(-1) + (qb * qb).sum()
    assert torch.allclose(gram_ss, (raw * raw).sum(-1), rtol=1e-4)
    _, cqn = O.cae_mod_n3q(res, so, z, torch.zeros(6 * D), lnw, lnb, qw, qb, eps, qn=(qnw, eps))
    assert torch.allclose((cqn / qnw).pow(2).mean(-1), torch.ones(M), atol=2e-2)
    # attention + o-projection, head-major operands
    H, hd, SK = 3, 16, 7
    q, k, v = r(H, M, hd), r(H, SK, hd), r(H, SK, hd)
    keep = torch.rand(M, SK, generator=g) > 0.3
    keep[:, 0] = True
    wo, bo = r(20, H * hd) / 7, r(20)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=keep[None]).transpose(0, 1).reshape(M, H * hd)
    assert torch.allclose(O.cae_attn_oproj(q, k, v, keep, wo, bo), F.linear(bf(ref), wo, bo), atol=1e-4)
    assert (O.cae_attn_oproj(q, k.transpose(1, 2).reshape(H, SK, hd), v, keep, wo, bo)
            - F.linear(bf(ref), wo, bo)).abs().max() > 1e-2
    # FFN fold
    x, oacc = bf(r(M, D)), r(M, D)
    w1, b1, w2, b2 = bf(r(64, D) / 6), bf(0.1 * r(64)), bf(r(D, 64) / 8), bf(0.1 * r(D))
    modc, modn = mod.clone(), bf(r(6 * D))
    modc[5 * D:] = 0
    t0 = tmod.clone()
    t0[5 * D:] = 0
    xn, nxt = O.cae_ffn_fold(x, oacc, modc, modn, t0, w1, b1, w2, b2, eps, eps)
    assert torch.equal(xn, x + oacc)
    assert torch.allclose(nxt, O.adaln(xn, modn[:D] + t0[:D], modn[D:2 * D] + t0[D:2 * D], eps), atol=1e-6)
    xf, _ = O.cae_ffn_fold(x, oacc, mod, modn, tmod, w1, b1, w2, b2, eps, eps)
    a = O.adaln(x + oacc, mod[3 * D:4 * D] + tmod[3 * D:4 * D], mod[4 * D:5 * D] + tmod[4 * D:5 * D], eps)
    assert torch.allclose(xf, x + oacc + (mod[5 * D:] + tmod[5 * D:]) * O.cae_ffn(a, w1, b1, w2, b2),
                          atol=0.05, rtol=0.02)
    # mask bias planes
    am = torch.rand(M, SK, generator=g) > 0.4
    am[:, 1] = True
    cm = torch.rand(1, 9, generator=g) > 0.5
    cm[0, 0] = True
    sb, xb = O.cae_mask_bias(am, cm, 8, 16, 12)
    assert sb.shape == (8, 16) and xb.shape == (8, 12)
    p = torch.softmax(r(8, 16) + sb, -1)
    assert torch.equal(p[:M, :SK] > 0, am) and (p[:M, SK:] == 0).all() and torch.equal(p[M:, 0], torch.ones(3))
    assert torch.equal(xb[:M, :9] == 0, cm.expand(M, 9)) and torch.isinf(xb[M:]).all() and torch.isinf(xb[:, 9:]).all()
    # fp8 rows
    y = r(6, 64) * torch.logspace(-3, 2, 6)[:, None]
    qy, s = O.vfp8_row_q8(y)
    deq = qy.float() * s
    assert torch.equal(qy.float().abs().amax(-1), torch.full((6,), 448.0))
    mul = (448.0 / y.abs().amax(-1, keepdim=True).double()).float()   # the correctly rounded fp32 quotient
    assert torch.equal(qy.float(), (y * mul).to(torch.float8_e4m3fn).float())
    assert ((deq - y).abs() <= (y.abs() * 2 ** -4 + s * 2 ** -9) * 1.0001).all()
    assert torch.equal(O.vfp8_gelu_q8(y)[0].float(), O.vfp8_quantize_rows(bf(O.gelu_tanh(y)))[0].float())
    sh, sc = bf(0.3 * r(64)), bf(0.3 * r(64))
    ql, sl = O.vfp8_ln_mod_q8(y, sh, sc, eps)
    want = O.adaln(y, sh, sc, eps)
    assert ((ql.float() * sl - want).abs() <= want.abs() * 0.07 + 0.05).all()
    y2 = bf(r(6, 64))
    xo, qa, sa = O.vfp8_add_ln_mod_q8(bf(y), y2, sh, sc, eps)
    assert torch.equal(xo, bf(bf(y) + y2))
    want = O.adaln(xo, sh, sc, eps)
    assert ((qa.float() * sa - want).abs() <= want.abs() * 0.07 + 0.05).all()

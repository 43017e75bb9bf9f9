"""CPU oracle for the FastWAM / DiT4DiT action-DiT denoising hot path.

TEST INFRASTRUCTURE ONLY.  This module restates, in plain PyTorch running on the
CPU, the arithmetic of the reference's eager path so that the HIP kernels can be
checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or as
the timed CPU baseline -- never as a substitute for the HIP library.

Every function names the reference file:line whose behaviour it restates.  Paths
are relative to the reference checkout:

    FB  = src/fastwam-baseline/fastwam/models/wan22
    FG  = src/fastwam-geak/fastwam/models/wan22
    CA  = src/cae-fastwam/fastwam/models/wan22
    SCH = FB/schedulers/scheduler_continuous.py

Functions operate in the dtype of their inputs, exactly like the reference's eager
modules: passing bfloat16 tensors reproduces the rounding points of the reference's
bf16 inference path (every torch op rounds its result to bf16), passing float32
gives the fp32 oracle the kernels are held to.  Attention and the RoPE rotation
compute internally in fp32 / fp64 as the reference does.

Pinning (what checks each function, see ``tests/test_oracle.py``):
  sinusoidal_embedding_1d   closed forms (pos 0, first/last frequency, unit pairs) + goldens
  precompute_freqs_cis(_3d) closed-form angles, |z| = 1, 3-D split sizes, goldens
  rope_apply                identity at pos 0, norm preservation, inverse rotation,
                            2x2 rotation-matrix brute force, goldens
  rms_norm / layer_norm     unit RMS / zero-mean-unit-var, scale invariance,
                            torch.nn.functional.layer_norm, goldens
  attention                 brute-force fp64 loops, F.scaled_dot_product_attention,
                            Sk=1 => v, key permutation invariance, masked keys
  build_inference_schedule  known answers (shift 5, N=10 / N=4; shift 1), sum(delta) = -1
  dit_block / action_dit_forward / denoise_loop
                            golden vectors written by tests/golden/make_golden.py from
                            the reference modules themselves (tiny seeded configs)
  mot_action_forward        golden vectors from the reference MoT (tiny seeded config)
  wan_vae_encode_first_frame golden vectors from the reference VideoVAE38_.encode (tiny seeded
                            config, two image sizes) + planted slips; vae_avg_down closed forms
  geak_res_ln / cae_*       against the pinned primitives they compose (layer_norm, attention,
                            rope_apply, time_mlp, ffn) with planted slips
  geak_split_combine / geak_qcomb
                            K-chunk planes of a product sum to the whole product (a matmul
                            closed form), sk-plane truncation, one bf16 rounding; qcomb against
                            unit RMS before the weight, with planted slips
  cae_mod_n3q / cae_attn_oproj / cae_n3q_xoproj / cae_ffn_fold / cae_mask_bias / vfp8_*
                            zero / unit gates (closed forms), F.layer_norm, the Gram identity of
                            the whole-row query norm, F.scaled_dot_product_attention + F.linear,
                            adaln / cae_ffn, softmax of the bias planes against the keep mask,
                            fp8 dequantisation within e4m3's step (tests/test_oracle.py)
"""
from __future__ import annotations

import math
from dataclasses import dataclass, asdict
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

Params = Dict[str, torch.Tensor]


# ---------------------------------------------------------------------------
# Configurations
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class ActionDiTConfig:
    """Hyper-parameters of the action expert (FB/action_dit.py:47-103)."""

    hidden_dim: int = 1024
    action_dim: int = 7
    ffn_dim: int = 4096
    text_dim: int = 1024
    freq_dim: int = 256
    eps: float = 1e-6
    num_heads: int = 16
    attn_head_dim: int = 64
    num_layers: int = 12

    @property
    def attn_dim(self) -> int:
        return self.num_heads * self.attn_head_dim

    def to_dict(self) -> dict:
        return asdict(self)


# ---------------------------------------------------------------------------
# Elementary functions
# ---------------------------------------------------------------------------
def sinusoidal_embedding_1d(dim: int, position: torch.Tensor) -> torch.Tensor:
    """cat(cos(p*f), sin(p*f)) with f_i = 10000^(-i/(dim/2)), fp64, cast to position's dtype.

    Restates FB/wan_video_dit.py:34-38 (FG/wan_video_dit.py:110-122).
    """
    half = dim // 2
    expo = torch.arange(half, dtype=torch.float64) / half
    freq = torch.pow(torch.tensor(10000.0, dtype=torch.float64), -expo)
    ang = position.to(torch.float64).reshape(-1, 1) * freq.reshape(1, -1)
    out = torch.cat([torch.cos(ang), torch.sin(ang)], dim=1)
    return out.to(position.dtype)


def precompute_freqs_cis(dim: int, end: int = 1024, theta: float = 10000.0) -> torch.Tensor:
    """complex128 table [end, dim/2]: exp(i * pos * theta^(-2j/dim)).

    Restates FB/wan_video_dit.py:49-55 (built through torch.polar, as the reference does,
    because cos/sin and polar differ in the last bits; CA/wan_video_dit.py:747-750).
    """
    j = torch.arange(0, dim, 2)[: dim // 2].to(torch.float64)
    inv = 1.0 / (theta ** (j / dim))
    ang = torch.arange(end).to(torch.float64).reshape(-1, 1) * inv.reshape(1, -1)
    return torch.polar(torch.ones_like(ang), ang)


def precompute_freqs_cis_3d(dim: int, end: int = 1024, theta: float = 10000.0):
    """Per-axis tables (frame, height, width) with dims (dim-2*(dim//3), dim//3, dim//3).

    Restates FB/wan_video_dit.py:41-46.
    """
    return (
        precompute_freqs_cis(dim - 2 * (dim // 3), end, theta),
        precompute_freqs_cis(dim // 3, end, theta),
        precompute_freqs_cis(dim // 3, end, theta),
    )


def video_freqs(freqs3d, f: int, h: int, w: int) -> torch.Tensor:
    """3-D RoPE table for an (f,h,w) token grid, [f*h*w, 1, Dh/2] complex.

    Restates the concatenation in FB/wan_video_dit.py:620-624 (token order f-major, then h, w).
    """
    ff, fh, fw = freqs3d
    a = ff[:f].reshape(f, 1, 1, -1).expand(f, h, w, -1)
    b = fh[:h].reshape(1, h, 1, -1).expand(f, h, w, -1)
    c = fw[:w].reshape(1, 1, w, -1).expand(f, h, w, -1)
    return torch.cat([a, b, c], dim=-1).reshape(f * h * w, 1, -1)


def action_freqs(attn_head_dim: int, seq_len: int, end: int = 1024) -> torch.Tensor:
    """1-D RoPE table for action tokens 0..S-1, [S, 1, Dh/2] complex (FB/action_dit.py:101, :291-295)."""
    if seq_len > end:
        raise ValueError(f"Action token length {seq_len} exceeds RoPE cache {end}.")
    return precompute_freqs_cis(attn_head_dim, end)[:seq_len].reshape(seq_len, 1, -1)


def rope_apply(x: torch.Tensor, freqs: torch.Tensor, num_heads: int) -> torch.Tensor:
    """Rotate interleaved pairs (x[2i], x[2i+1]) by the complex table, computed in fp64.

    x [B, S, H*Dh], freqs complex [S, 1, Dh/2].  Restates FB/wan_video_dit.py:58-70.
    """
    b, s, nd = x.shape
    xc = torch.view_as_complex(x.to(torch.float64).reshape(b, s, num_heads, nd // num_heads // 2, 2).contiguous())
    out = torch.view_as_real(xc * freqs.to(torch.complex128)).reshape(b, s, nd)
    return out.to(x.dtype)


def rope_tables_real(freqs: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) fp32 [S, Dh/2] from a complex [S, 1, Dh/2] table (FG/wan_video_dit.py:173-177)."""
    f = freqs.reshape(freqs.shape[0], -1)
    return f.real.to(torch.float32).contiguous(), f.imag.to(torch.float32).contiguous()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x*rsqrt(mean(x^2)+eps) in fp32, rounded to x.dtype, then times weight.

    Restates FB/wan_video_dit.py:156-167 (note the rounding before the weight multiply).
    """
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return y.to(x.dtype) * weight


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """nn.LayerNorm over the last dim (biased variance), optional affine (FB/wan_video_dit.py:258-261)."""
    xf = x.float()
    mu = xf.mean(dim=-1, keepdim=True)
    var = (xf - mu).pow(2).mean(dim=-1, keepdim=True)
    y = ((xf - mu) * torch.rsqrt(var + eps)).to(x.dtype)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return y


def modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """x*(1+scale)+shift (FB/wan_video_dit.py:30-31)."""
    return x * (1 + scale) + shift


def adaln(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float) -> torch.Tensor:
    """AdaLN-Zero: LayerNorm(x, affine=False)*(1+scale)+shift (FB/fused_adaln.py:522-523, eager branch)."""
    return layer_norm(x, None, None, eps) * (1 + scale) + shift


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """0.5x(1+tanh(sqrt(2/pi)(x+0.044715x^3))) (nn.GELU(approximate='tanh'), FB/wan_video_dit.py:262)."""
    xf = x.float()
    y = 0.5 * xf * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (xf + 0.044715 * xf * xf * xf)))
    return y.to(x.dtype)


def silu(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (xf / (1.0 + torch.exp(-xf))).to(x.dtype)


def linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor]) -> torch.Tensor:
    """y = x W^T + b (nn.Linear)."""
    return F.linear(x, w, b)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor] = None,
              scale: Optional[float] = None) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v over [B, H, S, Dh], fp32 inside, output in q.dtype.

    Semantics of F.scaled_dot_product_attention as called at FB/wan_video_dit.py:22: bool
    masks keep True entries, float masks are added; a query row with every key masked
    yields zeros (what torch's SDPA returns for such rows).
    """
    dh = q.shape[-1]
    sc = (1.0 / math.sqrt(dh)) if scale is None else scale
    s = torch.matmul(q.float(), k.float().transpose(-1, -2)) * sc
    if mask is not None:
        if mask.dtype == torch.bool:
            s = s.masked_fill(~mask, float("-inf"))
        else:
            s = s + mask.float()
    mx = s.amax(dim=-1, keepdim=True)
    dead = torch.isinf(mx) & (mx < 0)
    mx = torch.where(dead, torch.zeros_like(mx), mx)
    p = torch.exp(s - mx)
    l = p.sum(dim=-1, keepdim=True)
    p = p / torch.where(l > 0, l, torch.ones_like(l))
    out = torch.matmul(p, v.float())
    return out.to(q.dtype)


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
                    ctx_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[B,S,H*Dh] -> heads -> attention -> [B,Sq,H*Dh] (FB/wan_video_dit.py:17-26)."""
    def heads(t):
        b, s, nd = t.shape
        return t.reshape(b, s, num_heads, nd // num_heads).transpose(1, 2)

    o = attention(heads(q), heads(k), heads(v), ctx_mask)
    b, h, s, d = o.shape
    return o.transpose(1, 2).reshape(b, s, h * d)


# ---------------------------------------------------------------------------
# Flow-matching scheduler (SCH)
# ---------------------------------------------------------------------------
def build_inference_schedule(num_steps: int, shift: float, dtype=torch.float32,
                             num_train_timesteps: int = 1000) -> Tuple[torch.Tensor, torch.Tensor]:
    """sigma = s*u/(1+(s-1)u), u = linspace(1,0,N+1) in fp32; t = 1000*sigma[:-1]; delta = diff(sigma).

    Restates SCH:17-19 and SCH:63-80 (both results cast to `dtype`, as the reference casts to
    the latents' dtype).
    """
    if num_steps <= 0:
        raise ValueError(f"`num_inference_steps` must be positive, got {num_steps}")
    if shift <= 0:
        raise ValueError(f"`shift` must be positive, got {shift}")
    u = torch.linspace(1.0, 0.0, num_steps + 1, dtype=torch.float32)
    sigma = shift * u / (1.0 + (shift - 1.0) * u)
    t = sigma[:-1] * float(num_train_timesteps)
    d = sigma[1:] - sigma[:-1]
    return t.to(dtype), d.to(dtype)


def scheduler_step(model_output: torch.Tensor, delta: torch.Tensor, sample: torch.Tensor) -> torch.Tensor:
    """sample + model_output * delta, in sample's dtype (SCH:82-88)."""
    delta = delta.to(sample.dtype)
    if delta.ndim != 0:
        delta = delta.reshape(-1, *([1] * (sample.ndim - 1)))
    return sample + model_output * delta


# ---------------------------------------------------------------------------
# Parameters (state-dict key layout of FB/action_dit.py ActionDiT)
# ---------------------------------------------------------------------------
def action_dit_param_shapes(cfg: ActionDiTConfig) -> Dict[str, Tuple[int, ...]]:
    """Parameter names and shapes of ActionDiT (FB/action_dit.py:76-97, FB/wan_video_dit.py:180-265)."""
    H, A, Fd, T, Q = cfg.hidden_dim, cfg.attn_dim, cfg.ffn_dim, cfg.text_dim, cfg.freq_dim
    shapes: Dict[str, Tuple[int, ...]] = {
        "action_encoder.weight": (H, cfg.action_dim), "action_encoder.bias": (H,),
        "text_embedding.0.weight": (H, T), "text_embedding.0.bias": (H,),
        "text_embedding.2.weight": (H, H), "text_embedding.2.bias": (H,),
        "time_embedding.0.weight": (H, Q), "time_embedding.0.bias": (H,),
        "time_embedding.2.weight": (H, H), "time_embedding.2.bias": (H,),
        "time_projection.1.weight": (6 * H, H), "time_projection.1.bias": (6 * H,),
        "head.weight": (cfg.action_dim, H), "head.bias": (cfg.action_dim,),
    }
    for i in range(cfg.num_layers):
        p = f"blocks.{i}."
        for att in ("self_attn", "cross_attn"):
            for n in ("q", "k", "v"):
                shapes[p + f"{att}.{n}.weight"] = (A, H)
                shapes[p + f"{att}.{n}.bias"] = (A,)
            shapes[p + f"{att}.o.weight"] = (H, A)
            shapes[p + f"{att}.o.bias"] = (H,)
            shapes[p + f"{att}.norm_q.weight"] = (A,)
            shapes[p + f"{att}.norm_k.weight"] = (A,)
        shapes[p + "norm3.weight"] = (H,)
        shapes[p + "norm3.bias"] = (H,)
        shapes[p + "ffn.0.weight"] = (Fd, H)
        shapes[p + "ffn.0.bias"] = (Fd,)
        shapes[p + "ffn.2.weight"] = (H, Fd)
        shapes[p + "ffn.2.bias"] = (H,)
        shapes[p + "modulation"] = (1, 6, H)
    return shapes


NORM_AFFINE_STD = 0.2


def init_action_dit_params(cfg: ActionDiTConfig, seed: int, std: float = 0.02) -> Params:
    """Seeded synthetic weights: N(0,std) weights and biases, modulation randn/sqrt(H)
    (FB/wan_video_dit.py:264).  The norm affines are drawn away from the identity the reference
    initialises them to (a trained checkpoint carries its own): RMSNorm / LayerNorm weights
    N(1, 0.2), LayerNorm biases N(0, 0.2), so that a swapped, dropped or mis-indexed norm
    weight changes every output.  Drawn in sorted-name order from one CPU generator, fp32."""
    g = torch.Generator("cpu").manual_seed(seed)
    out: Params = {}
    for name, shape in sorted(action_dit_param_shapes(cfg).items()):
        if name.endswith("modulation"):
            out[name] = torch.randn(shape, generator=g) / math.sqrt(cfg.hidden_dim)
        elif ".norm_q." in name or ".norm_k." in name or name.endswith("norm3.weight"):
            out[name] = 1.0 + torch.randn(shape, generator=g) * NORM_AFFINE_STD
        elif name.endswith("norm3.bias"):
            out[name] = torch.randn(shape, generator=g) * NORM_AFFINE_STD
        else:
            out[name] = torch.randn(shape, generator=g) * std
    return out


def cast_params(p: Params, dtype) -> Params:
    return {k: v.to(dtype) for k, v in p.items()}


# ---------------------------------------------------------------------------
# Composite modules
# ---------------------------------------------------------------------------
def split_modulation(modulation: torch.Tensor, t_mod: torch.Tensor):
    """(modulation + t_mod).chunk(6) -> shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp.

    t_mod [B,6,D] gives [B,1,D] pieces; per-token t_mod [B,S,6,D] gives [B,S,D] pieces.
    Restates FB/wan_video_dit.py:271-280 and FB/mot.py:63-80.
    """
    has_seq = t_mod.dim() == 4
    m = modulation.to(t_mod.dtype) + t_mod
    parts = m.chunk(6, dim=2 if has_seq else 1)
    if has_seq:
        parts = tuple(x.squeeze(2) for x in parts)
    return parts


def self_attention(p: Params, pre: str, x: torch.Tensor, freqs: torch.Tensor, num_heads: int, eps: float,
                   mask: Optional[torch.Tensor] = None, trace: Optional[dict] = None) -> torch.Tensor:
    """SelfAttention.forward (FB/wan_video_dit.py:197-204).  `trace`, when given, records the
    rotated q, k, the v and the attention output before the o projection."""
    q = rms_norm(linear(x, p[pre + "q.weight"], p[pre + "q.bias"]), p[pre + "norm_q.weight"], eps)
    k = rms_norm(linear(x, p[pre + "k.weight"], p[pre + "k.bias"]), p[pre + "norm_k.weight"], eps)
    v = linear(x, p[pre + "v.weight"], p[pre + "v.bias"])
    q = rope_apply(q, freqs, num_heads)
    k = rope_apply(k, freqs, num_heads)
    o = flash_attention(q, k, v, num_heads, mask)
    if trace is not None:
        trace.update(q=q, k=k, v=v, self_attn=o)
    return linear(o, p[pre + "o.weight"], p[pre + "o.bias"])


def cross_kv(p: Params, pre: str, context: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """Context keys/values of CrossAttention: norm_k(k(ctx)), v(ctx) (FB/wan_video_dit.py:226-227)."""
    k = rms_norm(linear(context, p[pre + "k.weight"], p[pre + "k.bias"]), p[pre + "norm_k.weight"], eps)
    v = linear(context, p[pre + "v.weight"], p[pre + "v.bias"])
    return k, v


def cross_attention(p: Params, pre: str, x: torch.Tensor, context: torch.Tensor, num_heads: int, eps: float,
                    mask: Optional[torch.Tensor] = None, trace: Optional[dict] = None) -> torch.Tensor:
    """CrossAttention.forward (FB/wan_video_dit.py:224-229).  `trace` records the attention
    output before the o projection."""
    q = rms_norm(linear(x, p[pre + "q.weight"], p[pre + "q.bias"]), p[pre + "norm_q.weight"], eps)
    k, v = cross_kv(p, pre, context, eps)
    o = flash_attention(q, k, v, num_heads, mask)
    if trace is not None:
        trace.update(cross_attn=o)
    return linear(o, p[pre + "o.weight"], p[pre + "o.bias"])


def ffn(p: Params, pre: str, x: torch.Tensor) -> torch.Tensor:
    """Linear -> GELU(tanh) -> Linear (FB/wan_video_dit.py:262-263)."""
    h = gelu_tanh(linear(x, p[pre + "ffn.0.weight"], p[pre + "ffn.0.bias"]))
    return linear(h, p[pre + "ffn.2.weight"], p[pre + "ffn.2.bias"])


def dit_block(p: Params, idx: int, x: torch.Tensor, context: torch.Tensor, t_mod: torch.Tensor,
              freqs: torch.Tensor, num_heads: int, eps: float,
              context_mask: Optional[torch.Tensor] = None,
              self_attn_mask: Optional[torch.Tensor] = None, trace: Optional[dict] = None) -> torch.Tensor:
    """DiTBlock.forward (FB/wan_video_dit.py:267-286).

    context_mask: None, bool [B,Sq,L] (unsqueezed to [B,1,Sq,L] as at :268-269) or [B,1,Sq,L].
    trace: when given, records the branch values (q, k, v, self_attn, cross_attn: see
    self_attention / cross_attention) and the residual stream after each branch (x_self,
    x_cross), so a test can compare a block's inner values and not only its residual-dominated
    output.
    """
    pre = f"blocks.{idx}."
    if context_mask is not None and context_mask.dim() == 3:
        context_mask = context_mask.unsqueeze(1)
    sh_a, sc_a, g_a, sh_m, sc_m, g_m = split_modulation(p[pre + "modulation"], t_mod)
    h = adaln(x, sh_a, sc_a, eps)
    x = x + g_a * self_attention(p, pre + "self_attn.", h, freqs, num_heads, eps, self_attn_mask, trace)
    if trace is not None:
        trace.update(x_self=x)
    x = x + cross_attention(p, pre + "cross_attn.",
                            layer_norm(x, p[pre + "norm3.weight"], p[pre + "norm3.bias"], eps),
                            context, num_heads, eps, context_mask, trace)
    if trace is not None:
        trace.update(x_cross=x)
    h = adaln(x, sh_m, sc_m, eps)
    x = x + g_m * ffn(p, pre, h)
    return x


def time_mlp(p: Params, cfg: ActionDiTConfig, timestep: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """t = time_embedding(sinusoid(t)); t_mod = time_projection(t) viewed [B,6,H] (FB/action_dit.py:282-283)."""
    e = sinusoidal_embedding_1d(cfg.freq_dim, timestep)
    t = linear(silu(linear(e, p["time_embedding.0.weight"], p["time_embedding.0.bias"])),
               p["time_embedding.2.weight"], p["time_embedding.2.bias"])
    t_mod = linear(silu(t), p["time_projection.1.weight"], p["time_projection.1.bias"])
    return t, t_mod.unflatten(1, (6, cfg.hidden_dim))


def text_embedding(p: Params, context: torch.Tensor) -> torch.Tensor:
    """Linear -> GELU(tanh) -> Linear over the context (FB/action_dit.py:77-81, :286)."""
    h = gelu_tanh(linear(context, p["text_embedding.0.weight"], p["text_embedding.0.bias"]))
    return linear(h, p["text_embedding.2.weight"], p["text_embedding.2.bias"])


def action_dit_forward(p: Params, cfg: ActionDiTConfig, action_tokens: torch.Tensor, timestep: torch.Tensor,
                       context: torch.Tensor, context_mask: Optional[torch.Tensor] = None,
                       context_emb: Optional[torch.Tensor] = None) -> torch.Tensor:
    """ActionDiT.forward = pre_dit -> blocks -> head (FB/action_dit.py:228-353).

    context_emb, when given, is text_embedding(context) computed earlier (the same value
    pre_dit recomputes every call)."""
    b, s, _ = action_tokens.shape
    if timestep.shape[0] == 1 and b > 1:
        timestep = timestep.expand(b)
    _, t_mod = time_mlp(p, cfg, timestep)
    x = linear(action_tokens, p["action_encoder.weight"], p["action_encoder.bias"])
    ctx = text_embedding(p, context) if context_emb is None else context_emb
    cmask = None
    if context_mask is not None:
        cmask = context_mask.unsqueeze(1).expand(-1, s, -1)
    freqs = action_freqs(cfg.attn_head_dim, s)
    for i in range(cfg.num_layers):
        x = dit_block(p, i, x, ctx, t_mod, freqs, cfg.num_heads, cfg.eps, cmask)
    return linear(x, p["head.weight"], p["head.bias"])


def denoise_loop(p: Params, cfg: ActionDiTConfig, noise: torch.Tensor, context: torch.Tensor,
                 num_steps: int, shift: float, context_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Flow-matching Euler loop of the policy call (FB/fastwam.py:1040-1069) over the action expert.

    The latents, schedule and every op run in the dtype of `noise` (the reference casts the
    seeded CPU noise to the model dtype, FB/fastwam.py:971-977)."""
    dtype = noise.dtype
    ts, ds = build_inference_schedule(num_steps, shift, dtype)
    ctx_emb = text_embedding(p, context)
    x = noise
    for t, d in zip(ts, ds):
        v = action_dit_forward(p, cfg, x, t.reshape(1), context, context_mask, context_emb=ctx_emb)
        x = scheduler_step(v, d, x)
    return x


def mot_action_forward(p: Params, cfg: ActionDiTConfig, x: torch.Tensor, freqs: torch.Tensor,
                       t_mod: torch.Tensor, context: torch.Tensor, video_kv: Sequence[Tuple[torch.Tensor, torch.Tensor]],
                       joint_mask: torch.Tensor, video_seq_len: int,
                       context_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """MoT action branch over a cached video K/V prefix (FB/mot.py:378-478 and :104-189).

    Per layer: AdaLN -> q,k,v (RMSNorm + RoPE) -> attention of the action rows over
    cat(video K/V, action K/V) with the action rows of the joint mask -> o-proj + gate ->
    cross-attention -> AdaLN -> FFN + gate."""
    sa = x.shape[1]
    amask = joint_mask[video_seq_len:video_seq_len + sa, :video_seq_len + sa]
    cmask = context_mask
    if cmask is not None and cmask.dim() == 3:
        cmask = cmask.unsqueeze(1)
    for i in range(cfg.num_layers):
        pre = f"blocks.{i}."
        sh_a, sc_a, g_a, sh_m, sc_m, g_m = split_modulation(p[pre + "modulation"], t_mod)
        h = adaln(x, sh_a, sc_a, cfg.eps)
        sp = pre + "self_attn."
        q = rms_norm(linear(h, p[sp + "q.weight"], p[sp + "q.bias"]), p[sp + "norm_q.weight"], cfg.eps)
        k = rms_norm(linear(h, p[sp + "k.weight"], p[sp + "k.bias"]), p[sp + "norm_k.weight"], cfg.eps)
        v = linear(h, p[sp + "v.weight"], p[sp + "v.bias"])
        q = rope_apply(q, freqs, cfg.num_heads)
        k = rope_apply(k, freqs, cfg.num_heads)
        kv, vv = video_kv[i]
        mixed = flash_attention(q, torch.cat([kv, k], dim=1), torch.cat([vv, v], dim=1), cfg.num_heads, amask)
        x = x + g_a * linear(mixed, p[sp + "o.weight"], p[sp + "o.bias"])
        x = x + cross_attention(p, pre + "cross_attn.",
                                layer_norm(x, p[pre + "norm3.weight"], p[pre + "norm3.bias"], cfg.eps),
                                context, cfg.num_heads, cfg.eps, cmask)
        h = adaln(x, sh_m, sc_m, cfg.eps)
        x = x + g_m * ffn(p, pre, h)
    return x


def mot_prefill_video_cache(p: Params, cfg: ActionDiTConfig, x: torch.Tensor, freqs: torch.Tensor,
                            t_mod: torch.Tensor, context: Optional[torch.Tensor], video_mask: torch.Tensor,
                            context_mask: Optional[torch.Tensor] = None,
                            num_run: int = 0) -> List[Tuple[torch.Tensor, torch.Tensor]]:
    """MoT.prefill_video_cache (FB/mot.py:262-376): the video tokens through the first
    `num_run` blocks (all when 0 or >= num_layers), returning each block's attention K/V.

    Per block (`_prefill_one_layer`, :360-376, with :63-80, :104-189): AdaLN ->
    q, k (RMSNorm + RoPE), v -> attention under the [Sv, Sv] video mask -> x += g_msa * o ->
    (context given) x += cross_attention(norm3(x), context) -> AdaLN -> x += g_mlp * FFN.
    The cached k is the normalised, rotated key and v the raw value projection.  Blocks past
    `num_run` reuse the last computed block's K/V (video layer drafting, :345-351)."""
    L = cfg.num_layers
    n_run = L if num_run <= 0 or num_run > L else num_run
    cmask = context_mask
    if cmask is not None and cmask.dim() == 3:
        cmask = cmask.unsqueeze(1)
    cache: List[Tuple[torch.Tensor, torch.Tensor]] = []
    for i in range(n_run):
        pre = f"blocks.{i}."
        sh_a, sc_a, g_a, sh_m, sc_m, g_m = split_modulation(p[pre + "modulation"], t_mod)
        h = adaln(x, sh_a, sc_a, cfg.eps)
        sp = pre + "self_attn."
        q = rms_norm(linear(h, p[sp + "q.weight"], p[sp + "q.bias"]), p[sp + "norm_q.weight"], cfg.eps)
        k = rms_norm(linear(h, p[sp + "k.weight"], p[sp + "k.bias"]), p[sp + "norm_k.weight"], cfg.eps)
        v = linear(h, p[sp + "v.weight"], p[sp + "v.bias"])
        q = rope_apply(q, freqs, cfg.num_heads)
        k = rope_apply(k, freqs, cfg.num_heads)
        cache.append((k, v))
        mixed = flash_attention(q, k, v, cfg.num_heads, video_mask)
        x = x + g_a * linear(mixed, p[sp + "o.weight"], p[sp + "o.bias"])
        if context is not None:
            x = x + cross_attention(p, pre + "cross_attn.",
                                    layer_norm(x, p[pre + "norm3.weight"], p[pre + "norm3.bias"], cfg.eps),
                                    context, cfg.num_heads, cfg.eps, cmask)
        h = adaln(x, sh_m, sc_m, cfg.eps)
        x = x + g_m * ffn(p, pre, h)
    while len(cache) < L:
        cache.append(cache[-1])
    return cache


def mot_joint_mask(video_seq_len: int, action_seq_len: int, video_tokens_per_frame: int) -> torch.Tensor:
    """Joint [video+action] bool mask for first_frame_causal video (FB/fastwam.py:389-410,
    FB/wan_video_dit.py:493-498): video->video first-frame causal, action->action all,
    action->first video frame only."""
    n = video_seq_len + action_seq_len
    m = torch.zeros((n, n), dtype=torch.bool)
    vv = torch.ones((video_seq_len, video_seq_len), dtype=torch.bool)
    ff = min(video_tokens_per_frame, video_seq_len)
    vv[:ff, ff:] = False
    m[:video_seq_len, :video_seq_len] = vv
    m[video_seq_len:, video_seq_len:] = True
    m[video_seq_len:, :ff] = True
    return m


# ---------------------------------------------------------------------------
# WanVideoDiT: the video expert's pre_dit / post_dit around the blocks
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class WanVideoConfig:
    """Hyper-parameters of WanVideoDiT (FB/wan_video_dit.py:329-411) in the inference setting
    the reference supports (seperated_timestep, VAE embedding fused in the latents)."""
    hidden_dim: int = 3072
    in_dim: int = 48
    ffn_dim: int = 14336
    out_dim: int = 48
    text_dim: int = 4096
    freq_dim: int = 256
    eps: float = 1e-6
    patch_size: Tuple[int, int, int] = (1, 2, 2)
    num_heads: int = 24
    attn_head_dim: int = 128
    num_layers: int = 30

    @property
    def attn_dim(self) -> int:
        return self.num_heads * self.attn_head_dim

    def block_config(self) -> ActionDiTConfig:
        """The per-block hyper-parameters in the form dit_block's callers use."""
        return ActionDiTConfig(hidden_dim=self.hidden_dim, action_dim=1, ffn_dim=self.ffn_dim, text_dim=self.text_dim,
                               freq_dim=self.freq_dim, eps=self.eps, num_heads=self.num_heads,
                               attn_head_dim=self.attn_head_dim, num_layers=self.num_layers)


def wan_param_shapes(cfg: WanVideoConfig) -> Dict[str, Tuple[int, ...]]:
    """State-dict keys of WanVideoDiT (FB/wan_video_dit.py:385-401, Head :309-316)."""
    H = cfg.hidden_dim
    P = cfg.patch_size[0] * cfg.patch_size[1] * cfg.patch_size[2]
    shapes = {k: v for k, v in action_dit_param_shapes(cfg.block_config()).items() if k.startswith("blocks.")}
    shapes.update({
        "patch_embedding.weight": (H, cfg.in_dim) + tuple(cfg.patch_size), "patch_embedding.bias": (H,),
        "text_embedding.0.weight": (H, cfg.text_dim), "text_embedding.0.bias": (H,),
        "text_embedding.2.weight": (H, H), "text_embedding.2.bias": (H,),
        "time_embedding.0.weight": (H, cfg.freq_dim), "time_embedding.0.bias": (H,),
        "time_embedding.2.weight": (H, H), "time_embedding.2.bias": (H,),
        "time_projection.1.weight": (6 * H, H), "time_projection.1.bias": (6 * H,),
        "head.head.weight": (cfg.out_dim * P, H), "head.head.bias": (cfg.out_dim * P,),
        "head.modulation": (1, 2, H),
    })
    return shapes


def init_wan_params(cfg: WanVideoConfig, seed: int, std: float = 0.02) -> Params:
    """Seeded synthetic weights with init_action_dit_params' rules (the two modulations
    randn/sqrt(H), norm affines N(1, 0.2) / N(0, 0.2)), sorted-name draws, fp32."""
    g = torch.Generator("cpu").manual_seed(seed)
    out: Params = {}
    for name, shape in sorted(wan_param_shapes(cfg).items()):
        if name.endswith("modulation"):
            out[name] = torch.randn(shape, generator=g) / math.sqrt(cfg.hidden_dim)
        elif ".norm_q." in name or ".norm_k." in name or name.endswith("norm3.weight"):
            out[name] = 1.0 + torch.randn(shape, generator=g) * NORM_AFFINE_STD
        elif name.endswith("norm3.bias"):
            out[name] = torch.randn(shape, generator=g) * NORM_AFFINE_STD
        else:
            out[name] = torch.randn(shape, generator=g) * std
    return out


def wan_patchify(p: Params, x: torch.Tensor, patch) -> torch.Tensor:
    """nn.Conv3d(in_dim, H, kernel = stride = patch) of the latents [B, C, F, Hl, Wl] ->
    [B, H, f, h, w] (FB/wan_video_dit.py:385-386, 420-426)."""
    return F.conv3d(x, p["patch_embedding.weight"], p["patch_embedding.bias"], stride=tuple(patch))


def wan_pre_dit(p: Params, cfg: WanVideoConfig, x: torch.Tensor, timestep: torch.Tensor, context: torch.Tensor,
                context_mask: Optional[torch.Tensor] = None) -> dict:
    """WanVideoDiT.pre_dit with seperated_timestep and the VAE embedding fused in the latents
    (FB/wan_video_dit.py:527-648, no action conditioning): every token carries the timestep of
    its latent frame, the first frame's being 0 (:555-568); t = time_embedding(sinusoid) per
    token, t_mod = time_projection(t) [B, S, 6, H]; tokens = patchify(x) in (f, h, w) order;
    context = text_embedding(context); the context mask broadcast over the tokens; the 3-D RoPE
    table of the (f, h, w) grid (:642-646)."""
    B = x.shape[0]
    pt, ph, pw = cfg.patch_size
    tpf = (x.shape[3] // ph) * (x.shape[4] // pw)
    if timestep.shape[0] == 1 and B > 1:
        timestep = timestep.expand(B)
    tt = torch.ones((B, x.shape[2], tpf), dtype=timestep.dtype) * timestep.view(B, 1, 1)
    tt[:, 0, :] = 0
    tt = tt.reshape(B, -1)
    emb = sinusoidal_embedding_1d(cfg.freq_dim, tt.reshape(-1))
    t = linear(silu(linear(emb, p["time_embedding.0.weight"], p["time_embedding.0.bias"])),
               p["time_embedding.2.weight"], p["time_embedding.2.bias"]).reshape(B, -1, cfg.hidden_dim)
    t_mod = linear(silu(t), p["time_projection.1.weight"], p["time_projection.1.bias"]).unflatten(2, (6, cfg.hidden_dim))
    xp = wan_patchify(p, x, cfg.patch_size)
    f, h, w = xp.shape[2:]
    ctx = text_embedding(p, context)
    if context_mask is None:
        context_mask = torch.ones((context.shape[0], context.shape[1]), dtype=torch.bool)
    cmask = context_mask.unsqueeze(1).expand(-1, f * h * w, -1)
    tokens = xp.flatten(2).transpose(1, 2).contiguous()
    freqs = video_freqs(precompute_freqs_cis_3d(cfg.attn_head_dim), f, h, w)
    return {"tokens": tokens, "freqs": freqs, "t": t, "t_mod": t_mod, "context": ctx, "context_mask": cmask,
            "grid": (f, h, w), "tokens_per_frame": tpf}


def wan_head(p: Params, x: torch.Tensor, t: torch.Tensor, eps: float) -> torch.Tensor:
    """Head.forward with per-token t [B, S, H] (FB/wan_video_dit.py:318-322): shift, scale =
    modulation + t; Linear(LN(x) (1 + scale) + shift)."""
    m = p["head.modulation"].unsqueeze(0).to(t.dtype) + t.unsqueeze(2)
    shift, scale = m.chunk(2, dim=2)
    return linear(adaln(x, shift.squeeze(2), scale.squeeze(2), eps), p["head.head.weight"], p["head.head.bias"])


def wan_unpatchify(x: torch.Tensor, grid, patch, out_dim: int) -> torch.Tensor:
    """rearrange 'b (f h w) (x y z c) -> b c (f x) (h y) (w z)' (FB/wan_video_dit.py:428-433)."""
    f, h, w = grid
    pt, ph, pw = patch
    B = x.shape[0]
    y = x.reshape(B, f, h, w, pt, ph, pw, out_dim).permute(0, 7, 1, 4, 2, 5, 3, 6)
    return y.reshape(B, out_dim, f * pt, h * ph, w * pw)


def wan_forward(p: Params, cfg: WanVideoConfig, x: torch.Tensor, timestep: torch.Tensor, context: torch.Tensor,
                context_mask: Optional[torch.Tensor] = None, video_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """WanVideoDiT.forward = pre_dit -> blocks -> post_dit (FB/wan_video_dit.py:651-684);
    video_mask: the [S, S] self-attention mask (None for bidirectional)."""
    pre = wan_pre_dit(p, cfg, x, timestep, context, context_mask)
    xt = pre["tokens"]
    for i in range(cfg.num_layers):
        xt = dit_block(p, i, xt, pre["context"], pre["t_mod"], pre["freqs"], cfg.num_heads, cfg.eps,
                       pre["context_mask"], video_mask)
    y = wan_head(p, xt, pre["t"], cfg.eps)
    return wan_unpatchify(y, pre["grid"], cfg.patch_size, cfg.out_dim)


# ---------------------------------------------------------------------------
# CAE-FastWAM action-VAE decoder (fp32)
# ---------------------------------------------------------------------------
@dataclass
class CaeDecoderConfig:
    """The decoder's shape (CAm/action_ae.py:15-29): latent tokens x latent_dim -> horizon x action_dim."""
    latent_dim: int = 16
    num_tokens: int = 8
    action_horizon: int = 32
    action_dim: int = 7
    decoder_hidden: int = 128


def cae_strides(ratio: int) -> List[int]:
    """ActionEncoder._factorise_ratio (CAm/action_ae.py:90-101): factors 4, then 2, then 3, then
    the remainder."""
    if ratio == 1:
        return [1]
    out = []
    for f in (4, 2, 3):
        while ratio % f == 0:
            out.append(f)
            ratio //= f
    if ratio > 1:
        out.append(ratio)
    return out


def cae_decoder_param_shapes(cfg: CaeDecoderConfig) -> Dict[str, tuple]:
    """State-dict keys of ActionAE.decoder (CAm/action_ae.py:123-150): nn.Sequential `up` holds
    per stride [ConvTranspose1d, GroupNorm, SiLU, ResidualConv1dBlock(net: Conv1d, GN, SiLU,
    Conv1d, GN)]."""
    C = cfg.decoder_hidden
    s = {"decoder.input_proj.weight": (C, cfg.latent_dim), "decoder.input_proj.bias": (C,),
         "decoder.output_proj.weight": (cfg.action_dim, C), "decoder.output_proj.bias": (cfg.action_dim,)}
    for j, st in enumerate(cae_strides(cfg.action_horizon // cfg.num_tokens)):
        u = f"decoder.up.{4 * j}"
        s[u + ".weight"], s[u + ".bias"] = (C, C, 2 * st), (C,)
        s[f"decoder.up.{4 * j + 1}.weight"] = s[f"decoder.up.{4 * j + 1}.bias"] = (C,)
        r = f"decoder.up.{4 * j + 3}.net."
        for k in ("0", "3"):
            s[r + k + ".weight"], s[r + k + ".bias"] = (C, C, 3), (C,)
        for k in ("1", "4"):
            s[r + k + ".weight"] = s[r + k + ".bias"] = (C,)
    return s


def init_cae_decoder_params(cfg: CaeDecoderConfig, seed: int) -> Params:
    """Seeded synthetic decoder weights (fp32), drawn in sorted-name order: weights with two or
    more dims N(0, 1/fan_in) with fan_in = prod(shape[1:]); GroupNorm weights 1 + N(0, 0.1) and
    biases N(0, 0.1); other biases N(0, 0.02)."""
    g = torch.Generator("cpu").manual_seed(seed)
    out: Params = {}
    for name, shape in sorted(cae_decoder_param_shapes(cfg).items()):
        parts = name.split(".")
        is_gn = (len(parts) == 4 and parts[1] == "up" and int(parts[2]) % 4 == 1) or \
            ".net.1." in name or ".net.4." in name
        if len(shape) >= 2:
            out[name] = torch.randn(shape, generator=g) / math.sqrt(math.prod(shape[1:]))
        elif is_gn and name.endswith(".weight"):
            out[name] = 1.0 + torch.randn(shape, generator=g) * 0.1
        elif is_gn:
            out[name] = torch.randn(shape, generator=g) * 0.1
        else:
            out[name] = torch.randn(shape, generator=g) * 0.02
    return out


def cae_decode(p: Params, cfg: CaeDecoderConfig, z: torch.Tensor, suite: Optional[torch.Tensor] = None,
               gn_eps: float = 1e-5) -> torch.Tensor:
    """ActionDecoder.forward (CAm/action_ae.py:152-166, ResidualConv1dBlock :32-48), fp32:
    z [B, num_tokens, latent_dim] -> [B, action_horizon, action_dim]; suite: optional [B, C]
    suite-embedding rows added after the input projection."""
    x = F.linear(z, p["decoder.input_proj.weight"], p["decoder.input_proj.bias"])
    if suite is not None:
        x = x + suite.unsqueeze(1)
    x = x.transpose(1, 2)
    C = x.shape[1]
    G = min(8, C)
    for j, st in enumerate(cae_strides(cfg.action_horizon // cfg.num_tokens)):
        u = f"decoder.up.{4 * j}"
        x = F.conv_transpose1d(x, p[u + ".weight"], p[u + ".bias"], stride=st, padding=st // 2)
        x = F.silu(F.group_norm(x, G, p[f"decoder.up.{4 * j + 1}.weight"], p[f"decoder.up.{4 * j + 1}.bias"], gn_eps))
        r = f"decoder.up.{4 * j + 3}.net."
        h = F.conv1d(x, p[r + "0.weight"], p[r + "0.bias"], padding=1)
        h = F.silu(F.group_norm(h, G, p[r + "1.weight"], p[r + "1.bias"], gn_eps))
        h = F.conv1d(h, p[r + "3.weight"], p[r + "3.bias"], padding=1)
        x = x + F.group_norm(h, G, p[r + "4.weight"], p[r + "4.bias"], gn_eps)
    T = x.shape[2]
    if T > cfg.action_horizon:
        x = x[:, :, :cfg.action_horizon]
    elif T < cfg.action_horizon:
        x = F.pad(x, (0, cfg.action_horizon - T))
    return F.linear(x.transpose(1, 2), p["decoder.output_proj.weight"], p["decoder.output_proj.bias"])


# ---------------------------------------------------------------------------
# DiT4DiT flow-matching action head (DB = src/dit4dit-baseline/DiT4DiT/model/modules/action_model)
# ---------------------------------------------------------------------------
# The head's transformer (DB/flow_matching_head/cross_attention_dit.py) is built from diffusers
# modules (Attention, FeedForward, Timesteps, TimestepEmbedding; diffusers 0.37.0.dev0 @3996788
# per scripts/dit4dit_diffusers_overlay.sh:7,35), which are not installed here.  Their published
# semantics are restated below.  No reference test or fixture holds this model; the composition
# is pinned by closed forms in tests/test_oracle.py (the AdaLayerNorm's (scale, shift) order, norm3
# without affine + the FFN, the output stage's (shift, scale) and eps, the action encoder's concat
# order, the two embeddings, the schedule and block wiring), each with its slipped alternative
# shown to fail; "parity unpinned" only as to diffusers' own code, which cannot run here.
@dataclass
class DiT4DiTHeadConfig:
    """DiT-B head of DB/ActionDiT.py:192-195 with the diffusion_model_cfg of
    DiT4DiT/config/real_robot/dit4dit_g1.yaml:25-49; state_dim 64 as in that file (:31) and the
    RoboCasa-GR1 config (LIBERO uses 16); 0 means no state encoder (DB/ActionDiT.py:235-239)."""
    action_dim: int = 32
    horizon: int = 16            # future_action_window_size + 1
    heads: int = 12              # DiT-B
    head_dim: int = 64
    num_layers: int = 16
    cross_dim: int = 2048        # VLM feature width
    output_dim: int = 2560       # DiT proj_out_2 width
    hidden_size: int = 2560      # action decoder hidden width
    max_seq_len: int = 1024      # position embedding table
    num_steps: int = 4           # num_inference_timesteps
    buckets: int = 1000          # num_timestep_buckets
    interleave_self_attention: bool = True
    ff_mult: int = 4             # diffusers FeedForward default inner_dim = 4 * dim
    norm_eps: float = 1e-5       # AdaLayerNorm / norm3 (cross_attention_dit.py:47-57, 207)
    out_eps: float = 1e-6        # norm_out (cross_attention_dit.py:253)
    state_dim: int = 64          # state_encoder input width (0: no state encoder)

    @property
    def dim(self) -> int:
        return self.heads * self.head_dim

    def is_cross(self, idx: int) -> bool:
        """Odd blocks are self-attention when interleaved (cross_attention_dit.py:231-233, 285)."""
        return not (self.interleave_self_attention and idx % 2 == 1)


def d4d_param_shapes(cfg: DiT4DiTHeadConfig) -> Dict[str, Tuple[int, ...]]:
    """State-dict keys of FlowmatchingActionHead (DB/ActionDiT.py:197-236; diffusers Attention
    to_q/to_k/to_v/to_out.0, FeedForward net.0.proj / net.2, TimestepEmbedding linear_1/2)."""
    D, C = cfg.dim, cfg.cross_dim
    s = {
        "model.timestep_encoder.timestep_embedder.linear_1.weight": (D, 256),
        "model.timestep_encoder.timestep_embedder.linear_1.bias": (D,),
        "model.timestep_encoder.timestep_embedder.linear_2.weight": (D, D),
        "model.timestep_encoder.timestep_embedder.linear_2.bias": (D,),
        "model.proj_out_1.weight": (2 * D, D), "model.proj_out_1.bias": (2 * D,),
        "model.proj_out_2.weight": (cfg.output_dim, D), "model.proj_out_2.bias": (cfg.output_dim,),
        "action_encoder.layer1.weight": (D, cfg.action_dim), "action_encoder.layer1.bias": (D,),
        "action_encoder.layer2.weight": (D, 2 * D), "action_encoder.layer2.bias": (D,),
        "action_encoder.layer3.weight": (D, D), "action_encoder.layer3.bias": (D,),
        "action_decoder.layer1.weight": (cfg.hidden_size, cfg.output_dim), "action_decoder.layer1.bias": (cfg.hidden_size,),
        "action_decoder.layer2.weight": (cfg.action_dim, cfg.hidden_size), "action_decoder.layer2.bias": (cfg.action_dim,),
        "position_embedding.weight": (cfg.max_seq_len, D),
    }
    if cfg.state_dim:
        # MLP(state_dim, hidden_size, D) (DB/ActionDiT.py:64-71, 235-239)
        s.update({"state_encoder.layer1.weight": (cfg.hidden_size, cfg.state_dim),
                  "state_encoder.layer1.bias": (cfg.hidden_size,),
                  "state_encoder.layer2.weight": (D, cfg.hidden_size), "state_encoder.layer2.bias": (D,)})
    for i in range(cfg.num_layers):
        b = f"model.transformer_blocks.{i}."
        kv_in = C if cfg.is_cross(i) else D
        s.update({
            b + "norm1.linear.weight": (2 * D, D), b + "norm1.linear.bias": (2 * D,),
            b + "attn1.to_q.weight": (D, D), b + "attn1.to_q.bias": (D,),
            b + "attn1.to_k.weight": (D, kv_in), b + "attn1.to_k.bias": (D,),
            b + "attn1.to_v.weight": (D, kv_in), b + "attn1.to_v.bias": (D,),
            b + "attn1.to_out.0.weight": (D, D), b + "attn1.to_out.0.bias": (D,),
            b + "ff.net.0.proj.weight": (cfg.ff_mult * D, D), b + "ff.net.0.proj.bias": (cfg.ff_mult * D,),
            b + "ff.net.2.weight": (D, cfg.ff_mult * D), b + "ff.net.2.bias": (D,),
        })
    return s


def init_d4d_params(cfg: DiT4DiTHeadConfig, seed: int, std: float = 0.02) -> Params:
    """Synthetic weights, N(0, std) for every tensor (sorted-name draws), fp32."""
    g = torch.Generator().manual_seed(seed)
    return {k: torch.randn(v, generator=g) * std for k, v in sorted(d4d_param_shapes(cfg).items())}


def d4d_tau_encoding(timesteps: torch.Tensor, dim: int) -> torch.Tensor:
    """SinusoidalPositionalEncoding (DB/flow_matching_head/action_encoder.py:21-37):
    cat(sin(t f), cos(t f)), f_i = exp(-i ln(10000) / (dim/2)), fp32.  timesteps [..]."""
    half = dim // 2
    f = torch.exp(-torch.arange(half, dtype=torch.float32) * (math.log(10000.0) / half))
    a = timesteps.float().unsqueeze(-1) * f
    return torch.cat([torch.sin(a), torch.cos(a)], dim=-1)


def d4d_timestep_proj(timesteps: torch.Tensor, channels: int = 256) -> torch.Tensor:
    """diffusers Timesteps(num_channels=256, flip_sin_to_cos=True, downscale_freq_shift=1) as used
    at DB/flow_matching_head/cross_attention_dit.py:34 (diffusers get_timestep_embedding):
    f_i = exp(-ln(10000) i / (half - 1)), emb = cat(cos(t f), sin(t f)), fp32.  timesteps [B]."""
    half = channels // 2
    f = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float32) / (half - 1))
    a = timesteps.float()[:, None] * f[None, :]
    return torch.cat([torch.cos(a), torch.sin(a)], dim=-1)


def d4d_temb(p: Params, timesteps: torch.Tensor, dtype) -> torch.Tensor:
    """TimestepEncoder (cross_attention_dit.py:31-41): TimestepEmbedding(linear_1, SiLU, linear_2)
    of the projection cast to the parameter dtype.  [B] -> [B, D]."""
    pre = "model.timestep_encoder.timestep_embedder."
    h = d4d_timestep_proj(timesteps).to(dtype)
    h = F.silu(F.linear(h, p[pre + "linear_1.weight"], p[pre + "linear_1.bias"]))
    return F.linear(h, p[pre + "linear_2.weight"], p[pre + "linear_2.bias"])


def d4d_action_encoder(p: Params, actions: torch.Tensor, timesteps: torch.Tensor) -> torch.Tensor:
    """ActionEncoder.forward (DB/ActionDiT.py:74-98): layer1(actions); tau = sinusoid(t) cast to
    that dtype; swish(layer2(cat(a, tau))); layer3.  actions [B, T, A], timesteps [B]."""
    B, T, _ = actions.shape
    a = F.linear(actions, p["action_encoder.layer1.weight"], p["action_encoder.layer1.bias"])
    tau = d4d_tau_encoding(timesteps[:, None].expand(B, T), a.shape[-1]).to(a.dtype)
    x = F.linear(torch.cat([a, tau], dim=-1), p["action_encoder.layer2.weight"], p["action_encoder.layer2.bias"])
    x = x * torch.sigmoid(x)
    return F.linear(x, p["action_encoder.layer3.weight"], p["action_encoder.layer3.bias"])


def d4d_block(p: Params, cfg: DiT4DiTHeadConfig, idx: int, x: torch.Tensor, ctx: torch.Tensor,
              temb: torch.Tensor) -> torch.Tensor:
    """BasicTransformerBlock.forward with norm_type 'ada_norm', no positional embedding
    (cross_attention_dit.py:150-187):
      AdaLayerNorm (:59-67): (scale, shift) = chunk(Linear(SiLU(temb)), 2); LN(x)(1 + scale) + shift
      diffusers Attention: q = to_q(h), k = to_k(c), v = to_v(c) with c = ctx (cross) or h (self),
        SDPA with scale 1/sqrt(head_dim), to_out.0 (dropout inactive at inference)
      x = attn + x;  norm3 = LN(no affine);  FeedForward 'gelu-approximate': net.2(GELU_tanh(net.0.proj(h)))
      x = ff + x."""
    b = f"model.transformer_blocks.{idx}."
    mod = F.linear(F.silu(temb), p[b + "norm1.linear.weight"], p[b + "norm1.linear.bias"])
    scale, shift = mod.chunk(2, dim=1)
    D = cfg.dim
    h = F.layer_norm(x, (D,), eps=cfg.norm_eps) * (1 + scale[:, None]) + shift[:, None]
    c = ctx if cfg.is_cross(idx) else h
    q = F.linear(h, p[b + "attn1.to_q.weight"], p[b + "attn1.to_q.bias"])
    k = F.linear(c, p[b + "attn1.to_k.weight"], p[b + "attn1.to_k.bias"])
    v = F.linear(c, p[b + "attn1.to_v.weight"], p[b + "attn1.to_v.bias"])
    o = flash_attention(q, k, v, cfg.heads)
    x = F.linear(o, p[b + "attn1.to_out.0.weight"], p[b + "attn1.to_out.0.bias"]) + x
    h = F.layer_norm(x, (D,), eps=cfg.norm_eps)
    h = gelu_tanh(F.linear(h, p[b + "ff.net.0.proj.weight"], p[b + "ff.net.0.proj.bias"]))
    return F.linear(h, p[b + "ff.net.2.weight"], p[b + "ff.net.2.bias"]) + x


def d4d_dit_forward(p: Params, cfg: DiT4DiTHeadConfig, x: torch.Tensor, ctx: torch.Tensor,
                    timesteps: torch.Tensor) -> torch.Tensor:
    """DiT.forward (cross_attention_dit.py:264-308): blocks, then (shift, scale) =
    chunk(proj_out_1(SiLU(temb)), 2), LN_1e-6(x)(1 + scale) + shift, proj_out_2."""
    temb = d4d_temb(p, timesteps, x.dtype)
    for i in range(cfg.num_layers):
        x = d4d_block(p, cfg, i, x, ctx, temb)
    shift, scale = F.linear(F.silu(temb), p["model.proj_out_1.weight"], p["model.proj_out_1.bias"]).chunk(2, dim=1)
    x = F.layer_norm(x, (cfg.dim,), eps=cfg.out_eps) * (1 + scale[:, None]) + shift[:, None]
    return F.linear(x, p["model.proj_out_2.weight"], p["model.proj_out_2.bias"])


def d4d_timesteps(cfg: DiT4DiTHeadConfig) -> List[int]:
    """Discrete timesteps of predict_action: int((1 - i/N) * buckets) (DB/ActionDiT.py:339-341)."""
    return [int((1.0 - i / float(cfg.num_steps)) * cfg.buckets) for i in range(cfg.num_steps)]


def d4d_mlp(p: Params, prefix: str, x: torch.Tensor) -> torch.Tensor:
    """MLP.forward (DB/ActionDiT.py:64-71): layer2(ReLU(layer1(x)))."""
    h = F.relu(F.linear(x, p[prefix + "layer1.weight"], p[prefix + "layer1.bias"]))
    return F.linear(h, p[prefix + "layer2.weight"], p[prefix + "layer2.bias"])


def d4d_predict_action(p: Params, cfg: DiT4DiTHeadConfig, vl_embs: torch.Tensor, noise: torch.Tensor,
                       state: Optional[torch.Tensor] = None) -> torch.Tensor:
    """FlowmatchingActionHead.predict_action (DB/ActionDiT.py:321-369): state features =
    state_encoder(state) once per call (:333) when a state [B, Ls, state_dim] is given; per step,
    encode (actions, t), add position embeddings (:349-352), prepend the state features (:355-356),
    DiT, action decoder MLP, actions = actions - dt * velocity[:, -horizon:] (dt = 1/N)."""
    B, T, _ = noise.shape
    actions = noise
    dt = 1.0 / cfg.num_steps
    pos = p["position_embedding.weight"][:T].unsqueeze(0)
    sfeat = d4d_mlp(p, "state_encoder.", state) if state is not None else None
    for t_disc in d4d_timesteps(cfg):
        ts = torch.full((B,), t_disc, dtype=torch.long)
        feats = d4d_action_encoder(p, actions, ts) + pos
        if sfeat is not None:
            feats = torch.cat([sfeat, feats], dim=1)
        out = d4d_dit_forward(p, cfg, feats, vl_embs, ts)
        pred = d4d_mlp(p, "action_decoder.", out)
        actions = actions - dt * pred[:, -cfg.horizon:]
    return actions


# ---------------------------------------------------------------------------
# Wan2.2 VAE (VAE38) encoder, first frame only (fp32)
# ---------------------------------------------------------------------------
@dataclass
class WanVaeConfig:
    """VideoVAE38_'s encoder shape (FB/wan_video_vae.py:1272-1295, Encoder3d_38 :619-676):
    dims = dim * [1] + dim_mult, two residual blocks per level, spatial /2 after every level
    but the last, temporal /2 after levels 1 and 2 (inert on the first frame)."""
    dim: int = 160
    z_dim: int = 48
    dim_mult: Tuple[int, ...] = (1, 2, 4, 4)
    num_res_blocks: int = 2
    temporal_downsample: Tuple[bool, ...] = (False, True, True)

    def dims(self) -> List[int]:
        return [self.dim * u for u in (1,) + tuple(self.dim_mult)]


def wan_vae_param_shapes(cfg: WanVaeConfig) -> Dict[str, Tuple[int, ...]]:
    """The encoder's state-dict entries that the first frame reads, under the reference's names
    (VideoVAE38_ state dict: "encoder.*", "conv1.*").  The downsample3d time_conv weights exist
    in the checkpoint but never run on the first chunk (Resample.forward, FB/wan_video_vae.py:162-167)."""
    d = cfg.dims()
    s = {"encoder.conv1.weight": (d[0], 12, 3, 3, 3), "encoder.conv1.bias": (d[0],)}

    def res(pre, ci, co):
        s[pre + "residual.0.gamma"] = (ci, 1, 1, 1)
        s[pre + "residual.2.weight"] = (co, ci, 3, 3, 3)
        s[pre + "residual.2.bias"] = (co,)
        s[pre + "residual.3.gamma"] = (co, 1, 1, 1)
        s[pre + "residual.6.weight"] = (co, co, 3, 3, 3)
        s[pre + "residual.6.bias"] = (co,)
        if ci != co:
            s[pre + "shortcut.weight"] = (co, ci, 1, 1, 1)
            s[pre + "shortcut.bias"] = (co,)

    for i, (ci, co) in enumerate(zip(d[:-1], d[1:])):
        pre = f"encoder.downsamples.{i}.downsamples."
        for j in range(cfg.num_res_blocks):
            res(f"{pre}{j}.", ci if j == 0 else co, co)
        if i != len(cfg.dim_mult) - 1:
            s[f"{pre}{cfg.num_res_blocks}.resample.1.weight"] = (co, co, 3, 3)
            s[f"{pre}{cfg.num_res_blocks}.resample.1.bias"] = (co,)
    c = d[-1]
    res("encoder.middle.0.", c, c)
    s["encoder.middle.1.norm.gamma"] = (c, 1, 1)
    s["encoder.middle.1.to_qkv.weight"] = (3 * c, c, 1, 1)
    s["encoder.middle.1.to_qkv.bias"] = (3 * c,)
    s["encoder.middle.1.proj.weight"] = (c, c, 1, 1)
    s["encoder.middle.1.proj.bias"] = (c,)
    res("encoder.middle.2.", c, c)
    s["encoder.head.0.gamma"] = (c, 1, 1, 1)
    s["encoder.head.2.weight"] = (2 * cfg.z_dim, c, 3, 3, 3)
    s["encoder.head.2.bias"] = (2 * cfg.z_dim,)
    s["conv1.weight"] = (2 * cfg.z_dim, 2 * cfg.z_dim, 1, 1, 1)
    s["conv1.bias"] = (2 * cfg.z_dim,)
    return s


def init_wan_vae_params(cfg: WanVaeConfig, seed: int, std: float = 0.125) -> Params:
    """Seeded weights: convolutions N(0, std) scaled by 1/sqrt(fan_in / 64) (unit-scale outputs at
    the default std), biases N(0, std), RMS_norm gammas N(1, 0.2) (away from the identity, so that
    a misplaced gamma shows)."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for k, shape in wan_vae_param_shapes(cfg).items():
        if k.endswith("gamma"):
            out[k] = 1.0 + 0.2 * torch.randn(shape, generator=g)
        elif k.endswith("weight"):
            fan_in = math.prod(shape[1:])
            out[k] = torch.randn(shape, generator=g) * std / math.sqrt(max(fan_in, 64) / 64)
        else:
            out[k] = torch.randn(shape, generator=g) * std
    return out


def vae_patchify(x: torch.Tensor, patch: int = 2) -> torch.Tensor:
    """FB/wan_video_vae.py:196-208 on an image: 'b c (h q) (w r) -> b (c r q) h w'."""
    b, c, h, w = x.shape
    x = x.reshape(b, c, h // patch, patch, w // patch, patch)          # b c h q w r
    return x.permute(0, 1, 5, 3, 2, 4).reshape(b, c * patch * patch, h // patch, w // patch)


def vae_rms_norm(x: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    """RMS_norm (FB/wan_video_vae.py:55-70), channel-first: F.normalize over the channels
    (x / max(||x||_2, 1e-12)) * sqrt(C) * gamma."""
    return F.normalize(x, dim=1) * (x.shape[1] ** 0.5) * gamma.reshape(1, -1, 1, 1)


def vae_causal_conv_first(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """CausalConv3d (FB/wan_video_vae.py:33-52) on a single frame with no cache: the temporal
    padding is 2*pad zero frames in front, so only the last temporal tap sees the frame and the
    layer is a 2-D convolution with weight[:, :, -1] and 'same' spatial padding."""
    k = w.shape[-1]
    return F.conv2d(x, w[:, :, -1], b, padding=k // 2)


def vae_residual_block(p: Params, pre: str, x: torch.Tensor) -> torch.Tensor:
    """ResidualBlock (FB/wan_video_vae.py:267-301): shortcut (1x1x1 conv when the width changes)
    + [RMS_norm, SiLU, conv 3x3x3, RMS_norm, SiLU, (dropout), conv 3x3x3]."""
    h = x
    if pre + "shortcut.weight" in p:
        h = vae_causal_conv_first(x, p[pre + "shortcut.weight"], p[pre + "shortcut.bias"])
    y = F.silu(vae_rms_norm(x, p[pre + "residual.0.gamma"]))
    y = vae_causal_conv_first(y, p[pre + "residual.2.weight"], p[pre + "residual.2.bias"])
    y = F.silu(vae_rms_norm(y, p[pre + "residual.3.gamma"]))
    y = vae_causal_conv_first(y, p[pre + "residual.6.weight"], p[pre + "residual.6.bias"])
    return y + h


def vae_avg_down(x: torch.Tensor, out_channels: int, factor_t: int, factor_s: int) -> torch.Tensor:
    """AvgDown3D (FB/wan_video_vae.py:345-395) on one frame: the frame axis is front-padded with
    factor_t - 1 zero frames, space-time blocks of factor_t x factor_s^2 become channels
    (index c * F + t * fs^2 + i * fs + j), and each output channel is the mean of a group of
    C * F / out_channels consecutive ones."""
    b, c, h, w = x.shape
    f = factor_t * factor_s * factor_s
    xt = x.unsqueeze(2)
    if factor_t > 1:
        xt = torch.cat([torch.zeros(b, c, factor_t - 1, h, w, dtype=x.dtype), xt], 2)
    xt = xt.reshape(b, c, 1, factor_t, h // factor_s, factor_s, w // factor_s, factor_s)
    xt = xt.permute(0, 1, 3, 5, 7, 2, 4, 6).reshape(b, c * f, h // factor_s, w // factor_s)
    return xt.reshape(b, out_channels, c * f // out_channels, h // factor_s, w // factor_s).mean(dim=2)


def vae_attention_block(p: Params, pre: str, x: torch.Tensor) -> torch.Tensor:
    """AttentionBlock (FB/wan_video_vae.py:304-342): one head over the frame's h*w tokens with
    the full channel width, q | k | v = consecutive channel blocks of to_qkv."""
    b, c, h, w = x.shape
    y = vae_rms_norm(x, p[pre + "norm.gamma"])
    qkv = F.conv2d(y, p[pre + "to_qkv.weight"], p[pre + "to_qkv.bias"])           # b 3c h w
    qkv = qkv.reshape(b, 3 * c, h * w).transpose(1, 2)                             # b hw 3c
    q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
    o = attention(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1)).squeeze(1)       # b hw c
    o = o.transpose(1, 2).reshape(b, c, h, w)
    return F.conv2d(o, p[pre + "proj.weight"], p[pre + "proj.bias"]) + x


def wan_vae_encode_first_frame(p: Params, cfg: WanVaeConfig, image: torch.Tensor, mean: torch.Tensor,
                               std: torch.Tensor) -> torch.Tensor:
    """VideoVAE38_.encode (FB/wan_video_vae.py:1299-1323) of a single frame image [B, 3, H, W]
    (FB/fastwam.py:256-268 encodes the first frame this way): patchify 2x2, Encoder3d_38.forward
    (:678-732) on the first chunk, conv1, mu = first z_dim channels, (mu - mean) / std.
    Returns [B, z_dim, 1, H / 16, W / 16]."""
    d = cfg.dims()
    x = vae_patchify(image, 2)
    x = vae_causal_conv_first(x, p["encoder.conv1.weight"], p["encoder.conv1.bias"])
    nlev = len(cfg.dim_mult)
    for i, (ci, co) in enumerate(zip(d[:-1], d[1:])):
        pre = f"encoder.downsamples.{i}.downsamples."
        x_copy = x
        for j in range(cfg.num_res_blocks):
            x = vae_residual_block(p, f"{pre}{j}.", x)
        down = i != nlev - 1
        t_down = cfg.temporal_downsample[i] if i < len(cfg.temporal_downsample) else False
        if down:
            # Resample38 downsample2d / downsample3d (FB/wan_video_vae.py:245-262, :158-175):
            # ZeroPad2d((0, 1, 0, 1)) + 3x3 stride-2 conv; the time_conv waits for a second chunk
            x = F.conv2d(F.pad(x, (0, 1, 0, 1)), p[f"{pre}{cfg.num_res_blocks}.resample.1.weight"],
                         p[f"{pre}{cfg.num_res_blocks}.resample.1.bias"], stride=2)
        # Down_ResidualBlock (FB/wan_video_vae.py:442-474): + AvgDown3D of the level's input
        x = x + vae_avg_down(x_copy, co, 2 if t_down else 1, 2 if down else 1)
    x = vae_residual_block(p, "encoder.middle.0.", x)
    x = vae_attention_block(p, "encoder.middle.1.", x)
    x = vae_residual_block(p, "encoder.middle.2.", x)
    x = F.silu(vae_rms_norm(x, p["encoder.head.0.gamma"]))
    x = vae_causal_conv_first(x, p["encoder.head.2.weight"], p["encoder.head.2.bias"])
    x = F.conv2d(x, p["conv1.weight"][:, :, 0], p["conv1.bias"])
    mu = x[:, :cfg.z_dim]
    mu = (mu - mean.reshape(1, -1, 1, 1)) * (1.0 / std).reshape(1, -1, 1, 1)
    return mu.unsqueeze(2)


# ---------------------------------------------------------------------------
# The GEAK trees' fused operators (FG = src/fastwam-geak/fastwam/models/wan22, CA =
# src/cae-fastwam/fastwam/models/wan22): each restates the arithmetic of one Triton kernel in
# fp32 from the oracle's pinned primitives (layer_norm, rms_norm's RMS, attention, the
# sinusoid, gelu_tanh, silu); tests/test_oracle.py pins each against those primitives.
# ---------------------------------------------------------------------------
def geak_res_ln(x: torch.Tensor, parts: Sequence[torch.Tensor], gate: torch.Tensor, eps: float,
                ln: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                ada: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """_fw_resln_kernel (FG/mot.py:1769-1827): t = x + gate * parts[0] (+ parts[1]); returns
    (t, LN(t) * w + b) with ln = (w, b), or (t, LN(t) * (1 + scale) + shift) with
    ada = (shift, scale); gate / shift / scale broadcast over rows or given per row."""
    t = x + gate * parts[0]
    for extra in parts[1:]:
        t = t + extra
    n = layer_norm(t, None, None, eps)
    if ln is not None:
        return t, n * ln[0] + ln[1]
    return t, n * (1 + ada[1]) + ada[0]


def geak_split_combine(planes: torch.Tensor, bias: torch.Tensor, sk: int) -> torch.Tensor:
    """The split-K combine of _fw_reslnsk_kernel / _fw_qcomb_kernel (FG/mot.py:2112-2120,
    :2304-2311): the first sk fp32 planes summed in plane order, plus the bias, rounded to bf16
    once (returned in fp32)."""
    if not 1 <= sk <= planes.shape[0]:
        raise ValueError(f"sk={sk} outside [1, {planes.shape[0]}]")
    p = planes[0].float()
    for i in range(1, sk):
        p = p + planes[i].float()
    return (p + bias.float()).to(torch.bfloat16).float()


def geak_qcomb(planes: torch.Tensor, bias: torch.Tensor, wq: torch.Tensor, eps: float, sk: int) -> torch.Tensor:
    """_fw_qcomb_kernel (FG/mot.py:2290-2318): x = the split-K combine, then
    x * rsqrt(mean(x^2) + eps) * wq with no rounding between the norm and the weight."""
    x = geak_split_combine(planes, bias, sk)
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * wq.float()


def cae_qkv_post(qkv: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor, freqs: torch.Tensor, num_heads: int,
                 eps: float):
    """_fwam_qkvpost_kernel (CA/mot.py:1369-1456): from qkv [M, 3D]: RMSNorm over D of q and k
    with their weights, then each (2p, 2p + 1) pair rotated by (cos, sin) = freqs[t, 2p],
    freqs[t, 2p + 1] of token t; returns q, k, v as [H, M, hd] (head-major)."""
    M, D3 = qkv.shape
    D = D3 // 3
    hd = D // num_heads

    def nr(x, w):
        y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w
        y = y.reshape(M, num_heads, hd // 2, 2)
        c, s_ = freqs[:M, 0::2][:, None, :], freqs[:M, 1::2][:, None, :]
        r = torch.stack([y[..., 0] * c - y[..., 1] * s_, y[..., 0] * s_ + y[..., 1] * c], -1)
        return r.reshape(M, num_heads, hd).transpose(0, 1)
    q, k = nr(qkv[:, :D], qw), nr(qkv[:, D:2 * D], kw)
    return q, k, qkv[:, 2 * D:].reshape(M, num_heads, hd).transpose(0, 1)


def cae_xattn_qn(qr: torch.Tensor, qw: torch.Tensor, k: torch.Tensor, v: torch.Tensor, keep: torch.Tensor,
                 num_heads: int, eps: float) -> torch.Tensor:
    """_fwam_xattn_qn_kernel (CA/mot.py:2240-2305): q = qr rsqrt(mean(qr^2) + eps) qw over the whole
    row, then attention per head over [N, C] keys / values with keep [M, N]; [M, C]."""
    q = qr * torch.rsqrt((qr * qr).mean(-1, keepdim=True) + eps) * qw
    return flash_attention(q[None], k[None], v[None], num_heads, keep[None, None])[0]


def cae_ctx_kv_norm(g: torch.Tensor, nkw: torch.Tensor, nl: int, ahd: int, eps: float) -> torch.Tensor:
    """_fwam_ctxkv_norm_kernel (CA/mot.py:2119-2142): layer l's keys g[:, l ahd:(l + 1) ahd]
    RMS-normalised with nkw[l]; [nl, S, ahd]."""
    k = g[:, :nl * ahd].reshape(-1, nl, ahd)
    y = k * torch.rsqrt((k * k).mean(-1, keepdim=True) + eps) * nkw.reshape(nl, ahd)
    return y.transpose(0, 1)


def cae_ffn(x: torch.Tensor, w1, b1, w2, b2) -> torch.Tensor:
    """_fwam_ffn_kernel (CA/mot.py:2308-2343): W2 GELU(tanh)(W1 x + b1) + b2."""
    return linear(gelu_tanh(linear(x, w1, b1)), w2, b2)


def cae_adit_tmod(t: torch.Tensor, w0, b0, w1, b1, w2, b2, atok: torch.Tensor, aw, ab):
    """_fwam_adit_tmod_kernel (CA/action_dit.py:127-187): te = sinusoid(t) [FD], x = SiLU(W0 te + b0),
    tt = W1 x + b1, t_mod = W2 SiLU(tt) + b2, tokens = atok W_aw^T + ab; returns (tt, t_mod, tokens)."""
    te = sinusoidal_embedding_1d(w0.shape[1], t.reshape(1))
    tt = linear(silu(linear(te, w0, b0)), w1, b1)
    return tt, linear(silu(tt), w2, b2), linear(atok, aw, ab)


def _rbf(x: torch.Tensor) -> torch.Tensor:
    return x.float().to(torch.bfloat16).float()


def _mod_chunk(mod: torch.Tensor, tmod: torch.Tensor, i: int, n: int) -> torch.Tensor:
    """Chunk i (width n) of modulation + t_mod, one row shared by every token, fp32 sum."""
    return mod.reshape(-1)[i * n:(i + 1) * n].float() + tmod.reshape(-1)[i * n:(i + 1) * n].float()


def cae_mod_n3q(res: torch.Tensor, so: torch.Tensor, mod: torch.Tensor, tmod: torch.Tensor, lnw, lnb, qw, qb,
                eps: float, qn: Optional[Tuple[torch.Tensor, float]] = None):
    """_fwam_mod_n3q_kernel (CA/mot.py:2707-2780): the self-attention residual with gate_msa
    (chunk 2, rounded to bf16), norm3 (affine LayerNorm) and the cross-attention q projection:
        x = bf16(res + bf16(g bf16(so))),  n = bf16(LN(x) lnw + lnb),  cq = n qw^T + qb;
    with qn = (qnw, eps_q) the query's RMSNorm over the whole row of cq, its sum of squares taken
    on the unrounded product: cq = bf16(cq) rsqrt(mean(cq^2) + eps_q) qnw.  Returns (x, cq) fp32."""
    D = res.shape[-1]
    g = _rbf(_mod_chunk(mod, tmod, 2, D))
    x = _rbf(res.float() + _rbf(g * _rbf(so)))
    n = _rbf(layer_norm(x, None, None, eps) * lnw.float() + lnb.float())
    cq = linear(n, qw.float(), qb.float())
    if qn is not None:
        cq = _rbf(cq) * torch.rsqrt((cq * cq).mean(-1, keepdim=True) + qn[1]) * qn[0].float()
    return x, cq


def cae_attn_oproj(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, keep: torch.Tensor, wo, bo) -> torch.Tensor:
    """_fwam_attn_oproj_kernel (CA/mot.py:2563-2680): per head h, o_h = softmax(q_h k_h^T / sqrt(hd),
    keep) v_h rounded to bf16, contracted with head h's columns of wo; the sum over heads plus bo
    is what the kernel adds into its fp32 accumulator.  q [H, M, hd], k / v [H, SK, hd] (head-major),
    keep [M, SK]; returns [M, NO] fp32."""
    H, M, hd = q.shape

    def rows(t):
        return t.transpose(0, 1).reshape(1, t.shape[1], H * hd).float()
    o = flash_attention(rows(q), rows(k), rows(v), H, keep[None, None])[0]
    return linear(_rbf(o), wo.float(), bo.float())


def cae_n3q_xoproj(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, ck, cv, keep, wo, bo, nh: int, eps: float,
                   eps_q: float):
    """_fwam_n3q_xoproj_kernel (CA/mot.py:1556-1680): cae_mod_n3q with the whole-row query norm, the
    cross attention of that query (rounded to bf16) per head over ck / cv [NSEQ, NQ] rows with keep
    [M, NSEQ], and the cross o-projection.  Returns (x, the [M, NO] fp32 accumulator term)."""
    x, cq = cae_mod_n3q(res, so, mod, tmod, lnw, lnb, qw, qb, eps, qn=(qnw, eps_q))
    o = flash_attention(_rbf(cq)[None], ck[None].float(), cv[None].float(), nh, keep[None, None])[0]
    return x, linear(_rbf(o), wo.float(), bo.float())


def cae_ffn_fold(x: torch.Tensor, oacc: torch.Tensor, modc, modn, tmod, w1, b1, w2, b2, eps2: float, eps1: float):
    """_fwam_ffn_fold_kernel (CA/mot.py:2346-2430): v = x + oacc (the cross o-projection's fp32
    accumulator), norm2 AdaLN with (shift, scale) = chunks (3, 4) of modc + t_mod, the FFN on that
    (GELU(tanh) of the bf16 pre-activation), xn = v + gate_mlp (chunk 5) bf16(ffn); then the next
    block's AdaLN1 of xn with (shift, scale) = chunks (0, 1) of modn + t_mod.  Returns (xn, next
    AdaLN1 input) fp32."""
    H = x.shape[-1]
    v = x.float() + oacc.float()
    a = _rbf(adaln(v, _mod_chunk(modc, tmod, 3, H), _mod_chunk(modc, tmod, 4, H), eps2))
    h = _rbf(gelu_tanh(_rbf(linear(a, w1.float(), b1.float()))))
    xn = v + _mod_chunk(modc, tmod, 5, H) * _rbf(linear(h, w2.float(), b2.float()))
    return xn, adaln(xn, _mod_chunk(modn, tmod, 0, H), _mod_chunk(modn, tmod, 1, H), eps1)


def cae_mask_bias(am: torch.Tensor, cm: torch.Tensor, mp: int, skp: int, ncp: int):
    """_fwam_mbias_kernel (CA/mot.py:2525-2560): additive planes sb [mp, skp] (0 where row m < M
    keeps key c of am [M, SK]; padding rows keep key 0 only) and xb [mp, ncp] (0 where row m < M
    keeps context key c of cm [M or 1, NS]; padding rows none); -inf elsewhere."""
    M, SK = am.shape
    NS = cm.shape[-1]
    keep = torch.zeros(mp, skp, dtype=torch.bool)
    keep[:M, :SK] = am != 0
    keep[M:, 0] = True
    keep2 = torch.zeros(mp, ncp, dtype=torch.bool)
    keep2[:M, :NS] = torch.broadcast_to(cm != 0, (M, NS))
    ninf = torch.tensor(float("-inf"))
    return torch.where(keep, 0.0, ninf), torch.where(keep2, 0.0, ninf)


def vfp8_quantize_rows(y: torch.Tensor):
    """The per-row fp8 quantisation of CA/mot.py:3763-3850: a = max |y| per row, s = max(a, 1e-12)
    (1 / 448), q = e4m3(y (448 / max(a, 1e-12))); returns (q as float8_e4m3fn [M, D], s [M, 1])."""
    y = y.float()
    a = y.abs().amax(-1, keepdim=True).clamp_min(1e-12)
    s = a * (1.0 / 448.0)
    # a correctly rounded fp32 quotient, as the kernel's `AMAX / max(a, 1e-12)` (torch's
    # `448.0 / a` would take reciprocal(a) * 448, which rounds twice)
    mul = torch.div(torch.full_like(a, 448.0), a)
    q = (y * mul).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, s


def vfp8_row_q8(x: torch.Tensor):
    """_fwam_rowq8_kernel (CA/mot.py:3836-3849): the row as it is."""
    return vfp8_quantize_rows(x.reshape(-1, x.shape[-1]))


def vfp8_gelu_q8(x: torch.Tensor):
    """_fwam_geluq8_kernel (CA/mot.py:3817-3833): bf16(GELU_tanh(x)), quantised."""
    return vfp8_quantize_rows(_rbf(gelu_tanh(x.reshape(-1, x.shape[-1]).float())))


def vfp8_ln_mod_q8(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float):
    """_fwam_lnmodq8_kernel (CA/mot.py:3763-3787): bf16(bf16(LN(x)) (1 + scale) + shift), quantised."""
    x2 = x.reshape(-1, x.shape[-1]).float()
    n = _rbf(layer_norm(x2, None, None, eps))
    return vfp8_quantize_rows(_rbf(n * (1 + scale.reshape(-1).float()) + shift.reshape(-1).float()))


def vfp8_add_ln_mod_q8(a: torch.Tensor, b: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float):
    """_fwam_addlnmodq8_kernel (CA/mot.py:3789-3814): xo = bf16(a + b), then vfp8_ln_mod_q8 of xo;
    returns (xo, q, s)."""
    xo = _rbf(a.float() + b.float())
    q, s = vfp8_ln_mod_q8(xo, shift, scale, eps)
    return xo, q, s


# ---------------------------------------------------------------------------
# Cosmos-Predict2.5 backbone of DiT4DiT (config 4): diffusers' CosmosTransformer3DModel at
# 3996788 (scripts/dit4dit_diffusers_overlay.sh:7,35) as the reference patches it,
#   CP = src/dit4dit-geak/patches/diffusers-3996788-transformer_cosmos-geak.patch
# and as DB/modules/vlm/Cosmos25.py:60-160 drives it (the output of block extract_layer is the
# feature the head reads).  diffusers is not installed here and the reference holds no fixture
# of this model: the composition is restated from the patch (its stock and fast paths, which
# must agree, CP:2074-2130) and pinned by closed forms in tests/test_oracle.py (AdaLN-LoRA chunk
# order, the three gated sub-blocks, per-head RMSNorm, rotate-half RoPE, the 3-D table split);
# parity unpinned as to diffusers itself.
# ---------------------------------------------------------------------------
@dataclass
class CosmosConfig:
    """Cosmos-Predict2.5-2B-style transformer: hidden 2048 = 16 x 128 heads,
    28 blocks, MLP ratio 4, AdaLN-LoRA rank 256, patch (1, 2, 2), text features of width 1024
    (after the pipeline's crossattn_proj), eps 1e-6.  in_channels counts the latent channels plus
    the condition and padding masks the model concatenates (CP:2289-2360)."""
    hidden: int = 2048
    num_heads: int = 16
    head_dim: int = 128
    num_layers: int = 28
    mlp_ratio: int = 4
    in_channels: int = 18
    patch_size: Tuple[int, int, int] = (1, 2, 2)
    text_dim: int = 1024
    adaln_lora_dim: int = 256
    rope_scale: Tuple[float, float, float] = (1.0, 3.0, 3.0)
    base_fps: int = 24
    eps: float = 1e-6

    @property
    def attn_dim(self) -> int:
        return self.num_heads * self.head_dim


def cosmos_param_shapes(cfg: CosmosConfig) -> Dict[str, Tuple[int, ...]]:
    """diffusers state-dict keys of the modules the features path uses: patch_embed.proj
    (Linear, no bias), time_embed (t_embedder.linear_1 / linear_2 without bias, norm = RMSNorm),
    and per block norm{1,2,3}.linear_{1,2} (AdaLN-LoRA, no bias), attn1 / attn2 to_q / to_k /
    to_v / to_out.0 (no bias) with norm_q / norm_k (RMSNorm(head_dim)), ff.net.0.proj / ff.net.2
    (no bias)."""
    C, A, D, L = cfg.hidden, cfg.attn_dim, cfg.head_dim, cfg.adaln_lora_dim
    pt, ph, pw = cfg.patch_size
    s = {"patch_embed.proj.weight": (C, cfg.in_channels * pt * ph * pw),
         "time_embed.t_embedder.linear_1.weight": (C, C),
         "time_embed.t_embedder.linear_2.weight": (3 * C, C),
         "time_embed.norm.weight": (C,)}
    for i in range(cfg.num_layers):
        b = f"transformer_blocks.{i}."
        for n in ("norm1", "norm2", "norm3"):
            s[b + n + ".linear_1.weight"] = (L, C)
            s[b + n + ".linear_2.weight"] = (3 * C, L)
        for a, kv_in in (("attn1", C), ("attn2", cfg.text_dim)):
            s[b + a + ".to_q.weight"] = (A, C)
            s[b + a + ".to_k.weight"] = (A, kv_in)
            s[b + a + ".to_v.weight"] = (A, kv_in)
            s[b + a + ".to_out.0.weight"] = (C, A)
            s[b + a + ".norm_q.weight"] = (D,)
            s[b + a + ".norm_k.weight"] = (D,)
        s[b + "ff.net.0.proj.weight"] = (cfg.mlp_ratio * C, C)
        s[b + "ff.net.2.weight"] = (C, cfg.mlp_ratio * C)
    return s


def init_cosmos_params(cfg: CosmosConfig, seed: int, std: float = 0.02) -> Params:
    """Seeded synthetic weights, sorted-name draws, fp32: N(0, std), the RMSNorm weights N(1, 0.2)
    (away from the identity, so that a swapped or mis-indexed norm weight shows)."""
    g = torch.Generator("cpu").manual_seed(seed)
    out: Params = {}
    for name, shape in sorted(cosmos_param_shapes(cfg).items()):
        if name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or name == "time_embed.norm.weight":
            out[name] = 1.0 + torch.randn(shape, generator=g) * NORM_AFFINE_STD
        else:
            out[name] = torch.randn(shape, generator=g) * std
    return out


def cosmos_rope_tables(cfg: CosmosConfig, t: int, h: int, w: int, fps: Optional[float] = None):
    """CosmosRotaryPosEmbed.forward (CP:1953-1976): per head dim D the (t, h, w) split is
    D - 2 (D // 6 * 2), D // 6 * 2, D // 6 * 2 (128 -> 44 / 42 / 42); axis a has angles
    pos * theta_a^(-2j / dim_a), theta_a = 10000 * rope_scale[a]^(dim_a / (dim_a - 2)) (NTK);
    the temporal positions are scaled by base_fps / fps when an fps is given; freqs =
    cat([t, h, w] * 2) per token in (t, h, w) order -- the halves repeat, so pairs are
    (d, d + D / 2) -- and the tables are cos / sin in fp32, [t h w, D]."""
    D = cfg.head_dim
    dh = D // 6 * 2
    dw = dh
    dt = D - dh - dw
    rs_t, rs_h, rs_w = cfg.rope_scale

    def freqs(dim, scale):
        theta = 10000.0 * scale ** (dim / (dim - 2))
        rng = torch.arange(0, dim, 2, dtype=torch.float32)[: dim // 2] / dim
        return 1.0 / theta ** rng

    seq = torch.arange(max(t, h, w), dtype=torch.float32)
    tpos = seq[:t] if fps is None else seq[:t] / fps * cfg.base_fps
    et = torch.outer(tpos, freqs(dt, rs_t))[:, None, None, :].expand(t, h, w, dt // 2)
    eh = torch.outer(seq[:h], freqs(dh, rs_h))[None, :, None, :].expand(t, h, w, dh // 2)
    ew = torch.outer(seq[:w], freqs(dw, rs_w))[None, None, :, :].expand(t, h, w, dw // 2)
    f = torch.cat([et, eh, ew] * 2, dim=-1).reshape(t * h * w, D).float()
    return torch.cos(f), torch.sin(f)


def cosmos_apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_heads: int) -> torch.Tensor:
    """apply_rotary_emb(use_real=True, use_real_unbind_dim=-2) as CP:1311-1316: per head,
    rotated = cat(-x[D/2:], x[:D/2]); out = x cos + rotated sin in fp32, cast back.
    x [B, S, H*D], cos / sin [S, D]."""
    b, s, nd = x.shape
    xh = x.reshape(b, s, num_heads, nd // num_heads).float()
    half = xh.shape[-1] // 2
    rot = torch.cat([-xh[..., half:], xh[..., :half]], dim=-1)
    out = xh * cos[None, :, None, :] + rot * sin[None, :, None, :]
    return out.reshape(b, s, nd).to(x.dtype)


def cosmos_head_rms_norm(x: torch.Tensor, weight: torch.Tensor, num_heads: int, eps: float) -> torch.Tensor:
    """RMSNorm(head_dim) over each head of x [B, S, H*D] (norm_q / norm_k of the Cosmos attention,
    CP:1289-1308: diffusers' RMSNorm, x rsqrt(mean(x^2) + eps) cast to the weight's dtype, then
    times the weight)."""
    b, s, nd = x.shape
    return rms_norm(x.reshape(b, s, num_heads, nd // num_heads), weight, eps).reshape(b, s, nd)


def cosmos_timestep_proj(timesteps: torch.Tensor, dim: int) -> torch.Tensor:
    """diffusers Timesteps(dim, flip_sin_to_cos=True, downscale_freq_shift=0) of CosmosEmbedding:
    f_i = exp(-ln(10000) i / (dim / 2)), cat(cos(t f), sin(t f)), fp32.  [N] -> [N, dim]."""
    half = dim // 2
    f = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float32) / half)
    a = timesteps.float()[:, None] * f[None, :]
    return torch.cat([torch.cos(a), torch.sin(a)], dim=-1)


def cosmos_time_embed(p: Params, cfg: CosmosConfig, timesteps: torch.Tensor, dtype=torch.float32):
    """CosmosEmbedding (time_embed; CP:2015-2030 memoises it): the projection cast to the model
    dtype; temb = linear_2(SiLU(linear_1(proj))) [N, 3C] (the AdaLN-LoRA residual);
    embedded_timestep = RMSNorm(proj) [N, C]."""
    pr = cosmos_timestep_proj(timesteps, cfg.hidden).to(dtype)
    h = silu(F.linear(pr, p["time_embed.t_embedder.linear_1.weight"]))
    temb = F.linear(h, p["time_embed.t_embedder.linear_2.weight"])
    et = rms_norm(pr, p["time_embed.norm.weight"], cfg.eps)
    return temb, et


def cosmos_modulation(p: Params, pre: str, et: torch.Tensor, temb: torch.Tensor):
    """CosmosAdaLayerNormZero's modulation (CP:2091 restates it; fused over all units at
    CP:2148-2182): linear_2(linear_1(SiLU(e))) + temb, chunked into (shift, scale, gate)."""
    m = F.linear(F.linear(silu(et), p[pre + "linear_1.weight"]), p[pre + "linear_2.weight"]) + temb
    return m.chunk(3, dim=-1)


def cosmos_attention(p: Params, pre: str, x: torch.Tensor, ctx: Optional[torch.Tensor], cos, sin,
                     cfg: CosmosConfig, mask: Optional[torch.Tensor] = None,
                     trace: Optional[dict] = None, tag: str = "") -> torch.Tensor:
    """CosmosAttnProcessor2_0 (CP:1525-1710 stock path): q = to_q(x), k = to_k(c), v = to_v(c)
    with c = x (self) or the text (cross); per-head RMSNorm of q and k; rotate-half RoPE on both
    for self attention; SDPA; to_out.0.  No biases."""
    c = x if ctx is None else ctx
    nh = cfg.num_heads
    q = cosmos_head_rms_norm(F.linear(x, p[pre + "to_q.weight"]), p[pre + "norm_q.weight"], nh, cfg.eps)
    k = cosmos_head_rms_norm(F.linear(c, p[pre + "to_k.weight"]), p[pre + "norm_k.weight"], nh, cfg.eps)
    v = F.linear(c, p[pre + "to_v.weight"])
    if cos is not None:
        q = cosmos_apply_rope(q, cos, sin, nh)
        k = cosmos_apply_rope(k, cos, sin, nh)
    o = flash_attention(q, k, v, nh, mask)
    if trace is not None:
        trace.update({f"q{tag}": q, f"k{tag}": k, f"v{tag}": v, f"attn{tag}": o})
    return F.linear(o, p[pre + "to_out.0.weight"])


def cosmos_block(p: Params, cfg: CosmosConfig, idx: int, x: torch.Tensor, ctx: torch.Tensor,
                 et: torch.Tensor, temb: torch.Tensor, cos, sin, ctx_mask: Optional[torch.Tensor] = None,
                 trace: Optional[dict] = None) -> torch.Tensor:
    """CosmosTransformerBlock.forward (CP:1851-1879 restates the stock order): three AdaLN-Zero
    sub-blocks, each x = x + gate * f(LN(x) (1 + scale) + shift) with its own LoRA modulation,
    LN without affine at eps 1e-6: self attention (RoPE), cross attention to the text, and the
    FeedForward net.2(GELU(net.0.proj(h))) with the exact (erf) GELU.  et [B, S, C] and temb
    [B, S, 3C] per token (the frame's rows expanded, CP:2378-2400).  trace records q / k / v /
    attn of the self attention (suffix "") and the cross attention ("_x"), and x after each
    sub-block (x_self, x_cross)."""
    b = f"transformer_blocks.{idx}."

    def sub(n, x, f):
        shift, scale, gate = cosmos_modulation(p, b + n + ".", et, temb)
        h = layer_norm(x, None, None, cfg.eps) * (1 + scale) + shift
        return x + gate * f(h)

    x = sub("norm1", x, lambda h: cosmos_attention(p, b + "attn1.", h, None, cos, sin, cfg, None, trace, ""))
    if trace is not None:
        trace.update(x_self=x)
    x = sub("norm2", x, lambda h: cosmos_attention(p, b + "attn2.", h, ctx, None, None, cfg, ctx_mask, trace, "_x"))
    if trace is not None:
        trace.update(x_cross=x)
    return sub("norm3", x, lambda h: F.linear(F.gelu(F.linear(h, p[b + "ff.net.0.proj.weight"])),
                                             p[b + "ff.net.2.weight"]))


def cosmos_patch_embed(p: Params, cfg: CosmosConfig, latents: torch.Tensor) -> torch.Tensor:
    """CosmosPatchEmbed: [B, C, T, H, W] -> (t, h, w)-major tokens of (C, pt, ph, pw) features ->
    Linear without bias (diffusers; CP:1282).  Returns [B, S, hidden]."""
    B, C, T, H, W = latents.shape
    pt, ph, pw = cfg.patch_size
    x = latents.reshape(B, C, T // pt, pt, H // ph, ph, W // pw, pw).permute(0, 2, 4, 6, 1, 3, 5, 7)
    x = x.reshape(B, (T // pt) * (H // ph) * (W // pw), C * pt * ph * pw)
    return F.linear(x, p["patch_embed.proj.weight"])


def cosmos_features(p: Params, cfg: CosmosConfig, latents: torch.Tensor, timestep: torch.Tensor,
                    ctx: torch.Tensor, stop_layer: Optional[int] = None, ctx_mask: Optional[torch.Tensor] = None,
                    fps: Optional[float] = None, traces: Optional[list] = None) -> torch.Tensor:
    """CosmosTransformer3DModel.forward up to the output of block stop_layer (CP:2289-2490, the
    stop_at_layer the reference adds; DB/modules/vlm/Cosmos25.py:150-160 hooks that block):
    patch embedding, the time embedding of one timestep per latent frame ([B, T], the 5-D
    timestep of CP:2378-2400, expanded over each frame's tokens), the 3-D RoPE tables, blocks
    0 .. stop_layer.  latents [B, in_channels, T, H, W]; ctx [B, Lc, text_dim]."""
    B, _, T, H, W = latents.shape
    pt, ph, pw = cfg.patch_size
    t, h, w = T // pt, H // ph, W // pw
    x = cosmos_patch_embed(p, cfg, latents)
    ts = timestep.reshape(B, -1).expand(B, t).reshape(-1)
    temb, et = cosmos_time_embed(p, cfg, ts, x.dtype)
    temb = temb.reshape(B, t, 1, -1).expand(B, t, h * w, temb.shape[-1]).reshape(B, t * h * w, -1)
    et = et.reshape(B, t, 1, -1).expand(B, t, h * w, et.shape[-1]).reshape(B, t * h * w, -1)
    cos, sin = cosmos_rope_tables(cfg, t, h, w, fps)
    last = cfg.num_layers - 1 if stop_layer is None else stop_layer
    mask = None if ctx_mask is None else ctx_mask.reshape(B, 1, 1, -1)
    for i in range(last + 1):
        tr = {} if traces is not None else None
        x = cosmos_block(p, cfg, i, x, ctx, et, temb, cos, sin, mask, tr)
        if traces is not None:
            traces.append(tr)
    return x

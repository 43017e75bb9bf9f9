"""Drop-in operators for the reference's call sites, each backed by one C-ABI entry point.

The functions keep the reference signatures so that they replace the originals inside the
existing PyTorch modules:

    adaln_forward(x, norm, shift, scale)           FB/fused_adaln.py:513-523
    layer_norm(x, weight, bias, eps)               nn.LayerNorm (norm3, FB/wan_video_dit.py:261)
    rms_norm(x, weight, eps) / RMSNorm             FB/wan_video_dit.py:156-167
    rope_apply(x, freqs, num_heads)                FB/wan_video_dit.py:58-70, FG/wan_video_dit.py:193-215
    rope_apply_cae(x, freqs, num_heads, force_complex=False)
                                                   CA/wan_video_dit.py:769-799
    flash_attention(q, k, v, num_heads, ctx_mask=None, compatibility_mode=True)
                                                   FB/wan_video_dit.py:17-26, FG:18-39, CA:569-587
    linear(x, weight, bias)                        nn.Linear on the hot path
    euler_step(model_output, delta, sample)        WanContinuousFlowMatchScheduler.step, SCH:82-88

(FB = src/fastwam-baseline/fastwam/models/wan22, FG = src/fastwam-geak/..., CA =
src/cae-fastwam/..., SCH = FB/schedulers/scheduler_continuous.py.)

Tensors must be bf16 CUDA (HIP) tensors with a contiguous last dimension; anything else
raises -- there is no fallback implementation.  Outputs are new tensors allocated on the
input's device, launches go to torch's current stream.

Each of these functions is a thin wrapper over a ``torch.library`` custom operator in the
``fam`` namespace (``torch.ops.fam.adaln``, ``rope``, ``attention``, ``linear``,
``euler_step``) with a fake implementation, so ``torch.compile(fullgraph=True)`` and
``torch.export`` trace through them as single graph nodes, the way the reference's own
``fastwam::*`` operators are traced (FG/wan_video_dit.py:1680-1721).  The reference's
``fastwam::*`` operator forms themselves are in ``fam.fastwam_ops``.
"""
from __future__ import annotations

import ctypes as C
import math
from collections import OrderedDict
from typing import Dict, Optional, Tuple

import torch

from . import _capi
from ._capi import call

_BF16 = torch.bfloat16


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(t: torch.Tensor, name: str, dtype=_BF16, device: bool = True) -> None:
    """dtype / last-dim checks, and (device=True) that t lives on a HIP device.  The fake
    implementations run the same checks with device=False, so a traced graph rejects what the
    real operator would."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if device and t.device.type != "cuda":
        raise ValueError(f"{name} must be on a HIP device (got {t.device})")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if t.dim() > 0 and t.stride(-1) != 1 and t.shape[-1] != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")


def _rows(x: torch.Tensor) -> Tuple[torch.Tensor, int, int, int]:
    """View x as [B*S, D]; returns (2-D view, rows, rows_per_batch, D)."""
    D = x.shape[-1]
    if x.dim() == 3:
        B, S = x.shape[0], x.shape[1]
    elif x.dim() == 2:
        B, S = 1, x.shape[0]
    else:
        raise ValueError(f"expected a 2-D or 3-D tensor, got shape {tuple(x.shape)}")
    x2 = x.reshape(B * S, D)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2, B * S, S, D


# --------------------------------------------------------------------------- norms
def _broadcast_mod(t: torch.Tensor, x: torch.Tensor, name: str) -> Tuple[torch.Tensor, int, int]:
    """Broadcast shift/scale to x's shape; returns (tensor, batch stride, row stride)."""
    _check(t, name)
    tb = torch.broadcast_to(t, x.shape)
    if tb.stride(-1) != 1:
        tb = tb.contiguous()
    if x.dim() == 3:
        bs, rs = tb.stride(0), tb.stride(1)
    else:
        bs, rs = 0, tb.stride(0)
    if bs % 8 or rs % 8 or tb.data_ptr() % 16:
        tb = tb.contiguous()
        bs, rs = (tb.stride(0), tb.stride(1)) if x.dim() == 3 else (0, tb.stride(0))
    return tb, bs, rs


def _adaln_launch(x: torch.Tensor, shift, scale, weight, bias, eps: float) -> torch.Tensor:
    _check(x, "x")
    x2, rows, rpb, D = _rows(x)
    y = torch.empty((rows, D), dtype=_BF16, device=x.device)
    sh_p = sc_p = None
    bs = rs = 0
    if shift is not None:
        sh, bs, rs = _broadcast_mod(shift, x, "shift")
        sc, bs2, rs2 = _broadcast_mod(scale, x, "scale")
        if (bs, rs) != (bs2, rs2):
            sc = torch.broadcast_to(scale, x.shape).contiguous()
            sh = torch.broadcast_to(shift, x.shape).contiguous()
            bs, rs = (sh.stride(0), sh.stride(1)) if x.dim() == 3 else (0, sh.stride(0))
        sh_p, sc_p = sh.data_ptr(), sc.data_ptr()
    # every temporary whose pointer is passed stays referenced until the launch is enqueued
    wc = bc = None
    if weight is not None:
        _check(weight, "ln weight")
        wc = weight.contiguous()
    if bias is not None:
        _check(bias, "ln bias")
        bc = bias.contiguous()
    call("fam_adaln", x2.data_ptr(), x2.stride(0), sh_p, sc_p, bs, rs,
         wc.data_ptr() if wc is not None else None, bc.data_ptr() if bc is not None else None,
         y.data_ptr(), D, rows, rpb, D, float(eps), _stream(x))
    return y.reshape(x.shape)


@torch.library.custom_op("fam::adaln", mutates_args=())
def _adaln_op(x: torch.Tensor, shift: Optional[torch.Tensor], scale: Optional[torch.Tensor],
              weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """LayerNorm over the last dim (optional affine), then optional modulation (1 + scale), + shift."""
    if (shift is None) != (scale is None):
        raise ValueError("adaln: shift and scale go together")
    return _adaln_launch(x, shift, scale, weight, bias, eps)


@_adaln_op.register_fake
def _adaln_fake(x, shift, scale, weight, bias, eps):
    _check(x, "x", device=False)
    if x.dim() not in (2, 3):
        raise ValueError(f"expected a 2-D or 3-D tensor, got shape {tuple(x.shape)}")
    if (shift is None) != (scale is None):
        raise ValueError("adaln: shift and scale go together")
    return x.new_empty(x.shape)


def adaln_forward(x: torch.Tensor, norm: torch.nn.LayerNorm, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """norm(x) * (1 + scale) + shift in one kernel (FB/fused_adaln.py:513-523).

    `norm` is the block's nn.LayerNorm (its eps and, if elementwise_affine, weight/bias are
    used); shift/scale broadcast as [B,1,D] (per sample) or [B,S,D] (per token)."""
    w = norm.weight if getattr(norm, "elementwise_affine", False) else None
    b = norm.bias if getattr(norm, "elementwise_affine", False) else None
    return torch.ops.fam.adaln(x, shift, scale, w, b, float(norm.eps))


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """nn.LayerNorm forward over the last dim (FB/wan_video_dit.py:258-261)."""
    return torch.ops.fam.adaln(x, None, None, weight, bias, float(eps))


def modulate_layer_norm(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """modulate(LayerNorm(x, affine=False), shift, scale) -- the CAE form (CA/wan_video_dit.py:590-591)."""
    return torch.ops.fam.adaln(x, shift, scale, None, None, float(eps))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward: bf16(x*rsqrt(mean(x^2)+eps)) * weight (FB/wan_video_dit.py:156-167)."""
    return torch.ops.fam.rope(x, None, 1, "none", weight, float(eps))


class RMSNorm(torch.nn.Module):
    """Module form with the reference's parameter layout (`weight` [dim], eps)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.weight, self.eps)


# --------------------------------------------------------------------------- rope
# (source tensor, cos, sin, row stride, element stride) per source; the entry holds the source
# itself, so its address cannot be handed to another tensor while the entry exists and the key
# (address, shape, strides, dtype, version) names one content
_TABLES: "OrderedDict[tuple, tuple]" = OrderedDict()
_TABLES_MAX = 64


def _check_pair_layout(f: torch.Tensor, layout: str, src_dtype: torch.dtype = torch.float32) -> None:
    """Reject a real table whose (cos, sin) pairs are not where `layout` says: FG packs
    cat(cos, sin) per row, CA interleaves (cos, sin) pairs, and both are [S, 1, Dh] -- read
    with the other convention, every position rotates the wrong pairs.  The pairs of the right
    layout have unit modulus up to the rounding of the table's own dtype (FG's pack_rope_real
    takes a dtype: a bf16 table is off by up to ~8e-3); position 0 of the other layout pairs
    (1, 1) or (0, 0), a deviation of 1."""
    tol = max(1e-3, 8.0 * torch.finfo(src_dtype).eps) if src_dtype.is_floating_point else 1e-3
    half = f.shape[1] // 2
    c, s_ = (f[:, :half], f[:, half:]) if layout == "cat" else (f[:, 0::2], f[:, 1::2])
    dev = (c.double() ** 2 + s_.double() ** 2 - 1.0).abs().max().item() if f.numel() else 0.0
    if dev > tol:
        other = "rope_apply_cae (CA's interleaved (cos, sin) table)" if layout == "cat" else \
            "rope_apply (FG's packed cat(cos, sin) table)"
        raise ValueError(f"freqs is not a {layout!r} RoPE table (|cos|^2 + |sin|^2 deviates from 1 by {dev:.3g}); "
                         f"a table in the other packing belongs to {other}")


def rope_tables(freqs: torch.Tensor, layout: str, device: torch.device):
    """(cos, sin, row stride, element stride) fp32 device tables for a RoPE `freqs` tensor.

    layout 'complex'     complex [S, 1, Dh/2] (FB/wan_video_dit.py:49-55)
           'cat'         real [S, 1, Dh] = cat(cos, sin) (FG/wan_video_dit.py:173-177)
           'interleaved' real [S, 1, Dh] = (cos0, sin0, cos1, sin1, ...) (CA/wan_video_dit.py:736-766)

    A real fp32 table already on `device` with unit-stride rows is used in place (views of the
    source, no copy).  Anything else (complex, fp64, host) is converted once per source tensor
    and cached; the first use of a real table checks its packing (a host sync), so a caller that
    captures a graph makes one eager call per table first."""
    if layout not in ("complex", "cat", "interleaved"):
        raise ValueError(f"unknown RoPE layout {layout!r}")
    if layout == "complex" and not freqs.is_complex():
        raise ValueError("layout 'complex' needs a complex freqs tensor")
    if layout != "complex" and freqs.is_complex():
        raise ValueError(f"layout {layout!r} needs a real freqs tensor")
    key = (freqs.data_ptr(), tuple(freqs.shape), tuple(freqs.stride()), freqs.dtype, str(freqs.device),
           freqs._version, layout, str(device))
    hit = _TABLES.get(key)
    if hit is not None:
        _TABLES.move_to_end(key)
        return hit[1:]
    S = freqs.shape[0]
    if layout == "complex":
        f = freqs.reshape(S, -1)
        cos = f.real.to(device=device, dtype=torch.float32).contiguous()
        sin = f.imag.to(device=device, dtype=torch.float32).contiguous()
        res = (cos, sin, cos.shape[1], 1)
    else:
        f = freqs.reshape(S, -1)
        if not (f.dtype == torch.float32 and f.device == torch.device(device) and f.stride(-1) == 1
                and f.data_ptr() % 16 == 0):
            f = f.to(device=device, dtype=torch.float32).contiguous()
        _check_pair_layout(f, layout, freqs.dtype)
        half = f.shape[1] // 2
        if layout == "cat":
            res = (f, f[:, half:], f.stride(0), 1)
        else:
            res = (f, f[:, 1:], f.stride(0), 2)
    _TABLES[key] = (freqs,) + res
    while len(_TABLES) > _TABLES_MAX:
        _TABLES.popitem(last=False)
    return res


def _rope_launch(x: torch.Tensor, freqs: Optional[torch.Tensor], num_heads: int, layout: str,
                 weight: Optional[torch.Tensor] = None, eps: float = 0.0) -> torch.Tensor:
    _check(x, "x")
    if weight is not None:
        _check(weight, "weight")
    x2, rows, S, D = _rows(x)
    y = torch.empty((rows, D), dtype=_BF16, device=x.device)
    wc = weight.contiguous() if weight is not None else None
    w_p = wc.data_ptr() if wc is not None else None
    if layout == "none":
        call("fam_rmsnorm_rope", x2.data_ptr(), x2.stride(0), y.data_ptr(), D, rows, 1, D, w_p, float(eps),
             None, None, 0, 0, 0, _stream(x))
        return y.reshape(x.shape)
    _rope_shape(x, freqs, num_heads)
    cos, sin, trs, tes = rope_tables(freqs, layout, x.device)
    call("fam_rmsnorm_rope", x2.data_ptr(), x2.stride(0), y.data_ptr(), D, rows, S, D, w_p, float(eps),
         cos.data_ptr(), sin.data_ptr(), trs, tes, D // num_heads, _stream(x))
    return y.reshape(x.shape)


def _rope_shape(x: torch.Tensor, freqs: Optional[torch.Tensor], num_heads: int) -> None:
    if x.dim() != 3:
        raise ValueError(f"x must be [B, S, H*Dh], got {tuple(x.shape)}")
    if freqs is None:
        raise ValueError("a RoPE layout needs freqs")
    B, S, ND = x.shape
    if num_heads <= 0 or ND % num_heads:
        raise ValueError(f"last dim {ND} not divisible by num_heads {num_heads}")
    if freqs.shape[0] < S:
        raise ValueError(f"freqs has {freqs.shape[0]} positions, need {S}")


@torch.library.custom_op("fam::rope", mutates_args=())
def _rope_op(x: torch.Tensor, freqs: Optional[torch.Tensor], num_heads: int, layout: str,
             weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """Optional RMSNorm (weight given; bf16 rounding before the weight) then the rotation of
    `layout` ('complex', 'cat', 'interleaved', or 'none' for the norm alone)."""
    if layout not in ("none", "complex", "cat", "interleaved"):
        raise ValueError(f"unknown RoPE layout {layout!r}")
    return _rope_launch(x, freqs, num_heads, layout, weight, eps)


@_rope_op.register_fake
def _rope_fake(x, freqs, num_heads, layout, weight, eps):
    _check(x, "x", device=False)
    if layout not in ("none", "complex", "cat", "interleaved"):
        raise ValueError(f"unknown RoPE layout {layout!r}")
    if layout != "none":
        _rope_shape(x, freqs, num_heads)
    elif x.dim() not in (2, 3):
        raise ValueError(f"expected a 2-D or 3-D tensor, got shape {tuple(x.shape)}")
    return x.new_empty(x.shape)


def rope_apply(x: torch.Tensor, freqs: torch.Tensor, num_heads: int) -> torch.Tensor:
    """Rotary embedding with the FB/FG call signature: freqs complex [S,1,Dh/2] or packed
    real cat(cos, sin) [S,1,Dh] (FB/wan_video_dit.py:58-70, FG/wan_video_dit.py:193-215).
    A real table in CA's interleaved packing is rejected (it belongs to rope_apply_cae)."""
    return torch.ops.fam.rope(x, freqs, int(num_heads), "complex" if freqs.is_complex() else "cat", None, 0.0)


def rope_apply_cae(x: torch.Tensor, freqs: torch.Tensor, num_heads: int, force_complex: bool = False) -> torch.Tensor:
    """Rotary embedding with the CAE call signature: freqs complex or interleaved real
    (cos, sin) pairs [S,1,Dh] (CA/wan_video_dit.py:769-799).  force_complex only selects the
    reference's arithmetic route; the rotation is the same.  A real table in FG's
    cat(cos, sin) packing is rejected (it belongs to rope_apply)."""
    del force_complex
    return torch.ops.fam.rope(x, freqs, int(num_heads), "complex" if freqs.is_complex() else "interleaved", None,
                              0.0)


def rms_norm_rope(x: torch.Tensor, weight: torch.Tensor, eps: float, freqs: torch.Tensor, num_heads: int,
                  layout: str = "complex") -> torch.Tensor:
    """rope_apply(RMSNorm(x), freqs) in one kernel (the q/k post-processing, FG/mot.py:786-816)."""
    return torch.ops.fam.rope(x, freqs, int(num_heads), layout, weight, float(eps))


# --------------------------------------------------------------------------- attention
def _mask_args(mask: Optional[torch.Tensor], B: int, H: int, Sq: int, Sk: int):
    if mask is None:
        return None, _capi.FAM_MASK_NONE, 0, 0, 0, None
    if mask.device.type != "cuda":
        raise ValueError("ctx_mask must be on the device of q")
    if mask.dtype == torch.bool:
        kind = _capi.FAM_MASK_BOOL
        m = mask
    elif mask.dtype == torch.float32:
        kind, m = _capi.FAM_MASK_ADD_F32, mask
    elif mask.dtype == torch.bfloat16:
        kind, m = _capi.FAM_MASK_ADD_BF16, mask
    else:
        kind, m = _capi.FAM_MASK_ADD_F32, mask.float()
    m4 = torch.broadcast_to(m, (B, H, Sq, Sk))
    if m4.stride(-1) != 1:
        m4 = m4.contiguous()
    return m4.data_ptr(), kind, m4.stride(0), m4.stride(1), m4.stride(2), m4


def _attn_desc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
               mask: Optional[torch.Tensor] = None, scale: Optional[float] = None,
               k_prefix: Optional[torch.Tensor] = None, v_prefix: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None, qk_norm: Optional[dict] = None):
    """fam_attn_desc for [B, S, H*Dh] tensors (see attention_bshd); returns (desc, out, keep),
    keep = tensors the descriptor points into (a converted mask) that must outlive the launch."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n)
        if t.dim() != 3:
            raise ValueError(f"{n} must be [B, S, H*Dh], got {tuple(t.shape)}")
    B, Sq, ND = q.shape
    Dh = ND // num_heads
    if ND % num_heads or k.shape[-1] != ND or v.shape[-1] != ND:
        raise ValueError("q/k/v last dims must equal num_heads * head_dim")
    if k.shape[:2] != v.shape[:2]:
        raise ValueError("k and v must have the same [B, S]")
    if k.shape[0] != B and k.shape[0] != 1:
        raise ValueError("k batch must equal q batch (or 1 to broadcast)")
    segs = []
    if k_prefix is not None:
        _check(k_prefix, "k_prefix")
        _check(v_prefix, "v_prefix")
        segs.append((k_prefix, v_prefix))
    segs.append((k, v))
    Sk = sum(s[0].shape[1] for s in segs)
    if out is None:
        out = torch.empty((B, Sq, ND), dtype=_BF16, device=q.device)
    d = _capi.AttnDesc()
    d.q, d.q_bs, d.q_rs, d.q_hs = q.data_ptr(), q.stride(0), q.stride(1), Dh
    (k0, v0) = segs[0]
    d.k0, d.k0_bs, d.k0_rs, d.k0_hs = k0.data_ptr(), (k0.stride(0) if k0.shape[0] == B else 0), k0.stride(1), Dh
    d.v0, d.v0_bs, d.v0_rs, d.v0_hs = v0.data_ptr(), (v0.stride(0) if v0.shape[0] == B else 0), v0.stride(1), Dh
    d.sk0 = k0.shape[1]
    if len(segs) > 1:
        (k1, v1) = segs[1]
        d.k1, d.k1_bs, d.k1_rs, d.k1_hs = k1.data_ptr(), (k1.stride(0) if k1.shape[0] == B else 0), k1.stride(1), Dh
        d.v1, d.v1_bs, d.v1_rs, d.v1_hs = v1.data_ptr(), (v1.stride(0) if v1.shape[0] == B else 0), v1.stride(1), Dh
        d.sk1 = k1.shape[1]
    d.o, d.o_bs, d.o_rs, d.o_hs = out.data_ptr(), out.stride(0), out.stride(1), Dh
    d.batch, d.heads, d.sq, d.head_dim = B, num_heads, Sq, Dh
    d.scale = (1.0 / math.sqrt(Dh)) if scale is None else float(scale)
    mp, kind, mbs, mhs, mqs, keep = _mask_args(mask, B, num_heads, Sq, Sk)
    d.mask, d.mask_kind, d.mask_bs, d.mask_hs, d.mask_qs = mp, kind, mbs, mhs, mqs
    if qk_norm is not None:
        # on-load RMSNorm (+ RoPE) of q / k from fam_gemm_final sums of squares (include/fam_hip.h)
        n = qk_norm
        d.qk_norm = 1
        qs, ks = n.get("q_sumsq"), n.get("k_sumsq")
        ss = qs if qs is not None else ks
        d.q_sumsq = qs.data_ptr() if qs is not None else None
        d.k_sumsq = ks.data_ptr() if ks is not None else None
        d.ss_row_stride, d.ss_batch_rows = ss.stride(0), n["ss_batch_rows"]
        d.q_group0, d.k_group0, d.norm_width = n.get("q_group0", 0), n.get("k_group0", 0), n["norm_width"]
        d.q_norm_w = n["q_norm_w"].data_ptr() if qs is not None else None
        d.k_norm_w = n["k_norm_w"].data_ptr() if ks is not None else None
        d.norm_eps = float(n.get("eps", 1e-6))
        if n.get("rope") is not None:
            cs, sn, trs = n["rope"]
            d.rope_cos, d.rope_sin, d.rope_row_stride = cs.data_ptr(), sn.data_ptr(), trs
    return d, out, keep


def _attention_launch(q, k, v, num_heads, mask, scale, k_prefix, v_prefix, out, num_splits, qk_norm):
    d, out, keep = _attn_desc(q, k, v, num_heads, mask, scale, k_prefix, v_prefix, out, qk_norm)
    B, Sq, ND = q.shape
    Dh = ND // num_heads
    if num_splits > 1:
        # key splits over workgroups: per-split partials, then an ordered merge
        nq = B * num_heads * Sq
        part_o = torch.empty(num_splits * nq * Dh, dtype=torch.float32, device=q.device)
        part_ml = torch.empty(num_splits * nq * 2, dtype=torch.float32, device=q.device)
        d.num_splits, d.part_o, d.part_ml = num_splits, part_o.data_ptr(), part_ml.data_ptr()
    call("fam_attention", C.byref(d), _stream(q))
    if num_splits > 1:
        call("fam_attention_combine", C.byref(d), _stream(q))
    del keep
    return out


@torch.library.custom_op("fam::attention", mutates_args=())
def _attention_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor], num_heads: int,
                  scale: Optional[float], k_prefix: Optional[torch.Tensor], v_prefix: Optional[torch.Tensor],
                  num_splits: int) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v over [B, S, H*Dh] tensors, keys cat(k_prefix, k)."""
    return _attention_launch(q, k, v, num_heads, mask, scale, k_prefix, v_prefix, None, num_splits, None)


@_attention_op.register_fake
def _attention_fake(q, k, v, mask, num_heads, scale, k_prefix, v_prefix, num_splits):
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n, device=False)
        if t.dim() != 3:
            raise ValueError(f"{n} must be [B, S, H*Dh], got {tuple(t.shape)}")
    if num_heads <= 0 or q.shape[-1] % num_heads or k.shape[-1] != q.shape[-1] or v.shape[-1] != q.shape[-1]:
        raise ValueError("q/k/v last dims must equal num_heads * head_dim")
    return q.new_empty(q.shape)


def attention_bshd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
                   mask: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                   k_prefix: Optional[torch.Tensor] = None, v_prefix: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None, num_splits: int = 1,
                   qk_norm: Optional[dict] = None) -> torch.Tensor:
    """Attention on [B, S, H*Dh] tensors; keys/values are cat(k_prefix, k) when a prefix is
    given (the MoT joint attention over a cached video K/V, FB/mot.py:446-478) without
    materialising the concatenation.  With `out` or `qk_norm` (the fused models' on-load
    normalisation from fam_gemm_final sums of squares) the launch is direct, not an operator."""
    if out is not None or qk_norm is not None:
        return _attention_launch(q, k, v, num_heads, mask, scale, k_prefix, v_prefix, out, num_splits, qk_norm)
    return torch.ops.fam.attention(q, k, v, mask, int(num_heads), scale, k_prefix, v_prefix, int(num_splits))


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
                    ctx_mask: Optional[torch.Tensor] = None, compatibility_mode: bool = True) -> torch.Tensor:
    """softmax(q k^T / sqrt(Dh) + mask) v over [B, S, H*Dh] tensors -> [B, Sq, H*Dh]
    (FB/wan_video_dit.py:17-26).  Bool masks keep True entries; float masks are added."""
    if not compatibility_mode:
        raise NotImplementedError("Only compatibility mode is implemented for flash attention. "
                                  "Please set compatibility_mode=True.")
    return torch.ops.fam.attention(q, k, v, ctx_mask, int(num_heads), None, None, None, 1)


# --------------------------------------------------------------------------- linear
@torch.library.custom_op("fam::linear", mutates_args=())
def _linear_op(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
    """y = x W^T + b, bf16 in and out, fp32 accumulation."""
    _check(x, "x")
    _check(weight, "weight")
    K = x.shape[-1]
    N = weight.shape[0]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise ValueError(f"weight {tuple(weight.shape)} does not match input features {K}")
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    w = weight if weight.is_contiguous() else weight.contiguous()
    b = None
    if bias is not None:
        _check(bias, "bias")
        b = bias.contiguous()
    y = torch.empty((M, N), dtype=_BF16, device=x.device)
    aligned = (K % 8 == 0 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0)
    if not aligned:
        if K > 64:
            x2 = x2.contiguous()
            if x2.data_ptr() % 16 or K % 8:
                raise ValueError(f"linear: unsupported K={K} (needs K % 8 == 0 or K <= 64)")
        else:
            call("fam_linear_smallk", x2.data_ptr(), x2.stride(0), 0, w.data_ptr(),
                 b.data_ptr() if b is not None else None, y.data_ptr(), N, M, N, K, _stream(x))
            return y.reshape(*x.shape[:-1], N)
    gemm(x2, w, b, y)
    return y.reshape(*x.shape[:-1], N)


@_linear_op.register_fake
def _linear_fake(x, weight, bias):
    _check(x, "x", device=False)
    _check(weight, "weight", device=False)
    if weight.dim() != 2 or weight.shape[1] != x.shape[-1]:
        raise ValueError(f"weight {tuple(weight.shape)} does not match input features {x.shape[-1]}")
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x W^T + b for bf16 x [..., K], W [N, K] (nn.Linear)."""
    return torch.ops.fam.linear(x, weight, bias)


def gemm(a: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], out: torch.Tensor, *,
         prologue: int = _capi.FAM_PRO_NONE, pro_w=None, pro_b=None, pro_shift=None, pro_scale=None,
         pro_mod_bs: int = 0, pro_mod_rs: int = 0, pro_eps: float = 1e-6, act: int = _capi.FAM_ACT_NONE,
         res: Optional[torch.Tensor] = None, gate: Optional[torch.Tensor] = None, gate_bs: int = 0,
         gate_rs: int = 0, gate_ns: int = 1, rows_per_batch: Optional[int] = None, out_f32: bool = False,
         ws: Optional[torch.Tensor] = None) -> None:
    """Fused GEMM on 2-D views (see fam_gemm in include/fam_hip.h): a [M, K], w [N, K], out [M, N].
    With prologue=FAM_PRO_LN_FOLDED, pro_w is the fp32 [N] column-sum vector of `fold_layernorm`.
    ws: an fp32 workspace (fam_gemm_ws): the library may then split K over workgroups (sized by
    `gemm_ws_floats(M, N, K)`; a smaller one limits the splits)."""
    M, K = a.shape
    N = w.shape[0]
    if prologue == _capi.FAM_PRO_LN_FOLDED:
        if pro_w is None or pro_w.dtype != torch.float32 or pro_w.numel() != N or not pro_w.is_contiguous():
            raise ValueError("FAM_PRO_LN_FOLDED needs pro_w = fp32 contiguous [N] column sums of w")
    d = _capi.GemmDesc()
    d.a, d.lda = a.data_ptr(), a.stride(0)
    d.w, d.ldw = w.data_ptr(), w.stride(0)
    d.bias = bias.data_ptr() if bias is not None else None
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    d.M, d.N, d.K = M, N, K
    d.prologue = prologue
    d.pro_w = pro_w.data_ptr() if pro_w is not None else None
    d.pro_b = pro_b.data_ptr() if pro_b is not None else None
    d.pro_shift = pro_shift.data_ptr() if pro_shift is not None else None
    d.pro_scale = pro_scale.data_ptr() if pro_scale is not None else None
    d.pro_mod_bs, d.pro_mod_rs, d.pro_eps = pro_mod_bs, pro_mod_rs, float(pro_eps)
    d.act = act
    d.res, d.ldr = (res.data_ptr(), res.stride(0)) if res is not None else (None, 0)
    d.gate = gate.data_ptr() if gate is not None else None
    d.gate_bs, d.gate_rs, d.gate_ns = gate_bs, gate_rs, gate_ns
    d.rows_per_batch = rows_per_batch if rows_per_batch is not None else max(M, 1)
    d.out_f32 = int(out_f32)
    if ws is not None:
        if ws.dtype != torch.float32 or not ws.is_contiguous() or ws.device != a.device:
            raise ValueError("ws must be a contiguous fp32 tensor on the device of a")
        call("fam_gemm_ws", C.byref(d), ws.data_ptr(), ws.numel(), _stream(a))
    else:
        call("fam_gemm", C.byref(d), _stream(a))


def gemm_ws_floats(M: int, N: int, K: int) -> int:
    """Workspace (fp32 elements) with which fam_gemm_ws may choose any K split for this shape."""
    return int(_capi.load().fam_gemm_ws_floats(M, N, K))


def fold_layernorm(w: torch.Tensor, bias: Optional[torch.Tensor] = None, *, ln_weight: Optional[torch.Tensor] = None,
                   ln_bias: Optional[torch.Tensor] = None, scale: Optional[torch.Tensor] = None,
                   shift: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fold what follows a LayerNorm and precedes a linear layer -- its affine (ln_weight,
    ln_bias) and an AdaLN modulation (1 + scale, shift), each one [K] vector for every row --
    into the layer, for fam_gemm's FAM_PRO_LN_FOLDED:

        ((LN(x) * ln_weight + ln_bias) * (1 + scale) + shift) w^T + bias
          = rstd * (x w'^T - mean * colsum) + bias'

    with w' = w diag(g), g = ln_weight (1 + scale); bias' = bias + w c, c = ln_bias (1 + scale)
    + shift; colsum[n] = sum_k w'[n, k] of the bf16 w' (fp32).  Returns (w' bf16, bias' bf16,
    colsum fp32), all on w's device.  A weight-preparation step (run once per weight and
    modulation), not a hot-path op."""
    N, K = w.shape
    dev = w.device
    g = torch.ones(K, dtype=torch.float64, device=dev)
    c = torch.zeros(K, dtype=torch.float64, device=dev)
    if ln_weight is not None:
        g = ln_weight.to(torch.float64).reshape(K)
    if ln_bias is not None:
        c = ln_bias.to(torch.float64).reshape(K)
    if scale is not None:
        s1 = 1.0 + scale.to(torch.float64).reshape(K)
        g, c = g * s1, c * s1
    if shift is not None:
        c = c + shift.to(torch.float64).reshape(K)
    w64 = w.to(torch.float64)
    w2 = (w64 * g[None, :]).to(_BF16).contiguous()
    b2 = w64 @ c
    if bias is not None:
        b2 = b2 + bias.to(torch.float64).reshape(N)
    colsum = w2.to(torch.float64).sum(dim=1).to(torch.float32).contiguous()
    return w2, b2.to(_BF16).contiguous(), colsum


def gemm_partial(a: torch.Tensor, w: torch.Tensor):
    """Split-K partials of a [M, K] x w [N, K]^T: returns ([S, M, N] fp32, S) (the shapes
    fam_gemm_partial takes; S = 0 for one it does not)."""
    _check(a, "a")
    _check(w, "w")
    M, K = a.shape
    N = w.shape[0]
    S = _capi.lib().fam_gemm_partial_splits(M, N, K)
    if S <= 0:
        raise ValueError(f"fam_gemm_partial does not take M={M} N={N} K={K} (fam_gemm_partial_splits is 0)")
    part = torch.empty((S, M, N), dtype=torch.float32, device=a.device)
    call("fam_gemm_partial", a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), part.data_ptr(), M, N, K,
         _stream(a))
    return part, S


def gemm_final(a: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor] = None, act: int = _capi.FAM_ACT_NONE,
               out: Optional[torch.Tensor] = None, want_sumsq: bool = False):
    """act(a w^T + bias) for M <= 64 in one kernel; with want_sumsq also the per-row sum of
    squares of each 16-column group of the (bf16) output, [M, ceil(N/16)] fp32."""
    _check(a, "a")
    _check(w, "w")
    M, K = a.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=_BF16, device=a.device)
    ss = torch.empty((M, (N + 15) // 16), dtype=torch.float32, device=a.device) if want_sumsq else None
    call("fam_gemm_final", a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
         bias.data_ptr() if bias is not None else None, act, out.data_ptr(), out.stride(0),
         ss.data_ptr() if ss is not None else None, M, N, K, _stream(a))
    return (out, ss) if want_sumsq else out


def rowop(out: torch.Tensor, *, partials: Optional[torch.Tensor] = None, x_in: Optional[torch.Tensor] = None,
          w_in: Optional[torch.Tensor] = None, bias=None, act: int = _capi.FAM_ACT_NONE, res=None, gate=None,
          gate_strides=(0, 0, 1), rows_per_batch: Optional[int] = None, norm: int = _capi.FAM_ROWNORM_NONE,
          eps: float = 1e-6, ln_w=None, ln_b=None, shift=None, scale=None, mod_strides=(0, 0), segs=(),
          seg_width: int = 0, rope=None, nout: Optional[torch.Tensor] = None, col0: int = 0) -> None:
    """Row kernel (fam_rowop in include/fam_hip.h) on 2-D row-major tensors.  `partials` is the
    [S, M, P] output of gemm_partial, of which columns [col0, col0 + N) are read (P may exceed
    N); `rope` is (cos, sin, row_stride, elem_stride, head_dim, seq_len) with fp32 tables."""
    M, N = out.shape
    d = _capi.RowopDesc()
    keep = []
    if partials is not None:
        S, Mp, P = partials.shape
        if Mp != M or not partials.is_contiguous() or col0 < 0 or col0 + N > P:
            raise ValueError(f"rowop: partials {tuple(partials.shape)} do not hold columns [{col0}, {col0 + N}) "
                             f"of {M} rows")
        d.src, d.partials, d.splits = _capi.FAM_ROWSRC_PARTIALS, partials.data_ptr() + 4 * col0, S
        d.split_stride, d.ldp = M * P, P
    else:
        d.src = _capi.FAM_ROWSRC_SMALLK
        d.x_in, d.ldx, d.k_in, d.w_in = x_in.data_ptr(), x_in.stride(0), w_in.shape[1], w_in.data_ptr()
    d.M, d.N = M, N
    d.bias = bias.data_ptr() if bias is not None else None
    d.act = act
    if res is not None:
        d.res, d.ldr = res.data_ptr(), res.stride(0)
    d.gate = gate.data_ptr() if gate is not None else None
    d.gate_bs, d.gate_rs, d.gate_ns = gate_strides
    d.rows_per_batch = rows_per_batch or M
    d.out, d.ldo, d.out_f32 = out.data_ptr(), out.stride(0), int(out.dtype == torch.float32)
    d.norm, d.eps = norm, float(eps)
    d.ln_weight = ln_w.data_ptr() if ln_w is not None else None
    d.ln_bias = ln_b.data_ptr() if ln_b is not None else None
    d.shift = shift.data_ptr() if shift is not None else None
    d.scale = scale.data_ptr() if scale is not None else None
    d.mod_bs, d.mod_rs = mod_strides
    d.nseg = len(segs)
    for i, (c0, wt) in enumerate(segs):
        d.seg_col0[i], d.seg_weight[i] = c0, wt.data_ptr()
    d.seg_width = seg_width
    if rope is not None:
        cs, sn, trs, tes, hd, seq = rope
        d.rope_cos, d.rope_sin, d.rope_row_stride, d.rope_elem_stride = cs.data_ptr(), sn.data_ptr(), trs, tes
        d.head_dim, d.seq_len = hd, seq
    if nout is not None:
        d.nout, d.ldn = nout.data_ptr(), nout.stride(0)
    call("fam_rowop", C.byref(d), _stream(out))
    del keep


# --------------------------------------------------------------------------- sampler
def _euler_launch(model_output, delta, sample, out=None):
    _check(sample, "sample")
    _check(model_output, "model_output")
    if model_output.shape != sample.shape:
        raise ValueError("model_output and sample must have the same shape")
    delta = delta.to(device=sample.device, dtype=_BF16).contiguous()
    n = sample.numel()
    if delta.numel() == 1:
        inner = max(n, 1)
    else:
        if delta.numel() != sample.shape[0]:
            raise ValueError("delta must be a scalar or have one value per batch row")
        inner = max(n // sample.shape[0], 1)
    s = sample.contiguous()
    v = model_output.contiguous()
    if out is None:
        out = torch.empty_like(s)
    call("fam_euler_step", s.data_ptr(), v.data_ptr(), delta.data_ptr(), out.data_ptr(), n, inner, _stream(s))
    return out


@torch.library.custom_op("fam::euler_step", mutates_args=())
def _euler_op(model_output: torch.Tensor, delta: torch.Tensor, sample: torch.Tensor) -> torch.Tensor:
    """sample + model_output * delta in bf16 with the reference's two roundings."""
    return _euler_launch(model_output, delta, sample)


@_euler_op.register_fake
def _euler_fake(model_output, delta, sample):
    _check(sample, "sample", device=False)
    _check(model_output, "model_output", device=False)
    if model_output.shape != sample.shape:
        raise ValueError("model_output and sample must have the same shape")
    return torch.empty_like(sample, memory_format=torch.contiguous_format)


def euler_step(model_output: torch.Tensor, delta: torch.Tensor, sample: torch.Tensor,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sample + model_output * delta in bf16 (SCH:82-88); delta a scalar or per-batch [B].
    With `out` the launch is direct (writes into it), otherwise it is the fam::euler_step
    operator."""
    if not isinstance(delta, torch.Tensor):
        delta = torch.tensor(float(delta))
    if out is not None:
        return _euler_launch(model_output, delta, sample, out)
    return torch.ops.fam.euler_step(model_output, delta, sample)


class WanContinuousFlowMatchScheduler:
    """Inference half of the reference scheduler (SCH:4-88): the shifted schedule and the
    Euler `step`, the latter on the device through fam_euler_step."""

    def __init__(self, num_train_timesteps: int = 1000, shift: float = 5.0, eps: float = 1e-10):
        if num_train_timesteps <= 0:
            raise ValueError(f"`num_train_timesteps` must be positive, got {num_train_timesteps}")
        if shift <= 0:
            raise ValueError(f"`shift` must be positive, got {shift}")
        self.num_train_timesteps = int(num_train_timesteps)
        self.shift = float(shift)
        self.eps = float(eps)

    @staticmethod
    def _phi(u: torch.Tensor, shift: float) -> torch.Tensor:
        return shift * u / (1.0 + (shift - 1.0) * u)

    def build_inference_schedule(self, num_inference_steps: int, device, dtype, shift_override=None):
        """(timesteps, deltas) in `dtype` on `device`; fp32 arithmetic on the host (SCH:63-80)."""
        if num_inference_steps <= 0:
            raise ValueError(f"`num_inference_steps` must be positive, got {num_inference_steps}")
        shift = self.shift if shift_override is None else float(shift_override)
        if shift <= 0:
            raise ValueError(f"`shift` must be positive, got {shift}")
        u = torch.linspace(1.0, 0.0, num_inference_steps + 1, dtype=torch.float32)
        sigma = self._phi(u, shift)
        t = sigma[:-1] * float(self.num_train_timesteps)
        d = sigma[1:] - sigma[:-1]
        return t.to(device=device, dtype=dtype), d.to(device=device, dtype=dtype)

    @staticmethod
    def step(model_output: torch.Tensor, delta: torch.Tensor, sample: torch.Tensor) -> torch.Tensor:
        return euler_step(model_output, delta, sample)

"""The reference's ``fastwam::`` custom operators, on the gfx950 kernels.

The GEAK-optimised FastWAM tree calls its Triton kernels through ``torch.library`` operators
from inside ``torch.compile`` regions (FG/wan_video_dit.py:1680-1721, :2174-2208;
FG/mot.py:682-720, :948-1010, :1207-1348).  Importing this module defines operators with the
same names, schemas and output shapes in the ``fastwam`` namespace, each with a fake
implementation, so those call sites (``torch.ops.fastwam.short_attn.default(...)`` etc.) run
on this library unchanged once the reference's own definitions are not imported.  Defining an
operator that already exists raises: the reference's Triton module and this one cannot both
own the name.

    fastwam::short_attn(q, k, v, mask, num_heads)           FG/wan_video_dit.py:1680-1721
    fastwam::short_attn_bsd(q, k, v, mask, num_heads)       FG/mot.py:682-720
    fastwam::qrms_attn(qraw, wq, k, v, mask, num_heads, eps) FG/wan_video_dit.py:2174-2208
    fastwam::qkv_post(qkv, wqk, freqs, sgn, kbuf, vbuf, kv_off, head, eps)
                                                            FG/mot.py:948-965 (mutates kbuf, vbuf)
    fastwam::qk_post(qkv, wqk, freqs, sgn, head, eps)       FG/mot.py:993-1010
    fastwam::skmm(x, w)                                     FG/mot.py:1207-1243
    fastwam::skpost(a, w, bias, res, modg, moda, tmod, lnw, lnb, gi, si, hi, eps, xdt)
                                                            FG/mot.py:1315-1348

(FG = src/fastwam-geak/fastwam/models/wan22.)

Numerics follow the reference's eager modules (src/fastwam-baseline), which the GEAK kernels
approximate: RMSNorm rounds to bf16 before its weight (FB/wan_video_dit.py:156-167), and
``modulation + t_mod`` is a bf16 sum (FB/wan_video_dit.py:271-274).  ``sgn`` is the constant
[-1, +1] pair-sign vector the reference always passes (FG/wan_video_dit.py:183-190); the
kernels apply that rotation and read only its shape.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import List, Optional, Tuple

import torch

from . import _capi
from ._capi import call
from .ops import _check, _stream, gemm, gemm_partial, rope_tables, rowop

_BF16 = torch.bfloat16


def _mask_plane(mask: Optional[torch.Tensor], Sq: int, Sk: int):
    """A [Sq, Sk] mask plane (bool = keep, or additive) -> (pointer, kind, query stride, keep)."""
    if mask is None:
        return None, _capi.FAM_MASK_NONE, 0, None
    m = mask
    while m.dim() > 2:
        if m.shape[0] != 1:
            raise ValueError(f"mask must broadcast to one [Sq, Sk] plane, got {tuple(mask.shape)}")
        m = m[0]
    if tuple(m.shape) != (Sq, Sk):
        m = torch.broadcast_to(m, (Sq, Sk))
    if m.dtype == torch.bool:
        kind = _capi.FAM_MASK_BOOL
    elif m.dtype == torch.bfloat16:
        kind = _capi.FAM_MASK_ADD_BF16
    else:
        kind, m = _capi.FAM_MASK_ADD_F32, m.float()
    if m.stride(-1) != 1:
        m = m.contiguous()
    return m.data_ptr(), kind, m.stride(0), m


def _launch_attention(q, q_strides, k, k_strides, v, v_strides, o, o_strides, B, H, Sq, Sk, D, mask):
    """One fam_attention launch over explicit (batch, row, head) element strides."""
    d = _capi.AttnDesc()
    d.q, (d.q_bs, d.q_rs, d.q_hs) = q.data_ptr(), q_strides
    d.k0, (d.k0_bs, d.k0_rs, d.k0_hs) = k.data_ptr(), k_strides
    d.v0, (d.v0_bs, d.v0_rs, d.v0_hs) = v.data_ptr(), v_strides
    d.o, (d.o_bs, d.o_rs, d.o_hs) = o.data_ptr(), o_strides
    d.batch, d.heads, d.sq, d.sk0, d.sk1, d.head_dim = B, H, Sq, Sk, 0, D
    d.scale = 1.0 / math.sqrt(D)
    mp, kind, qs, keep = _mask_plane(mask, Sq, Sk)
    d.mask, d.mask_kind, d.mask_bs, d.mask_hs, d.mask_qs = mp, kind, 0, 0, qs
    d.num_splits = 1
    call("fam_attention", C.byref(d), _stream(q))
    del keep


def _bhsd_strides(t: torch.Tensor) -> Tuple[int, int, int]:
    return t.stride(0), t.stride(2), t.stride(1)


def _bshd_strides(t: torch.Tensor, D: int) -> Tuple[int, int, int]:
    return t.stride(0), t.stride(1), D


# --------------------------------------------------------------------------- attention
@torch.library.custom_op("fastwam::short_attn", mutates_args=())
def short_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
               num_heads: int) -> torch.Tensor:
    """softmax(q k^T / sqrt(D) + mask) v; q/k/v [B, H, S, D] (output [B, H, Sq, D]) or
    [B, S, H*D] (output [B, Sq, H*D]); mask one [Sq, Sk] plane, bool or additive."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n)
    if q.dim() == 4:
        B, H, Sq, D = q.shape
        Sk = k.shape[2]
        o = torch.empty((B, H, Sq, D), dtype=q.dtype, device=q.device)
        _launch_attention(q, _bhsd_strides(q), k, _bhsd_strides(k), v, _bhsd_strides(v), o, _bhsd_strides(o),
                          B, H, Sq, Sk, D, mask)
    else:
        B, Sq, HD = q.shape
        H = int(num_heads)
        D = HD // H
        Sk = k.shape[1]
        o = torch.empty((B, Sq, HD), dtype=q.dtype, device=q.device)
        _launch_attention(q, _bshd_strides(q, D), k, _bshd_strides(k, D), v, _bshd_strides(v, D), o,
                          _bshd_strides(o, D), B, H, Sq, Sk, D, mask)
    return o


@short_attn.register_fake
def _(q, k, v, mask, num_heads):
    return q.new_empty(q.shape)


@torch.library.custom_op("fastwam::short_attn_bsd", mutates_args=())
def short_attn_bsd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor],
                   num_heads: int) -> torch.Tensor:
    """short_attn on [B, H, S, D] inputs with the output in [B, Sq, H*D]."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    o = torch.empty((B, Sq, H * D), dtype=q.dtype, device=q.device)
    _launch_attention(q, _bhsd_strides(q), k, _bhsd_strides(k), v, _bhsd_strides(v), o, _bshd_strides(o, D),
                      B, H, Sq, Sk, D, mask)
    return o


@short_attn_bsd.register_fake
def _(q, k, v, mask, num_heads):
    B, H, Sq, D = q.shape
    return q.new_empty((B, Sq, H * D))


def _rms(x2: torch.Tensor, y2: torch.Tensor, weight: torch.Tensor, eps: float, rope=None) -> None:
    """y2 = [RoPE](bf16(RMSNorm(x2)) * weight) on 2-D row views (one RMS per row)."""
    rows, D = x2.shape
    if rope is None:
        call("fam_rmsnorm_rope", x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0), rows, 1, D,
             weight.data_ptr(), float(eps), None, None, 0, 0, 0, _stream(x2))
    else:
        cos, sin, trs, tes, head = rope
        call("fam_rmsnorm_rope", x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0), rows, rows, D,
             weight.data_ptr(), float(eps), cos.data_ptr(), sin.data_ptr(), trs, tes, head, _stream(x2))


@torch.library.custom_op("fastwam::qrms_attn", mutates_args=())
def qrms_attn(qraw: torch.Tensor, wq: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
              mask: Optional[torch.Tensor], num_heads: int, eps: float) -> torch.Tensor:
    """flash_attention(RMSNorm(qraw) * wq, k, v) on [B, S, H*D] tensors (the cross-attention
    query norm folded into the attention call, FG/wan_video_dit.py:2211-2248)."""
    for t, n in ((qraw, "qraw"), (wq, "wq"), (k, "k"), (v, "v")):
        _check(t, n)
    B, Sq, HD = qraw.shape
    q = torch.empty((B * Sq, HD), dtype=_BF16, device=qraw.device)
    _rms(qraw.reshape(B * Sq, HD), q, wq.contiguous(), eps)
    H = int(num_heads)
    D = HD // H
    o = torch.empty((B, Sq, HD), dtype=qraw.dtype, device=qraw.device)
    q3 = q.view(B, Sq, HD)
    _launch_attention(q3, _bshd_strides(q3, D), k, _bshd_strides(k, D), v, _bshd_strides(v, D), o,
                      _bshd_strides(o, D), B, H, Sq, k.shape[1], D, mask)
    return o


@qrms_attn.register_fake
def _(qraw, wq, k, v, mask, num_heads, eps):
    return qraw.new_empty(qraw.shape)


# --------------------------------------------------------------------------- q/k post-processing
def _qk_tables(freqs: torch.Tensor, head: int, S: int, device):
    """The packed per-token cat(cos, sin) table [S, head] (fp32) of the qkv_post call sites."""
    if freqs.shape[0] < S or freqs.shape[-1] != head:
        raise ValueError(f"freqs must be [S, head] = [{S}, {head}], got {tuple(freqs.shape)}")
    cos, sin, trs, tes = rope_tables(freqs.reshape(freqs.shape[0], 1, head), "cat", device)
    return cos, sin, trs, tes, head


def _check_qkv(qkv, wqk, sgn, head):
    _check(qkv, "qkv")
    _check(wqk, "wqk")
    if qkv.dim() != 2 or qkv.shape[1] % 3:
        raise ValueError(f"qkv must be [S, 3N], got {tuple(qkv.shape)}")
    N = qkv.shape[1] // 3
    if wqk.numel() != 2 * N:
        raise ValueError(f"wqk must hold the q and k norm weights [2, {N}], got {tuple(wqk.shape)}")
    if sgn.numel() != 2:
        raise ValueError("sgn must be the [-1, +1] pair-sign vector")
    if head <= 0 or head % 2 or N % head:
        raise ValueError(f"head {head} must be even and divide N={N}")
    return N


@torch.library.custom_op("fastwam::qkv_post", mutates_args={"kbuf", "vbuf"})
def qkv_post(qkv: torch.Tensor, wqk: torch.Tensor, freqs: torch.Tensor, sgn: torch.Tensor,
             kbuf: torch.Tensor, vbuf: torch.Tensor, kv_off: int, head: int, eps: float) -> torch.Tensor:
    """From a fused projection qkv [S, 3N]: q = RoPE(RMSNorm(q) w_q) returned [1, S, N];
    RoPE(RMSNorm(k) w_k) and v written into rows [kv_off, kv_off + S) of the joint K/V cache
    buffers kbuf / vbuf ([1, Sv + S, N], contiguous), FG/mot.py:948-965 / :3068-3082."""
    S = qkv.shape[0]
    N = _check_qkv(qkv, wqk, sgn, head)
    for t, n in ((kbuf, "kbuf"), (vbuf, "vbuf")):
        _check(t, n)
        if not t.is_contiguous() or t.numel() < (kv_off + S) * N:
            raise ValueError(f"{n} must be contiguous with at least {kv_off + S} rows of {N}")
    tab = _qk_tables(freqs, head, S, qkv.device)
    w2 = wqk.reshape(2, N)
    q = torch.empty((1, S, N), dtype=qkv.dtype, device=qkv.device)
    _rms(qkv[:, :N], q.view(S, N), w2[0].contiguous(), eps, tab)
    kdst = kbuf.view(-1, N)[kv_off:kv_off + S]
    _rms(qkv[:, N:2 * N], kdst, w2[1].contiguous(), eps, tab)
    vbuf.view(-1, N)[kv_off:kv_off + S].copy_(qkv[:, 2 * N:])
    return q


@qkv_post.register_fake
def _(qkv, wqk, freqs, sgn, kbuf, vbuf, kv_off, head, eps):
    S, qn = qkv.shape
    return qkv.new_empty((1, S, qn // 3))


@torch.library.custom_op("fastwam::qk_post", mutates_args=())
def qk_post(qkv: torch.Tensor, wqk: torch.Tensor, freqs: torch.Tensor, sgn: torch.Tensor, head: int,
            eps: float) -> List[torch.Tensor]:
    """qkv_post's q and k as two new [1, S, N] tensors (the video prefill's form, FG/mot.py:993-1010)."""
    S = qkv.shape[0]
    N = _check_qkv(qkv, wqk, sgn, head)
    tab = _qk_tables(freqs, head, S, qkv.device)
    w2 = wqk.reshape(2, N)
    q = torch.empty((1, S, N), dtype=qkv.dtype, device=qkv.device)
    k = torch.empty((1, S, N), dtype=qkv.dtype, device=qkv.device)
    _rms(qkv[:, :N], q.view(S, N), w2[0].contiguous(), eps, tab)
    _rms(qkv[:, N:2 * N], k.view(S, N), w2[1].contiguous(), eps, tab)
    return [q, k]


@qk_post.register_fake
def _(qkv, wqk, freqs, sgn, head, eps):
    S, qn = qkv.shape
    return [qkv.new_empty((1, S, qn // 3)), qkv.new_empty((1, S, qn // 3))]


# --------------------------------------------------------------------------- projections
def _rows2d(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    return x2 if x2.stride(-1) == 1 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0 else x2.contiguous()


@torch.library.custom_op("fastwam::skmm", mutates_args=())
def skmm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x w^T without bias, [.., M, K] x [N, K] -> [1, M, N] (the action tokens' projections)."""
    _check(x, "x")
    _check(w, "w")
    x2 = _rows2d(x)
    out = torch.empty((1, x2.shape[0], w.shape[0]), dtype=x.dtype, device=x.device)
    gemm(x2, w.contiguous(), None, out.view(x2.shape[0], w.shape[0]))
    return out


@skmm.register_fake
def _(x, w):
    return x.new_empty((1, x.shape[-2], w.shape[0]))


@torch.library.custom_op("fastwam::skpost", mutates_args=())
def skpost(a: torch.Tensor, w: torch.Tensor, bias: torch.Tensor, res: torch.Tensor, modg: torch.Tensor,
           moda: torch.Tensor, tmod: torch.Tensor, lnw: Optional[torch.Tensor], lnb: Optional[torch.Tensor],
           gi: int, si: int, hi: int, eps: float, xdt: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """The projection and what follows it in a block (FG/mot.py:1315-1348):

        y = a w^T + bias;  x = res + g * y  (g = chunk gi of modg + tmod; no gate when gi < 0)
        o = LayerNorm(x) * lnw + lnb   (lnw given)   or   LN(x) * (1 + chunk si) + chunk hi
            of moda + tmod
    returns (x [1, M, N] bf16, or fp32 when xdt != 0; o [1, M, N]).  A split-K product whose
    partials are summed by one row launch that also applies bias, gate, residual and the norm."""
    for t, n in ((a, "a"), (w, "w"), (bias, "bias"), (res, "res"), (modg, "modg"), (moda, "moda"), (tmod, "tmod")):
        _check(t, n)
    a2 = _rows2d(a)
    M, N = a2.shape[0], w.shape[0]

    def chunk(mod, i):
        # modulation + t_mod in bf16 as the reference's eager split (FB/wan_video_dit.py:271-274)
        return (mod.reshape(-1)[i * N:(i + 1) * N] + tmod.reshape(-1)[i * N:(i + 1) * N]).contiguous()

    gate = chunk(modg, gi) if gi >= 0 else None
    if M <= 64 and a2.shape[1] % 8 == 0:
        part, splits = gemm_partial(a2, w.contiguous())
    else:
        part = torch.empty((1, M, N), dtype=torch.float32, device=a.device)
        gemm(a2, w.contiguous(), None, part.view(M, N), out_f32=True)
    xo = torch.empty((1, M, N), dtype=torch.float32 if xdt else a.dtype, device=a.device)
    yo = torch.empty((1, M, N), dtype=a.dtype, device=a.device)
    r2 = _rows2d(res)
    # the row kernel normalises bf16 rows: with xdt the bf16 x feeds the norm (as in the
    # reference's eager block, whose residual stream is bf16) and a second row launch stores
    # the fp32 x
    xb = torch.empty((M, N), dtype=a.dtype, device=a.device) if xdt else xo.view(M, N)
    if lnw is not None:
        rowop(xb, partials=part, bias=bias, res=r2, gate=gate, norm=_capi.FAM_ROWNORM_LAYERNORM, eps=eps,
              ln_w=lnw, ln_b=lnb, nout=yo.view(M, N))
    else:
        rowop(xb, partials=part, bias=bias, res=r2, gate=gate, norm=_capi.FAM_ROWNORM_ADALN, eps=eps,
              shift=chunk(moda, hi), scale=chunk(moda, si), nout=yo.view(M, N))
    if xdt:
        rowop(xo.view(M, N), partials=part, bias=bias, res=r2.float(), gate=gate)
    return xo, yo


@skpost.register_fake
def _(a, w, bias, res, modg, moda, tmod, lnw, lnb, gi, si, hi, eps, xdt=0):
    n = w.shape[0]
    xd = torch.float32 if xdt else a.dtype
    return a.new_empty((1, a.shape[-2], n), dtype=xd), a.new_empty((1, a.shape[-2], n))

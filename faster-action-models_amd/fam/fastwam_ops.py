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

The GEAK tree's prefill (FG/mot.py:1693-1905) and the CAE-FastWAM tree's action expert
(CA = src/cae-fastwam/fastwam/models/wan22; CA/mot.py:2793-3010, :3585-3712,
CA/action_dit.py:127-231) add:

    fastwam::pf_mm(x, w, b), pf_mm_gelu(x, w, b)            FG/mot.py:1693-1710
    fastwam::res_ln1(x, o, mb, tm, wn, bn, go, eps)         FG/mot.py:1829-1844
    fastwam::res_ln2(x, o1, o2, mb, mb2, tm, go, sho, sco, eps)   FG/mot.py:1846-1862
    fastwam::res_ln_tail(x, o, mb, mb2, tm, go, sho, sco, eps)    FG/mot.py:1883-1899
    fastwam::pf_skmm(x, w), pf_skmm_big(x, w)               FG/mot.py:2031-2074
    fastwam::res_ln1_sk(x, p, bi, mb, tm, wn, bn, go, eps, sk)    FG/mot.py:2155-2173
    fastwam::res_ln2_sk(x, o1, p, bi, mb, mb2, tm, go, sho, sco, eps, sk)
                                                            FG/mot.py:2175-2194
    fastwam::res_ln_tail_sk(x, p, bi, mb, mb2, tm, go, sho, sco, eps, sk)
                                                            FG/mot.py:2227-2244
    fastwam::pf_qcomb(p, bi, wq, eps, sk)                   FG/mot.py:2320-2333
    fastwam::mot_attn(q, k, v, msk, nh, hd, head_major)     CA/mot.py:2948-2976
    fastwam::mot_qkv_post(qkv, qw, kw, freqs, kbuf, vbuf, sv, eps)  CA/mot.py:2793-2822
    fastwam::xattn_qn(qr, qw, k, v, msk, nh, hd, eps)       CA/mot.py:3673-3700
    fastwam::ctx_kv_norm(g, nkw, nl, ahd, eps)              CA/mot.py:3585-3608
    fastwam::mot_oproj(a, w, b), mot_ffn(x, w1, b1, w2, b2) CA/mot.py:2904-2946
    fastwam::adit_tmod(te, inv, w0, b0, w1, b1, w2, b2, atok, aw, ab, fuse_sin)
                                                            CA/action_dit.py:191-225

and the CAE tree's fused levers and fp8 rows (CA/mot.py:2830-3980):

    fastwam::mask_bias(am, cm, mp, skp, ncp)                CA/mot.py:3342-3369
    fastwam::mot_attn_oproj(q, k, v, msk, wo, bo, acc, nh, hd)       (mutates acc)  :2864-2900
    fastwam::mod_n3q(res, so, mod, tmod, lnw, lnb, qw, qb, eps)                     :2978-3008
    fastwam::mod_n3q_qn(... qw, qb, qnw, gram, eps, eps_q)                          :3227-3262
    fastwam::n3q_xoproj(... qnw, gram, ck, cv, msk, wo, bo, acc, nh, eps, eps_q)    :3414-3470
    fastwam::mot_ffn_fold(x, oacc, modc, modn, tmod, w1, b1, w2, b2, eps2, eps1, hasnext)
                                                                                    :3086-3122
    fastwam::mot_sa_qkv(xin, w, b, qgr, kgr, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps)
                                                                                    :3285-3322
    fastwam::mot_ffn_sa_qkv(xp, oacc, ..., za, zb, sv, eps, eps2, eps1)             :3498-3565
    fastwam::mot_qkv_post_z(qkv, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps)        :2830-2860
    fastwam::mot_qkv_gemm_post_z(xin, wt, bqkv, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps)
                                                                                    :3032-3070
    fastwam::mot_l0_qkv_rope(q, k, v, qw, kw, freqs, kbuf, vbuf, sv, eps)           :3142-3172
    fastwam::mot_l0_qkv_rope_z(... kbuf, vbuf, oaccx, sv, eps)                      :3180-3210
    fastwam::ctx_kv_norm_into(g, nkw, out, nl, ahd, eps)                            :3621-3638
    fastwam::ctx_kv_gemm_norm_into(e, w, b, nkw, out, nl, ahd, eps, has_b)          :3641-3662
    fastwam::vqkv_post(qkv, qw, kw, freqs, kbuf, vbuf, eps)                         :3713-3750
    fastwam::row_q8(x), gelu_q8(x), ln_mod_q8(x, shift, scale, eps),
             add_ln_mod_q8(a, b, shift, scale, eps)                                 :3859-3960

Per-operator rounding differences from the Triton kernels they stand in for (all within one
bf16 rounding of an intermediate; the GPU tests hold each against an eager restatement of the
reference kernel at 2e-2):
  res_ln*   the norm reads the bf16-rounded residual (the reference takes its statistics from
            the fp32 sum); the gate / shift / scale sums modulation + t_mod in fp32 as it does;
            the *_sk forms round the split-K combine + bias to bf16 once, as the reference does;
  pf_skmm*  the product sits whole in plane 0 and the other planes are zero (the reference
            spreads K over its configured count of planes): any sk sums to the same product;
  pf_qcomb  RMSNorm rounds to bf16 before the weight (the reference kernel does not);
  mot_qkv_post, xattn_qn, ctx_kv_norm
            RMSNorm rounds to bf16 before the weight (the eager module's order); the CAE
            kernels of xattn_qn and ctx_kv_norm multiply the weight before their one rounding;
  mot_ffn, pf_mm_gelu, adit_tmod, mot_ffn_fold
            the activation runs on the fp32 accumulator (+ bias) and rounds once; the
            reference kernels round the pre-activation to bf16 first;
  mod_n3q*, n3q_xoproj, mot_ffn_fold
            the gated residual is formed in fp32 and rounded once (the reference rounds the
            gate, so and gate * so first), the norms read the bf16 residual; the FFN's output
            enters xout unrounded;
  mod_n3q_qn, n3q_xoproj, mot_sa_qkv, mot_ffn_sa_qkv
            the whole-row q / k norm sums the squares of the (bf16) row itself instead of the
            Gram form of the unrounded product (gram / qgr / kgr are checked for shape only);
  mot_l0_qkv_rope, vqkv_post and the *_z forms
            as mot_qkv_post (bf16 before the norm weight);
  gelu_q8   exp through the hardware exp2 (a handful of fp8 codes one step apart);
            row_q8, ln_mod_q8 and add_ln_mod_q8 give the reference's codes.
ctx_kv_norm returns the K half only ([1, nl, 1, S, ahd]), the reference's default
(FASTWAM_R2_NORM_V unset, CA/mot.py:578).  adit_tmod computes the sinusoid with the library's
own fp64 frequencies; `inv` must be 10000^(-j / (FD/2)), which is what the call site passes.

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


# --------------------------------------------------------------------------- prefill projections (FG)
@torch.library.custom_op("fastwam::pf_mm", mutates_args=())
def pf_mm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """F.linear(x, w, b) for the prefill's 98-row projections (FG/mot.py:1693-1700)."""
    for t, n in ((x, "x"), (w, "w"), (b, "b")):
        _check(t, n)
    x2 = _rows2d(x)
    out = torch.empty(tuple(x.shape[:-1]) + (w.shape[0],), dtype=x.dtype, device=x.device)
    gemm(x2, w.contiguous(), b.contiguous(), out.view(x2.shape[0], w.shape[0]))
    return out


@pf_mm.register_fake
def _(x, w, b):
    return x.new_empty(tuple(x.shape[:-1]) + (int(w.shape[0]),))


@torch.library.custom_op("fastwam::pf_mm_gelu", mutates_args=())
def pf_mm_gelu(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """GELU(tanh)(x w^T + b) (aten _addmm_activation(use_gelu=True), FG/mot.py:1703-1707)."""
    for t, n in ((x, "x"), (w, "w"), (b, "b")):
        _check(t, n)
    x2 = _rows2d(x)
    out = torch.empty(tuple(x.shape[:-1]) + (w.shape[0],), dtype=x.dtype, device=x.device)
    gemm(x2, w.contiguous(), b.contiguous(), out.view(x2.shape[0], w.shape[0]), act=_capi.FAM_ACT_GELU_TANH)
    return out


@pf_mm_gelu.register_fake
def _(x, w, b):
    return x.new_empty(tuple(x.shape[:-1]) + (int(w.shape[0]),))


def _mod_rows(mb: torch.Tensor, tm: torch.Tensor, off: int, S: int, N: int) -> torch.Tensor:
    """(modulation + per-token t_mod) chunk at column `off`: [S, N], summed in fp32 and rounded
    once (the reference kernel adds the two bf16 loads in fp32, FG/mot.py:1783-1795)."""
    if tm.dim() != 2 or tm.shape[0] < S or tm.shape[1] < off + N:
        raise ValueError(f"t_mod must be [S, >= {off + N}] rows, got {tuple(tm.shape)}")
    return (mb.reshape(-1)[off:off + N].float()[None, :] + tm[:S, off:off + N].float()).to(_BF16).contiguous()


def _res_norm(x, parts, gate, eps, ln=None, ada=None):
    """x + gate * parts[0] (+ parts[1]) in fp32, stored bf16, then LayerNorm (affine, ln = (w, b))
    or AdaLN (ada = (shift rows, scale rows)) of that row into a second bf16 tensor."""
    S, N = x.shape[1], x.shape[2]
    p = parts[0].reshape(S, N).float() * gate.float()
    for extra in parts[1:]:
        p = p + extra.reshape(S, N).float()
    p = p.reshape(1, S, N).contiguous()
    xo = torch.empty((1, S, N), dtype=x.dtype, device=x.device)
    no = torch.empty((1, S, N), dtype=x.dtype, device=x.device)
    kw = dict(partials=p, res=_rows2d(x), eps=eps, nout=no.view(S, N))
    if ln is not None:
        rowop(xo.view(S, N), norm=_capi.FAM_ROWNORM_LAYERNORM, ln_w=ln[0].contiguous(), ln_b=ln[1].contiguous(), **kw)
    else:
        rowop(xo.view(S, N), norm=_capi.FAM_ROWNORM_ADALN, shift=ada[0], scale=ada[1], mod_strides=(0, N), **kw)
    return xo, no


@torch.library.custom_op("fastwam::res_ln1", mutates_args=())
def res_ln1(x: torch.Tensor, o: torch.Tensor, mb: torch.Tensor, tm: torch.Tensor, wn: torch.Tensor,
            bn: torch.Tensor, go: int, eps: float) -> torch.Tensor:
    """LayerNorm(x + g o) * wn + bn per token, g = chunk `go` of modulation mb + t_mod row tm[s]
    (the prefill's norm3 after the self-attention residual, FG/mot.py:1829-1844); [1, S, N]."""
    for t, n in ((x, "x"), (o, "o"), (mb, "mb"), (tm, "tm"), (wn, "wn"), (bn, "bn")):
        _check(t, n)
    S, N = x.shape[1], x.shape[2]
    _, no = _res_norm(x, [o], _mod_rows(mb, tm, go, S, N), eps, ln=(wn, bn))
    return no


@res_ln1.register_fake
def _(x, o, mb, tm, wn, bn, go, eps):
    return x.new_empty((1, int(x.shape[1]), int(x.shape[2])))


@torch.library.custom_op("fastwam::res_ln2", mutates_args=())
def res_ln2(x: torch.Tensor, o1: torch.Tensor, o2: torch.Tensor, mb: torch.Tensor, mb2: torch.Tensor,
            tm: torch.Tensor, go: int, sho: int, sco: int, eps: float) -> List[torch.Tensor]:
    """[xo, no]: xo = x + g o1 + o2, no = LN(xo) (1 + scale) + shift, g / shift / scale the chunks
    `go` of mb and `sho` / `sco` of mb2, each plus t_mod row tm[s] (FG/mot.py:1846-1862)."""
    for t, n in ((x, "x"), (o1, "o1"), (o2, "o2"), (mb, "mb"), (mb2, "mb2"), (tm, "tm")):
        _check(t, n)
    S, N = x.shape[1], x.shape[2]
    xo, no = _res_norm(x, [o1, o2], _mod_rows(mb, tm, go, S, N), eps,
                       ada=(_mod_rows(mb2, tm, sho, S, N), _mod_rows(mb2, tm, sco, S, N)))
    return [xo, no]


@res_ln2.register_fake
def _(x, o1, o2, mb, mb2, tm, go, sho, sco, eps):
    S, N = int(x.shape[1]), int(x.shape[2])
    return [x.new_empty((1, S, N)), x.new_empty((1, S, N))]


@torch.library.custom_op("fastwam::res_ln_tail", mutates_args=())
def res_ln_tail(x: torch.Tensor, o: torch.Tensor, mb: torch.Tensor, mb2: torch.Tensor, tm: torch.Tensor,
                go: int, sho: int, sco: int, eps: float) -> List[torch.Tensor]:
    """res_ln2 without the second output term: the layer boundary x + gate_mlp ffn, then the next
    block's AdaLN1 (FG/mot.py:1883-1899)."""
    for t, n in ((x, "x"), (o, "o"), (mb, "mb"), (mb2, "mb2"), (tm, "tm")):
        _check(t, n)
    S, N = x.shape[1], x.shape[2]
    xo, no = _res_norm(x, [o], _mod_rows(mb, tm, go, S, N), eps,
                       ada=(_mod_rows(mb2, tm, sho, S, N), _mod_rows(mb2, tm, sco, S, N)))
    return [xo, no]


@res_ln_tail.register_fake
def _(x, o, mb, mb2, tm, go, sho, sco, eps):
    S, N = int(x.shape[1]), int(x.shape[2])
    return [x.new_empty((1, S, N)), x.new_empty((1, S, N))]


# --------------------------------------------------------------------------- prefill split-K planes (FG)
# The prefill's o-projections and ffn.2 return fp32 planes [SKMAX, M, N] (SKMAX 8, and 16 for
# ffn.2: fixed so the fake shape does not follow the split count) of which the consumer sums the
# first `sk`, sk being the count its caller configured (FG/mot.py:1944-1961, :2017-2074).  Here
# the product lands whole in plane 0 and every other plane holds zeros, so the first sk planes
# sum to it for every sk in [1, SKMAX].  As the reference's default (FASTWAM_PFSKSHARE), one
# buffer per (device, SKMAX, M, N) serves every call: its zero planes are written once, when it
# is allocated, a call rewrites plane 0 only, and a result is valid until the next call of the
# same shape.
_PF_PARTS: dict = {}


def _pf_planes(x: torch.Tensor, w: torch.Tensor, skmax: int) -> torch.Tensor:
    _check(x, "x")
    _check(w, "w")
    x2 = _rows2d(x)
    M, K, N = x2.shape[0], x2.shape[1], w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"pf_skmm: x has K={K} columns, w is {tuple(w.shape)}")
    key = (x.device.type, x.device.index, skmax, M, N)
    part = _PF_PARTS.get(key)
    if part is None:
        part = torch.zeros((skmax, M, N), dtype=torch.float32, device=x.device)
        if not torch.cuda.is_current_stream_capturing():
            _PF_PARTS[key] = part
    gemm(x2, w.contiguous(), None, part[0], out_f32=True)
    return part


@torch.library.custom_op("fastwam::pf_skmm", mutates_args=())
def pf_skmm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x w^T as [8, M, N] fp32 split planes (FG/mot.py:2031-2043)."""
    return _pf_planes(x, w, 8)


@pf_skmm.register_fake
def _(x, w):
    return x.new_empty((8, int(x.shape[-2]), int(w.shape[0])), dtype=torch.float32)


@torch.library.custom_op("fastwam::pf_skmm_big", mutates_args=())
def pf_skmm_big(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x w^T as [16, M, N] fp32 split planes, the ffn.2 site's (FG/mot.py:2057-2069)."""
    return _pf_planes(x, w, 16)


@pf_skmm_big.register_fake
def _(x, w):
    return x.new_empty((16, int(x.shape[-2]), int(w.shape[0])), dtype=torch.float32)


def _pf_combine_planes(p: torch.Tensor, sk: int, S: int, N: int) -> torch.Tensor:
    """The first sk planes of a split-plane operand, checked."""
    if not p.is_cuda or p.dim() != 3 or p.dtype != torch.float32 or not p.is_contiguous() or p.shape[1] != S or \
            p.shape[2] != N:
        raise ValueError(f"split planes must be contiguous fp32 CUDA [SKMAX, {S}, {N}], got {tuple(p.shape)} "
                         f"{p.dtype} on {p.device}")
    if not 1 <= sk <= p.shape[0]:
        raise ValueError(f"sk={sk} outside [1, {p.shape[0]}]")
    return p[:sk]


def _pf_combine(p: torch.Tensor, bi: torch.Tensor, sk: int, S: int, N: int) -> torch.Tensor:
    """bf16(sum of the first sk planes + bias), [S, N]: the reference kernels round the
    combined product once, where a bf16 GEMM output would have been (FG/mot.py:2112-2120)."""
    _check(bi, "bi")
    planes = _pf_combine_planes(p, sk, S, N)
    pb = torch.empty((S, N), dtype=_BF16, device=p.device)
    rowop(pb, partials=planes, bias=bi.contiguous())
    return pb


@torch.library.custom_op("fastwam::res_ln1_sk", mutates_args=())
def res_ln1_sk(x: torch.Tensor, p: torch.Tensor, bi: torch.Tensor, mb: torch.Tensor, tm: torch.Tensor,
               wn: torch.Tensor, bn: torch.Tensor, go: int, eps: float, sk: int) -> List[torch.Tensor]:
    """[LN(x + g o) wn + bn, o] with o = bf16(sum of sk planes of p + bi): the self-attention
    o-projection's split-K combine, its residual and norm3 (FG/mot.py:2155-2168)."""
    S, N = x.shape[1], x.shape[2]
    o = _pf_combine(p, bi, sk, S, N)
    _check(x, "x")
    _, no = _res_norm(x, [o], _mod_rows(mb, tm, go, S, N), eps, ln=(wn, bn))
    return [no, o.view(1, S, N)]


@res_ln1_sk.register_fake
def _(x, p, bi, mb, tm, wn, bn, go, eps, sk):
    S, N = int(x.shape[1]), int(x.shape[2])
    return [x.new_empty((1, S, N)), x.new_empty((1, S, N))]


@torch.library.custom_op("fastwam::res_ln2_sk", mutates_args=())
def res_ln2_sk(x: torch.Tensor, o1: torch.Tensor, p: torch.Tensor, bi: torch.Tensor, mb: torch.Tensor,
               mb2: torch.Tensor, tm: torch.Tensor, go: int, sho: int, sco: int, eps: float,
               sk: int) -> List[torch.Tensor]:
    """res_ln2 with its second term the split-K combine of the cross-attention o-projection:
    [xo, no], xo = x + g o1 + bf16(sum of sk planes of p + bi) (FG/mot.py:2175-2189)."""
    S, N = x.shape[1], x.shape[2]
    o2 = _pf_combine(p, bi, sk, S, N)
    for t, n in ((x, "x"), (o1, "o1"), (mb, "mb"), (mb2, "mb2"), (tm, "tm")):
        _check(t, n)
    xo, no = _res_norm(x, [o1, o2], _mod_rows(mb, tm, go, S, N), eps,
                       ada=(_mod_rows(mb2, tm, sho, S, N), _mod_rows(mb2, tm, sco, S, N)))
    return [xo, no]


@res_ln2_sk.register_fake
def _(x, o1, p, bi, mb, mb2, tm, go, sho, sco, eps, sk):
    S, N = int(x.shape[1]), int(x.shape[2])
    return [x.new_empty((1, S, N)), x.new_empty((1, S, N))]


@torch.library.custom_op("fastwam::res_ln_tail_sk", mutates_args=())
def res_ln_tail_sk(x: torch.Tensor, p: torch.Tensor, bi: torch.Tensor, mb: torch.Tensor, mb2: torch.Tensor,
                   tm: torch.Tensor, go: int, sho: int, sco: int, eps: float, sk: int) -> List[torch.Tensor]:
    """res_ln_tail on the split-K combine of ffn.2: [xo, no], xo = x + g bf16(sum of sk planes
    of p + bi), no = the next block's AdaLN1 of xo (FG/mot.py:2227-2239)."""
    S, N = x.shape[1], x.shape[2]
    o = _pf_combine(p, bi, sk, S, N)
    for t, n in ((x, "x"), (mb, "mb"), (mb2, "mb2"), (tm, "tm")):
        _check(t, n)
    xo, no = _res_norm(x, [o], _mod_rows(mb, tm, go, S, N), eps,
                       ada=(_mod_rows(mb2, tm, sho, S, N), _mod_rows(mb2, tm, sco, S, N)))
    return [xo, no]


@res_ln_tail_sk.register_fake
def _(x, p, bi, mb, mb2, tm, go, sho, sco, eps, sk):
    S, N = int(x.shape[1]), int(x.shape[2])
    return [x.new_empty((1, S, N)), x.new_empty((1, S, N))]


@torch.library.custom_op("fastwam::pf_qcomb", mutates_args=())
def pf_qcomb(p: torch.Tensor, bi: torch.Tensor, wq: torch.Tensor, eps: float, sk: int) -> torch.Tensor:
    """RMSNorm(bf16(sum of sk planes of p + bi)) * wq, [1, S, N]: the prefill cross-attention
    query's split-K combine and norm_q (FG/mot.py:2290-2329)."""
    S, N = p.shape[1], p.shape[2]
    _check(wq, "wq")
    if wq.numel() != N:
        raise ValueError(f"pf_qcomb: wq has {wq.numel()} entries for rows of {N}")
    q = torch.empty((S, N), dtype=_BF16, device=p.device)
    qn = torch.empty((1, S, N), dtype=_BF16, device=p.device)
    rowop(q, partials=_pf_combine_planes(p, sk, S, N), bias=bi.contiguous(), norm=_capi.FAM_ROWNORM_RMS, eps=eps,
          segs=((0, wq.contiguous()),), seg_width=N, nout=qn.view(S, N))
    return qn


@pf_qcomb.register_fake
def _(p, bi, wq, eps, sk):
    return bi.new_empty((1, int(p.shape[1]), int(p.shape[2])))


# --------------------------------------------------------------------------- CAE action expert (CA)
def _keep_plane(msk: torch.Tensor, M: int, SK: int) -> torch.Tensor:
    """The [M, SK] keep plane (nonzero = attend) of a CAE mask operand, as bool."""
    m = msk
    while m.dim() > 2:
        m = m[0]
    if m.dim() == 1:
        m = m[None, :]
    return torch.broadcast_to(m != 0, (M, SK))


@torch.library.custom_op("fastwam::mot_attn", mutates_args=())
def mot_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, msk: torch.Tensor, nh: int, hd: int,
             head_major: bool) -> torch.Tensor:
    """softmax(q k^T / sqrt(hd), keys where msk != 0) v per head (CA/mot.py:2948-2976): q [1, H, M,
    hd] and k / v [1, H, SK, hd] when head_major, else [1, M, H*hd] / [1, SK, H*hd] rows;
    output [1, M, H*hd]."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n)
    H, D = int(nh), int(hd)
    if head_major:
        M, SK = q.shape[2], k.shape[2]
        qs, ks, vs = _bhsd_strides(q), _bhsd_strides(k), _bhsd_strides(v)
    else:
        M, SK = q.shape[1], k.shape[1]
        qs, ks, vs = (0, q.stride(1), D), (0, k.stride(1), D), (0, v.stride(1), D)
    o = torch.empty((1, M, H * D), dtype=q.dtype, device=q.device)
    _launch_attention(q, qs, k, ks, v, vs, o, _bshd_strides(o, D), 1, H, M, SK, D, _keep_plane(msk, M, SK))
    return o


@mot_attn.register_fake
def _(q, k, v, msk, nh, hd, head_major):
    m = q.shape[2] if head_major else q.shape[1]
    return q.new_empty((1, m, nh * hd))


@torch.library.custom_op("fastwam::mot_qkv_post", mutates_args={"kbuf", "vbuf"})
def mot_qkv_post(qkv: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor, freqs: torch.Tensor, kbuf: torch.Tensor,
                 vbuf: torch.Tensor, sv: int, eps: float) -> torch.Tensor:
    """The CAE expert's q / k post-processing (CA/mot.py:2793-2822, kernel :1369-1456): from the
    fused projection qkv [1, M, 3D] (D = H hd), RMSNorm over D of q and k with their weights,
    then the interleaved rotation by freqs [M, hd] (cos at 2p, sin at 2p + 1 of each token's row);
    q returned head-major [1, H, M, hd], k and v written to rows sv .. sv + M of the head-major
    cache buffers kbuf / vbuf [1, H, SKV, hd]."""
    _check(qkv, "qkv")
    M, D3 = qkv.shape[1], qkv.shape[2]
    D = D3 // 3
    x2 = qkv.reshape(M, D3)
    qn = _cae_qkv_rows(x2[:, :D], x2[:, D:2 * D], x2[:, 2 * D:], qw, kw, freqs, kbuf, vbuf, sv, eps)
    return _head_major(qn, kbuf.shape[1])


def _head_major(rows: torch.Tensor, H: int) -> torch.Tensor:
    """[M, H hd] token rows -> [1, H, M, hd] contiguous."""
    M, D = rows.shape
    return rows.view(M, H, D // H).transpose(0, 1).contiguous().unsqueeze(0)


def _cae_qkv_rows(q2: torch.Tensor, k2: torch.Tensor, v2: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor,
                  freqs: torch.Tensor, kbuf: torch.Tensor, vbuf: torch.Tensor, sv: int, eps: float,
                  q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The CAE q / k / v post-processing on [M, D] row views: RMSNorm over D of q and k with their
    weights and the interleaved rotation by freqs [M, hd] (cos at 2p, sin at 2p + 1), k and v
    written head-major to rows sv .. sv + M of kbuf / vbuf [1, H, SKV, hd]; returns the rotated q
    rows [M, D] (into q_out when given)."""
    for t, n in ((q2, "q"), (k2, "k"), (v2, "v"), (qw, "qw"), (kw, "kw"), (kbuf, "kbuf"), (vbuf, "vbuf")):
        _check(t, n)
    M, D = q2.shape
    H, hd, SKV = kbuf.shape[1], kbuf.shape[3], kbuf.shape[2]
    if H * hd != D or k2.shape != (M, D) or v2.shape != (M, D) or sv < 0 or sv + M > SKV or vbuf.shape != kbuf.shape:
        raise ValueError(f"kbuf {tuple(kbuf.shape)} does not take {M} rows of {D} at row {sv}")
    f = freqs.reshape(-1, hd).float().contiguous()
    if f.shape[0] < M:
        raise ValueError(f"freqs must hold {M} rows of {hd}, got {tuple(freqs.shape)}")
    q2, k2 = (t if t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0 else t.contiguous() for t in (q2, k2))
    qn = q_out if q_out is not None else torch.empty((M, D), dtype=q2.dtype, device=q2.device)
    kn = torch.empty((M, D), dtype=q2.dtype, device=q2.device)
    for src, dst, w in ((q2, qn, qw), (k2, kn, kw)):
        call("fam_rmsnorm_rope", src.data_ptr(), src.stride(0), dst.data_ptr(), dst.stride(0), M, M, D,
             w.contiguous().data_ptr(), float(eps), f.data_ptr(), f[:, 1:].data_ptr(), hd, 2, hd, _stream(src))
    kbuf[0, :, sv:sv + M, :].copy_(kn.view(M, H, hd).transpose(0, 1))
    vbuf[0, :, sv:sv + M, :].copy_(v2.reshape(M, H, hd).transpose(0, 1))
    return qn


@mot_qkv_post.register_fake
def _(qkv, qw, kw, freqs, kbuf, vbuf, sv, eps):
    return qkv.new_empty((1, kbuf.shape[1], qkv.shape[1], kbuf.shape[3]))


@torch.library.custom_op("fastwam::xattn_qn", mutates_args=())
def xattn_qn(qr: torch.Tensor, qw: torch.Tensor, k: torch.Tensor, v: torch.Tensor, msk: torch.Tensor, nh: int,
             hd: int, eps: float) -> torch.Tensor:
    """Cross attention with the query's RMSNorm over its whole C-wide row (CA/mot.py:3673-3700,
    kernel :2240-2305): q = RMSNorm(qr) qw; o = softmax(q k^T / sqrt(hd), keys where msk != 0) v
    per head over [1, N, C] rows of k / v; output [1, M, C]."""
    for t, n in ((qr, "qr"), (qw, "qw"), (k, "k"), (v, "v")):
        _check(t, n)
    M, Cw = qr.shape[1], qr.shape[2]
    N, H, D = k.shape[1], int(nh), int(hd)
    q = torch.empty((M, Cw), dtype=qr.dtype, device=qr.device)
    _rms(_rows2d(qr), q, qw.contiguous(), eps)
    o = torch.empty((1, M, Cw), dtype=qr.dtype, device=qr.device)
    q3 = q.view(1, M, Cw)
    _launch_attention(q3, _bshd_strides(q3, D), k, (0, k.stride(1), D), v, (0, v.stride(1), D), o,
                      _bshd_strides(o, D), 1, H, M, N, D, _keep_plane(msk, M, N))
    return o


@xattn_qn.register_fake
def _(qr, qw, k, v, msk, nh, hd, eps):
    return torch.empty_like(qr)


@torch.library.custom_op("fastwam::ctx_kv_norm", mutates_args=())
def ctx_kv_norm(g: torch.Tensor, nkw: torch.Tensor, nl: int, ahd: int, eps: float) -> torch.Tensor:
    """RMSNorm of every layer's context keys (CA/mot.py:3585-3608, kernel :2119-2142): g [S, 2 nl ahd]
    holds the keys of layer l at columns l ahd and the values after all keys; returns the keys
    normalised with nkw [nl, ahd], [1, nl, 1, S, ahd]."""
    _check(g, "g")
    _check(nkw, "nkw")
    S, nl, ahd = g.shape[0], int(nl), int(ahd)
    if g.dim() != 2 or g.shape[1] != 2 * nl * ahd or nkw.numel() != nl * ahd:
        raise ValueError(f"g must be [S, {2 * nl * ahd}] and nkw [{nl}, {ahd}]")
    keys = g[:, :nl * ahd].reshape(S * nl, ahd).contiguous()    # row (s, l): layer l's key of token s
    y = torch.empty_like(keys)
    call("fam_rmsnorm_grouped", keys.data_ptr(), ahd, y.data_ptr(), ahd, S * nl, ahd,
         nkw.reshape(nl, ahd).contiguous().data_ptr(), nl, float(eps), _stream(g))
    return y.view(S, nl, ahd).transpose(0, 1).contiguous().view(1, nl, 1, S, ahd)


@ctx_kv_norm.register_fake
def _(g, nkw, nl, ahd, eps):
    return g.new_empty((1, nl, 1, g.shape[0], ahd))


@torch.library.custom_op("fastwam::mot_oproj", mutates_args=())
def mot_oproj(a: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a w^T + b on the M action rows, [1, M, K] -> [1, M, N] (CA/mot.py:2929-2946)."""
    for t, n in ((a, "a"), (w, "w"), (b, "b")):
        _check(t, n)
    a2 = _rows2d(a)
    out = torch.empty((1, a2.shape[0], w.shape[0]), dtype=a.dtype, device=a.device)
    gemm(a2, w.contiguous(), b.contiguous(), out.view(a2.shape[0], w.shape[0]))
    return out


@mot_oproj.register_fake
def _(a, w, b):
    return a.new_empty((1, a.shape[1], w.shape[0]))


@torch.library.custom_op("fastwam::mot_ffn", mutates_args=())
def mot_ffn(x: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor) -> torch.Tensor:
    """W2 GELU(tanh)(W1 x + b1) + b2 on the action rows (CA/mot.py:2904-2927, kernel :2308-2343)."""
    for t, n in ((x, "x"), (w1, "w1"), (b1, "b1"), (w2, "w2"), (b2, "b2")):
        _check(t, n)
    x2 = _rows2d(x)
    M = x2.shape[0]
    hid = torch.empty((M, w1.shape[0]), dtype=x.dtype, device=x.device)
    gemm(x2, w1.contiguous(), b1.contiguous(), hid, act=_capi.FAM_ACT_GELU_TANH)
    out = torch.empty_like(x)
    gemm(hid, w2.contiguous(), b2.contiguous(), out.view(M, w2.shape[0]))
    return out


@mot_ffn.register_fake
def _(x, w1, b1, w2, b2):
    return torch.empty_like(x)


@torch.library.custom_op("fastwam::adit_tmod", mutates_args=())
def adit_tmod(te: torch.Tensor, inv: torch.Tensor, w0: torch.Tensor, b0: torch.Tensor, w1: torch.Tensor,
              b1: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor, atok: torch.Tensor, aw: torch.Tensor,
              ab: torch.Tensor, fuse_sin: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The action expert's time MLP and action encoder (CA/action_dit.py:127-225): te the timestep
    (fuse_sin: its sinusoidal embedding is formed here) or that embedding [FD]; returns
    t = W1 SiLU(W0 te + b0) + b1 [1, H], t_mod = W2 SiLU(t) + b2 [1, 6H] and the encoded action
    tokens atok [1, S, A] W_aw^T + ab [1, S, H]."""
    for t, n in ((w0, "w0"), (w1, "w1"), (w2, "w2"), (atok, "atok"), (aw, "aw")):
        _check(t, n)
    dev, odt = atok.device, atok.dtype
    FD, H, H6 = w0.shape[1], w0.shape[0], w2.shape[0]
    if fuse_sin:
        emb = torch.empty((1, FD), dtype=odt, device=dev)
        pos = te.reshape(1).to(odt).contiguous()
        call("fam_sinusoid", pos.data_ptr(), emb.data_ptr(), 1, FD, _stream(atok))
    else:
        emb = te.reshape(1, FD).to(odt).contiguous()
    h0 = torch.empty((1, H), dtype=odt, device=dev)
    gemm(emb, w0.contiguous(), b0.contiguous(), h0, act=_capi.FAM_ACT_SILU)
    t = torch.empty((1, H), dtype=odt, device=dev)
    gemm(h0, w1.contiguous(), b1.contiguous(), t)
    st = torch.empty((1, H), dtype=odt, device=dev)
    call("fam_act_rows", t.data_ptr(), H, st.data_ptr(), H, 1, H, _capi.FAM_ACT_SILU, _stream(atok))
    tm = torch.empty((1, H6), dtype=odt, device=dev)
    gemm(st, w2.contiguous(), b2.contiguous(), tm)
    S, A = atok.shape[1], atok.shape[2]
    tk = torch.empty((1, S, H), dtype=odt, device=dev)
    a2 = atok.reshape(S, A).contiguous()
    call("fam_linear_smallk", a2.data_ptr(), A, 0, aw.contiguous().data_ptr(), ab.contiguous().data_ptr(),
         tk.data_ptr(), H, S, H, A, _stream(atok))
    return t, tm, tk


@adit_tmod.register_fake
def _(te, inv, w0, b0, w1, b1, w2, b2, atok, aw, ab, fuse_sin):
    return (atok.new_empty((1, w0.shape[0])), atok.new_empty((1, w2.shape[0])),
            atok.new_empty((1, atok.shape[1], w0.shape[0])))


# --------------------------------------------------------------------------- CAE fused levers (CA)
def _mod_vec(mod: torch.Tensor, tmod: torch.Tensor, i: int, n: int) -> torch.Tensor:
    """Chunk i (width n) of modulation + t_mod, one row for every token: the fp32 sum the CAE
    kernels form, rounded once to bf16 for the row kernel."""
    m, t = mod.reshape(-1), tmod.reshape(-1)
    if m.numel() < (i + 1) * n or t.numel() < (i + 1) * n:
        raise ValueError(f"modulation / t_mod hold fewer than {i + 1} chunks of {n}")
    return (m[i * n:(i + 1) * n].float() + t[i * n:(i + 1) * n].float()).to(_BF16).contiguous()


def _plane(t: torch.Tensor, M: int, N: int, name: str) -> torch.Tensor:
    """An fp32 [1, M, N] partial plane of t (the fp32 accumulators are used in place)."""
    if t.numel() != M * N:
        raise ValueError(f"{name} must hold {M} x {N} values, got {tuple(t.shape)}")
    if t.dtype != torch.float32 or not t.is_contiguous():
        t = t.float().contiguous()
    return t.view(1, M, N)


def _zero_rows(z: torch.Tensor, rows: int, name: str) -> None:
    """Rows [0, rows) of an fp32 [.., ZN] accumulator set to zero (the reference kernels clear
    the next layer's o-projection accumulators in passing)."""
    if z.dtype != torch.float32 or not z.is_contiguous() or z.numel() < rows * z.shape[-1]:
        raise ValueError(f"{name} must be a contiguous fp32 [>= {rows}, ZN] accumulator")
    z.view(-1, z.shape[-1])[:rows].zero_()


def _acc_add(acc: torch.Tensor, a2: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> None:
    """acc[:M] += a2 w^T + b in fp32 (the reference's o-projections accumulate into acc)."""
    _check(w, "wo")
    _check(b, "bo")
    M, K = a2.shape
    N = w.shape[0]
    if acc.dtype != torch.float32 or not acc.is_contiguous() or acc.numel() < M * N or acc.shape[-1] != N:
        raise ValueError(f"acc must be a contiguous fp32 [.., >= {M}, {N}] accumulator, got {tuple(acc.shape)}")
    acc2 = acc.view(-1, N)[:M]
    if M <= 64 and K % 8 == 0 and _capi.lib().fam_gemm_partial_splits(M, N, K) > 0:
        part, _ = gemm_partial(a2, w.contiguous())
    else:
        part = torch.empty((1, M, N), dtype=torch.float32, device=a2.device)
        gemm(a2, w.contiguous(), None, part.view(M, N), out_f32=True)
    rowop(acc2, partials=part, bias=b.contiguous(), res=acc2)


def _cae_mask(msk: torch.Tensor, M: int, SK: int, bias_form: bool):
    """The attention mask operand: the additive 0 / -inf fp32 plane of fastwam::mask_bias when
    bias_form (read in place, row stride kept), else a keep plane (nonzero = attend)."""
    if bias_form:
        return msk[:M, :SK]
    return _keep_plane(msk, M, SK)


def _pow2(n: int) -> int:
    return 1 << (int(n) - 1).bit_length()


@torch.library.custom_op("fastwam::mask_bias", mutates_args=())
def mask_bias(am: torch.Tensor, cm: torch.Tensor, mp: int, skp: int, ncp: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """The CAE expert's two additive attention-bias planes in one launch (CA/mot.py:3342-3369):
    sb [mp, skp] fp32, 0 where row m < M keeps action key c of am [M, SK] (padding rows keep key 0
    only), and xb [mp, ncp], 0 where row m < M keeps context key c of cm ([M, NS], or [1, NS] for
    every row); -inf elsewhere."""
    if am.dim() != 2 or cm.dim() != 2:
        raise ValueError("am must be [M, SK] and cm [M or 1, NS]")
    M, SK = am.shape
    NS = cm.shape[1]
    if cm.shape[0] not in (1, M):
        raise ValueError(f"cm must have 1 or {M} rows, got {tuple(cm.shape)}")

    def u8(t):
        t = t.contiguous() if t.dtype in (torch.bool, torch.uint8) else (t != 0).contiguous()
        return t.view(torch.uint8) if t.dtype == torch.bool else t
    a8, c8 = u8(am), u8(cm)
    cms = 0 if cm.shape[0] == 1 and M != 1 else NS
    sb = torch.empty((mp, skp), dtype=torch.float32, device=am.device)
    xb = torch.empty((mp, ncp), dtype=torch.float32, device=am.device)
    call("fam_mask_bias", a8.data_ptr(), c8.data_ptr(), cms, M, SK, NS, mp, skp, ncp, sb.data_ptr(), xb.data_ptr(),
         _stream(sb))
    return sb, xb


@mask_bias.register_fake
def _(am, cm, mp, skp, ncp):
    return am.new_empty((mp, skp), dtype=torch.float32), am.new_empty((mp, ncp), dtype=torch.float32)


@torch.library.custom_op("fastwam::mot_attn_oproj", mutates_args={"acc"})
def mot_attn_oproj(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, msk: torch.Tensor, wo: torch.Tensor,
                   bo: torch.Tensor, acc: torch.Tensor, nh: int, hd: int) -> None:
    """The self attention of head-major q [1, H, M, hd] over k / v [1, H, SK, hd] with its o
    projection added into the fp32 accumulator: acc[:M] += attn wo^T + bo (CA/mot.py:2864-2900,
    kernel :2563-2680).  msk is a keep plane (nonzero = attend) or, as [mp, skp] fp32 with mp =
    max(16, pow2(M)) and skp = pow2(SK), fastwam::mask_bias's additive plane."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _check(t, n)
    H, D = int(nh), int(hd)
    M, SK = q.shape[2], k.shape[2]
    bias_form = msk.dim() == 2 and msk.dtype == torch.float32 and tuple(msk.shape) == (max(16, _pow2(M)), _pow2(SK))
    o = torch.empty((1, M, H * D), dtype=q.dtype, device=q.device)
    _launch_attention(q, _bhsd_strides(q), k, _bhsd_strides(k), v, _bhsd_strides(v), o, _bshd_strides(o, D), 1, H,
                      M, SK, D, _cae_mask(msk, M, SK, bias_form))
    _acc_add(acc, o.view(M, H * D), wo, bo)


@mot_attn_oproj.register_fake
def _(q, k, v, msk, wo, bo, acc, nh, hd):
    return None


def _n3q(res, so, mod, tmod, lnw, lnb, qw, qb, eps):
    """x = res + gate_msa so (chunk 2), n = norm3(x) with its affine, cq = n qw^T + qb; bf16."""
    for t, n in ((res, "res"), (mod, "mod"), (tmod, "tmod"), (lnw, "lnw"), (lnb, "lnb"), (qw, "qw"), (qb, "qb")):
        _check(t, n)
    D = res.shape[-1]
    M = res.numel() // D
    r2 = _rows2d(res)
    x = torch.empty((1, M, D), dtype=_BF16, device=res.device)
    n = torch.empty((M, D), dtype=_BF16, device=res.device)
    rowop(x.view(M, D), partials=_plane(so, M, D, "so"), res=r2, gate=_mod_vec(mod, tmod, 2, D),
          norm=_capi.FAM_ROWNORM_LAYERNORM, eps=eps, ln_w=lnw.contiguous(), ln_b=lnb.contiguous(), nout=n)
    cq = torch.empty((1, M, qw.shape[0]), dtype=_BF16, device=res.device)
    gemm(n, qw.contiguous(), qb.contiguous(), cq.view(M, qw.shape[0]))
    return x, cq


def _check_gram(gram: torch.Tensor, D: int) -> None:
    if gram.numel() != D * D + D + 1:
        raise ValueError(f"gram must hold [[Wq^T Wq], [Wq^T bq], [|bq|^2]] = {D * D + D + 1} values, "
                         f"got {gram.numel()}")


@torch.library.custom_op("fastwam::mod_n3q", mutates_args=())
def mod_n3q(res: torch.Tensor, so: torch.Tensor, mod: torch.Tensor, tmod: torch.Tensor, lnw: torch.Tensor,
            lnb: torch.Tensor, qw: torch.Tensor, qb: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """(x, cq): x = res + gate_msa so (so the self-attention o-projection, bf16 or its fp32
    accumulator), cq = LN3(x) lnw + lnb projected by the cross-attention q (CA/mot.py:2978-3008,
    kernel :2707-2780)."""
    return _n3q(res, so, mod, tmod, lnw, lnb, qw, qb, eps)


@mod_n3q.register_fake
def _(res, so, mod, tmod, lnw, lnb, qw, qb, eps):
    d = int(res.shape[-1])
    m = int(res.shape[-2])
    return res.new_empty((1, m, d)), res.new_empty((1, m, int(qw.shape[0])))


def _n3q_qn(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, eps, eps_q):
    _check(qnw, "qnw")
    _check_gram(gram, res.shape[-1])
    x, cq = _n3q(res, so, mod, tmod, lnw, lnb, qw, qb, eps)
    M, N = cq.shape[1], cq.shape[2]
    cqn = torch.empty_like(cq)
    _rms(cq.view(M, N), cqn.view(M, N), qnw.contiguous(), eps_q)
    return x, cqn


@torch.library.custom_op("fastwam::mod_n3q_qn", mutates_args=())
def mod_n3q_qn(res: torch.Tensor, so: torch.Tensor, mod: torch.Tensor, tmod: torch.Tensor, lnw: torch.Tensor,
               lnb: torch.Tensor, qw: torch.Tensor, qb: torch.Tensor, qnw: torch.Tensor, gram: torch.Tensor,
               eps: float, eps_q: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """mod_n3q with the cross-attention norm_q (RMSNorm over the whole q row, weight qnw) applied
    to cq (CA/mot.py:3227-3262).  The reference takes the row's sum of squares from the Gram
    block gram; here the row kernel sums the squares of the row itself (the same quantity; gram
    is checked for its shape only)."""
    return _n3q_qn(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, eps, eps_q)


@mod_n3q_qn.register_fake
def _(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, eps, eps_q):
    d = int(res.shape[-1])
    m = int(res.shape[-2])
    return res.new_empty((1, m, d)), res.new_empty((1, m, int(qw.shape[0])))


@torch.library.custom_op("fastwam::n3q_xoproj", mutates_args={"acc"})
def n3q_xoproj(res: torch.Tensor, so: torch.Tensor, mod: torch.Tensor, tmod: torch.Tensor, lnw: torch.Tensor,
               lnb: torch.Tensor, qw: torch.Tensor, qb: torch.Tensor, qnw: torch.Tensor, gram: torch.Tensor,
               ck: torch.Tensor, cv: torch.Tensor, msk: torch.Tensor, wo: torch.Tensor, bo: torch.Tensor,
               acc: torch.Tensor, nh: int, eps: float, eps_q: float) -> torch.Tensor:
    """mod_n3q_qn, then the cross attention of that query per head over the context keys / values
    ck / cv [1, NSEQ, NQ] (row stride ck.stride(1), so a layer's slice of a stacked buffer reads
    in place) and the cross o-projection added into acc: acc[:M] += attn wo^T + bo; returns x
    (CA/mot.py:3414-3470, kernel :1556-1680).  msk: a [1, M, NSEQ] keep plane, or fastwam::
    mask_bias's fp32 plane (2-D, at least max(16, pow2(M)) rows and NSEQ columns)."""
    _check(ck, "ck")
    _check(cv, "cv")
    x, cqn = _n3q_qn(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, eps, eps_q)
    M, NQ = cqn.shape[1], cqn.shape[2]
    H = int(nh)
    hd, NSEQ = NQ // H, ck.shape[1]
    if H * hd != NQ or ck.shape[-1] != NQ or cv.shape[1] != NSEQ or cv.shape[-1] != NQ:
        raise ValueError(f"ck / cv must be [1, {NSEQ}, {NQ}] for {H} heads")
    bias_form = msk.dim() == 2 and msk.dtype == torch.float32 and msk.shape[0] >= max(16, _pow2(M)) and \
        msk.shape[1] >= NSEQ
    o = torch.empty((1, M, NQ), dtype=_BF16, device=res.device)
    _launch_attention(cqn, _bshd_strides(cqn, hd), ck, (0, ck.stride(1), hd), cv, (0, cv.stride(1), hd), o,
                      _bshd_strides(o, hd), 1, H, M, NSEQ, hd, _cae_mask(msk, M, NSEQ, bias_form))
    _acc_add(acc, o.view(M, NQ), wo, bo)
    return x


@n3q_xoproj.register_fake
def _(res, so, mod, tmod, lnw, lnb, qw, qb, qnw, gram, ck, cv, msk, wo, bo, acc, nh, eps, eps_q):
    d = int(res.shape[-1])
    return res.new_empty((1, int(res.shape[-2]), d))


def _ffn_fold(x, oacc, modc, modn, tmod, w1, b1, w2, b2, eps2, eps1, hasnext):
    for t, n in ((x, "x"), (modc, "modc"), (modn, "modn"), (tmod, "tmod"), (w1, "w1"), (b1, "b1"), (w2, "w2"),
                 (b2, "b2")):
        _check(t, n)
    H = x.shape[-1]
    M = x.numel() // H
    x2 = _rows2d(x)
    v = torch.empty((M, H), dtype=_BF16, device=x.device)
    a = torch.empty((M, H), dtype=_BF16, device=x.device)
    rowop(v, partials=_plane(oacc, M, H, "oacc"), res=x2, norm=_capi.FAM_ROWNORM_ADALN, eps=eps2,
          shift=_mod_vec(modc, tmod, 3, H), scale=_mod_vec(modc, tmod, 4, H), mod_strides=(0, 0), nout=a)
    hid = torch.empty((M, w1.shape[0]), dtype=_BF16, device=x.device)
    gemm(a, w1.contiguous(), b1.contiguous(), hid, act=_capi.FAM_ACT_GELU_TANH)
    f = torch.empty((1, M, H), dtype=torch.float32, device=x.device)
    gemm(hid, w2.contiguous(), b2.contiguous(), f.view(M, H), out_f32=True)
    xout = torch.empty((1, M, H), dtype=_BF16, device=x.device)
    ai = torch.empty((1, M, H), dtype=_BF16, device=x.device)
    kw = dict(partials=f, res=v, gate=_mod_vec(modc, tmod, 5, H))
    if hasnext:
        rowop(xout.view(M, H), norm=_capi.FAM_ROWNORM_ADALN, eps=eps1, shift=_mod_vec(modn, tmod, 0, H),
              scale=_mod_vec(modn, tmod, 1, H), mod_strides=(0, 0), nout=ai.view(M, H), **kw)
    else:
        rowop(xout.view(M, H), **kw)
    return xout, ai


@torch.library.custom_op("fastwam::mot_ffn_fold", mutates_args=())
def mot_ffn_fold(x: torch.Tensor, oacc: torch.Tensor, modc: torch.Tensor, modn: torch.Tensor, tmod: torch.Tensor,
                 w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor, eps2: float, eps1: float,
                 hasnext: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(xout, aiout): v = x + oacc (the cross o-projection's fp32 accumulator), the FFN on
    norm2's AdaLN of v (shift / scale chunks 3 / 4 of modc + t_mod), xout = v + gate_mlp (chunk
    5) ffn; with hasnext, aiout = the next block's AdaLN1 of xout (chunks 0 / 1 of modn + t_mod),
    else aiout is not written, as in the reference (CA/mot.py:3086-3122, kernel :2346-2430)."""
    return _ffn_fold(x, oacc, modc, modn, tmod, w1, b1, w2, b2, eps2, eps1, hasnext)


@mot_ffn_fold.register_fake
def _(x, oacc, modc, modn, tmod, w1, b1, w2, b2, eps2, eps1, hasnext):
    d = int(x.shape[-1])
    m = int(x.numel()) // d if x.numel() > 0 else int(x.shape[-2])
    return x.new_empty((1, m, d)), x.new_empty((1, m, d))


def _sa_qkv(xin, w, b, qgr, kgr, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps):
    for t, n in ((xin, "xin"), (w, "w"), (b, "b")):
        _check(t, n)
    K = xin.shape[-1]
    _check_gram(qgr, K)
    _check_gram(kgr, K)
    x2 = _rows2d(xin)
    M, D3 = x2.shape[0], w.shape[0]
    D = D3 // 3
    qkv = torch.empty((M, D3), dtype=_BF16, device=xin.device)
    gemm(x2, w.contiguous(), b.contiguous(), qkv)
    _zero_rows(za, M, "za")
    _zero_rows(zb, M, "zb")
    return _head_major(_cae_qkv_rows(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], qw, kw, freqs, kbuf, vbuf, sv,
                                     eps), kbuf.shape[1])


@torch.library.custom_op("fastwam::mot_sa_qkv", mutates_args={"kbuf", "vbuf", "za", "zb"})
def mot_sa_qkv(xin: torch.Tensor, w: torch.Tensor, b: torch.Tensor, qgr: torch.Tensor, kgr: torch.Tensor,
               qw: torch.Tensor, kw: torch.Tensor, freqs: torch.Tensor, kbuf: torch.Tensor, vbuf: torch.Tensor,
               za: torch.Tensor, zb: torch.Tensor, sv: int, eps: float) -> torch.Tensor:
    """The fused q / k / v projection of the hidden-K action rows (w [3D, K], b [3D]) and
    mot_qkv_post's normalisation, rotation and K / V cache writes; rows [0, M) of the fp32
    accumulators za / zb cleared; q returned head-major (CA/mot.py:3285-3322, kernel
    :1458-1553).  qgr / kgr are the reference's Gram blocks of the q / k norms (checked for
    shape; the row kernel sums the row's own squares)."""
    return _sa_qkv(xin, w, b, qgr, kgr, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps)


@mot_sa_qkv.register_fake
def _(xin, w, b, qgr, kgr, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps):
    return xin.new_empty((1, kbuf.shape[1], xin.numel() // xin.shape[-1], kbuf.shape[3]))


@torch.library.custom_op("fastwam::mot_ffn_sa_qkv", mutates_args={"kbuf", "vbuf", "za", "zb"})
def mot_ffn_sa_qkv(xp: torch.Tensor, oacc: torch.Tensor, modc: torch.Tensor, modn: torch.Tensor, tmod: torch.Tensor,
                   f1w: torch.Tensor, f1b: torch.Tensor, f2w: torch.Tensor, f2b: torch.Tensor, w: torch.Tensor,
                   b: torch.Tensor, qgr: torch.Tensor, kgr: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor,
                   freqs: torch.Tensor, kbuf: torch.Tensor, vbuf: torch.Tensor, za: torch.Tensor, zb: torch.Tensor,
                   sv: int, eps: float, eps2: float, eps1: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """mot_ffn_fold of layer L (with the next block's AdaLN1) followed by mot_sa_qkv of layer L + 1
    on that input: returns (xout, q head-major) (CA/mot.py:3498-3565)."""
    xout, ai = _ffn_fold(xp, oacc, modc, modn, tmod, f1w, f1b, f2w, f2b, eps2, eps1, 1)
    return xout, _sa_qkv(ai, w, b, qgr, kgr, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps)


@mot_ffn_sa_qkv.register_fake
def _(xp, oacc, modc, modn, tmod, f1w, f1b, f2w, f2b, w, b, qgr, kgr, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps,
      eps2, eps1):
    k = int(xp.shape[-1])
    m = int(xp.numel()) // k
    return xp.new_empty((1, m, k)), xp.new_empty((1, kbuf.shape[1], m, kbuf.shape[3]))


@torch.library.custom_op("fastwam::mot_qkv_post_z", mutates_args={"kbuf", "vbuf", "za", "zb"})
def mot_qkv_post_z(qkv: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor, freqs: torch.Tensor, kbuf: torch.Tensor,
                   vbuf: torch.Tensor, za: torch.Tensor, zb: torch.Tensor, sv: int, eps: float) -> torch.Tensor:
    """mot_qkv_post, and rows [0, M) of the fp32 accumulators za / zb cleared (CA/mot.py:2830-2860)."""
    _check(qkv, "qkv")
    M, D3 = qkv.shape[1], qkv.shape[2]
    D = D3 // 3
    x2 = qkv.reshape(M, D3)
    _zero_rows(za, M, "za")
    _zero_rows(zb, M, "zb")
    return _head_major(_cae_qkv_rows(x2[:, :D], x2[:, D:2 * D], x2[:, 2 * D:], qw, kw, freqs, kbuf, vbuf, sv, eps),
                       kbuf.shape[1])


@mot_qkv_post_z.register_fake
def _(qkv, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps):
    return qkv.new_empty((1, kbuf.shape[1], qkv.shape[1], kbuf.shape[3]))


@torch.library.custom_op("fastwam::mot_qkv_gemm_post_z", mutates_args={"kbuf", "vbuf", "za", "zb"})
def mot_qkv_gemm_post_z(xin: torch.Tensor, wt: torch.Tensor, bqkv: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor,
                        freqs: torch.Tensor, kbuf: torch.Tensor, vbuf: torch.Tensor, za: torch.Tensor,
                        zb: torch.Tensor, sv: int, eps: float) -> torch.Tensor:
    """mot_qkv_post_z on qkv = xin wt + bqkv, wt the transposed [K, 3D] projection weight
    (CA/mot.py:3032-3070, kernel :1369-1456 with GK = K)."""
    _check(xin, "xin")
    _check(wt, "wt")
    _check(bqkv, "bqkv")
    x2 = _rows2d(xin)
    M, D3 = x2.shape[0], wt.shape[1]
    D = D3 // 3
    qkv = torch.empty((M, D3), dtype=_BF16, device=xin.device)
    gemm(x2, wt.t().contiguous(), bqkv.contiguous(), qkv)
    _zero_rows(za, M, "za")
    _zero_rows(zb, M, "zb")
    return _head_major(_cae_qkv_rows(qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], qw, kw, freqs, kbuf, vbuf, sv,
                                     eps), kbuf.shape[1])


@mot_qkv_gemm_post_z.register_fake
def _(xin, wt, bqkv, qw, kw, freqs, kbuf, vbuf, za, zb, sv, eps):
    return xin.new_empty((1, kbuf.shape[1], xin.shape[-2], kbuf.shape[3]))


def _l0_qkv(q, k, v, qw, kw, freqs, kbuf, vbuf, sv, eps):
    _check(q, "q")
    M, D = q.shape[1], q.shape[2]
    qout = torch.empty_like(q, memory_format=torch.contiguous_format)
    _cae_qkv_rows(q.reshape(M, D), k.reshape(M, D), v.reshape(M, D), qw, kw, freqs, kbuf, vbuf, sv, eps,
                  q_out=qout.view(M, D))
    return qout


@torch.library.custom_op("fastwam::mot_l0_qkv_rope", mutates_args={"kbuf", "vbuf"})
def mot_l0_qkv_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor,
                    freqs: torch.Tensor, kbuf: torch.Tensor, vbuf: torch.Tensor, sv: int, eps: float) -> torch.Tensor:
    """Layer 0's q / k / v post-processing from separate [1, M, D] projections: the q rows
    normalised and rotated, token-major like q; k / v to rows sv .. sv + M of the head-major
    caches (CA/mot.py:3142-3172, kernel :2430-2480)."""
    return _l0_qkv(q, k, v, qw, kw, freqs, kbuf, vbuf, sv, eps)


@mot_l0_qkv_rope.register_fake
def _(q, k, v, qw, kw, freqs, kbuf, vbuf, sv, eps):
    return torch.empty_like(q)


@torch.library.custom_op("fastwam::mot_l0_qkv_rope_z", mutates_args={"kbuf", "vbuf", "oaccx"})
def mot_l0_qkv_rope_z(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor,
                      freqs: torch.Tensor, kbuf: torch.Tensor, vbuf: torch.Tensor, oaccx: torch.Tensor, sv: int,
                      eps: float) -> torch.Tensor:
    """mot_l0_qkv_rope, and rows [0, M) of layer 0's cross o-projection accumulator oaccx [M, NO]
    cleared (CA/mot.py:3180-3210)."""
    qout = _l0_qkv(q, k, v, qw, kw, freqs, kbuf, vbuf, sv, eps)
    _zero_rows(oaccx, q.shape[1], "oaccx")
    return qout


@mot_l0_qkv_rope_z.register_fake
def _(q, k, v, qw, kw, freqs, kbuf, vbuf, oaccx, sv, eps):
    return torch.empty_like(q)


def _ctx_kv_into(g: torch.Tensor, nkw: torch.Tensor, out: torch.Tensor, nl: int, ahd: int, eps: float) -> None:
    """out [2, nl, 1, S, ahd]: [0] the normalised keys of every layer, [1] the values."""
    S = g.shape[0]
    if out.shape != (2, nl, 1, S, ahd) or out.dtype != _BF16 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous bf16 [2, {nl}, 1, {S}, {ahd}] tensor, got {tuple(out.shape)}")
    out[0].copy_(ctx_kv_norm(g, nkw, nl, ahd, eps)[0])
    out[1].copy_(g[:, nl * ahd:].reshape(S, nl, ahd).transpose(0, 1).unsqueeze(1))


@torch.library.custom_op("fastwam::ctx_kv_norm_into", mutates_args=("out",))
def ctx_kv_norm_into(g: torch.Tensor, nkw: torch.Tensor, out: torch.Tensor, nl: int, ahd: int, eps: float) -> None:
    """ctx_kv_norm with the values too, into out [2, nl, 1, S, ahd]: [0] the RMS-normalised keys,
    [1] the values, layer-major (CA/mot.py:3621-3638)."""
    _ctx_kv_into(g, nkw, out, int(nl), int(ahd), eps)


@ctx_kv_norm_into.register_fake
def _(g, nkw, out, nl, ahd, eps):
    return None


@torch.library.custom_op("fastwam::ctx_kv_gemm_norm_into", mutates_args=("out",))
def ctx_kv_gemm_norm_into(e: torch.Tensor, w: torch.Tensor, b: torch.Tensor, nkw: torch.Tensor, out: torch.Tensor,
                          nl: int, ahd: int, eps: float, has_b: bool) -> None:
    """ctx_kv_norm_into on g = e w^T (+ b with has_b): the whole stack's context K / V projection
    (w [2 nl ahd, C], keys of every layer before the values) and its key norm
    (CA/mot.py:3641-3662, kernel :2166-2210)."""
    _check(e, "e")
    _check(w, "w")
    S, nl, ahd = e.shape[0], int(nl), int(ahd)
    if w.shape[0] != 2 * nl * ahd:
        raise ValueError(f"w must have {2 * nl * ahd} rows, got {tuple(w.shape)}")
    g = torch.empty((S, w.shape[0]), dtype=_BF16, device=e.device)
    gemm(_rows2d(e), w.contiguous(), b.contiguous() if has_b else None, g)
    _ctx_kv_into(g, nkw, out, nl, ahd, eps)


@ctx_kv_gemm_norm_into.register_fake
def _(e, w, b, nkw, out, nl, ahd, eps, has_b):
    return None


@torch.library.custom_op("fastwam::vqkv_post", mutates_args={"kbuf", "vbuf"})
def vqkv_post(qkv: torch.Tensor, qw: torch.Tensor, kw: torch.Tensor, freqs: torch.Tensor, kbuf: torch.Tensor,
              vbuf: torch.Tensor, eps: float) -> torch.Tensor:
    """The video prefill's q / k / v post-processing: returns [3, 1, M, D] (q, k normalised and
    rotated, v as is, token-major) and writes k / v head-major to rows [0, M) of kbuf / vbuf
    [1, H, SKV, hd], clearing rows [M, SKV) (CA/mot.py:3713-3750, kernel :2015-2077)."""
    _check(qkv, "qkv")
    M, D3 = qkv.shape[1], qkv.shape[2]
    D = D3 // 3
    x2 = qkv.reshape(M, D3)
    out = torch.empty((3, 1, M, D), dtype=qkv.dtype, device=qkv.device)
    _cae_qkv_rows(x2[:, :D], x2[:, D:2 * D], x2[:, 2 * D:], qw, kw, freqs, kbuf, vbuf, 0, eps,
                  q_out=out[0, 0])
    H, hd = kbuf.shape[1], kbuf.shape[3]
    out[1, 0].view(M, H, hd).copy_(kbuf[0, :, :M].transpose(0, 1))
    out[2, 0].copy_(x2[:, 2 * D:])
    kbuf[0, :, M:].zero_()
    vbuf[0, :, M:].zero_()
    return out


@vqkv_post.register_fake
def _(qkv, qw, kw, freqs, kbuf, vbuf, eps):
    d = int(kbuf.shape[1]) * int(kbuf.shape[3])
    return qkv.new_empty((3, 1, int(qkv.shape[1]), d))


# --------------------------------------------------------------------------- fp8 rows (CA video prefill)
_FP8 = torch.float8_e4m3fn


def _row_q8(mode: int, x: torch.Tensor, x2: Optional[torch.Tensor] = None, shift=None, scale=None, eps: float = 0.0):
    _check(x, "x")
    D = x.shape[-1]
    xc = x.contiguous()
    M = xc.numel() // D
    y = torch.empty((M, D), dtype=_FP8, device=x.device)
    s = torch.empty((M, 1), dtype=torch.float32, device=x.device)
    d = _capi.RowQ8Desc()
    d.mode, d.x, d.ldx, d.M, d.D = mode, xc.data_ptr(), D, M, D
    d.y, d.ldy, d.s = y.data_ptr(), D, s.data_ptr()
    keep = [xc]
    if shift is not None:
        sh, sc = shift.reshape(-1).contiguous(), scale.reshape(-1).contiguous()
        for t, n in ((sh, "shift"), (sc, "scale")):
            _check(t, n)
            if t.numel() != D:
                raise ValueError(f"{n} must hold {D} values, got {t.numel()}")
        d.shift, d.scale, d.eps = sh.data_ptr(), sc.data_ptr(), float(eps)
        keep += [sh, sc]
    xo = None
    if x2 is not None:
        _check(x2, "b")
        if x2.shape != x.shape:
            raise ValueError(f"a and b must have one shape, got {tuple(x.shape)} and {tuple(x2.shape)}")
        b2 = x2.contiguous()
        xo = torch.empty_like(xc)
        d.x2, d.ldx2, d.xo, d.ldxo = b2.data_ptr(), D, xo.data_ptr(), D
        keep += [b2]
    call("fam_row_q8", C.byref(d), _stream(x))
    del keep
    return xo, y, s


@torch.library.custom_op("fastwam::row_q8", mutates_args=())
def row_q8(x: torch.Tensor) -> List[torch.Tensor]:
    """[q, s]: the rows of x [.., D] quantised to fp8 e4m3 with a per-row scale s [M, 1]
    (q s = x to e4m3's precision; CA/mot.py:3936-3960, kernel :3836-3849)."""
    _, y, s = _row_q8(_capi.FAM_Q8_ROW, x)
    return [y, s]


@row_q8.register_fake
def _(x):
    d = int(x.shape[-1])
    m = x.numel() // d
    return [x.new_empty((m, d), dtype=_FP8), x.new_empty((m, 1), dtype=torch.float32)]


@torch.library.custom_op("fastwam::gelu_q8", mutates_args=())
def gelu_q8(x: torch.Tensor) -> List[torch.Tensor]:
    """[q, s] of bf16(GELU_tanh(x)), the activation between the video FFN's two fp8 GEMMs
    (CA/mot.py:3914-3934, kernel :3817-3833)."""
    _, y, s = _row_q8(_capi.FAM_Q8_GELU, x)
    return [y, s]


@gelu_q8.register_fake
def _(x):
    d = int(x.shape[-1])
    m = x.numel() // d
    return [x.new_empty((m, d), dtype=_FP8), x.new_empty((m, 1), dtype=torch.float32)]


@torch.library.custom_op("fastwam::ln_mod_q8", mutates_args=())
def ln_mod_q8(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, eps: float) -> List[torch.Tensor]:
    """[q, s] of bf16(bf16(LN(x)) (1 + scale) + shift), shift / scale [D] for every row
    (CA/mot.py:3859-3883, kernel :3763-3787)."""
    _, y, s = _row_q8(_capi.FAM_Q8_LN_MOD, x, shift=shift, scale=scale, eps=eps)
    return [y, s]


@ln_mod_q8.register_fake
def _(x, shift, scale, eps):
    d = int(x.shape[-1])
    m = x.numel() // d
    return [x.new_empty((m, d), dtype=_FP8), x.new_empty((m, 1), dtype=torch.float32)]


@torch.library.custom_op("fastwam::add_ln_mod_q8", mutates_args=())
def add_ln_mod_q8(a: torch.Tensor, b: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                  eps: float) -> List[torch.Tensor]:
    """[xo, q, s]: xo = bf16(a + b) (the cross-attention residual), then ln_mod_q8 of xo
    (CA/mot.py:3885-3912, kernel :3789-3814)."""
    xo, y, s = _row_q8(_capi.FAM_Q8_ADD_LN_MOD, a, x2=b, shift=shift, scale=scale, eps=eps)
    return [xo.view(a.shape), y, s]


@add_ln_mod_q8.register_fake
def _(a, b, shift, scale, eps):
    d = int(a.shape[-1])
    m = a.numel() // d
    return [torch.empty_like(a), a.new_empty((m, d), dtype=_FP8), a.new_empty((m, 1), dtype=torch.float32)]

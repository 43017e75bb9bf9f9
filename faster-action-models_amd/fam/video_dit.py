"""DiT block of the video backbone at long sequence length on the gfx950 kernels.

One `DiTBlock.forward` (FB/wan_video_dit.py:267-286) for the video tokens of the backbone
(Wan2.2-5B-style config: 1560 tokens = 2 latent frames x 30 x 26 patches with 3-D RoPE,
hidden 3072, 24 x 128 heads, FFN 14336, 512 text tokens, per-token AdaLN modulation,
FB/wan_video_dit.py:555-568), built from the library's kernels:

    mods   = modulation + t_mod                           fam_add_modulation
    h      = AdaLN1(x)   (per-token shift/scale)          fam_adaln
    qkv    = h Wqkv^T + b                                 fam_gemm (tiled, MFMA)
    q, k   = RoPE3D(RMSNorm(q)), RoPE3D(RMSNorm(k))       fam_rmsnorm_rope (in place)
    a      = softmax(q k^T / sqrt(Dh)) v                  fam_attention (64-query tiles)
    x      = x + g_msa * (a Wo^T + bo)                    fam_gemm epilogue (per-token gate)
    h      = LayerNorm3(x)                                fam_adaln (affine)
    qc     = RMSNorm(h Wq^T + bq)                         fam_gemm + fam_rmsnorm_rope
    kc, vc = RMSNorm(ctx Wk^T + bk), ctx Wv^T + bv        fam_gemm (fused k|v) + fam_rmsnorm_rope
    x      = x + (attn(qc, kc, vc) Wo^T + bo)             fam_attention + fam_gemm epilogue
    h      = AdaLN2(x)                                    fam_adaln
    x      = x + g_mlp * (GELU(h W1^T + b1) W2^T + b2)    fam_gemm (GELU epilogue), fam_gemm (gate)

Every launch is prebuilt once per shape; `run()` enqueues them on the current stream and
`capture()` records them in one HIP graph.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _capi
from .ops import rope_tables

_BF16 = torch.bfloat16


def video_freqs_3d(head_dim: int, f: int, h: int, w: int):
    """3-D RoPE table of an (f, h, w) grid, complex [f*h*w, 1, .]: per-axis tables over
    head_dim - 2*(head_dim//3), head_dim//3 and head_dim//3 dims (44/42/42 for head_dim 128),
    angles pos * 10000^(-2j/d) in fp64 through torch.polar, concatenated per token in f-major
    order (FB/wan_video_dit.py:41-55, 620-624)."""
    import torch
    dims = (head_dim - 2 * (head_dim // 3), head_dim // 3, head_dim // 3)

    def table(d, n):
        j = torch.arange(0, d, 2, dtype=torch.float64)[: d // 2]
        ang = torch.outer(torch.arange(n, dtype=torch.float64), 1.0 / (10000.0 ** (j / d)))
        return torch.polar(torch.ones_like(ang), ang)

    tf, th, tw = table(dims[0], f), table(dims[1], h), table(dims[2], w)
    grid = torch.cat([tf[:, None, None, :].expand(f, h, w, -1), th[None, :, None, :].expand(f, h, w, -1),
                      tw[None, None, :, :].expand(f, h, w, -1)], dim=-1)
    return grid.reshape(f * h * w, 1, -1)


class FusedVideoDiTBlock:
    """One DiT block (the reference's `blocks.{idx}.` parameters) for fixed (B, S, Lc).

    Optional, for the MoT video prefill (FB/mot.py:262-376):
        self_mask: bool [S, S] on the self-attention (True = attend), shared by batch and heads.
        ctx_mask: bool [B, S, Lc] on the cross-attention (the video context payload's mask).
        ctx_len = 0: no cross-attention (a prefill without a context payload).
        shared: buffers to use instead of allocating ("x", "tmod_in", "ctx" and the scratch
            "mods", "h", "attn", "qc", "ckv", "hid", "part"), so that blocks chain in place.
        ctx_kv: (buffer [B*Lc, W] bf16, column of this block's [k | v]): the context K/V of the
            cross-attention computed outside (one GEMM for every block of a prefill) with k
            already normalised; the block then skips its own context projection and K norm.
        kv_only: build only what the block's K/V need -- modulation, AdaLN1, the q/k/v
            projection and the key's RMSNorm + RoPE -- for a last prefill block whose output
            nobody reads.
        mods_ready: "mods" (may be a row-strided view, e.g. one block of a [rows, L, 6H]
            buffer) already holds this block's modulation + t_mod; no modulation launch.
        pre_normed: the block's AdaLN1 output ("h") was produced by the block before it (see
            next_mod); the block starts at its q/k/v projection.
        next_mod: the next block's ready "mods" view: this block's FFN-down row applies the
            next block's AdaLN1 into "h" (only with the split-K projections).
        mod_group: tokens that share one modulation row (t_mod and "mods" hold B*S / mod_group
            rows; consecutive groups of mod_group tokens read one row): 0 follows per_token_mod
            (1 or S); WanVideoDiT passes the tokens of one latent frame, whose timestep is one.
    `self.qkv` holds [q | k | v] per row; after `run()` its k (normalised, rotated) and v
    columns are the block's attention K/V (`kv()`).
    """

    def __init__(self, params: Dict[str, torch.Tensor], idx: int, *, hidden: int, num_heads: int, head_dim: int,
                 ffn_dim: int, batch: int, seq_len: int, ctx_len: int, freqs: torch.Tensor, eps: float = 1e-6,
                 per_token_mod: bool = True, device="cuda", self_mask: Optional[torch.Tensor] = None,
                 ctx_mask: Optional[torch.Tensor] = None, shared: Optional[Dict[str, torch.Tensor]] = None,
                 kv_only: bool = False, ctx_kv: Optional[tuple] = None, mods_ready: bool = False,
                 pre_normed: bool = False, next_mod: Optional[torch.Tensor] = None, mod_group: int = 0):
        dev = torch.device(device)
        self.kv_only = kv_only
        self.mods_ready, self.pre_normed, self.next_mod = mods_ready, pre_normed, next_mod
        self.ctx_kv = ctx_kv
        self.lib = _capi.load()
        self.B, self.S, self.Lc = batch, seq_len, ctx_len
        self.H, self.nh, self.Dh, self.F = hidden, num_heads, head_dim, ffn_dim
        self.A = A = num_heads * head_dim
        self.eps = float(eps)
        self.mod_group = g = mod_group if mod_group > 0 else (1 if per_token_mod else seq_len)
        if seq_len % g:
            raise ValueError(f"mod_group {g} must divide seq_len {seq_len}")
        H, F = hidden, ffn_dim
        M = batch * seq_len
        pre = f"blocks.{idx}."

        def P(n):
            return params[pre + n].to(device=dev, dtype=_BF16).contiguous()

        def cat(ns):
            return torch.cat([params[pre + n].float() for n in ns], 0).to(device=dev, dtype=_BF16).contiguous()

        self.w = w = {
            "qkv_w": cat([f"self_attn.{n}.weight" for n in "qkv"]), "qkv_b": cat([f"self_attn.{n}.bias" for n in "qkv"]),
            "o_w": P("self_attn.o.weight"), "o_b": P("self_attn.o.bias"),
            "nq": P("self_attn.norm_q.weight"), "nk": P("self_attn.norm_k.weight"),
            "cq_w": P("cross_attn.q.weight"), "cq_b": P("cross_attn.q.bias"),
            "ckv_w": cat(["cross_attn.k.weight", "cross_attn.v.weight"]),
            "ckv_b": cat(["cross_attn.k.bias", "cross_attn.v.bias"]),
            "co_w": P("cross_attn.o.weight"), "co_b": P("cross_attn.o.bias"),
            "cnq": P("cross_attn.norm_q.weight"), "cnk": P("cross_attn.norm_k.weight"),
            "n3_w": P("norm3.weight"), "n3_b": P("norm3.bias"),
            "f0_w": P("ffn.0.weight"), "f0_b": P("ffn.0.bias"), "f2_w": P("ffn.2.weight"), "f2_b": P("ffn.2.bias"),
            "mod": P("modulation").reshape(6 * H).contiguous(),
        }
        cos, sin, trs, tes = rope_tables(freqs, "complex", dev)
        self.rope = (cos, sin, trs, tes)

        sh = shared or {}

        def buf(name, *shape, row_strided=False):
            t = sh.get(name)
            if t is None:
                return torch.zeros(*shape, dtype=_BF16, device=dev)
            dense = t.is_contiguous() or (row_strided and t.stride(1) == 1 and t.stride(0) >= shape[1]
                                          and t.stride(0) % 8 == 0)
            if tuple(t.shape) != tuple(shape) or t.dtype != _BF16 or not dense:
                raise ValueError(f"shared buffer {name!r} must be {'row-strided' if row_strided else 'contiguous'} "
                                 f"bf16 {tuple(shape)}")
            return t
        self.x = buf("x", M, H)
        self.tmod_in = buf("tmod_in", M // g, 6 * H)
        self.ctx = buf("ctx", batch * ctx_len, H)
        self.mods = buf("mods", M // g, 6 * H, row_strided=True)
        self.h = buf("h", M, H)
        self.qkv = torch.zeros(M, 3 * A, dtype=_BF16, device=dev)   # per block: its K/V cache
        self.attn = buf("attn", M, A)
        self.qc = buf("qc", M, A)
        self.ckv = buf("ckv", batch * ctx_len, 2 * A)
        self.hid = buf("hid", M, F)
        # <= 128 rows (the video prefill at 98 tokens): the N = hidden projections stream their
        # weights through fam_gemm_partial (split-K over >= 256 workgroups, every load issued
        # at once) and a row kernel applies bias / gate / residual (and the cross query's
        # RMSNorm); the tiled GEMM's k-loop would wait on memory once per 64-wide k-block
        self.splitk = M <= 128 and H <= 4096 and A <= 4096
        if self.splitk:
            need = max(self.lib.fam_gemm_partial_splits(M, n_, k_) * M * n_
                       for n_, k_ in ((H, A), (A, H), (H, F), (3 * A, H), (F, H)))
            t = sh.get("part")
            if t is not None and (t.dtype != torch.float32 or t.numel() < need):
                raise ValueError(f"shared buffer 'part' must be fp32 with >= {need} elements")
            self.part = t if t is not None else torch.zeros(need, dtype=torch.float32, device=dev)
        # above 128 rows: the fp32 planes of the large-M products the GEMM plan splits along K
        # (fam_gemm_ws; at config 2 only FFN down, whose 3072 output columns leave the big tiles
        # too few), one workspace shared by the blocks of a stack
        self.ws = None
        if not self.splitk:
            need = max([self.lib.fam_gemm_ws_floats(M, n_, k_)
                        for n_, k_ in ((3 * A, H), (H, A), (A, H), (F, H), (H, F))] +
                       [self.lib.fam_gemm_ws_floats(batch * ctx_len, 2 * A, H)] + [0])
            if need > 0:
                t = sh.get("ws")
                if t is not None and (t.dtype != torch.float32 or t.numel() < need or t.data_ptr() % 16):
                    raise ValueError(f"shared buffer 'ws' must be 16-byte aligned fp32 with >= {need} elements")
                self.ws = t if t is not None else torch.zeros(need, dtype=torch.float32, device=dev)
        if self_mask is not None:
            self_mask = self_mask.to(device=dev, dtype=torch.bool).contiguous()
            if tuple(self_mask.shape) != (seq_len, seq_len):
                raise ValueError(f"self_mask must be bool [S, S] = [{seq_len}, {seq_len}]")
        if ctx_mask is not None:
            # [B, S, Lc], or [B, Lc] shared by every query of a sample (read in place: a caller
            # may update it between calls)
            ctx_mask = ctx_mask.to(device=dev, dtype=torch.bool).contiguous()
            if tuple(ctx_mask.shape) not in ((batch, seq_len, ctx_len), (batch, ctx_len)):
                raise ValueError(f"ctx_mask must be bool [B, S, Lc] = [{batch}, {seq_len}, {ctx_len}] or "
                                 f"[B, Lc] = [{batch}, {ctx_len}]")
        self.self_mask, self.ctx_mask = self_mask, ctx_mask
        self._descs: List = []
        self.steps: List = []
        self.meta: List[dict] = []
        self._build()
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ launches
    def _add(self, name, fname, args, kind, flops=0):
        f, lib = getattr(self.lib, fname), self.lib

        def run(stream):
            rc = f(*args, stream)
            if rc != 0:
                raise _capi.FamError(f"{fname}[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.steps.append(run)
        self.meta.append({"name": name, "kernel": kind, "flops": int(flops)})

    def _gemm(self, name, a, w, bias, out, act=_capi.FAM_ACT_NONE, res=None, gate=None, gate_strides=(0, 0, 1)):
        d = _capi.GemmDesc()
        M, K = a.shape
        N = w.shape[0]
        d.a, d.lda, d.w, d.ldw = a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0)
        d.bias = bias.data_ptr() if bias is not None else None
        d.out, d.ldo = out.data_ptr(), out.stride(0)
        d.M, d.N, d.K = M, N, K
        d.act = act
        if res is not None:
            d.res, d.ldr = res.data_ptr(), res.stride(0)
        if gate is not None:
            d.gate = gate.data_ptr()
            d.gate_bs, d.gate_rs, d.gate_ns = gate_strides
        d.rows_per_batch = self.mod_group if M == self.B * self.S else M   # the gate's modulation rows
        self._descs.append(d)
        if self.ws is not None and self.lib.fam_gemm_ws_floats(M, N, K) > 0:
            self._add(name, "fam_gemm_ws", (C.byref(d), self.ws.data_ptr(), self.ws.numel()), "gemm", 2 * M * N * K)
        else:
            self._add(name, "fam_gemm", (C.byref(d),), "gemm", 2 * M * N * K)

    def _partial(self, name, a, w):
        """Split-K partials of a [M, K] x w[N, K]^T into self.part; returns the plane count."""
        M, K = a.shape
        N = w.shape[0]
        splits = self.lib.fam_gemm_partial_splits(M, N, K)
        self._add(name, "fam_gemm_partial", (a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
                                             self.part.data_ptr(), M, N, K), "gemm_partial", 2 * M * N * K)
        return splits

    def _rowop(self, name, *, N, splits, bias, out, res=None, gate=None, gate_strides=(0, 0, 1), rms_w=None,
               rope=False, col0=0, ldp=0, act=_capi.FAM_ACT_NONE, segs=None, seg_width=0, ln=None, adaln=None,
               nout=None):
        """out = res + gate * act(sum of the partial planes + bias) (or act(sum + bias)), then
        one normalisation of the stored row: rms_w, RMSNorm over the N columns in place; segs
        [(col0, weight)] of seg_width, RMSNorm per segment in place; ln (weight, bias),
        LayerNorm into nout; adaln (shift, scale) [rows, H] views, AdaLN into nout; RoPE on the
        RMS segments with rope.  col0 / ldp: columns [col0, col0 + N) of planes whose rows are
        ldp wide."""
        M = self.B * self.S
        ldp = ldp or N
        d = _capi.RowopDesc()
        d.src = _capi.FAM_ROWSRC_PARTIALS
        d.partials, d.splits, d.split_stride = self.part.data_ptr() + 4 * col0, splits, M * ldp
        d.ldp = ldp
        d.M, d.N = M, N
        d.bias = bias.data_ptr()
        d.act = act
        if res is not None:
            d.res, d.ldr = res.data_ptr(), res.stride(0)
        d.gate = gate.data_ptr() if gate is not None else None
        d.gate_bs, d.gate_rs, d.gate_ns = gate_strides
        d.rows_per_batch = self.mod_group   # rows per gate / modulation row (RoPE positions use seq_len)
        d.out, d.ldo, d.out_f32 = out.data_ptr(), out.stride(0), 0
        d.eps = self.eps
        if rms_w is not None:
            segs, seg_width = [(0, rms_w)], N
        if ln is not None:
            d.norm = _capi.FAM_ROWNORM_LAYERNORM
            d.ln_weight, d.ln_bias = ln[0].data_ptr(), ln[1].data_ptr()
            d.nout, d.ldn = nout.data_ptr(), nout.stride(0)
        elif adaln is not None:
            d.norm = _capi.FAM_ROWNORM_ADALN
            d.shift, d.scale = adaln[0].data_ptr(), adaln[1].data_ptr()
            d.mod_bs, d.mod_rs = self._mod_strides()
            d.nout, d.ldn = nout.data_ptr(), nout.stride(0)
        elif segs:
            d.norm = _capi.FAM_ROWNORM_RMS
            d.nseg = len(segs)
            for i, (c0, wt) in enumerate(segs):
                d.seg_col0[i], d.seg_weight[i] = c0, wt.data_ptr()
            d.seg_width = seg_width
            d.nout, d.ldn = out.data_ptr(), out.stride(0)
            if rope:
                cos, sin, trs, tes = self.rope
                d.rope_cos, d.rope_sin = cos.data_ptr(), sin.data_ptr()
                d.rope_row_stride, d.rope_elem_stride = trs, tes
                d.head_dim, d.seq_len = self.Dh, self.S
        self._descs.append(d)
        self._add(name, "fam_rowop", (C.byref(d),), "rowop")

    def _proj(self, name, a, w, bias, out, res=None, gate=None, gate_strides=(0, 0, 1), rms_w=None,
              act=_capi.FAM_ACT_NONE, ln=None, adaln=None, nout=None):
        """out = [res +] [gate *] act(a w^T + bias) [then RMSNorm in place, or LayerNorm / AdaLN
        of the stored row into nout]: split-K + row kernel at <= 128 rows, otherwise one
        fam_gemm followed by the norm's own kernel."""
        if self.splitk:
            sp = self._partial(name, a, w)
            self._rowop(name + "_row", N=w.shape[0], splits=sp, bias=bias, out=out, res=res, gate=gate,
                        gate_strides=gate_strides, rms_w=rms_w, act=act, ln=ln, adaln=adaln, nout=nout)
        else:
            self._gemm(name, a, w, bias, out, act=act, res=res, gate=gate, gate_strides=gate_strides)
            if rms_w is not None:
                self._rms(name + "_norm", out.data_ptr(), out.stride(0), out.shape[0], self.S, rms_w, False)
            if ln is not None:
                self._adaln(name + "_ln", out, nout, lw=ln[0], lb=ln[1])
            if adaln is not None:
                self._adaln(name + "_adaln", out, nout, shift=adaln[0], scale=adaln[1])

    def _mod_strides(self, mods=None):
        """(group, row) element strides of a modulation chunk view: row r of the activations reads
        modulation row r / mod_group (consumers take rows_per_batch = mod_group)."""
        rs = (self.mods if mods is None else mods).stride(0)
        return (rs, 0)

    def _adaln(self, name, x, y, shift=None, scale=None, lw=None, lb=None):
        M, H = x.shape
        mbs, mrs = self._mod_strides()
        args = (x.data_ptr(), x.stride(0), shift.data_ptr() if shift is not None else None,
                scale.data_ptr() if scale is not None else None, mbs, mrs,
                lw.data_ptr() if lw is not None else None, lb.data_ptr() if lb is not None else None,
                y.data_ptr(), y.stride(0), M, self.mod_group, H, self.eps)
        self._add(name, "fam_adaln", args, "adaln")

    def _rms(self, name, x_ptr, ld, rows, seq, weight, rope):
        A, Dh = self.A, self.Dh
        cs, sn, trs, tes = self.rope if rope else (None, None, 0, 0)
        args = (x_ptr, ld, x_ptr, ld, rows, seq, A, weight.data_ptr(), self.eps,
                cs.data_ptr() if cs is not None else None, sn.data_ptr() if sn is not None else None, trs, tes, Dh)
        self._add(name, "fam_rmsnorm_rope", args, "rmsnorm_rope")

    def _attention(self, name, q, q_rs, k, k_rs, v, v_rs, sq, sk, kv_batch_rows, mask=None, mask_strides=(0, 0, 0)):
        d = _capi.AttnDesc()
        A, Dh = self.A, self.Dh
        d.q, d.q_bs, d.q_rs, d.q_hs = q, sq * q_rs, q_rs, Dh
        d.k0, d.k0_bs, d.k0_rs, d.k0_hs = k, kv_batch_rows * k_rs, k_rs, Dh
        d.v0, d.v0_bs, d.v0_rs, d.v0_hs = v, kv_batch_rows * v_rs, v_rs, Dh
        d.o, d.o_bs, d.o_rs, d.o_hs = self.attn.data_ptr(), sq * A, A, Dh
        d.batch, d.heads, d.sq, d.sk0, d.sk1, d.head_dim = self.B, self.nh, sq, sk, 0, Dh
        d.scale = 1.0 / math.sqrt(Dh)
        d.num_splits = 1
        if mask is not None:   # bool, [b, q, k] strides (mask_bs, mask_qs) and no head stride
            d.mask, d.mask_kind = mask.data_ptr(), _capi.FAM_MASK_BOOL
            d.mask_bs, d.mask_hs, d.mask_qs = mask_strides
        self._descs.append(d)
        self._add(name, "fam_attention", (C.byref(d),), "attention", 4 * self.B * self.nh * sq * sk * Dh)

    def _build(self):
        w, H, A, S, Lc = self.w, self.H, self.A, self.S, self.Lc
        M = self.B * S
        rows = self.mods.shape[0]
        if not self.mods_ready:
            self._add("modulation", "fam_add_modulation",
                      (self.tmod_in.data_ptr(), w["mod"].data_ptr(), self.mods.data_ptr(), rows, 1, 6 * H),
                      "modulation")

        def mod(i, mods=None):  # chunk i of (modulation + t_mod), [rows, H] view with row stride 6H
            return (self.mods if mods is None else mods)[:, i * H:(i + 1) * H]

        gstr = (*self._mod_strides(), 1)
        # self-attention
        if not self.pre_normed:
            self._adaln("adaln1", self.x, self.h, shift=mod(0), scale=mod(1))
        qp = self.qkv.data_ptr()
        if self.splitk:
            # one split-K product for q|k|v; one row launch finishes it, q and k RMS-normalised
            # and rotated in their own workgroups, v with its bias (a q|k|v row tiles when the
            # head width A is 1024, 2048, 3072 or 4096, otherwise one launch per segment)
            sp = self._partial("qkv", self.h, w["qkv_w"])
            b = w["qkv_b"]
            if A % 1024 == 0 and A <= 4096:
                self._rowop("qkv_row", N=3 * A, splits=sp, bias=b, out=self.qkv, segs=[(0, w["nq"]), (A, w["nk"])],
                            seg_width=A, rope=True)
                if self.kv_only:
                    return
            else:
                self._rowop("k_row", N=A, splits=sp, bias=b[A:2 * A], out=self.qkv[:, A:2 * A], rms_w=w["nk"],
                            rope=True, col0=A, ldp=3 * A)
                self._rowop("v_row", N=A, splits=sp, bias=b[2 * A:], out=self.qkv[:, 2 * A:], col0=2 * A, ldp=3 * A)
                if self.kv_only:
                    return
                self._rowop("q_row", N=A, splits=sp, bias=b[:A], out=self.qkv[:, :A], rms_w=w["nq"], rope=True,
                            col0=0, ldp=3 * A)
        else:
            self._gemm("qkv", self.h, w["qkv_w"], w["qkv_b"], self.qkv)
            self._rms("k_norm_rope", qp + 2 * A, 3 * A, M, S, w["nk"], True)
            if self.kv_only:
                return
            self._rms("q_norm_rope", qp, 3 * A, M, S, w["nq"], True)
        self._attention("self_attn", qp, 3 * A, qp + 2 * A, 3 * A, qp + 4 * A, 3 * A, S, S, S,
                        mask=self.self_mask, mask_strides=(0, 0, S))
        # the o row also normalises for what follows: norm3 (LayerNorm) before the cross
        # attention, else the FFN's AdaLN
        if Lc > 0:
            self._proj("o", self.attn, w["o_w"], w["o_b"], self.x, res=self.x, gate=mod(2), gate_strides=gstr,
                       ln=(w["n3_w"], w["n3_b"]), nout=self.h)
        else:
            self._proj("o", self.attn, w["o_w"], w["o_b"], self.x, res=self.x, gate=mod(2), gate_strides=gstr,
                       adaln=(mod(3), mod(4)), nout=self.h)
        # cross-attention
        if Lc > 0:
            self._proj("cross_q", self.h, w["cq_w"], w["cq_b"], self.qc, rms_w=w["cnq"])
            if self.ctx_kv is None:
                self._gemm("cross_kv", self.ctx, w["ckv_w"], w["ckv_b"], self.ckv)
                kp, kld = self.ckv.data_ptr(), 2 * A
                self._rms("cross_k_norm", kp, kld, self.B * Lc, Lc, w["cnk"], False)
            else:
                buf, col = self.ctx_kv
                kp, kld = buf.data_ptr() + 2 * col, buf.stride(0)
            cms = (S * Lc, 0, Lc) if self.ctx_mask is None or self.ctx_mask.dim() == 3 else (Lc, 0, 0)
            self._attention("cross_attn", self.qc.data_ptr(), A, kp, kld, kp + 2 * A, kld, S, Lc, Lc,
                            mask=self.ctx_mask, mask_strides=cms)
            self._proj("cross_o", self.attn, w["co_w"], w["co_b"], self.x, res=self.x, adaln=(mod(3), mod(4)),
                       nout=self.h)
        # FFN (its AdaLN came with the last projection's row)
        self._proj("ffn_up", self.h, w["f0_w"], w["f0_b"], self.hid, act=_capi.FAM_ACT_GELU_TANH)
        if self.next_mod is not None:
            if not self.splitk:
                raise ValueError("next_mod needs the split-K projections (<= 128 rows, widths <= 4096)")
            nmods = self.next_mod
            if nmods.stride(0) != self.mods.stride(0):
                raise ValueError("next_mod must have the row stride of this block's mods")
            self._proj("ffn_down", self.hid, w["f2_w"], w["f2_b"], self.x, res=self.x, gate=mod(5), gate_strides=gstr,
                       adaln=(mod(0, nmods), mod(1, nmods)), nout=self.h)
        else:
            self._proj("ffn_down", self.hid, w["f2_w"], w["f2_b"], self.x, res=self.x, gate=mod(5),
                       gate_strides=gstr)

    # ------------------------------------------------------------------ execution
    def set_inputs(self, x: torch.Tensor, t_mod: torch.Tensor, context: torch.Tensor) -> None:
        """x [B, S, H]; t_mod [B, S, 6, H] (per token) or [B, 6, H]; context [B, Lc, H] (bf16)."""
        self.x.copy_(x.reshape(self.x.shape))
        self.tmod_in.copy_(t_mod.reshape(self.tmod_in.shape))
        self.ctx.copy_(context.reshape(self.ctx.shape))

    def run(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            s = torch.cuda.current_stream().cuda_stream
            for f in self.steps:
                f(s)

    def capture(self) -> None:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in self.steps:
                f(s.cuda_stream)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            st = torch.cuda.current_stream().cuda_stream
            for f in self.steps:
                f(st)
        self.graph = g

    def run_until(self, name: str) -> None:
        """Eager launches of this block up to and including its step `name`, to inspect the
        buffers in between: after "self_attn" / "cross_attn", `attn` [B*S, A] holds that
        attention's output before its o projection; after "o", `x` holds the residual stream
        after the self-attention branch."""
        names = [m["name"] for m in self.meta]
        if name not in names:
            raise ValueError(f"no step {name!r} in this block (steps: {names})")
        s = torch.cuda.current_stream().cuda_stream
        for f in self.steps[:names.index(name) + 1]:
            f(s)

    def forward(self, x: torch.Tensor, t_mod: torch.Tensor, context: torch.Tensor) -> torch.Tensor:
        """One block forward; returns a copy of the new x, [B, S, H]."""
        self.set_inputs(x, t_mod, context)
        self.run()
        return self.x.clone().view(self.B, self.S, self.H)

    def kv(self):
        """The block's attention K (normalised, rotated) and V as [B, S, A] views of `qkv`."""
        q3 = self.qkv.view(self.B, self.S, 3 * self.A)
        return q3[:, :, self.A:2 * self.A], q3[:, :, 2 * self.A:]


class FusedVideoPrefill:
    """MoT.prefill_video_cache (FB/mot.py:262-376) of the video expert for fixed (B, Sv, Lc):
    the video tokens through the expert's first `num_run` blocks (all when 0), keeping each
    block's attention K/V.  The blocks share the residual stream, t_mod, context and scratch
    buffers and run back to back (one graph with `capture()`); each keeps its own q/k/v buffer,
    whose k and v columns are the cache (`kv_cache()`, views valid until the next run).  The
    last block run builds only its K/V -- its output is not part of the cache -- and blocks
    past `num_run` reuse that block's K/V (video layer drafting, FB/mot.py:345-351).

    Args: as FusedVideoDiTBlock, plus num_layers (the expert's depth), video_mask bool [Sv, Sv]
    (None: every key), ctx_mask bool [B, Sv, Lc] or [B, Lc] (None: every context token), ctx_len
    0 for a prefill without a context payload.  keep_output: every block runs in full, so that
    after `run()` the shared "x" holds the last block's output (the block stack of
    WanVideoDiT.forward, FB/wan_video_dit.py:667-682) besides the K/V cache.
    """

    def __init__(self, params: Dict[str, torch.Tensor], *, num_layers: int, hidden: int, num_heads: int,
                 head_dim: int, ffn_dim: int, batch: int, video_len: int, ctx_len: int, freqs: torch.Tensor,
                 eps: float = 1e-6, per_token_mod: bool = True, video_mask: Optional[torch.Tensor] = None,
                 ctx_mask: Optional[torch.Tensor] = None, num_run: int = 0, device="cuda",
                 keep_output: bool = False, mod_group: int = 0):
        dev = torch.device(device)
        self.keep_output = keep_output
        self.L = num_layers
        self.n_run = num_layers if num_run <= 0 or num_run > num_layers else num_run
        self.B, self.S, self.Lc, self.H, self.A = batch, video_len, ctx_len, hidden, num_heads * head_dim
        M = batch * video_len
        z = lambda *s: torch.zeros(*s, dtype=_BF16, device=dev)  # noqa: E731
        g = mod_group if mod_group > 0 else (1 if per_token_mod else video_len)
        rows = M // g   # modulation rows: one per group of g tokens
        self.shared = {"x": z(M, hidden), "tmod_in": z(rows, 6 * hidden), "ctx": z(batch * ctx_len, hidden),
                       "mods": z(rows, 6 * hidden), "h": z(M, hidden), "attn": z(M, self.A), "qc": z(M, self.A),
                       "ckv": z(batch * ctx_len, 2 * self.A), "hid": z(M, ffn_dim)}
        self.lib = lib = _capi.load()
        if M <= 128:   # one split-K partial buffer for every block
            need = max(lib.fam_gemm_partial_splits(M, n_, k_) * M * n_
                       for n_, k_ in ((hidden, self.A), (self.A, hidden), (hidden, ffn_dim), (3 * self.A, hidden),
                                      (ffn_dim, hidden)))
            self.shared["part"] = torch.zeros(need, dtype=torch.float32, device=dev)
        else:          # one split-K workspace of the large-M products for every block
            need = max([lib.fam_gemm_ws_floats(M, n_, k_)
                        for n_, k_ in ((3 * self.A, hidden), (hidden, self.A), (self.A, hidden), (ffn_dim, hidden),
                                       (hidden, ffn_dim))] +
                       [lib.fam_gemm_ws_floats(batch * ctx_len, 2 * self.A, hidden), 0])
            if need > 0:
                self.shared["ws"] = torch.zeros(need, dtype=torch.float32, device=dev)
        # the context K/V of every block that cross-attends, in one GEMM per call: the context
        # does not change between blocks, only the weights do
        # (without keep_output the last block run builds only its K/V)
        ncross = (self.n_run if keep_output else self.n_run - 1) if ctx_len > 0 else 0
        self.steps, self.meta, self._descs = [], [], []
        if ncross > 0:
            def cat(names):
                return torch.cat([params[f"blocks.{i}.cross_attn.{n}"].to(device=dev, dtype=torch.float32)
                                  for i in range(ncross) for n in names], 0).to(_BF16).contiguous()
            self.ckv_w = cat(["k.weight", "v.weight"])
            self.ckv_b = cat(["k.bias", "v.bias"])
            self.ctxkv = z(batch * ctx_len, ncross * 2 * self.A)
            self.cnk = [params[f"blocks.{i}.cross_attn.norm_k.weight"].to(device=dev, dtype=_BF16).contiguous()
                        for i in range(ncross)]
            self._ctx_launches(batch * ctx_len, ctx_len, head_dim, eps)
        # the modulation + t_mod of every block comes from one launch into a [rows, blocks, 6H]
        # buffer (up to 256 MB of it; per block otherwise), and at <= 128 rows each block's
        # FFN-down row also applies the next block's AdaLN1
        chain = M <= 128 and hidden <= 4096 and self.A <= 4096     # the blocks' split-K condition
        one_mod = chain or rows * self.n_run * 6 * hidden * 2 <= (256 << 20)
        if one_mod:
            self.mod_table = torch.stack([params[f"blocks.{i}.modulation"].reshape(6 * hidden)
                                          for i in range(self.n_run)]).to(device=dev, dtype=_BF16).contiguous()
            self.mods_all = z(rows, self.n_run, 6 * hidden)
            self._add_step("modulation_all", "fam_add_modulation",
                           (self.shared["tmod_in"].data_ptr(), self.mod_table.data_ptr(), self.mods_all.data_ptr(),
                            rows, self.n_run, 6 * hidden), "modulation")

        def mods(i):
            return self.mods_all[:, i, :] if one_mod else self.shared["mods"]

        self.blocks = [FusedVideoDiTBlock(params, i, hidden=hidden, num_heads=num_heads, head_dim=head_dim,
                                          ffn_dim=ffn_dim, batch=batch, seq_len=video_len, ctx_len=ctx_len,
                                          freqs=freqs, eps=eps, per_token_mod=per_token_mod, mod_group=g,
                                          device=dev,
                                          self_mask=video_mask, ctx_mask=ctx_mask,
                                          shared={**self.shared, "mods": mods(i)},
                                          kv_only=(i == self.n_run - 1 and not keep_output),
                                          ctx_kv=(self.ctxkv, i * 2 * self.A) if i < ncross else None,
                                          mods_ready=one_mod, pre_normed=chain and i > 0,
                                          next_mod=mods(i + 1) if chain and i + 1 < self.n_run else None)
                       for i in range(self.n_run)]
        self.steps += [f for b in self.blocks for f in b.steps]
        self.meta += [m for b in self.blocks for m in b.meta]
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    def _add_step(self, name, fname, args, kind):
        f = getattr(self.lib, fname)
        lib = self.lib

        def run(stream):
            rc = f(*args, stream)
            if rc != 0:
                raise _capi.FamError(f"{fname}[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.steps.append(run)
        self.meta.append({"name": name, "kernel": kind})

    def _ctx_launches(self, rows, seq, head_dim, eps):
        """ctxkv = ctx [k|v weights of every block]^T + bias, then each block's K RMSNorm."""
        lib, A = self.lib, self.A
        d = _capi.GemmDesc()
        ctx = self.shared["ctx"]
        d.a, d.lda, d.w, d.ldw = ctx.data_ptr(), ctx.stride(0), self.ckv_w.data_ptr(), self.ckv_w.stride(0)
        d.bias = self.ckv_b.data_ptr()
        d.out, d.ldo = self.ctxkv.data_ptr(), self.ctxkv.stride(0)
        d.M, d.N, d.K = rows, self.ckv_w.shape[0], ctx.shape[1]
        d.rows_per_batch = rows
        self._descs.append(d)

        add = self._add_step
        N, K = self.ckv_w.shape[0], ctx.shape[1]
        sp = lib.fam_gemm_partial_splits(rows, N, K) if 64 < rows <= 144 else 0
        if sp > 1:
            # up to 144 context rows: the streaming split-K kernel reads the 1 GB of stacked
            # weights once; the large-M GEMM's 256-row tiles would double the products of 129 rows
            self.ctx_part = torch.empty(sp * rows * N, dtype=torch.float32, device=ctx.device)
            add("ctx_kv_all", "fam_gemm_partial", (ctx.data_ptr(), ctx.stride(0), self.ckv_w.data_ptr(),
                                                    self.ckv_w.stride(0), self.ctx_part.data_ptr(), rows, N, K),
                "gemm_partial")
            r = _capi.RowopDesc()
            r.src, r.partials, r.splits, r.split_stride = _capi.FAM_ROWSRC_PARTIALS, self.ctx_part.data_ptr(), sp, rows * N
            r.M, r.N, r.bias, r.rows_per_batch = rows, N, self.ckv_b.data_ptr(), rows
            r.out, r.ldo = self.ctxkv.data_ptr(), self.ctxkv.stride(0)
            self._descs.append(r)
            add("ctx_kv_all_row", "fam_rowop", (C.byref(r),), "rowop")
        else:
            # (one split: fam_gemm runs the same streaming kernel and stores the bf16 rows with
            # their bias itself, no fp32 plane and no row launch)
            add("ctx_kv_all", "fam_gemm", (C.byref(d),), "gemm")
        # every block's context keys in one launch: rows (context row, block) with the block's
        # k columns 2A apart, normalised with that block's norm_k weight
        nb = len(self.cnk)
        self.cnk_all = torch.stack(self.cnk).contiguous()
        p = self.ctxkv.data_ptr()
        add("cross_k_norm_all", "fam_rmsnorm_grouped",
            (p, 2 * A, p, 2 * A, rows * nb, A, self.cnk_all.data_ptr(), nb, float(eps)), "rmsnorm_rope")

    @property
    def num_launches(self) -> int:
        return len(self.steps)

    def set_inputs(self, x: torch.Tensor, t_mod: torch.Tensor, context: Optional[torch.Tensor]) -> None:
        """x [B, Sv, H]; t_mod [B, Sv, 6, H] (per token) or [B, 6, H]; context [B, Lc, H] (bf16)."""
        sh = self.shared
        sh["x"].copy_(x.reshape(sh["x"].shape))
        sh["tmod_in"].copy_(t_mod.reshape(sh["tmod_in"].shape))
        if self.Lc > 0:
            sh["ctx"].copy_(context.reshape(sh["ctx"].shape))

    def run(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            s = torch.cuda.current_stream().cuda_stream
            for f in self.steps:
                f(s)

    def capture(self) -> None:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in self.steps:
                f(s.cuda_stream)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            st = torch.cuda.current_stream().cuda_stream
            for f in self.steps:
                f(st)
        self.graph = g

    def kv_cache(self):
        """[(k, v)] for every one of the expert's num_layers blocks, [B, Sv, A] views."""
        kv = [b.kv() for b in self.blocks]
        return kv + [kv[-1]] * (self.L - self.n_run)

    def prefill(self, x: torch.Tensor, t_mod: torch.Tensor, context: Optional[torch.Tensor]):
        self.set_inputs(x, t_mod, context)
        self.run()
        return self.kv_cache()


@dataclass
class WanVideoConfig:
    """WanVideoDiT's hyper-parameters (FB/wan_video_dit.py:329-411) as FusedWanVideoDiT reads
    them; the defaults are the Wan2.2-TI2V-5B video expert of FastWAM (configs 2 and the
    prefill).  The config-4 backbone is WanVideoConfig(hidden_dim=2048, in_dim=16, ffn_dim=8192,
    out_dim=16, text_dim=1024, num_heads=16, num_layers=28)."""
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


class FusedWanVideoDiT:
    """WanVideoDiT (FB/wan_video_dit.py:328-684) of the video expert on the library for a fixed
    call shape: latents [B, in_dim, F, Hl, Wl], one timestep per sample, Lc context tokens.

    pre_dit (:527-648, seperated_timestep with the VAE embedding fused in the latents):
        patches = patch gather of the latents                      fam_patchify
        tokens  = patches conv_w^T + conv_b                        fam_gemm
        t, t_mod of the two distinct token timesteps per sample (the first latent frame at 0,
            the others at the sample's timestep): sinusoid -> Linear, SiLU, Linear -> SiLU,
            Linear, each row computed once      fam_sinusoid, fam_gemm (SiLU epilogues)
        per-token t_mod (and t for the head) by row gather       fam_gather_rows
        context = Linear(GELU(Linear(text)))                      fam_gemm (GELU epilogue)
    blocks: the chain of FusedVideoPrefill (keep_output with mode "forward"), reading the
        tokens, the per-token t_mod and the embedded context in place; the context mask [B, Lc]
        is broadcast over the tokens inside the attention.
    post_dit (mode "forward", :650-654, Head :309-325):
        shift, scale = head.modulation + t (per token)           fam_add_modulation
        y = Linear(LN(x) (1 + scale) + shift)                     fam_adaln, fam_gemm
        out = unpatchify(y)                                       fam_unpatchify

    mode "prefill" stops after the blocks and exposes their K/V (`kv_cache()`): the video half of
    FastWAM.infer_action (FB/fastwam.py:1018-1041), whose first latent frame runs at t = 0.
    mode "features" runs every block in full and stops before the head: `features()` is the last
    block's output, the backbone.hidden_states[-1] a DiT4DiT head consumes
    (DB/framework/DiT4DiT.py:205-222).
    video_mask: bool [S, S] on the self-attention (None: every key).
    """

    def __init__(self, cfg: WanVideoConfig, params: Dict[str, torch.Tensor], *, batch: int, frames: int, height: int,
                 width: int, ctx_len: int, video_mask: Optional[torch.Tensor] = None, mode: str = "forward",
                 device="cuda"):
        if mode not in ("forward", "prefill", "features"):
            raise ValueError(f"mode must be 'forward', 'prefill' or 'features', got {mode!r}")
        dev = torch.device(device)
        self.mode, self.cfg, self.device = mode, cfg, dev
        pt, ph, pw = cfg.patch_size
        if frames % pt or height % ph or width % pw:
            raise ValueError(f"latent shape ({frames}, {height}, {width}) not divisible by the patch {cfg.patch_size}")
        f, h, w = frames // pt, height // ph, width // pw
        self.grid, self.tpf = (f, h, w), h * w
        B, H, C, Lc = batch, cfg.hidden_dim, cfg.in_dim, ctx_len
        S = f * h * w
        P = pt * ph * pw
        self.B, self.S, self.Lc = B, S, Lc
        self.lib = lib = _capi.load()
        z = lambda *s: torch.zeros(*s, dtype=_BF16, device=dev)  # noqa: E731

        def Pm(n):
            if n not in params:
                raise KeyError(f"missing parameter {n}")
            return params[n].to(device=dev, dtype=_BF16).contiguous()
        self.w = w_ = {
            "patch_w": Pm("patch_embedding.weight").reshape(H, C * P).contiguous(), "patch_b": Pm("patch_embedding.bias"),
            "te0_w": Pm("time_embedding.0.weight"), "te0_b": Pm("time_embedding.0.bias"),
            "te2_w": Pm("time_embedding.2.weight"), "te2_b": Pm("time_embedding.2.bias"),
            "tp_w": Pm("time_projection.1.weight"), "tp_b": Pm("time_projection.1.bias"),
            "txt0_w": Pm("text_embedding.0.weight"), "txt0_b": Pm("text_embedding.0.bias"),
            "txt2_w": Pm("text_embedding.2.weight"), "txt2_b": Pm("text_embedding.2.bias"),
        }
        if mode == "forward":
            w_["head_w"], w_["head_b"] = Pm("head.head.weight"), Pm("head.head.bias")
            w_["head_mod"] = Pm("head.modulation").reshape(2, H).contiguous()

        # inputs (static, for graph replay)
        self.x_in = z(B, C, frames, height, width)
        self.ts_in = z(B)
        self.ts2 = z(2 * B)                       # (0, t_b) per sample: the distinct token timesteps
        self.ctx_in = z(B * Lc, cfg.text_dim)
        self.cmask = torch.ones(B, Lc, dtype=torch.bool, device=dev)
        # the timestep, hence t and t_mod, is one per latent frame: the modulation tables hold a
        # row per (sample, frame) -- gathered from the two distinct rows, frame 0 -> 2b, later
        # frames -> 2b + 1 -- and every consumer reads row (token / tokens per frame)
        self.nf = f
        fr = torch.arange(f)
        idx = (2 * torch.arange(B)[:, None] + (fr[None, :] > 0).long()).reshape(-1)
        self.row_idx = idx.to(device=dev, dtype=torch.int32).contiguous()

        freqs = video_freqs_3d(cfg.attn_head_dim, f, h, w)
        self.freqs = freqs
        self.blocks = FusedVideoPrefill(params, num_layers=cfg.num_layers, hidden=H, num_heads=cfg.num_heads,
                                        head_dim=cfg.attn_head_dim, ffn_dim=cfg.ffn_dim, batch=B, video_len=S,
                                        ctx_len=Lc, freqs=freqs, eps=cfg.eps, video_mask=video_mask,
                                        ctx_mask=self.cmask if Lc > 0 else None, device=dev,
                                        keep_output=(mode != "prefill"), mod_group=self.tpf)
        sh = self.blocks.shared
        self.patches = z(B * S, C * P)
        self.emb = z(2 * B, cfg.freq_dim)
        self.t1 = z(2 * B, H)
        self.t2s = z(2 * B, H)                    # SiLU(t) of the distinct rows
        self.tmod2 = z(2 * B, 6 * H)
        self.ctx_h = z(B * Lc, H)
        self.steps: List = []
        self.meta: List[dict] = []
        self._descs: List = []
        add = self._add
        add("patchify", "fam_patchify", (self.x_in.data_ptr(), B, C, frames, height, width, pt, ph, pw,
                                         self.patches.data_ptr()), "patchify", 4 * self.x_in.numel())
        self._gemm("patch_embed", self.patches, w_["patch_w"], w_["patch_b"], sh["x"])
        add("sinusoid", "fam_sinusoid", (self.ts2.data_ptr(), self.emb.data_ptr(), 2 * B, cfg.freq_dim), "sinusoid")
        self._gemm("time_emb0", self.emb, w_["te0_w"], w_["te0_b"], self.t1, act=_capi.FAM_ACT_SILU)
        self._gemm("time_emb2_silu", self.t1, w_["te2_w"], w_["te2_b"], self.t2s, act=_capi.FAM_ACT_SILU)
        self._gemm("time_proj", self.t2s, w_["tp_w"], w_["tp_b"], self.tmod2)
        add("tmod_frames", "fam_gather_rows", (self.tmod2.data_ptr(), 6 * H, 2 * B, self.row_idx.data_ptr(),
                                               sh["tmod_in"].data_ptr(), 6 * H, B * f, 6 * H), "gather")
        if mode == "forward":
            self.t2 = z(2 * B, H)
            self.t_frm = z(B * f, H)
            self._gemm("time_emb2", self.t1, w_["te2_w"], w_["te2_b"], self.t2)
            add("t_frames", "fam_gather_rows", (self.t2.data_ptr(), H, 2 * B, self.row_idx.data_ptr(),
                                                self.t_frm.data_ptr(), H, B * f, H), "gather")
        if Lc > 0:
            self._gemm("text_emb0", self.ctx_in, w_["txt0_w"], w_["txt0_b"], self.ctx_h, act=_capi.FAM_ACT_GELU_TANH)
            self._gemm("text_emb2", self.ctx_h, w_["txt2_w"], w_["txt2_b"], sh["ctx"])
        self.steps += self.blocks.steps
        self.meta += self.blocks.meta
        if mode == "forward":
            self.head_mod = z(B * f, 2, H)
            self.hn = z(B * S, H)
            self.head_out = z(B * S, cfg.out_dim * P)
            self.out = z(B, cfg.out_dim, frames, height, width)
            add("head_modulation", "fam_add_modulation", (self.t_frm.data_ptr(), w_["head_mod"].data_ptr(),
                                                          self.head_mod.data_ptr(), B * f, 2, H), "modulation")
            hm = self.head_mod.data_ptr()
            add("head_adaln", "fam_adaln", (sh["x"].data_ptr(), H, hm, hm + 2 * H, 2 * H, 0, None, None,
                                            self.hn.data_ptr(), H, B * S, self.tpf, H, float(cfg.eps)), "adaln")
            self._gemm("head", self.hn, w_["head_w"], w_["head_b"], self.head_out)
            add("unpatchify", "fam_unpatchify", (self.head_out.data_ptr(), B, cfg.out_dim, f, h, w, pt, ph, pw,
                                                 self.out.data_ptr()), "patchify", 4 * self.out.numel())
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ plan building
    def _add(self, name, fname, args, kind, nbytes=0):
        f, lib = getattr(self.lib, fname), self.lib

        def run(stream):
            rc = f(*args, stream)
            if rc != 0:
                raise _capi.FamError(f"{fname}[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.steps.append(run)
        self.meta.append({"name": name, "kernel": kind, "bytes": int(nbytes)})

    def _gemm(self, name, a, w, bias, out, act=_capi.FAM_ACT_NONE):
        d = _capi.GemmDesc()
        d.a, d.lda, d.w, d.ldw = a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0)
        d.bias = bias.data_ptr() if bias is not None else None
        d.out, d.ldo = out.data_ptr(), out.stride(0)
        d.M, d.N, d.K = a.shape[0], w.shape[0], w.shape[1]
        d.act = act
        d.rows_per_batch = max(a.shape[0], 1)
        self._descs.append(d)
        self._add(name, "fam_gemm", (C.byref(d),), "gemm", 2 * (a.numel() + w.numel() + out.numel()))

    # ------------------------------------------------------------------ execution
    def set_inputs(self, latents: torch.Tensor, timestep: torch.Tensor, context: Optional[torch.Tensor] = None,
                   context_mask: Optional[torch.Tensor] = None) -> None:
        """latents [B, in_dim, F, Hl, Wl]; timestep [B] or [1]; context [B, Lc, text_dim];
        context_mask bool [B, Lc] (None: every token), all copied into the static buffers."""
        self.x_in.copy_(latents.reshape(self.x_in.shape))
        t = timestep.reshape(-1).to(device=self.device, dtype=_BF16)
        self.ts_in.copy_(t.expand(self.B) if t.numel() == 1 else t)
        ts2 = self.ts2.view(self.B, 2)
        ts2[:, 0].zero_()
        ts2[:, 1].copy_(self.ts_in if self.grid[0] > 1 else torch.zeros_like(self.ts_in))
        if self.Lc > 0:
            self.ctx_in.copy_(context.reshape(self.ctx_in.shape))
            if context_mask is None:
                self.cmask.fill_(True)
            else:
                self.cmask.copy_(context_mask.reshape(self.cmask.shape))

    def run(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            s = torch.cuda.current_stream(self.device).cuda_stream
            for f in self.steps:
                f(s)

    def capture(self) -> None:
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for f in self.steps:
                f(s.cuda_stream)
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            st = torch.cuda.current_stream(self.device).cuda_stream
            for f in self.steps:
                f(st)
        self.graph = g

    def forward(self, latents, timestep, context=None, context_mask=None) -> torch.Tensor:
        """WanVideoDiT.forward: the predicted latents [B, out_dim, F, Hl, Wl] (a copy)."""
        if self.mode != "forward":
            raise RuntimeError("forward() needs mode='forward'")
        self.set_inputs(latents, timestep, context, context_mask)
        self.run()
        return self.out.clone()

    def run_until(self, name: str, block: int) -> None:
        """Eager launches from pre_dit up to and including step `name` of block `block` (inputs
        from `set_inputs`), to inspect the shared buffers there: after "self_attn" /
        "cross_attn" the stack's "attn" holds that block's attention output before its o
        projection (see FusedVideoDiTBlock.run_until)."""
        blk = self.blocks.blocks[block]
        names = [m["name"] for m in blk.meta]
        if name not in names:
            raise ValueError(f"no step {name!r} in block {block} (steps: {names})")
        target = blk.steps[names.index(name)]
        end = next(i for i, f in enumerate(self.steps) if f is target)
        s = torch.cuda.current_stream(self.device).cuda_stream
        for f in self.steps[:end + 1]:
            f(s)

    def prefill(self, latents, timestep, context=None, context_mask=None):
        """pre_dit + every block's K/V: [(k, v)] per layer, [B, S, A] views valid until the next run."""
        self.set_inputs(latents, timestep, context, context_mask)
        self.run()
        return self.kv_cache()

    def kv_cache(self):
        return self.blocks.kv_cache()

    def features(self) -> torch.Tensor:
        """The last block's output [B, S, H] (a view of the residual stream, valid until the next
        run); modes "forward" and "features"."""
        if self.mode == "prefill":
            raise RuntimeError("the prefill mode does not run its last block in full")
        return self.blocks.shared["x"].view(self.B, self.S, self.cfg.hidden_dim)

    def pre_state(self):
        """The pre_dit outputs in the reference's layout (FB/wan_video_dit.py:642-648): tokens
        [B, S, H] (before the blocks ran), t_mod [B, S, 6, H], context [B, Lc, H], freqs."""
        sh = self.blocks.shared
        H = self.cfg.hidden_dim
        # per-token views of the per-frame tables (host-side expansion, for inspection)
        tm = sh["tmod_in"].view(self.B, self.nf, 6, H).repeat_interleave(self.tpf, dim=1)
        t = self.t_frm.view(self.B, self.nf, H).repeat_interleave(self.tpf, dim=1) if self.mode == "forward" else None
        return {"tokens": sh["x"].view(self.B, self.S, H), "t_mod": tm,
                "context": sh["ctx"].view(self.B, self.Lc, H), "freqs": self.freqs, "t": t}

    @property
    def num_launches(self) -> int:
        return len(self.steps)

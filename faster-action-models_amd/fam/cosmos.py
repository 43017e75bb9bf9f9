"""The Cosmos-Predict2.5 backbone of DiT4DiT on the gfx950 kernels.

DiT4DiT reads the output of one block of diffusers' CosmosTransformer3DModel (the hook on
`transformer_blocks[extract_layer]`, DB = src/dit4dit-baseline/DiT4DiT/model,
DB/modules/vlm/Cosmos25.py:150-160; the reference's GEAK patch stops the forward there,
CP = src/dit4dit-geak/patches/diffusers-3996788-transformer_cosmos-geak.patch:2289-2490).
This module runs that forward for a fixed call shape as one chain of library launches:

per call (the timestep is one per latent frame: R = B * frames modulation rows)
    patches = patch gather of the latents                    fam_patchify
    x       = patches Wp^T                                   fam_gemm
    tp      = cat(cos(t f), sin(t f))                        fam_sinusoid
    temb    = Linear2(SiLU(Linear1(tp)))        [R, 3C]      fam_gemm (SiLU epilogue), fam_gemm
    e       = SiLU(RMSNorm(tp))                 [R, C]       fam_rmsnorm_rope, fam_act_rows
    hl      = e W1all^T (every AdaLN unit's LoRA down)       fam_gemm
    mods    = hl_u W2_u^T + temb per unit (shift|scale|gate) fam_gemm (residual epilogue), 3 L launches
    ctxkv   = ctx [Wk2; Wv2 of every block]^T; per-head RMSNorm of every block's keys
                                                             fam_gemm, fam_headnorm_rope
per block (CosmosTransformerBlock.forward, CP:1851-1879), three gated AdaLN-Zero sub-blocks:
    h   = LN(x) (1 + scale1) + shift1                        fam_adaln (per-frame rows)
    qkv = h Wqkv^T;  q, k = RoPE(RMSNorm_head(q | k))        fam_gemm, fam_headnorm_rope
    x  += gate1 * (attn(q, k, v) Wo^T)                        fam_attention, fam_gemm epilogue
    h   = LN(x) (1 + scale2) + shift2                        fam_adaln
    qc  = RMSNorm_head(h Wq2^T)                               fam_gemm, fam_headnorm_rope
    x  += gate2 * (attn(qc, ctx k, ctx v) Wo2^T)              fam_attention (text key mask), fam_gemm
    h   = LN(x) (1 + scale3) + shift3                        fam_adaln
    x  += gate3 * (GELU_erf(h W1^T) W2^T)                     fam_gemm (exact-GELU epilogue), fam_gemm

No projection has a bias.  The 3-D RoPE tables are computed once on the host in fp32, as
diffusers' CosmosRotaryPosEmbed does (CP:1953-1976).  Parameters take diffusers' state-dict
keys (`transformer_blocks.{i}.attn1.to_q.weight`, ...).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _capi
from .video_dit import FusedVideoDiTBlock

_BF16 = torch.bfloat16


@dataclass
class CosmosConfig:
    """CosmosTransformer3DModel's hyper-parameters as this module reads them; the defaults are
    the Cosmos-Predict2.5-2B shape of config 4 (hidden 2048 = 16 x 128 heads, 28 blocks, MLP
    ratio 4, AdaLN-LoRA rank 256, patch (1, 2, 2), text features 1024 wide).  in_channels counts
    the latent channels plus the condition and padding masks the model concatenates."""
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


def cosmos_rope_tables(cfg: CosmosConfig, t: int, h: int, w: int, fps: Optional[float] = None,
                       device="cuda") -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos / sin [t h w, head_dim] of CosmosRotaryPosEmbed.forward (CP:1953-1976): the head
    dims split (t, h, w) as D - 2 (D // 6 * 2), D // 6 * 2, D // 6 * 2; axis a rotates by
    pos * theta_a^(-2j / dim_a) with the NTK-scaled theta_a = 10000 rope_scale[a]^(dim_a /
    (dim_a - 2)); temporal positions scale by base_fps / fps when fps is given; the per-token
    angles are cat([t, h, w] * 2), so the two halves of a head share them."""
    D = cfg.head_dim
    dh = dw = D // 6 * 2
    dt = D - dh - dw
    rs = cfg.rope_scale

    def inv(dim, scale):
        theta = 10000.0 * scale ** (dim / (dim - 2))
        return 1.0 / theta ** (torch.arange(0, dim, 2, dtype=torch.float32)[: dim // 2] / dim)

    seq = torch.arange(max(t, h, w), dtype=torch.float32)
    tpos = seq[:t] if fps is None else seq[:t] / fps * cfg.base_fps
    et = torch.outer(tpos, inv(dt, rs[0]))[:, None, None, :].expand(t, h, w, dt // 2)
    eh = torch.outer(seq[:h], inv(dh, rs[1]))[None, :, None, :].expand(t, h, w, dh // 2)
    ew = torch.outer(seq[:w], inv(dw, rs[2]))[None, None, :, :].expand(t, h, w, dw // 2)
    f = torch.cat([et, eh, ew] * 2, dim=-1).reshape(t * h * w, D).float()
    return torch.cos(f).to(device).contiguous(), torch.sin(f).to(device).contiguous()


def param_shapes(cfg: CosmosConfig) -> Dict[str, Tuple[int, ...]]:
    """diffusers state-dict keys and shapes of what the features path reads: patch_embed.proj,
    time_embed (t_embedder.linear_1 / linear_2, norm), and per block norm{1,2,3}.linear_{1,2}
    (AdaLN-LoRA), attn1 / attn2 to_q / to_k / to_v / to_out.0 with norm_q / norm_k, ff.net.0.proj /
    ff.net.2.  No biases."""
    C, A, D, L = cfg.hidden, cfg.attn_dim, cfg.head_dim, cfg.adaln_lora_dim
    pt, ph, pw = cfg.patch_size
    s = {"patch_embed.proj.weight": (C, cfg.in_channels * pt * ph * pw),
         "time_embed.t_embedder.linear_1.weight": (C, C), "time_embed.t_embedder.linear_2.weight": (3 * C, C),
         "time_embed.norm.weight": (C,)}
    for i in range(cfg.num_layers):
        b = f"transformer_blocks.{i}."
        for n in ("norm1", "norm2", "norm3"):
            s[b + n + ".linear_1.weight"], s[b + n + ".linear_2.weight"] = (L, C), (3 * C, L)
        for a, kv_in in (("attn1", C), ("attn2", cfg.text_dim)):
            s.update({b + a + ".to_q.weight": (A, C), b + a + ".to_k.weight": (A, kv_in),
                      b + a + ".to_v.weight": (A, kv_in), b + a + ".to_out.0.weight": (C, A),
                      b + a + ".norm_q.weight": (D,), b + a + ".norm_k.weight": (D,)})
        s[b + "ff.net.0.proj.weight"] = (cfg.mlp_ratio * C, C)
        s[b + "ff.net.2.weight"] = (C, cfg.mlp_ratio * C)
    return s


def synthetic_params(cfg: CosmosConfig, seed: int, device="cuda", std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Seeded synthetic bf16 weights drawn on `device`: N(0, std), the RMSNorm weights N(1, 0.2)."""
    g = torch.Generator(device=device).manual_seed(seed)
    out = {}
    for k, shape in sorted(param_shapes(cfg).items()):
        t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
        norm = k.endswith("norm_q.weight") or k.endswith("norm_k.weight") or k == "time_embed.norm.weight"
        out[k] = (1.0 + 0.2 * t if norm else t * std).to(_BF16)
    return out


def _gemm_desc(a, w, out, bias=None, act=_capi.FAM_ACT_NONE, res=None, rows_per_batch=0):
    d = _capi.GemmDesc()
    d.a, d.lda, d.w, d.ldw = a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0)
    d.bias = bias.data_ptr() if bias is not None else None
    d.out, d.ldo = out.data_ptr(), out.stride(0)
    d.M, d.N, d.K = a.shape[0], w.shape[0], w.shape[1]
    d.act = act
    if res is not None:
        d.res, d.ldr = res.data_ptr(), res.stride(0)
    d.rows_per_batch = rows_per_batch or max(a.shape[0], 1)
    return d


class FusedCosmosBlock(FusedVideoDiTBlock):
    """One CosmosTransformerBlock (`transformer_blocks.{idx}.`) for fixed (B, S, Lc), chained in
    place on the stack's shared buffers (x, h, qc, attn, hid, ws).  Its launches reuse the video
    block's GEMM / AdaLN / attention plans; `mods` is this block's [R, 9C] row-strided view of
    the stack's modulation table (units 1, 2, 3 x (shift, scale, gate)); `ctx_kv` is
    (buffer [B Lc, W], column of this block's [k | v]) with k already normalised."""

    def __init__(self, params: Dict[str, torch.Tensor], idx: int, cfg: CosmosConfig, *, batch: int, seq_len: int,
                 ctx_len: int, rope: Tuple[torch.Tensor, torch.Tensor], mod_group: int,
                 shared: Dict[str, torch.Tensor], mods: torch.Tensor, ctx_kv: Optional[tuple],
                 ctx_mask: Optional[torch.Tensor], device):
        dev = torch.device(device)
        self.lib = _capi.load()
        self.cfg = cfg
        self.B, self.S, self.Lc = batch, seq_len, ctx_len
        self.H, self.nh, self.Dh, self.F = cfg.hidden, cfg.num_heads, cfg.head_dim, cfg.mlp_ratio * cfg.hidden
        self.A = A = cfg.attn_dim
        self.eps = float(cfg.eps)
        self.mod_group = mod_group
        self.splitk = False
        self.kv_only, self.mods_ready, self.pre_normed, self.next_mod = False, True, False, None
        pre = f"transformer_blocks.{idx}."

        def P(n):
            return params[pre + n].to(device=dev, dtype=_BF16).contiguous()

        def cat(ns):
            return torch.cat([params[pre + n].float() for n in ns], 0).to(device=dev, dtype=_BF16).contiguous()

        self.w = {
            "qkv_w": cat([f"attn1.to_{n}.weight" for n in "qkv"]), "o_w": P("attn1.to_out.0.weight"),
            "qk_norm": cat(["attn1.norm_q.weight", "attn1.norm_k.weight"]),
            "cq_w": P("attn2.to_q.weight"), "cq_norm": P("attn2.norm_q.weight"), "co_w": P("attn2.to_out.0.weight"),
            "f0_w": P("ff.net.0.proj.weight"), "f2_w": P("ff.net.2.weight"),
        }
        self.rope_cs = rope
        M = batch * seq_len
        sh = shared
        self.x, self.h, self.attn, self.qc, self.hid = sh["x"], sh["h"], sh["attn"], sh["qc"], sh["hid"]
        self.mods = mods
        self.qkv = torch.zeros(M, 3 * A, dtype=_BF16, device=dev)
        self.ws = sh.get("ws")
        self.ctx_kv = ctx_kv
        self.ctx_mask = ctx_mask
        self.self_mask = None
        self._descs: List = []
        self.steps: List = []
        self.meta: List[dict] = []
        self._build()
        self.graph = None

    def _headnorm(self, name, buf, nseg, weight, rope):
        """Per-head RMSNorm (+ rotate-half RoPE) of nseg A-wide segments of buf's rows, in place."""
        A, Dh = self.A, self.Dh
        cs, sn = self.rope_cs if rope else (None, None)
        args = (buf.data_ptr(), buf.stride(0), buf.data_ptr(), buf.stride(0), buf.shape[0], self.S, nseg, A, A, Dh,
                weight.data_ptr(), Dh, self.eps, cs.data_ptr() if rope else None, sn.data_ptr() if rope else None,
                Dh if rope else 0)
        self._add(name, "fam_headnorm_rope", args, "headnorm_rope")

    def _build(self):
        w, H, A, S, Lc = self.w, self.H, self.A, self.S, self.Lc
        mods = self.mods

        def m(unit, j):   # shift (0), scale (1), gate (2) of AdaLN unit 0..2, [R, H] views
            c0 = (3 * unit + j) * H
            return mods[:, c0:c0 + H]

        gstr = (*self._mod_strides(), 1)
        qp = self.qkv.data_ptr()
        # 1. self attention
        self._adaln("adaln1", self.x, self.h, shift=m(0, 0), scale=m(0, 1))
        self._gemm("qkv", self.h, w["qkv_w"], None, self.qkv)
        self._headnorm("qk_norm_rope", self.qkv, 2, w["qk_norm"], True)
        self._attention("self_attn", qp, 3 * A, qp + 2 * A, 3 * A, qp + 4 * A, 3 * A, S, S, S)
        self._gemm("o", self.attn, w["o_w"], None, self.x, res=self.x, gate=m(0, 2), gate_strides=gstr)
        # 2. cross attention (keys / values of every block come from the stack's one projection)
        self._adaln("adaln2", self.x, self.h, shift=m(1, 0), scale=m(1, 1))
        self._gemm("cross_q", self.h, w["cq_w"], None, self.qc)
        self._headnorm("cross_q_norm", self.qc, 1, w["cq_norm"], False)
        buf, col = self.ctx_kv
        kp, kld = buf.data_ptr() + 2 * col, buf.stride(0)
        cms = (Lc, 0, 0)
        self._attention("cross_attn", self.qc.data_ptr(), A, kp, kld, kp + 2 * A, kld, S, Lc, Lc,
                        mask=self.ctx_mask, mask_strides=cms)
        self._gemm("cross_o", self.attn, w["co_w"], None, self.x, res=self.x, gate=m(1, 2), gate_strides=gstr)
        # 3. feed forward (exact GELU)
        self._adaln("adaln3", self.x, self.h, shift=m(2, 0), scale=m(2, 1))
        self._gemm("ffn_up", self.h, w["f0_w"], None, self.hid, act=_capi.FAM_ACT_GELU_ERF)
        self._gemm("ffn_down", self.hid, w["f2_w"], None, self.x, res=self.x, gate=m(2, 2), gate_strides=gstr)

    def set_inputs(self, *a, **k):
        raise RuntimeError("a Cosmos block runs inside FusedCosmosBackbone; set the backbone's inputs")


class FusedCosmosBackbone:
    """CosmosTransformer3DModel.forward up to the output of block `stop_layer` (every block when
    None) for a fixed call shape: latents [B, in_channels, T, Hl, Wl], one timestep per sample or
    per latent frame, Lc text tokens of width text_dim with an optional [B, Lc] key mask.
    `features()` is that block's output [B, S, hidden] -- what DiT4DiT's head reads
    (DB/framework/DiT4DiT.py:205-222).  run() / capture() as the other fused models."""

    def __init__(self, cfg: CosmosConfig, params: Dict[str, torch.Tensor], *, batch: int, frames: int, height: int,
                 width: int, ctx_len: int, stop_layer: Optional[int] = None, fps: Optional[float] = None,
                 device="cuda"):
        dev = torch.device(device)
        self.cfg, self.device = cfg, dev
        pt, ph, pw = cfg.patch_size
        if frames % pt or height % ph or width % pw:
            raise ValueError(f"latent shape ({frames}, {height}, {width}) not divisible by the patch {cfg.patch_size}")
        if ctx_len < 1:
            raise ValueError("the Cosmos blocks cross-attend: ctx_len must be >= 1")
        t, h, w = frames // pt, height // ph, width // pw
        self.grid = (t, h, w)
        B, Cm, A, Lr = batch, cfg.hidden, cfg.attn_dim, cfg.adaln_lora_dim
        S, R = t * h * w, batch * t
        self.B, self.S, self.Lc, self.R = B, S, ctx_len, R
        last = cfg.num_layers - 1 if stop_layer is None else int(stop_layer)
        if not 0 <= last < cfg.num_layers:
            raise ValueError(f"stop_layer {stop_layer} outside 0 .. {cfg.num_layers - 1}")
        self.n = n = last + 1
        self.lib = lib = _capi.load()
        z = lambda *s: torch.zeros(*s, dtype=_BF16, device=dev)  # noqa: E731

        def Pm(name):
            if name not in params:
                raise KeyError(f"missing parameter {name}")
            return params[name].to(device=dev, dtype=_BF16).contiguous()

        P = pt * ph * pw
        self.w = {"patch_w": Pm("patch_embed.proj.weight"),
                  "te1_w": Pm("time_embed.t_embedder.linear_1.weight"),
                  "te2_w": Pm("time_embed.t_embedder.linear_2.weight"), "tn_w": Pm("time_embed.norm.weight")}
        if tuple(self.w["patch_w"].shape) != (Cm, cfg.in_channels * P):
            raise ValueError(f"patch_embed.proj.weight must be [{Cm}, {cfg.in_channels * P}]")
        units = [f"transformer_blocks.{i}.norm{u}." for i in range(n) for u in (1, 2, 3)]
        self.lora1 = torch.cat([params[u + "linear_1.weight"].float() for u in units], 0).to(dev, _BF16).contiguous()
        self.lora2 = [Pm(u + "linear_2.weight") for u in units]
        self.ckv_w = torch.cat([params[f"transformer_blocks.{i}.attn2.to_{c}.weight"].float()
                                for i in range(n) for c in "kv"], 0).to(dev, _BF16).contiguous()
        self.cnk = torch.stack([params[f"transformer_blocks.{i}.attn2.norm_k.weight"].float()
                                for i in range(n)]).to(dev, _BF16).contiguous()

        # static inputs and per-call buffers
        self.x_in = z(B, cfg.in_channels, frames, height, width)
        self.ts = z(R)
        self.ctx_in = z(B * ctx_len, cfg.text_dim)
        self.cmask = torch.ones(B, ctx_len, dtype=torch.bool, device=dev)
        self.patches = z(B * S, cfg.in_channels * P)
        self.tp, self.t1, self.et, self.es = z(R, Cm), z(R, Cm), z(R, Cm), z(R, Cm)
        self.temb = z(R, 3 * Cm)
        self.hl = z(R, 3 * n * Lr)
        self.mods = z(R, n, 9 * Cm)
        self.ctxkv = z(B * ctx_len, n * 2 * A)
        M = B * S
        self.shared = {"x": z(M, Cm), "h": z(M, Cm), "attn": z(M, A), "qc": z(M, A), "hid": z(M, cfg.mlp_ratio * Cm)}
        need = max([lib.fam_gemm_ws_floats(M, n_, k_) for n_, k_ in
                    ((3 * A, Cm), (Cm, A), (A, Cm), (cfg.mlp_ratio * Cm, Cm), (Cm, cfg.mlp_ratio * Cm))] + [0])
        if need > 0:
            self.shared["ws"] = torch.zeros(need, dtype=torch.float32, device=dev)
        self.rope = cosmos_rope_tables(cfg, t, h, w, fps, dev)

        self.steps: List = []
        self.meta: List[dict] = []
        self._descs: List = []
        sh = self.shared
        self._add("patchify", "fam_patchify", (self.x_in.data_ptr(), B, cfg.in_channels, frames, height, width,
                                               pt, ph, pw, self.patches.data_ptr()), "patchify")
        self._gemm("patch_embed", self.patches, self.w["patch_w"], sh["x"])
        self._add("sinusoid", "fam_sinusoid", (self.ts.data_ptr(), self.tp.data_ptr(), R, Cm), "sinusoid")
        self._gemm("time_emb1", self.tp, self.w["te1_w"], self.t1, act=_capi.FAM_ACT_SILU)
        self._gemm("time_emb2", self.t1, self.w["te2_w"], self.temb)
        self._add("time_norm", "fam_rmsnorm_rope", (self.tp.data_ptr(), Cm, self.et.data_ptr(), Cm, R, 1, Cm,
                                                    self.w["tn_w"].data_ptr(), float(cfg.eps), None, None, 0, 0, 0),
                  "rmsnorm_rope")
        self._add("time_silu", "fam_act_rows", (self.et.data_ptr(), Cm, self.es.data_ptr(), Cm, R, Cm,
                                                _capi.FAM_ACT_SILU), "act")
        self._gemm("lora_down_all", self.es, self.lora1, self.hl)
        for j, w2 in enumerate(self.lora2):
            i, u = divmod(j, 3)
            self._gemm(f"lora_up_{i}_{u}", self.hl[:, j * Lr:(j + 1) * Lr], w2,
                       self.mods[:, i, u * 3 * Cm:(u + 1) * 3 * Cm], res=self.temb)
        self._gemm("ctx_kv_all", self.ctx_in, self.ckv_w, self.ctxkv)
        kv = self.ctxkv
        self._add("ctx_k_norm_all", "fam_headnorm_rope",
                  (kv.data_ptr(), kv.stride(0), kv.data_ptr(), kv.stride(0), B * ctx_len, ctx_len, n, 2 * A, A,
                   cfg.head_dim, self.cnk.data_ptr(), cfg.head_dim, float(cfg.eps), None, None, 0), "headnorm_rope")
        self.blocks = [FusedCosmosBlock(params, i, cfg, batch=B, seq_len=S, ctx_len=ctx_len, rope=self.rope,
                                        mod_group=h * w, shared=sh, mods=self.mods[:, i, :],
                                        ctx_kv=(self.ctxkv, i * 2 * A), ctx_mask=self.cmask, device=dev)
                       for i in range(n)]
        for b in self.blocks:
            self.steps += b.steps
            self.meta += b.meta
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ plan building
    def _add(self, name, fname, args, kind):
        f, lib = getattr(self.lib, fname), self.lib

        def run(stream):
            rc = f(*args, stream)
            if rc != 0:
                raise _capi.FamError(f"{fname}[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.steps.append(run)
        self.meta.append({"name": name, "kernel": kind})

    def _gemm(self, name, a, w, out, act=_capi.FAM_ACT_NONE, res=None):
        d = _gemm_desc(a, w, out, act=act, res=res)
        self._descs.append(d)
        M, N, K = a.shape[0], w.shape[0], w.shape[1]
        self._add(name, "fam_gemm", (C.byref(d),), "gemm")
        self.meta[-1]["flops"] = 2 * M * N * K

    # ------------------------------------------------------------------ execution
    def set_inputs(self, latents: torch.Tensor, timestep: torch.Tensor, context: torch.Tensor,
                   context_mask: Optional[torch.Tensor] = None) -> None:
        """latents [B, in_channels, T, Hl, Wl]; timestep [B] (every frame) or [B, T]; context
        [B, Lc, text_dim]; context_mask bool [B, Lc] (None: every token).  Copied into the
        static buffers."""
        self.x_in.copy_(latents.reshape(self.x_in.shape))
        t = timestep.to(device=self.device, dtype=_BF16).reshape(self.B, -1)
        self.ts.view(self.B, -1).copy_(t.expand(self.B, self.grid[0]))
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

    def run_until(self, name: str, block: int) -> None:
        """Eager launches up to and including step `name` of block `block` (see
        FusedVideoDiTBlock.run_until): after "self_attn" / "cross_attn" the shared "attn" holds
        that attention's output before its o projection, after "qk_norm_rope" the block's `qkv`
        holds the rotated q and k."""
        blk = self.blocks[block]
        names = [m["name"] for m in blk.meta]
        if name not in names:
            raise ValueError(f"no step {name!r} in block {block} (steps: {names})")
        target = blk.steps[names.index(name)]
        end = next(i for i, f in enumerate(self.steps) if f is target)
        s = torch.cuda.current_stream(self.device).cuda_stream
        for f in self.steps[:end + 1]:
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

    def forward(self, latents, timestep, context, context_mask=None) -> torch.Tensor:
        """The output of block stop_layer, [B, S, hidden] (a view, valid until the next run)."""
        self.set_inputs(latents, timestep, context, context_mask)
        self.run()
        return self.features()

    def features(self) -> torch.Tensor:
        return self.shared["x"].view(self.B, self.S, self.cfg.hidden)

    def pre_state(self):
        """Per-call values for inspection: the embedded tokens before the blocks ran are not kept
        (the residual stream is updated in place); temb [R, 3C], embedded_timestep [R, C],
        the modulation table [R, blocks, 9C] and the RoPE tables."""
        return {"temb": self.temb, "embedded_timestep": self.et, "mods": self.mods, "rope": self.rope}

    @property
    def num_launches(self) -> int:
        return len(self.steps)

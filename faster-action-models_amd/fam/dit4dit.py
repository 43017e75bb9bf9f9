"""DiT4DiT flow-matching action head on the gfx950 kernels.

`FusedDiT4DiTHead` runs `FlowmatchingActionHead.predict_action` (state=None) of
src/dit4dit-baseline/DiT4DiT/model/modules/action_model/ActionDiT.py:321-369 for a fixed call
shape, on the library's GEMM, LayerNorm-prologue, attention and Euler kernels:

  per step (t = int((1 - i/N) * 1000)):
    ActionEncoder (ActionDiT.py:74-98): layer1 -> [a | tau] -> swish(layer2) -> layer3 (+ position
      embedding, ActionDiT.py:349-352)
    16 blocks of the head DiT (flow_matching_head/cross_attention_dit.py:150-187, 276-299):
      AdaLayerNorm prologue (scale, shift from Linear(SiLU(temb))) on the q (cross) or q/k/v (self)
      projection; attention over the VLM tokens (even blocks) or the action tokens (odd blocks,
      interleave_self_attention); to_out with the residual in the epilogue; LayerNorm prologue +
      GELU(tanh) on the FFN up projection; FFN down with the residual
    output AdaLN (cross_attention_dit.py:301-304) as the prologue of proj_out_2; action decoder
      MLP (layer1 + ReLU, layer2); actions -= dt * velocity (fam_euler_step, bf16 as the reference)

Everything that depends only on the weights and the fixed schedule -- the timestep embeddings
(diffusers Timesteps / TimestepEmbedding semantics), every block's AdaLN (scale, shift), the
output (shift, scale) and the action encoder's sinusoidal tau rows -- is computed once at
construction; the VLM K/V of all cross blocks is one GEMM per call.  The whole call can be
captured into one graph.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _capi, ops

_BF16 = torch.bfloat16


@dataclass
class DiT4DiTHeadConfig:
    """DiT-B head (ActionDiT.py:192-195) with the diffusion_model_cfg of
    DiT4DiT/config/real_robot/dit4dit_g1.yaml:25-49."""
    action_dim: int = 32
    horizon: int = 16
    heads: int = 12
    head_dim: int = 64
    num_layers: int = 16
    cross_dim: int = 2048
    output_dim: int = 2560
    hidden_size: int = 2560
    max_seq_len: int = 1024
    num_steps: int = 4
    buckets: int = 1000
    interleave_self_attention: bool = True
    ff_mult: int = 4
    norm_eps: float = 1e-5
    out_eps: float = 1e-6
    state_dim: int = 64      # state_encoder input (dit4dit_g1.yaml:31; LIBERO 16); 0: none


def param_shapes(cfg) -> Dict[str, Tuple[int, ...]]:
    """FlowmatchingActionHead state-dict keys and shapes (ActionDiT.py:197-236, diffusers
    Attention / FeedForward / TimestepEmbedding submodule names)."""
    D = cfg.heads * cfg.head_dim
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
        "action_decoder.layer1.weight": (cfg.hidden_size, cfg.output_dim),
        "action_decoder.layer1.bias": (cfg.hidden_size,),
        "action_decoder.layer2.weight": (cfg.action_dim, cfg.hidden_size), "action_decoder.layer2.bias": (cfg.action_dim,),
        "position_embedding.weight": (cfg.max_seq_len, D),
    }
    if cfg.state_dim:
        s.update({"state_encoder.layer1.weight": (cfg.hidden_size, cfg.state_dim),
                  "state_encoder.layer1.bias": (cfg.hidden_size,),
                  "state_encoder.layer2.weight": (D, cfg.hidden_size), "state_encoder.layer2.bias": (D,)})
    for i in range(cfg.num_layers):
        b = f"model.transformer_blocks.{i}."
        kv_in = D if (cfg.interleave_self_attention and i % 2 == 1) else cfg.cross_dim
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


def synthetic_params(cfg, seed: int, std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Seeded N(0, std) weights for every tensor (sorted-name draws on the CPU), fp32."""
    g = torch.Generator().manual_seed(seed)
    return {k: torch.randn(v, generator=g) * std for k, v in sorted(param_shapes(cfg).items())}


def _tau_rows(t: float, dim: int) -> torch.Tensor:
    """SinusoidalPositionalEncoding of one timestep (flow_matching_head/action_encoder.py:21-37),
    cat(sin, cos), computed in fp64 on the host."""
    half = dim // 2
    f = torch.exp(-torch.arange(half, dtype=torch.float64) * (math.log(10000.0) / half))
    a = t * f
    return torch.cat([torch.sin(a), torch.cos(a)])


def _timestep_proj(t: float, channels: int = 256) -> torch.Tensor:
    """diffusers Timesteps(256, flip_sin_to_cos=True, downscale_freq_shift=1) of one timestep
    (cross_attention_dit.py:34): cat(cos, sin) with f_i = exp(-ln(10000) i / (half - 1)), fp64."""
    half = channels // 2
    f = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float64) / (half - 1))
    a = t * f
    return torch.cat([torch.cos(a), torch.sin(a)])


class FusedDiT4DiTHead:
    """predict_action of the DiT4DiT head for `batch` action chunks, `vl_len` VLM tokens and
    `state_len` state tokens per chunk (0: the state=None call).

    Rows are token-major: sequence position j of chunk b is row j * batch + b, with the state
    tokens first (DB/ActionDiT.py:355-356), so the action rows of all chunks are one contiguous
    [horizon * batch, D] block for the encoder, the output projection and the decoder.  The
    actions buffer is [horizon, batch, action_dim] for the same reason; `set_inputs` and
    `predict_action` take and return the reference's [batch, horizon, action_dim].

    Args:
        cfg: DiT4DiTHeadConfig (or any object with its fields).
        params: state dict in the reference's key layout (FlowmatchingActionHead), any float
            dtype; converted to bf16 on `device`.
        state_len: state tokens per chunk (the reference's state is [B, 1, state_dim]);
            default 1 when cfg.state_dim > 0.
        fold_norms: evaluate every LayerNorm / AdaLN that feeds a projection as
            rstd * (x W'^T - mean * colsum(W')) with the (fixed-schedule) modulation folded into
            W' and the bias at construction (fam_gemm FAM_PRO_LN_FOLDED, <= 64 rows); otherwise
            normalise the rows in the GEMM prologue.
    """

    def __init__(self, cfg, params: Dict[str, torch.Tensor], *, batch: int, vl_len: int,
                 device: torch.device, attn_splits: Optional[int] = None, state_len: Optional[int] = None,
                 fold_norms: bool = True):
        self.cfg, self.B, self.L, self.device = cfg, batch, vl_len, device
        D, T, A = cfg.heads * cfg.head_dim, cfg.horizon, cfg.action_dim
        Ls = (1 if cfg.state_dim else 0) if state_len is None else state_len
        if Ls and not cfg.state_dim:
            raise ValueError("DiT4DiT head: state tokens need a state encoder (cfg.state_dim > 0)")
        self.D, self.T, self.Ls = D, T, Ls
        self.Sq = Ls + T                       # sequence length of the head DiT
        self.M, self.R = batch * T, batch * self.Sq   # action rows, all rows
        if D % 8 or cfg.cross_dim % 8 or cfg.output_dim % 8 or cfg.hidden_size % 8:
            raise ValueError("DiT4DiT head: feature widths must be multiples of 8")
        if Ls and cfg.state_dim % 8:
            raise ValueError("DiT4DiT head: state_dim must be a multiple of 8")
        if A > 64:
            raise ValueError("DiT4DiT head: action_dim must be <= 64")
        if self.Sq > 32:
            raise ValueError("DiT4DiT head: state_len + horizon must be <= 32")
        p = {k: v.to(device=device, dtype=_BF16).contiguous() for k, v in params.items()}
        self.p = p
        nb = cfg.num_layers
        cross = [i for i in range(nb) if not (cfg.interleave_self_attention and i % 2 == 1)]
        self.cross_ids = cross
        blk = lambda i, n: p[f"model.transformer_blocks.{i}.{n}"]
        # self blocks: q/k/v stacked into one [3D, D] projection
        self.wqkv = {i: torch.cat([blk(i, "attn1.to_q.weight"), blk(i, "attn1.to_k.weight"), blk(i, "attn1.to_v.weight")]).contiguous()
                     for i in range(nb) if i not in cross}
        self.bqkv = {i: torch.cat([blk(i, "attn1.to_q.bias"), blk(i, "attn1.to_k.bias"), blk(i, "attn1.to_v.bias")]).contiguous()
                     for i in range(nb) if i not in cross}
        # cross blocks: the VLM K/V of every cross block in one [n_cross * 2D, cross_dim] GEMM
        self.wkv = torch.cat([torch.cat([blk(i, "attn1.to_k.weight"), blk(i, "attn1.to_v.weight")]) for i in cross]).contiguous()
        self.bkv = torch.cat([torch.cat([blk(i, "attn1.to_k.bias"), blk(i, "attn1.to_v.bias")]) for i in cross]).contiguous()

        S = cfg.num_steps
        self.t_disc = [int((1.0 - i / float(S)) * cfg.buckets) for i in range(S)]
        self.dt = 1.0 / S
        # ---- per-call constants (weights and the fixed schedule only)
        proj = torch.stack([_timestep_proj(float(t)) for t in self.t_disc]).to(device=device, dtype=_BF16)
        pre = "model.timestep_encoder.timestep_embedder."
        h1 = torch.empty(S, D, dtype=_BF16, device=device)
        ops.gemm(proj, p[pre + "linear_1.weight"], p[pre + "linear_1.bias"], h1, act=_capi.FAM_ACT_SILU)
        self.stemb = torch.empty(S, D, dtype=_BF16, device=device)   # SiLU(temb): every consumer applies SiLU first
        ops.gemm(h1, p[pre + "linear_2.weight"], p[pre + "linear_2.bias"], self.stemb, act=_capi.FAM_ACT_SILU)
        # per (step, block) AdaLayerNorm rows [scale | shift] (cross_attention_dit.py:64-66)
        wmod = torch.cat([blk(i, "norm1.linear.weight") for i in range(nb)]).contiguous()
        bmod = torch.cat([blk(i, "norm1.linear.bias") for i in range(nb)]).contiguous()
        self.mods = torch.empty(S, nb * 2 * D, dtype=_BF16, device=device)
        ops.gemm(self.stemb, wmod, bmod, self.mods)
        # output rows [shift | scale] (cross_attention_dit.py:302)
        self.omods = torch.empty(S, 2 * D, dtype=_BF16, device=device)
        ops.gemm(self.stemb, p["model.proj_out_1.weight"], p["model.proj_out_1.bias"], self.omods)
        # action encoder input rows [a | tau]: tau is fixed per step
        M = self.M
        self.x2 = torch.empty(S, M, 2 * D, dtype=_BF16, device=device)
        for s, t in enumerate(self.t_disc):
            self.x2[s, :, D:] = _tau_rows(float(t), D).to(device=device, dtype=_BF16)
        self.posx = p["position_embedding.weight"][:T].repeat_interleave(batch, dim=0).contiguous()   # [M, D]
        # folded normalisations: per (step, block) the AdaLN of that step's timestep inside the
        # q / qkv weights; FFN up's plain LayerNorm needs only column sums; per step the output
        # AdaLN inside proj_out_2
        self.fold = fold_norms and self.R <= 64
        if self.fold:
            self.fq: List[List[tuple]] = []
            for s in range(S):
                row = []
                for i in range(nb):
                    shift, scale = self._mod(s, i)
                    w, b = ((blk(i, "attn1.to_q.weight"), blk(i, "attn1.to_q.bias")) if i in cross
                            else (self.wqkv[i], self.bqkv[i]))
                    row.append(ops.fold_layernorm(w, b, scale=scale, shift=shift))
                self.fq.append(row)
            self.fup_cs = [ops.fold_layernorm(blk(i, "ff.net.0.proj.weight"))[2] for i in range(nb)]
            self.fout = [ops.fold_layernorm(p["model.proj_out_2.weight"], p["model.proj_out_2.bias"],
                                            scale=self.omods[s, D:], shift=self.omods[s, :D]) for s in range(S)]
        # ---- activations (token-major rows)
        R = self.R
        self.actions = torch.empty(T, batch, A, dtype=_BF16, device=device)
        self.vl_in = torch.empty(batch, vl_len, cfg.cross_dim, dtype=_BF16, device=device)
        self.ctxkv = torch.empty(batch * vl_len, len(cross) * 2 * D, dtype=_BF16, device=device)
        if Ls:
            self.st_in = torch.empty(Ls, batch, cfg.state_dim, dtype=_BF16, device=device)
            self.st_hid = torch.empty(Ls * batch, cfg.hidden_size, dtype=_BF16, device=device)
            self.st_feat = torch.empty(Ls * batch, D, dtype=_BF16, device=device)
        self.h = torch.empty(R, D, dtype=_BF16, device=device)
        self.e = torch.empty(M, D, dtype=_BF16, device=device)
        self.qkv = torch.empty(R, 3 * D, dtype=_BF16, device=device)
        self.attn = torch.empty(R, D, dtype=_BF16, device=device)
        self.up = torch.empty(R, cfg.ff_mult * D, dtype=_BF16, device=device)
        # FFN down (D x ff_mult*D): at <= 64 rows a split-K product over >= 256 workgroups,
        # finished by the row kernel with bias and residual; the whole-K GEMM of D = 768
        # output columns would run on only D / 16 workgroups
        self.ff_split = R <= 64
        if self.ff_split:
            S = _capi.lib().fam_gemm_partial_splits(R, D, cfg.ff_mult * D)
            self.ff_part = torch.empty(S, R, D, dtype=torch.float32, device=device)
        self.y = torch.empty(M, cfg.output_dim, dtype=_BF16, device=device)
        self.z = torch.empty(M, cfg.hidden_size, dtype=_BF16, device=device)
        self.vel = torch.empty(T, batch, A, dtype=_BF16, device=device)
        self.delta = torch.tensor(-self.dt, dtype=_BF16, device=device)
        self.splits = (attn_splits if attn_splits is not None else
                       int(_capi.lib().fam_attention_key_splits(batch, cfg.heads, self.Sq, vl_len, cfg.head_dim)))
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ one policy call
    def _mod(self, s: int, i: int):
        D = self.D
        row = self.mods[s, i * 2 * D:(i + 1) * 2 * D]
        return row[D:], row[:D]   # shift, scale

    def _enqueue(self) -> None:
        cfg, p, D, T, B, M, R, Sq = self.cfg, self.p, self.D, self.T, self.B, self.M, self.R, self.Sq
        blk = lambda i, n: p[f"model.transformer_blocks.{i}.{n}"]
        ns = self.Ls * B                     # state rows come first
        h_act = self.h[ns:]
        # VLM K/V of every cross block
        ops.gemm(self.vl_in.view(B * self.L, cfg.cross_dim), self.wkv, self.bkv, self.ctxkv)
        kv_w = self.ctxkv.shape[1]
        if ns:
            # state_encoder MLP, once per call (DB/ActionDiT.py:333)
            ops.gemm(self.st_in.view(ns, cfg.state_dim), p["state_encoder.layer1.weight"], p["state_encoder.layer1.bias"],
                     self.st_hid, act=_capi.FAM_ACT_RELU)
            ops.gemm(self.st_hid, p["state_encoder.layer2.weight"], p["state_encoder.layer2.bias"], self.st_feat)
        # [B, Sq, .] views of the token-major row buffers
        q3 = self.qkv.view(Sq, B, 3 * D).transpose(0, 1)
        o3 = self.attn.view(Sq, B, D).transpose(0, 1)
        for s in range(cfg.num_steps):
            # ActionEncoder: layer1 into the a-half of [a | tau], swish(layer2), layer3 + position rows
            x2 = self.x2[s]
            _capi.call("fam_linear_smallk", self.actions.data_ptr(), cfg.action_dim, 0,
                       p["action_encoder.layer1.weight"].data_ptr(), p["action_encoder.layer1.bias"].data_ptr(),
                       x2.data_ptr(), 2 * D, M, D, cfg.action_dim, torch.cuda.current_stream(self.device).cuda_stream)
            ops.gemm(x2, p["action_encoder.layer2.weight"], p["action_encoder.layer2.bias"], self.e, act=_capi.FAM_ACT_SILU)
            ops.gemm(self.e, p["action_encoder.layer3.weight"], p["action_encoder.layer3.bias"], h_act, res=self.posx)
            if ns:
                self.h[:ns].copy_(self.st_feat)
            for i in range(cfg.num_layers):
                if self.fold:
                    wq, bq, cq = self.fq[s][i]
                    qproj = lambda out: ops.gemm(self.h, wq, bq, out, prologue=_capi.FAM_PRO_LN_FOLDED, pro_w=cq,
                                                 pro_eps=cfg.norm_eps)
                else:
                    shift, scale = self._mod(s, i)
                    ada = dict(prologue=_capi.FAM_PRO_ADALN, pro_shift=shift, pro_scale=scale, pro_mod_bs=0,
                               pro_mod_rs=0, pro_eps=cfg.norm_eps, rows_per_batch=R)
                    wq, bq = ((blk(i, "attn1.to_q.weight"), blk(i, "attn1.to_q.bias")) if i in self.cross_ids
                              else (self.wqkv[i], self.bqkv[i]))
                    qproj = lambda out: ops.gemm(self.h, wq, bq, out, **ada)
                if i in self.cross_ids:
                    c = self.cross_ids.index(i)
                    qproj(self.qkv[:, :D])
                    kv = self.ctxkv.view(B, self.L, kv_w)
                    k = kv[:, :, c * 2 * D:c * 2 * D + D]
                    v = kv[:, :, c * 2 * D + D:(c + 1) * 2 * D]
                    ops.attention_bshd(q3[:, :, :D], k, v, cfg.heads, out=o3, num_splits=self.splits)
                else:
                    qproj(self.qkv)
                    ops.attention_bshd(q3[:, :, :D], q3[:, :, D:2 * D], q3[:, :, 2 * D:], cfg.heads, out=o3)
                ops.gemm(self.attn, blk(i, "attn1.to_out.0.weight"), blk(i, "attn1.to_out.0.bias"), self.h,
                         res=self.h)
                if self.fold:
                    ops.gemm(self.h, blk(i, "ff.net.0.proj.weight"), blk(i, "ff.net.0.proj.bias"), self.up,
                             prologue=_capi.FAM_PRO_LN_FOLDED, pro_w=self.fup_cs[i], pro_eps=cfg.norm_eps,
                             act=_capi.FAM_ACT_GELU_TANH)
                else:
                    ops.gemm(self.h, blk(i, "ff.net.0.proj.weight"), blk(i, "ff.net.0.proj.bias"), self.up,
                             prologue=_capi.FAM_PRO_LAYERNORM, pro_eps=cfg.norm_eps, act=_capi.FAM_ACT_GELU_TANH)
                if self.ff_split:
                    w2 = blk(i, "ff.net.2.weight")
                    _capi.call("fam_gemm_partial", self.up.data_ptr(), self.up.stride(0), w2.data_ptr(), w2.stride(0),
                               self.ff_part.data_ptr(), self.R, self.D, w2.shape[1],
                               torch.cuda.current_stream().cuda_stream)
                    ops.rowop(self.h, partials=self.ff_part, bias=blk(i, "ff.net.2.bias"), res=self.h)
                else:
                    ops.gemm(self.up, blk(i, "ff.net.2.weight"), blk(i, "ff.net.2.bias"), self.h, res=self.h)
            # output AdaLN (shift, scale order) + proj_out_2, action decoder, Euler step; the state
            # rows' outputs are dropped by the reference (pred[:, -horizon:]) and not computed here
            if self.fold:
                wo, bo, co = self.fout[s]
                ops.gemm(h_act, wo, bo, self.y, prologue=_capi.FAM_PRO_LN_FOLDED, pro_w=co, pro_eps=cfg.out_eps)
            else:
                om = self.omods[s]
                ops.gemm(h_act, p["model.proj_out_2.weight"], p["model.proj_out_2.bias"], self.y,
                         prologue=_capi.FAM_PRO_ADALN, pro_shift=om[:D], pro_scale=om[D:], pro_mod_bs=0,
                         pro_mod_rs=0, pro_eps=cfg.out_eps, rows_per_batch=M)
            ops.gemm(self.y, p["action_decoder.layer1.weight"], p["action_decoder.layer1.bias"], self.z, act=_capi.FAM_ACT_RELU)
            ops.gemm(self.z, p["action_decoder.layer2.weight"], p["action_decoder.layer2.bias"], self.vel.view(M, -1))
            ops.euler_step(self.vel, self.delta, self.actions, out=self.actions)

    def set_inputs(self, noise: torch.Tensor, vl_embs: torch.Tensor, state: Optional[torch.Tensor] = None) -> None:
        """noise [B, horizon, action_dim], vl_embs [B, L, cross_dim], state [B, state_len, state_dim]
        (required exactly when state_len > 0)."""
        B, T = self.B, self.T
        self.actions.copy_(noise.reshape(B, T, -1).transpose(0, 1))
        self.vl_in.copy_(vl_embs.reshape(self.vl_in.shape))
        if self.Ls:
            if state is None:
                raise ValueError("DiT4DiT head was built for state tokens; pass state [B, state_len, state_dim]")
            self.st_in.copy_(state.reshape(B, self.Ls, -1).transpose(0, 1))
        elif state is not None:
            raise ValueError("DiT4DiT head was built with state_len=0; state must be None")

    def run(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            self._enqueue()

    def capture(self, warmup: int = 1) -> None:
        """Capture one policy call into a graph (the inputs are the static buffers)."""
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self._enqueue()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._enqueue()
        self.graph = g

    def result(self) -> torch.Tensor:
        """The denoised actions [B, horizon, action_dim] (bf16, a copy)."""
        return self.actions.transpose(0, 1).contiguous()

    def predict_action(self, vl_embs: torch.Tensor, noise: torch.Tensor,
                       state: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One call of FlowmatchingActionHead.predict_action (noise drawn by the caller)."""
        self.set_inputs(noise, vl_embs, state)
        self.run()
        return self.result()

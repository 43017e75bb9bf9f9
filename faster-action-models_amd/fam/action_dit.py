"""The action expert of FastWAM on the fused HIP kernels, and its flow-matching denoise loop.

Semantics follow the reference's eager modules (paths under src/fastwam-baseline/fastwam/
models/wan22, "FB"):

    ActionDiT.pre_dit / forward / post_dit    FB/action_dit.py:228-353
    DiTBlock.forward                           FB/wan_video_dit.py:267-286
    SelfAttention / CrossAttention             FB/wan_video_dit.py:180-229
    FastWAM.infer_action denoise loop          FB/fastwam.py:1040-1069
    WanContinuousFlowMatchScheduler            FB/schedulers/scheduler_continuous.py:63-88

The model is organised for one GPU and a fixed call shape (batch, action tokens, context
length, number of steps), so that every buffer is allocated once and one policy call is a
fixed sequence of launches -- a "plan" -- that replays eagerly or from a captured HIP graph.
Per policy call the plan runs:

  prologue (once per call, work that is identical for every denoise step):
    sinusoid(t_0..t_{T-1}) -> time MLP for all T steps (three GEMMs with SiLU epilogues)
    -> t_mod + modulation of every block; context embedding (GEMM+GELU, GEMM); the context
    K/V of every block from one GEMM over the concatenated weights; RMSNorm of each K.
  per step:
    [action encoder (7 -> H) + AdaLN1] -> 12 x block -> [head GEMM] -> [Euler update].
  per block (15 launches): every projection is a split-K GEMM writing fp32 partials, and the
  row kernel after it sums them and runs the epilogue plus the next normalisation:
    qkv GEMM -> [bias, RMSNorm+RoPE of q and k] -> self-attention ->
    o GEMM -> [bias, x += gate_msa*o, LayerNorm3] -> cross-q GEMM -> [bias, RMSNorm(q)] ->
    cross-attention (keys split over workgroups) -> combine ->
    cross-o GEMM -> [bias, x += o, AdaLN2] -> FFN-up GEMM -> [bias, GELU] ->
    FFN-down GEMM -> [bias, x += gate_mlp*ffn, AdaLN1 of the next block].

The per-call prologue replaces work the reference repeats inside every step (time MLP,
text embedding, context K/V projection): the values are identical at every step of one
call, so computing them once per call is the same arithmetic (the GEAK tree hoists the
same work, FG/action_dit.py:419-447, FG/mot.py:2580-2593).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, asdict
from typing import Callable, Dict, List, Optional

import torch

from . import _capi
from ._capi import FamError

_BF16 = torch.bfloat16


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


def param_shapes(cfg: ActionDiTConfig) -> Dict[str, tuple]:
    """Parameter names (the reference's state-dict keys) and shapes of ActionDiT
    (FB/action_dit.py:76-97, FB/wan_video_dit.py:180-265)."""
    H, A, Fd = cfg.hidden_dim, cfg.attn_dim, cfg.ffn_dim
    shapes = {
        "action_encoder.weight": (H, cfg.action_dim), "action_encoder.bias": (H,),
        "text_embedding.0.weight": (H, cfg.text_dim), "text_embedding.0.bias": (H,),
        "text_embedding.2.weight": (H, H), "text_embedding.2.bias": (H,),
        "time_embedding.0.weight": (H, cfg.freq_dim), "time_embedding.0.bias": (H,),
        "time_embedding.2.weight": (H, H), "time_embedding.2.bias": (H,),
        "time_projection.1.weight": (6 * H, H), "time_projection.1.bias": (6 * H,),
        "head.weight": (cfg.action_dim, H), "head.bias": (cfg.action_dim,),
    }
    for i in range(cfg.num_layers):
        p = f"blocks.{i}."
        for att in ("self_attn", "cross_attn"):
            for n in "qkv":
                shapes[p + f"{att}.{n}.weight"], shapes[p + f"{att}.{n}.bias"] = (A, H), (A,)
            shapes[p + f"{att}.o.weight"], shapes[p + f"{att}.o.bias"] = (H, A), (H,)
            shapes[p + f"{att}.norm_q.weight"] = shapes[p + f"{att}.norm_k.weight"] = (A,)
        shapes[p + "norm3.weight"] = shapes[p + "norm3.bias"] = (H,)
        shapes[p + "ffn.0.weight"], shapes[p + "ffn.0.bias"] = (Fd, H), (Fd,)
        shapes[p + "ffn.2.weight"], shapes[p + "ffn.2.bias"] = (H, Fd), (H,)
        shapes[p + "modulation"] = (1, 6, H)
    return shapes


def synthetic_params(cfg: ActionDiTConfig, seed: int, std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Seeded random weights for benchmarking (no checkpoints are available offline):
    N(0, std) weights and biases, modulation randn/sqrt(H) as the reference initialises it
    (FB/wan_video_dit.py:264), RMSNorm/LayerNorm weights N(1, 0.2) and LayerNorm biases
    N(0, 0.2) (a trained checkpoint's affines are not the identity); drawn in sorted-name
    order from one CPU generator, fp32."""
    g = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for name, shape in sorted(param_shapes(cfg).items()):
        if name.endswith("modulation"):
            out[name] = torch.randn(shape, generator=g) / math.sqrt(cfg.hidden_dim)
        elif ".norm_q." in name or ".norm_k." in name or name.endswith("norm3.weight"):
            out[name] = 1.0 + torch.randn(shape, generator=g) * 0.2
        elif name.endswith("norm3.bias"):
            out[name] = torch.randn(shape, generator=g) * 0.2
        else:
            out[name] = torch.randn(shape, generator=g) * std
    return out


def rope_1d_tables(head_dim: int, seq_len: int, theta: float = 10000.0, end: int = 1024):
    """cos/sin [S, Dh/2] fp32 of the 1-D action RoPE: angles pos * theta^(-2j/Dh) built in fp64
    through torch.polar like precompute_freqs_cis (FB/wan_video_dit.py:49-55, FB/action_dit.py:101)."""
    if seq_len > end:
        raise ValueError(f"Action token length {seq_len} exceeds RoPE cache {end}.")
    j = torch.arange(0, head_dim, 2)[: head_dim // 2].to(torch.float64)
    inv = 1.0 / (theta ** (j / head_dim))
    ang = torch.arange(seq_len).to(torch.float64).reshape(-1, 1) * inv.reshape(1, -1)
    z = torch.polar(torch.ones_like(ang), ang)
    return z.real.to(torch.float32).contiguous(), z.imag.to(torch.float32).contiguous()


def schedule(num_steps: int, shift: float, num_train_timesteps: int = 1000):
    """bf16 timesteps and deltas of the shifted flow-matching schedule (SCH:63-80)."""
    u = torch.linspace(1.0, 0.0, num_steps + 1, dtype=torch.float32)
    sigma = shift * u / (1.0 + (shift - 1.0) * u)
    return (sigma[:-1] * float(num_train_timesteps)).to(_BF16), (sigma[1:] - sigma[:-1]).to(_BF16)


class _Plan:
    """An ordered list of launches on prebuilt descriptors, each with its kernel class and
    algorithmic work (HBM bytes and flops that the operation must move/do at minimum)."""

    def __init__(self):
        self.steps: List[Callable[[int], None]] = []
        self.names: List[str] = []
        self.meta: List[dict] = []

    def add(self, name: str, fn: Callable[[int], None], kernel: str = "other", nbytes: int = 0,
            flops: int = 0) -> None:
        self.names.append(name)
        self.steps.append(fn)
        self.meta.append({"kernel": kernel, "bytes": int(nbytes), "flops": int(flops)})

    def run(self, stream: int) -> None:
        for fn in self.steps:
            fn(stream)


def _checked(lib, name: str, *args):
    f = getattr(lib, name)

    def run(stream: int):
        rc = f(*args, stream)
        if rc != 0:
            raise FamError(name, rc, lib.fam_last_error().decode(errors="replace"))
    return run


class FusedActionDiT:
    """ActionDiT + flow-matching loop on the gfx950 kernels, for a fixed call shape.

    Args:
        cfg: architecture.
        params: state dict in the reference's key layout (FB/action_dit.py ActionDiT), any
            float dtype; converted to bf16 on `device`.
        batch: B, action chunks denoised together (the context is shared by the batch).
        seq_len: action tokens per chunk (S).
        ctx_len: context tokens (L).
        num_steps / shift: the flow-matching schedule (SCH:63-80).
        video_len: Sv > 0 selects the MoT action step (FB/mot.py:378-478): the action tokens'
            self-attention runs over [cached video K/V of the layer ; action K/V]; the caches
            are given per call through `set_video_kv`.
        video_mask: optional bool [S, Sv + S], the action rows of the joint mask
            (FB/fastwam.py:388-410; True = attend); None = every key.
        video_kv: optional per-layer [(k, v)] device views [B, Sv, A] (bf16, unit last-dim
            stride, any row / batch stride) that the joint attention reads in place, e.g. the
            video prefill's cache (FusedVideoPrefill.kv_cache()); then no static copy exists and
            set_video_kv is not needed.  The views must stay valid while this model runs.
        tiny: run the blocks through fam_tiny_expert (two launches per block step; hidden 32
            only).  None (default) picks it whenever the library covers the shape.
        tiny_slice: the attention columns per workgroup of fam_tiny_expert (0: the library's
            choice, 128 or all A columns when A <= 128).
    """

    def __init__(self, cfg: ActionDiTConfig, params: Dict[str, torch.Tensor], *, batch: int, seq_len: int,
                 ctx_len: int, num_steps: int, shift: float = 5.0, device="cuda", mode: str = "denoise",
                 video_len: int = 0, video_mask: Optional[torch.Tensor] = None, video_kv=None,
                 tiny: Optional[bool] = None, tiny_slice: int = 0):
        if mode not in ("denoise", "forward"):
            raise ValueError(f"mode must be 'denoise' or 'forward', got {mode!r}")
        if mode == "forward" and num_steps != 1:
            raise ValueError("forward mode runs one ActionDiT.forward: num_steps must be 1")
        self.mode = mode
        self.cfg = cfg
        self.B, self.S, self.Lc, self.T = batch, seq_len, ctx_len, num_steps
        self.shift = shift
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.lib = _capi.load()
        H, A, Fd, L = cfg.hidden_dim, cfg.attn_dim, cfg.ffn_dim, cfg.num_layers
        dev = self.device

        def P(name):
            if name not in params:
                raise KeyError(f"missing parameter {name}")
            return params[name].to(device=dev, dtype=_BF16).contiguous()

        def cat(names):
            return torch.cat([params[n].to(dtype=torch.float32) for n in names], 0).to(device=dev, dtype=_BF16).contiguous()

        # ---- weights
        self.w = w = {}
        w["enc_w"], w["enc_b"] = P("action_encoder.weight"), P("action_encoder.bias")
        w["txt0_w"], w["txt0_b"] = P("text_embedding.0.weight"), P("text_embedding.0.bias")
        w["txt2_w"], w["txt2_b"] = P("text_embedding.2.weight"), P("text_embedding.2.bias")
        w["te0_w"], w["te0_b"] = P("time_embedding.0.weight"), P("time_embedding.0.bias")
        w["te2_w"], w["te2_b"] = P("time_embedding.2.weight"), P("time_embedding.2.bias")
        w["tp_w"], w["tp_b"] = P("time_projection.1.weight"), P("time_projection.1.bias")
        w["head_w"], w["head_b"] = P("head.weight"), P("head.bias")
        w["mod"] = torch.stack([P(f"blocks.{i}.modulation").reshape(6 * H) for i in range(L)]).contiguous()
        kv_w, kv_b = [], []
        for i in range(L):
            p = f"blocks.{i}."
            w[f"qkv_w{i}"] = cat([p + f"self_attn.{n}.weight" for n in "qkv"])
            w[f"qkv_b{i}"] = cat([p + f"self_attn.{n}.bias" for n in "qkv"])
            for n in ("o", "norm_q", "norm_k"):
                w[f"sa_{n}_w{i}"] = P(p + f"self_attn.{n}.weight")
            w[f"sa_o_b{i}"] = P(p + "self_attn.o.bias")
            w[f"ca_q_w{i}"], w[f"ca_q_b{i}"] = P(p + "cross_attn.q.weight"), P(p + "cross_attn.q.bias")
            w[f"ca_o_w{i}"], w[f"ca_o_b{i}"] = P(p + "cross_attn.o.weight"), P(p + "cross_attn.o.bias")
            w[f"ca_nq_w{i}"], w[f"ca_nk_w{i}"] = P(p + "cross_attn.norm_q.weight"), P(p + "cross_attn.norm_k.weight")
            w[f"n3_w{i}"], w[f"n3_b{i}"] = P(p + "norm3.weight"), P(p + "norm3.bias")
            w[f"ff0_w{i}"], w[f"ff0_b{i}"] = P(p + "ffn.0.weight"), P(p + "ffn.0.bias")
            w[f"ff2_w{i}"], w[f"ff2_b{i}"] = P(p + "ffn.2.weight"), P(p + "ffn.2.bias")
            kv_w += [p + "cross_attn.k.weight", p + "cross_attn.v.weight"]
            kv_b += [p + "cross_attn.k.bias", p + "cross_attn.v.bias"]
        w["ctxkv_w"], w["ctxkv_b"] = cat(kv_w), cat(kv_b)   # [L*2A, H]: layer-major (K_l, V_l)

        # ---- schedule and RoPE tables
        ts, ds = schedule(num_steps, shift)
        self.timesteps = ts.to(dev)
        self.deltas = ds.to(dev)
        cos, sin = rope_1d_tables(cfg.attn_head_dim, seq_len)
        self.rope_cos, self.rope_sin = cos.to(dev), sin.to(dev)

        # ---- activations (static, so a captured graph can replay them)
        M = batch * seq_len
        z = lambda *s: torch.zeros(*s, dtype=_BF16, device=dev)  # noqa: E731
        self.noise_in = z(batch, seq_len, cfg.action_dim)
        self.context_in = z(ctx_len, cfg.text_dim)
        # the chunk being denoised is carried in fp32 between steps (the reference rounds it to
        # bf16 after every step); it is the only state that survives a step
        self.latents = torch.zeros(batch, seq_len, cfg.action_dim, dtype=torch.float32, device=dev)
        self.x = z(M, H)
        self.qkv = z(M, 3 * A)
        self.attn = z(M, A)
        self.qc = z(M, A)
        self.hid = z(M, Fd)
        self.head_out = z(M, cfg.action_dim)
        self.t_emb = z(num_steps, cfg.freq_dim)
        self.t1 = z(num_steps, H)
        self.t2 = z(num_steps, H)
        self.tmod = z(num_steps, 6 * H)
        self.mods = z(num_steps, L, 6 * H)
        # the text embedding's second layer and the context K/V of every layer are GEMMs over
        # K = H; a hidden width that is not a multiple of 64 (the tiny experts' 32) is
        # zero-padded to the next one, so those products run on the large-M kernel (which takes
        # K in blocks of 64) instead of the generic tiled one: each activation lands in the first
        # H columns of its buffer, the rest stay zero, and the weights get zero columns
        Hp = H if H % 64 == 0 or ctx_len < 128 else (H + 63) // 64 * 64
        if Hp != H:
            for key in ("txt2_w", "ctxkv_w"):
                wt = w[key]
                w[key] = torch.cat([wt, torch.zeros(wt.shape[0], Hp - H, dtype=wt.dtype, device=wt.device)],
                                   dim=1).contiguous()
        self.ctx_h_pad = z(ctx_len, Hp)
        self.ctx_h = self.ctx_h_pad[:, :H]
        self.ctx_emb_pad = z(ctx_len, Hp)
        self.ctx_emb = self.ctx_emb_pad[:, :H]
        self.ctxkv = z(ctx_len, L * 2 * A)
        self.h = z(M, H)   # normalised input of the next projection
        # MoT: per-layer cached video K/V [L, B, Sv, A] and the action rows of the joint mask
        self.Sv = int(video_len)
        self.video_kv = None
        if self.Sv > 0:
            if video_kv is not None:
                if len(video_kv) != L:
                    raise ValueError(f"video_kv needs one (k, v) per layer ({L}), got {len(video_kv)}")
                for k_, v_ in video_kv:
                    for t_ in (k_, v_):
                        if (t_.dtype != _BF16 or t_.device != dev or tuple(t_.shape) != (batch, self.Sv, A)
                                or t_.stride(-1) != 1 or t_.stride(1) % 8 or t_.stride(0) % 8 or t_.data_ptr() % 16):
                            raise ValueError(f"video_kv entries must be bf16 [{batch}, {self.Sv}, {A}] views on "
                                             f"{dev} with unit last-dim stride and 16-byte aligned rows")
                self.video_kv = [(k_, v_) for k_, v_ in video_kv]
            else:
                self.video_k = z(L, batch, self.Sv, A)
                self.video_v = z(L, batch, self.Sv, A)
            self.video_mask = None
            if video_mask is not None:
                vm = video_mask.to(device=dev, dtype=torch.bool).contiguous()
                if tuple(vm.shape) != (seq_len, self.Sv + seq_len):
                    raise ValueError(f"video_mask must be [S, Sv + S] = [{seq_len}, {self.Sv + seq_len}]")
                self.video_mask = vm
        # per-row, per-16-column sums of squares of the raw q/k projections (fam_gemm_final)
        self.ss_qkv = torch.zeros(M, 3 * A // 16, dtype=torch.float32, device=dev)
        self.ss_q = torch.zeros(M, A // 16, dtype=torch.float32, device=dev)

        # split-K partials of the action projections (one buffer, reused launch after launch)
        part_need = 0
        for (n_, k_) in ((3 * A, H), (H, A), (A, H), (Fd, H), (H, Fd), (cfg.action_dim, H)):
            part_need = max(part_need, self._part_splits(M, n_, k_) * M * n_)
        self.part = torch.zeros(part_need, dtype=torch.float32, device=dev)
        # Above 64 rows the cross-attention query arrives normalised from its row kernel and every
        # batch row attends to the same (batch-shared) context K/V: the batch rows' queries are one
        # sequence of B*S queries per head, the long-sequence kernel's shape (no key splits, no
        # combine).  Otherwise key splits (1: a single launch, no combine) as the library advises.
        self.cross_flat = batch * seq_len > 64 and cfg.attn_head_dim in (64, 128) and batch > 1
        self.kv_splits = 1 if self.cross_flat else int(self.lib.fam_attention_key_splits(
            batch, cfg.num_heads, seq_len, ctx_len, cfg.attn_head_dim))
        nq = batch * cfg.num_heads * seq_len
        self.apart_o = torch.zeros(self.kv_splits * nq * cfg.attn_head_dim, dtype=torch.float32, device=dev)
        self.apart_ml = torch.zeros(self.kv_splits * nq * 2, dtype=torch.float32, device=dev)

        self._descs: list = []   # keeps ctypes descriptors alive
        self.tiny = None
        if mode == "denoise" and tiny is not False:
            self.tiny = self._tiny_setup(params, tiny_slice)
            if self.tiny is None and tiny:
                raise ValueError("tiny=True but fam_tiny_expert does not cover this shape: "
                                 + self.lib.fam_last_error().decode(errors="replace"))
        self.plan = self._build_plan()
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ plan building
    def _gemm(self, name, a, w, bias, out, *, prologue=_capi.FAM_PRO_NONE, pro_w=None, pro_b=None,
              shift=None, scale=None, act=_capi.FAM_ACT_NONE, res=None, gate=None, gate_strides=(0, 0, 1),
              rows_per_batch=None, M=None, K=None, lda=None, ldo=None, ldr=None, out_f32=False, ws=None):
        d = _capi.GemmDesc()
        Mv = a.shape[0] if M is None else M
        Kv = w.shape[1] if K is None else K
        d.a, d.lda = a.data_ptr(), (a.stride(0) if lda is None else lda)
        d.w, d.ldw = w.data_ptr(), w.stride(0)
        d.bias = bias.data_ptr() if bias is not None else None
        d.out, d.ldo = out.data_ptr(), (out.stride(0) if ldo is None else ldo)
        d.M, d.N, d.K = Mv, w.shape[0], Kv
        d.prologue = prologue
        d.pro_w = pro_w.data_ptr() if pro_w is not None else None
        d.pro_b = pro_b.data_ptr() if pro_b is not None else None
        d.pro_shift = shift.data_ptr() if shift is not None else None
        d.pro_scale = scale.data_ptr() if scale is not None else None
        d.pro_mod_bs = d.pro_mod_rs = 0   # one modulation vector for every row (per-sample t)
        d.pro_eps = float(self.cfg.eps)
        d.act = act
        if res is not None:
            d.res, d.ldr = res.data_ptr(), (res.stride(0) if ldr is None else ldr)
        d.gate = gate.data_ptr() if gate is not None else None
        d.gate_bs, d.gate_rs, d.gate_ns = gate_strides
        d.rows_per_batch = rows_per_batch or max(Mv, 1)
        d.out_f32 = int(out_f32)
        self._descs.append(d)
        lib = self.lib
        ref = C.byref(d)
        if ws is not None:
            # fam_gemm_ws: the planner may split K over the workspace (its planes summed by a row
            # launch that also applies the epilogue)
            f, wsp, wsn = self.lib.fam_gemm_ws, ws.data_ptr(), ws.numel()

            def run(stream):
                rc = f(ref, wsp, wsn, stream)
                if rc != 0:
                    raise FamError(f"fam_gemm_ws[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        else:
            f = self.lib.fam_gemm

            def run(stream):
                rc = f(ref, stream)
                if rc != 0:
                    raise FamError(f"fam_gemm[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        N = d.N
        nbytes = 2 * (Mv * Kv + N * Kv + Mv * N) + (2 * N if bias is not None else 0)
        nbytes += 2 * Mv * N if res is not None else 0
        nbytes += 2 * N if gate is not None else 0
        nbytes += 4 * Kv if prologue != _capi.FAM_PRO_NONE else 0
        self.plan.add(name, run, "gemm", nbytes, 2 * Mv * N * Kv)

    def _launch(self, name, fname, ref, kernel, nbytes, flops=0):
        f, lib = getattr(self.lib, fname), self.lib

        def run(stream):
            rc = f(ref, stream)
            if rc != 0:
                raise FamError(f"{fname}[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.plan.add(name, run, kernel, nbytes, flops)

    def _part_splits(self, M, N, K):
        # up to 64 rows the weight-streaming split; above 144 the large-M kernel's planes (split
        # along K where the planes cost less than idle CUs); else (or off the large-M kernel's
        # shapes) the GEMM writes a single fp32 plane
        if M <= 64:
            return self.lib.fam_gemm_partial_splits(M, N, K)
        return (self.lib.fam_gemm_partial_splits(M, N, K) or 1) if M > 144 else 1

    def _gemm_partial(self, name, a, w):
        """Split-K partials of a [M, K] x w[N, K]^T into self.part; returns the split count."""
        M, K = a.shape[0], w.shape[1]
        N = w.shape[0]
        if M > 64 and not (M > 144 and self.lib.fam_gemm_partial_splits(M, N, K) > 0):
            self._gemm(name, a, w, None, self.part, ldo=N, out_f32=True)
            return 1
        splits = self._part_splits(M, N, K)
        args = (a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), self.part.data_ptr(), M, N, K)
        self.plan.add(name, _checked(self.lib, "fam_gemm_partial", *args), "gemm_partial",
                      2 * (M * K + N * K) + 4 * splits * M * N, 2 * M * N * K)
        return splits

    def _gemm_final(self, name, a, w, bias, out, act=_capi.FAM_ACT_NONE, sumsq=None):
        """Whole-K projection with its bias/activation epilogue (M <= 64), no partials."""
        M, K = a.shape[0], w.shape[1]
        N = w.shape[0]
        args = (a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), bias.data_ptr() if bias is not None else None,
                act, out.data_ptr(), out.stride(0), sumsq.data_ptr() if sumsq is not None else None, M, N, K)
        self.plan.add(name, _checked(self.lib, "fam_gemm_final", *args), "gemm_final",
                      2 * (M * K + N * K + M * N), 2 * M * N * K)

    def _rowop(self, name, *, N, splits=1, src=_capi.FAM_ROWSRC_PARTIALS, x_in=None, w_in=None, bias=None,
               act=_capi.FAM_ACT_NONE, res=None, gate=None, gate_strides=(0, 0, 1), out=None, out_f32=False,
               norm=_capi.FAM_ROWNORM_NONE, ln_w=None, ln_b=None, shift=None, scale=None, segs=(), rope=False,
               nout=None):
        cfg = self.cfg
        M = self.B * self.S
        d = _capi.RowopDesc()
        d.src = src
        if src == _capi.FAM_ROWSRC_PARTIALS:
            d.partials, d.splits, d.split_stride = self.part.data_ptr(), splits, M * N
        else:
            d.x_in, d.ldx, d.k_in, d.w_in = x_in.data_ptr(), x_in.stride(0), w_in.shape[1], w_in.data_ptr()
        d.M, d.N = M, N
        d.bias = bias.data_ptr() if bias is not None else None
        d.act = act
        if res is not None:
            d.res, d.ldr = res.data_ptr(), res.stride(0)
        d.gate = gate.data_ptr() if gate is not None else None
        d.gate_bs, d.gate_rs, d.gate_ns = gate_strides
        d.rows_per_batch = self.S
        d.out, d.ldo, d.out_f32 = out.data_ptr(), out.stride(0), int(out_f32)
        d.norm, d.eps = norm, float(cfg.eps)
        d.ln_weight = ln_w.data_ptr() if ln_w is not None else None
        d.ln_bias = ln_b.data_ptr() if ln_b is not None else None
        d.shift = shift.data_ptr() if shift is not None else None
        d.scale = scale.data_ptr() if scale is not None else None
        d.mod_bs = d.mod_rs = 0   # one modulation vector for every row (the timestep is shared)
        d.nseg = len(segs)
        for g_, (c0, wt) in enumerate(segs):
            d.seg_col0[g_], d.seg_weight[g_] = c0, wt.data_ptr()
        d.seg_width = cfg.attn_dim
        if rope:
            d.rope_cos, d.rope_sin = self.rope_cos.data_ptr(), self.rope_sin.data_ptr()
            d.rope_row_stride, d.rope_elem_stride = cfg.attn_head_dim // 2, 1
            d.head_dim, d.seq_len = cfg.attn_head_dim, self.S
        if nout is not None:
            d.nout, d.ldn = nout.data_ptr(), nout.stride(0)
        self._descs.append(d)
        nbytes = (4 * splits * M * N if src == _capi.FAM_ROWSRC_PARTIALS else 4 * M * d.k_in) + 2 * M * N
        nbytes += (2 * M * N if res is not None else 0) + (2 * M * N if nout is not None else 0)
        self._launch(name, "fam_rowop", C.byref(d), "rowop", nbytes)

    def _attn_desc(self, q, q_bs, q_rs, k, k_bs, k_rs, v, v_bs, v_rs, out, sq, sk, splits=1, qk_norm=None,
                   batch=None):
        cfg = self.cfg
        Dh = cfg.attn_head_dim
        d = _capi.AttnDesc()
        d.q, d.q_bs, d.q_rs, d.q_hs = q, q_bs, q_rs, Dh
        d.k0, d.k0_bs, d.k0_rs, d.k0_hs = k, k_bs, k_rs, Dh
        d.v0, d.v0_bs, d.v0_rs, d.v0_hs = v, v_bs, v_rs, Dh
        d.o, d.o_bs, d.o_rs, d.o_hs = out.data_ptr(), sq * cfg.attn_dim, cfg.attn_dim, Dh
        d.batch, d.heads, d.sq, d.sk0, d.sk1, d.head_dim = self.B if batch is None else batch, cfg.num_heads, sq, sk, 0, Dh
        d.scale = 1.0 / math.sqrt(Dh)
        d.mask_kind = _capi.FAM_MASK_NONE
        d.num_splits = splits
        if splits > 1:
            d.part_o, d.part_ml = self.apart_o.data_ptr(), self.apart_ml.data_ptr()
        if qk_norm is not None:
            # q (and k) arrive raw from fam_gemm_final; RMSNorm (+ RoPE) happens on load
            n = qk_norm
            d.qk_norm = 1
            d.q_sumsq = n["ss"].data_ptr()
            d.k_sumsq = n["ss"].data_ptr() if n.get("k_w") is not None else None
            d.ss_row_stride, d.ss_batch_rows = n["ss"].stride(0), sq
            d.q_group0, d.k_group0, d.norm_width = 0, n.get("k_group0", 0), cfg.attn_dim
            d.q_norm_w = n["q_w"].data_ptr()
            d.k_norm_w = n["k_w"].data_ptr() if n.get("k_w") is not None else None
            d.norm_eps = float(cfg.eps)
            if n.get("rope"):
                d.rope_cos, d.rope_sin, d.rope_row_stride = self.rope_cos.data_ptr(), self.rope_sin.data_ptr(), Dh // 2
        self._descs.append(d)
        return d

    def _attn(self, name, q, q_bs, q_rs, k, k_bs, k_rs, v, v_bs, v_rs, out, sq, sk, splits=1, qk_norm=None,
              batch=None):
        cfg = self.cfg
        Dh = cfg.attn_head_dim
        B = self.B if batch is None else batch
        d = self._attn_desc(q, q_bs, q_rs, k, k_bs, k_rs, v, v_bs, v_rs, out, sq, sk, splits, qk_norm, batch=B)
        A = cfg.attn_dim
        kv_batches = B if k_bs else 1   # a batch-broadcast context is read once
        nbytes = 2 * (2 * B * sq * A + 2 * kv_batches * sk * A)
        self._launch(name, "fam_attention", C.byref(d), "attention", nbytes,
                     4 * B * cfg.num_heads * sq * sk * Dh)
        if splits > 1:
            nq = B * cfg.num_heads * sq
            self._launch(name + "_combine", "fam_attention_combine", C.byref(d), "attn_combine",
                         splits * nq * (4 * Dh + 8) + 2 * nq * Dh)

    def _attn_joint(self, name, l, out):
        """MoT self-attention of the action rows over [video K/V cache of layer l ; action K/V]
        with the action rows of the joint mask (FB/mot.py:446-478): two key segments read in
        place, no concat."""
        cfg = self.cfg
        A, Dh, S, Sv = cfg.attn_dim, cfg.attn_head_dim, self.S, self.Sv
        qkvp = self.qkv.data_ptr()
        d = _capi.AttnDesc()
        d.q, d.q_bs, d.q_rs, d.q_hs = qkvp, S * 3 * A, 3 * A, Dh
        vk, vv = self.video_kv[l] if self.video_kv is not None else (self.video_k[l], self.video_v[l])
        d.k0, d.k0_bs, d.k0_rs, d.k0_hs = vk.data_ptr(), vk.stride(0), vk.stride(1), Dh
        d.v0, d.v0_bs, d.v0_rs, d.v0_hs = vv.data_ptr(), vv.stride(0), vv.stride(1), Dh
        d.k1, d.k1_bs, d.k1_rs, d.k1_hs = qkvp + 2 * A, S * 3 * A, 3 * A, Dh
        d.v1, d.v1_bs, d.v1_rs, d.v1_hs = qkvp + 4 * A, S * 3 * A, 3 * A, Dh
        d.o, d.o_bs, d.o_rs, d.o_hs = out.data_ptr(), S * A, A, Dh
        d.batch, d.heads, d.sq, d.sk0, d.sk1, d.head_dim = self.B, cfg.num_heads, S, Sv, S, Dh
        d.scale = 1.0 / math.sqrt(Dh)
        if self.video_mask is not None:
            d.mask, d.mask_kind = self.video_mask.data_ptr(), _capi.FAM_MASK_BOOL
            d.mask_bs, d.mask_hs, d.mask_qs = 0, 0, Sv + S
        d.num_splits = 1
        self._descs.append(d)
        nbytes = 2 * (2 * self.B * S * A + 2 * self.B * (Sv + S) * A)
        self._launch(name, "fam_attention", C.byref(d), "attention", nbytes,
                     4 * self.B * cfg.num_heads * S * (Sv + S) * Dh)

    # ------------------------------------------------------------------ tiny-hidden path
    def _tiny_setup(self, params: Dict[str, torch.Tensor], slice_: int):
        """Layer-major weight stacks, the Gram matrices of the q / k / cross-q projections and
        the state buffers of fam_tiny_expert; None when the library does not cover the shape
        (checked with an empty phase range, which validates without launching)."""
        cfg, dev = self.cfg, self.device
        H, A, Fd, L, Dh = cfg.hidden_dim, cfg.attn_dim, cfg.ffn_dim, cfg.num_layers, cfg.attn_head_dim
        B, S, T = self.B, self.S, self.T
        if H != 32:
            return None
        W = slice_ if slice_ > 0 else (A if A <= 128 else 128)
        if W <= 0 or A % W:
            return None
        G = A // W

        def stack(fmt):
            return torch.stack([params[fmt.format(i)].to(torch.float32) for i in range(L)]).to(
                device=dev, dtype=_BF16).contiguous()

        tw = {}
        tw["qkv_w"] = torch.stack([torch.cat([params[f"blocks.{i}.self_attn.{n}.weight"].to(torch.float32)
                                              for n in "qkv"]) for i in range(L)]).to(device=dev, dtype=_BF16).contiguous()
        tw["qkv_b"] = torch.stack([torch.cat([params[f"blocks.{i}.self_attn.{n}.bias"].to(torch.float32)
                                              for n in "qkv"]) for i in range(L)]).to(device=dev, dtype=_BF16).contiguous()
        for key, fmt in (("nq_w", "blocks.{}.self_attn.norm_q.weight"), ("nk_w", "blocks.{}.self_attn.norm_k.weight"),
                         ("o_w", "blocks.{}.self_attn.o.weight"), ("o_b", "blocks.{}.self_attn.o.bias"),
                         ("n3_w", "blocks.{}.norm3.weight"), ("n3_b", "blocks.{}.norm3.bias"),
                         ("cq_w", "blocks.{}.cross_attn.q.weight"), ("cq_b", "blocks.{}.cross_attn.q.bias"),
                         ("cnq_w", "blocks.{}.cross_attn.norm_q.weight"), ("co_w", "blocks.{}.cross_attn.o.weight"),
                         ("co_b", "blocks.{}.cross_attn.o.bias"), ("ff0_w", "blocks.{}.ffn.0.weight"),
                         ("ff0_b", "blocks.{}.ffn.0.bias"), ("ff2_w", "blocks.{}.ffn.2.weight"),
                         ("ff2_b", "blocks.{}.ffn.2.bias")):
            tw[key] = stack(fmt)
        # a slice wider than the 32-wide rows attends in the space of the context rows: the cross
        # key weight transposed, the value weight and both biases per layer
        folded = W > H
        if folded:
            tw["ck_wt"] = torch.stack([params[f"blocks.{i}.cross_attn.k.weight"].to(torch.float32).t()
                                       for i in range(L)]).to(device=dev, dtype=_BF16).contiguous()
            for key, fmt in (("ck_b", "blocks.{}.cross_attn.k.bias"), ("cv_w", "blocks.{}.cross_attn.v.weight"),
                             ("cv_b", "blocks.{}.cross_attn.v.bias")):
                tw[key] = stack(fmt)
        # sum_j q_j^2 = h G h + 2 h.c + beta for q = h Wq^T + bq, from the bf16 weights in fp64:
        # G = Wq^T Wq as hi + lo bf16 parts, c = Wq^T bq, beta = |bq|^2 (self q, self k, cross q,
        # cross k)
        gram = torch.zeros(L, 4, 2, H, H, dtype=_BF16)
        gc = torch.zeros(L, 4, H, dtype=torch.float32)
        gb = torch.zeros(L, 4, dtype=torch.float32)
        qkw, qkb = tw["qkv_w"].cpu().double(), tw["qkv_b"].cpu().double()
        cqw, cqb = tw["cq_w"].cpu().double(), tw["cq_b"].cpu().double()
        ckw = torch.stack([params[f"blocks.{i}.cross_attn.k.weight"].to(torch.float32) for i in range(L)]).to(
            _BF16).double()
        ckb = torch.stack([params[f"blocks.{i}.cross_attn.k.bias"].to(torch.float32) for i in range(L)]).to(
            _BF16).double()
        for l in range(L):
            for j, (wm, bv) in enumerate(((qkw[l, :A], qkb[l, :A]), (qkw[l, A:2 * A], qkb[l, A:2 * A]),
                                          (cqw[l], cqb[l]), (ckw[l], ckb[l]))):
                g = wm.t() @ wm
                hi = g.to(_BF16)
                gram[l, j, 0], gram[l, j, 1] = hi, (g - hi.double()).to(_BF16)
                gc[l, j] = (wm.t() @ bv).float()
                gb[l, j] = float(bv @ bv)
        tw["gram"], tw["gram_c"], tw["gram_b"] = gram.to(dev), gc.to(dev), gb.to(dev)
        tw["nk_stack"] = stack("blocks.{}.cross_attn.norm_k.weight")
        # state
        f32 = dict(dtype=torch.float32, device=dev)
        tw["lat"] = torch.zeros(2, B, S, cfg.action_dim, **f32)
        tw["xa"] = torch.zeros(B, S, H, **f32)
        tw["xb"] = torch.zeros(B, S, H, **f32)
        tw["part_s"] = torch.zeros(B, G, S, H, **f32)
        tw["part_c"] = torch.zeros(B, G, S, H, **f32)
        d = _capi.TinyDesc()
        d.batch, d.seq, d.hidden, d.heads, d.head_dim = B, S, H, cfg.num_heads, Dh
        d.ffn, d.action_dim, d.layers, d.steps = Fd, cfg.action_dim, L, T
        d.video_len, d.ctx_len, d.slice = self.Sv, self.Lc, W
        d.eps, d.scale = float(cfg.eps), 1.0 / math.sqrt(Dh)
        d.noise, d.mods, d.deltas = self.noise_in.data_ptr(), self.mods.data_ptr(), self.deltas.data_ptr()
        d.rope_cos, d.rope_sin = self.rope_cos.data_ptr(), self.rope_sin.data_ptr()
        if folded:
            tw["ctx_rs"] = torch.zeros(L, (self.Lc + 31) // 32 * 32, **f32)
            d.ctx_emb, d.ctx_emb_ld = self.ctx_emb_pad.data_ptr(), self.ctx_emb_pad.stride(0)
            for key in ("ck_wt", "ck_b", "cv_w", "cv_b", "ctx_rs"):
                setattr(d, key, tw[key].data_ptr())
            d.cnk_w = tw["nk_stack"].data_ptr()
        else:
            d.ctxkv, d.ctx_ld = self.ctxkv.data_ptr(), L * 2 * A
        if self.Sv > 0:
            kvs = (self.video_kv if self.video_kv is not None else
                   [(self.video_k[l], self.video_v[l]) for l in range(L)])
            bs, rs = kvs[0][0].stride(0), kvs[0][0].stride(1)
            if any(t_.stride(0) != bs or t_.stride(1) != rs for kv in kvs for t_ in kv):
                return None
            tw["vk_tab"] = torch.tensor([kv[0].data_ptr() for kv in kvs], dtype=torch.int64, device=dev)
            tw["vv_tab"] = torch.tensor([kv[1].data_ptr() for kv in kvs], dtype=torch.int64, device=dev)
            d.video_k, d.video_v = tw["vk_tab"].data_ptr(), tw["vv_tab"].data_ptr()
            d.video_bs, d.video_rs = bs, rs
            if self.video_mask is not None:
                d.video_mask, d.mask_rs = self.video_mask.data_ptr(), self.Sv + S
        w = self.w
        d.enc_w, d.enc_b, d.head_w, d.head_b = (w["enc_w"].data_ptr(), w["enc_b"].data_ptr(), w["head_w"].data_ptr(),
                                                w["head_b"].data_ptr())
        for key in ("qkv_w", "qkv_b", "nq_w", "nk_w", "o_w", "o_b", "n3_w", "n3_b", "cq_w", "cq_b", "cnq_w", "co_w",
                    "co_b", "ff0_w", "ff0_b", "ff2_w", "ff2_b", "gram", "gram_c", "gram_b", "lat", "xa", "xb",
                    "part_s", "part_c"):
            setattr(d, key, tw[key].data_ptr())
        d.out = self.latents.data_ptr()
        # context splits of the cross phases (one 32-wide slice, few batch rows): the library's choice
        ks = self.lib.fam_tiny_key_splits(C.byref(d))
        if ks < 0:
            return None
        if ks > 1:
            tw["part_x"] = torch.zeros(B * ks * 32 * (W + 4), **f32)
            d.part_x = tw["part_x"].data_ptr()
        tw["KS"] = ks
        if self.lib.fam_tiny_expert(C.byref(d), 0, 0, None) != 0:
            return None
        tw["desc"] = d
        tw["G"], tw["folded"] = G, folded
        return tw

    def _tiny_plan(self, plan: _Plan) -> None:
        """The blocks, head and Euler updates of every step as fam_tiny_expert phases: per block
        step a self phase and a cross phase, then the final phase (last FFN, head, last update)."""
        cfg, tw = self.cfg, self.tiny
        H, A, L, T, S, B = cfg.hidden_dim, cfg.attn_dim, cfg.num_layers, self.T, self.S, self.B
        G, Sv, Lc, Fd = tw["G"], self.Sv, self.Lc, cfg.ffn_dim
        ref = C.byref(tw["desc"])
        f, lib = self.lib.fam_tiny_expert, self.lib
        rows = B * S

        def phase(p):
            def run(stream):
                rc = f(ref, p, p + 1, stream)
                if rc != 0:
                    raise FamError(f"fam_tiny_expert[{p}]", rc, lib.fam_last_error().decode(errors="replace"))
            return run
        # algorithmic bytes: the weights a phase streams once (bf16), the K/V (or the context rows
        # and the keys' factors) it reads, the partials
        w_self = 2 * (3 * A * H + 2 * A + H * A) + 2 * (2 * Fd * H)
        w_cross = 2 * (A * H + A + H * A)
        if tw["folded"]:
            w_cross += 2 * (2 * A * H + 3 * A) + 2 * Lc * H + 4 * Lc
        else:
            w_cross += 2 * 2 * Lc * A
        for t in range(T):
            for l in range(L):
                p = 2 * (t * L + l)
                plan.add(f"s{t}.b{l}.tiny_self", phase(p), "tiny_self",
                         w_self + 2 * 2 * B * Sv * A + 4 * 2 * G * rows * H, 4 * B * cfg.num_heads * S * (Sv + S) * cfg.attn_head_dim)
                plan.add(f"s{t}.b{l}.tiny_cross", phase(p + 1), "tiny_cross",
                         w_cross + 4 * 2 * G * rows * H, 4 * B * cfg.num_heads * S * Lc * cfg.attn_head_dim)
        plan.add("tiny_final", phase(2 * L * T), "tiny_final", 2 * (2 * Fd * H) + 4 * G * rows * H)

    def set_video_kv(self, keys, values) -> None:
        """Copy the per-layer cached video K/V (each [B, Sv, A] or [Sv, A], already normalised
        and rotated as the video expert's prefill leaves them) into the static buffers."""
        if self.Sv == 0:
            raise ValueError("this model was built without a video prefix (video_len=0)")
        if self.video_kv is not None:
            raise ValueError("this model reads its video K/V in place (video_kv); there is no static copy")
        for l, (k, v) in enumerate(zip(keys, values)):
            self.video_k[l].copy_(k.reshape(self.video_k[l].shape) if k.dim() == 3 else k.expand_as(self.video_k[l]))
            self.video_v[l].copy_(v.reshape(self.video_v[l].shape) if v.dim() == 3 else v.expand_as(self.video_v[l]))

    def _build_plan(self) -> _Plan:
        cfg, lib = self.cfg, self.lib
        H, A, L, Dh, Fd = cfg.hidden_dim, cfg.attn_dim, cfg.num_layers, cfg.attn_head_dim, cfg.ffn_dim
        B, S, Lc, T = self.B, self.S, self.Lc, self.T
        M = B * S
        self.plan = plan = _Plan()
        w = self.w
        eps = float(cfg.eps)

        # -- input copy and per-call prologue
        if self.tiny is None:
            plan.add("latents<-noise", lambda s: self.latents.copy_(self.noise_in), "copy", 4 * self.latents.numel())
        plan.add("sinusoid", _checked(lib, "fam_sinusoid", self.timesteps.data_ptr(), self.t_emb.data_ptr(), T,
                                      cfg.freq_dim), "sinusoid", 2 * T * (1 + cfg.freq_dim))
        self._gemm("time_emb0", self.t_emb, w["te0_w"], w["te0_b"], self.t1, act=_capi.FAM_ACT_SILU)
        self._gemm("time_emb2", self.t1, w["te2_w"], w["te2_b"], self.t2, act=_capi.FAM_ACT_SILU)
        self._gemm("time_proj", self.t2, w["tp_w"], w["tp_b"], self.tmod)
        plan.add("modulation", _checked(lib, "fam_add_modulation", self.tmod.data_ptr(), w["mod"].data_ptr(),
                                        self.mods.data_ptr(), T, L, 6 * H), "modulation",
                 2 * 6 * H * (T + L + T * L))
        # the text embedding's first layer (ctx_len x H x text_dim: few output tiles, a long K) may
        # split K over a workspace
        nws = int(lib.fam_gemm_ws_floats(Lc, H, cfg.text_dim))
        self.ctx_ws = torch.empty(max(nws, 1), dtype=torch.float32, device=self.device) if nws > 0 else None
        self._gemm("ctx_emb0", self.context_in, w["txt0_w"], w["txt0_b"], self.ctx_h, act=_capi.FAM_ACT_GELU_TANH,
                   ws=self.ctx_ws)
        self._gemm("ctx_emb2", self.ctx_h_pad, w["txt2_w"], w["txt2_b"], self.ctx_emb)
        if self.tiny is not None and self.tiny["folded"]:
            # the tiny expert's wide slices attend in the space of the context rows: only the
            # keys' RMS factors are computed here (no context K/V)
            ref = C.byref(self.tiny["desc"])
            plan.add("tiny_context", _checked(lib, "fam_tiny_context", ref), "tiny_context",
                     2 * Lc * H + 4 * L * self.tiny["ctx_rs"].shape[1] + 2 * L * (2 * H * H + 4 * H + 4))
            self._tiny_plan(plan)
            return plan
        self._gemm("ctx_kv", self.ctx_emb_pad, w["ctxkv_w"], w["ctxkv_b"], self.ctxkv)
        kvp = self.ctxkv.data_ptr()
        # RMSNorm of every block's context keys in one launch: row (i, l) = ctxkv[i, 2 A l ..]
        w["nk_stack"] = torch.stack([w[f"ca_nk_w{l}"] for l in range(L)]).contiguous()
        plan.add("ctx_knorm", _checked(lib, "fam_rmsnorm_grouped", kvp, 2 * A, kvp, 2 * A, Lc * L, A,
                                       w["nk_stack"].data_ptr(), L, eps), "rmsnorm_rope", 2 * (2 * Lc * L * A + L * A))
        if self.tiny is not None:
            self._tiny_plan(plan)
            return plan

        lat = self.latents.view(M, cfg.action_dim)
        x, qkv, attn, qc, hid, h = self.x, self.qkv, self.attn, self.qc, self.hid, self.h
        qkvp = qkv.data_ptr()
        kvp = self.ctxkv.data_ptr()
        RMS, LN, ADALN = _capi.FAM_ROWNORM_RMS, _capi.FAM_ROWNORM_LAYERNORM, _capi.FAM_ROWNORM_ADALN

        # M <= 64 rows, Sq <= 32 and an RMS width the on-load normaliser supports: q/k projections
        # are single kernels and their norms run inside the attention kernels
        fused_qk = M <= 64 and S <= 32 and A % 1024 == 0 and Dh in (64, 128) and self.Sv == 0
        # the cross-attention query alone (also in MoT mode): raw projection + sums of squares,
        # normalised as the attention loads it (the short-context kernel takes widths <= 4096)
        fused_q = M <= 64 and S <= 32 and A % 1024 == 0 and Dh in (64, 128) and (Lc > 256 or A <= 4096)

        def mod(t, l, i):   # chunk i of (modulation + t_mod) of block l at step t: [H]
            return self.mods[t, l, i * H:(i + 1) * H]

        for t in range(T):
            # action encoder (7 -> H) + AdaLN1 of block 0, one row per workgroup
            self._rowop(f"s{t}.encoder", N=H, src=_capi.FAM_ROWSRC_SMALLK, x_in=lat, w_in=w["enc_w"],
                        bias=w["enc_b"], out=x, norm=ADALN, shift=mod(t, 0, 0), scale=mod(t, 0, 1), nout=h)
            for l in range(L):
                tag = f"s{t}.b{l}"
                if fused_qk:
                    # raw q, k, v in one kernel (+ per-row sums of squares); the attention
                    # kernel applies RMSNorm + RoPE to q and k as it loads them
                    self._gemm_final(tag + ".qkv", h, w[f"qkv_w{l}"], w[f"qkv_b{l}"], qkv, sumsq=self.ss_qkv)
                    qkn = dict(ss=self.ss_qkv, q_w=w[f"sa_norm_q_w{l}"], k_w=w[f"sa_norm_k_w{l}"], k_group0=A // 16,
                               rope=True)
                    self._attn(tag + ".self_attn", qkvp, S * 3 * A, 3 * A, qkvp + 2 * A, S * 3 * A, 3 * A,
                               qkvp + 4 * A, S * 3 * A, 3 * A, attn, S, S, qk_norm=qkn)
                else:
                    # q, k, v projection; RMSNorm + RoPE of q and k in the row kernel
                    sp = self._gemm_partial(tag + ".qkv", h, w[f"qkv_w{l}"])
                    self._rowop(tag + ".qkv_row", N=3 * A, splits=sp, bias=w[f"qkv_b{l}"], out=qkv, norm=RMS,
                                segs=((0, w[f"sa_norm_q_w{l}"]), (A, w[f"sa_norm_k_w{l}"])), rope=True, nout=qkv)
                    if self.Sv > 0:
                        self._attn_joint(tag + ".joint_attn", l, attn)
                    else:
                        self._attn(tag + ".self_attn", qkvp, S * 3 * A, 3 * A, qkvp + 2 * A, S * 3 * A, 3 * A,
                                   qkvp + 4 * A, S * 3 * A, 3 * A, attn, S, S)
                # o projection; x += gate_msa * o; LayerNorm3 (affine) for the cross-attention query
                sp = self._gemm_partial(tag + ".o", attn, w[f"sa_o_w{l}"])
                self._rowop(tag + ".o_row", N=H, splits=sp, bias=w[f"sa_o_b{l}"], res=x, gate=mod(t, l, 2), out=x,
                            norm=LN, ln_w=w[f"n3_w{l}"], ln_b=w[f"n3_b{l}"], nout=h)
                kb = kvp + 2 * (l * 2 * A)
                if fused_q:
                    # raw cross-attention query; its RMSNorm happens as the attention loads it
                    self._gemm_final(tag + ".cross_q", h, w[f"ca_q_w{l}"], w[f"ca_q_b{l}"], qc, sumsq=self.ss_q)
                    self._attn(tag + ".cross_attn", qc.data_ptr(), S * A, A, kb, 0, L * 2 * A, kb + 2 * A, 0,
                               L * 2 * A, attn, S, Lc, splits=self.kv_splits,
                               qk_norm=dict(ss=self.ss_q, q_w=w[f"ca_nq_w{l}"]))
                else:
                    # cross-attention query + its RMSNorm
                    sp = self._gemm_partial(tag + ".cross_q", h, w[f"ca_q_w{l}"])
                    self._rowop(tag + ".cross_q_row", N=A, splits=sp, bias=w[f"ca_q_b{l}"], out=qc, norm=RMS,
                                segs=((0, w[f"ca_nq_w{l}"]),), nout=qc)
                    if self.cross_flat:
                        # the B*S normalised queries as one sequence over the shared context
                        self._attn(tag + ".cross_attn", qc.data_ptr(), 0, A, kb, 0, L * 2 * A, kb + 2 * A, 0,
                                   L * 2 * A, attn, B * S, Lc, batch=1)
                    else:
                        self._attn(tag + ".cross_attn", qc.data_ptr(), S * A, A, kb, 0, L * 2 * A, kb + 2 * A, 0,
                                   L * 2 * A, attn, S, Lc, splits=self.kv_splits)
                # cross o projection; x += o; AdaLN2 for the FFN
                sp = self._gemm_partial(tag + ".cross_o", attn, w[f"ca_o_w{l}"])
                self._rowop(tag + ".cross_o_row", N=H, splits=sp, bias=w[f"ca_o_b{l}"], res=x, out=x, norm=ADALN,
                            shift=mod(t, l, 3), scale=mod(t, l, 4), nout=h)
                # FFN: up + GELU, down; x += gate_mlp * ffn; AdaLN1 of the next block
                if M <= 64:
                    self._gemm_final(tag + ".ffn_up", h, w[f"ff0_w{l}"], w[f"ff0_b{l}"], hid,
                                     act=_capi.FAM_ACT_GELU_TANH)
                else:
                    sp = self._gemm_partial(tag + ".ffn_up", h, w[f"ff0_w{l}"])
                    self._rowop(tag + ".ffn_up_row", N=Fd, splits=sp, bias=w[f"ff0_b{l}"],
                                act=_capi.FAM_ACT_GELU_TANH, out=hid)
                sp = self._gemm_partial(tag + ".ffn_down", hid, w[f"ff2_w{l}"])
                if l + 1 < L:
                    self._rowop(tag + ".ffn_down_row", N=H, splits=sp, bias=w[f"ff2_b{l}"], res=x, gate=mod(t, l, 5),
                                out=x, norm=ADALN, shift=mod(t, l + 1, 0), scale=mod(t, l + 1, 1), nout=h)
                else:
                    self._rowop(tag + ".ffn_down_row", N=H, splits=sp, bias=w[f"ff2_b{l}"], res=x, gate=mod(t, l, 5),
                                out=x)
            # head; the row kernel's epilogue is the Euler update of the fp32 latents
            sp = self._gemm_partial(f"s{t}.head", x, w["head_w"])
            if self.mode == "forward":
                self._rowop(f"s{t}.head_row", N=cfg.action_dim, splits=sp, bias=w["head_b"], out=self.head_out)
            else:
                self._rowop(f"s{t}.head_euler", N=cfg.action_dim, splits=sp, bias=w["head_b"], res=lat,
                            gate=self.deltas[t:t + 1], gate_strides=(0, 0, 0), out=lat, out_f32=True)
        return plan

    # ------------------------------------------------------------------ execution
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def set_inputs(self, noise: torch.Tensor, context: torch.Tensor) -> None:
        """Copy one call's inputs into the static input buffers (noise [B,S,action_dim],
        context [L, text_dim] or [1, L, text_dim])."""
        self.noise_in.copy_(noise.reshape(self.noise_in.shape))
        self.context_in.copy_(context.reshape(self.context_in.shape))

    def run(self) -> None:
        """Enqueue one policy call on the current stream (graph replay if captured)."""
        if self.graph is not None:
            self.graph.replay()
        else:
            self.plan.run(self._stream())

    def capture(self, warmup: int = 1) -> None:
        """Capture the whole policy call into one HIP graph (kernel and copy nodes only)."""
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self.plan.run(s.cuda_stream)
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.plan.run(self._stream())
        self.graph = g

    def forward(self, action_tokens: torch.Tensor, timestep: float, context: torch.Tensor) -> torch.Tensor:
        """One ActionDiT.forward (mode='forward'): head output [B, S, action_dim] for the given
        noisy action tokens, timestep (rounded to bf16 as the reference's bf16 timestep) and context."""
        if self.mode != "forward":
            raise RuntimeError("forward() needs mode='forward'")
        self.timesteps.fill_(float(timestep))
        self.set_inputs(action_tokens, context)
        self.run()
        return self.head_out.view(self.B, self.S, self.cfg.action_dim).clone()

    def infer(self, noise: torch.Tensor, context: torch.Tensor) -> torch.Tensor:
        """One policy call: returns the denoised chunk [B, S, action_dim] (fp32, a copy; the
        reference returns its bf16 chunk converted to fp32, FB/fastwam.py:1071-1073)."""
        self.set_inputs(noise, context)
        self.run()
        return self.latents.clone()

    @property
    def num_launches(self) -> int:
        return len(self.plan.steps)

"""The Wan2.2 VAE (VAE38) encoder on the policy call's first frame, on the library.

FastWAM.infer_action encodes the first frame of the observation (FB/fastwam.py:256-268) with
VideoVAE38_.encode (FB/wan_video_vae.py:1299-1323): patchify 2x2, Encoder3d_38 (:619-732) on
the first chunk, conv1, mu = the first z_dim channels, (mu - mean) / std.  On a single frame
with an empty feature cache every CausalConv3d sees two zero frames in front of the frame, so
it is a 2-D convolution with its last temporal tap, and the downsample3d time_conv (which waits
for a second chunk, :162-167) does not run.

Layout: activations are channels-last rows, one per pixel ([h*w, C] bf16).  A 1x1 convolution
is one GEMM over the rows; a 3x3 convolution is fam_im2col3x3 (the pixel's neighbourhood, taps
outermost, zero-padded to a multiple of 64 columns) followed by a GEMM with the weight laid out
the same way; biases, the residual adds and the Down_ResidualBlock shortcut are GEMM epilogues.
The GEMMs go through fam_gemm_ws with one shared fp32 workspace, so the deep levels (392 to
1568 pixels, K up to 5760) split K over workgroups instead of leaving most CUs idle.  The middle AttentionBlock (one head, C = 640 wide, h*w tokens) is two fam_gemm
products around fam_softmax_rows: S = q k^T, P = softmax(S / sqrt(C)), O = P v0 + b_v, where
v0^T = W_v y^T is computed directly in the transposed layout the second product reads (the rows
of P sum to one, so the value bias moves after the product).

Every buffer is allocated once at construction (one image size per object); `capture()` records
the whole encode as one HIP graph.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from . import _capi

_BF16 = torch.bfloat16


@dataclass
class WanVaeConfig:
    """Encoder shape of WanVideoVAE38 (FB/wan_video_vae.py:1272-1295, :1355-1384)."""
    dim: int = 160
    z_dim: int = 48
    dim_mult: Tuple[int, ...] = (1, 2, 4, 4)
    num_res_blocks: int = 2
    temporal_downsample: Tuple[bool, ...] = (False, True, True)

    def dims(self) -> List[int]:
        return [self.dim * u for u in (1,) + tuple(self.dim_mult)]


# WanVideoVAE38's latent statistics (FB/wan_video_vae.py:1359-1378): mean, std per channel
WAN22_LATENT_MEAN = (
    -0.2289, -0.0052, -0.1323, -0.2339, -0.2799, 0.0174, 0.1838, 0.1557, -0.1382, 0.0542, 0.2813, 0.0891,
    0.1570, -0.0098, 0.0375, -0.1825, -0.2246, -0.1207, -0.0698, 0.5109, 0.2665, -0.2108, -0.2158, 0.2502,
    -0.2055, -0.0322, 0.1109, 0.1567, -0.0729, 0.0899, -0.2799, -0.1230, -0.0313, -0.1649, 0.0117, 0.0723,
    -0.2839, -0.2083, -0.0520, 0.3748, 0.0152, 0.1957, 0.1433, -0.2944, 0.3573, -0.0548, -0.1681, -0.0667)
WAN22_LATENT_STD = (
    0.4765, 1.0364, 0.4514, 1.1677, 0.5313, 0.4990, 0.4818, 0.5013, 0.8158, 1.0344, 0.5894, 1.0901,
    0.6885, 0.6165, 0.8454, 0.4978, 0.5759, 0.3523, 0.7135, 0.6804, 0.5833, 1.4146, 0.8986, 0.5659,
    0.7069, 0.5338, 0.4889, 0.4917, 0.4069, 0.4999, 0.6866, 0.4093, 0.5709, 0.6065, 0.6415, 0.4944,
    0.5726, 1.2042, 0.5458, 1.6887, 0.3971, 1.0600, 0.3943, 0.5537, 0.5444, 0.4089, 0.7468, 0.7744)


def _kpad(n: int) -> int:
    return (n + 63) // 64 * 64


def encoder_param_shapes(cfg: WanVaeConfig) -> Dict[str, Tuple[int, ...]]:
    """The state-dict entries the first-frame encode reads (reference names, VideoVAE38_ :1272-1295)."""
    d = cfg.dims()
    s = {"encoder.conv1.weight": (d[0], 12, 3, 3, 3), "encoder.conv1.bias": (d[0],)}

    def res(pre, ci, co):
        s.update({pre + "residual.0.gamma": (ci, 1, 1, 1), pre + "residual.2.weight": (co, ci, 3, 3, 3),
                  pre + "residual.2.bias": (co,), pre + "residual.3.gamma": (co, 1, 1, 1),
                  pre + "residual.6.weight": (co, co, 3, 3, 3), pre + "residual.6.bias": (co,)})
        if ci != co:
            s.update({pre + "shortcut.weight": (co, ci, 1, 1, 1), pre + "shortcut.bias": (co,)})

    for i, (ci, co) in enumerate(zip(d[:-1], d[1:])):
        pre = f"encoder.downsamples.{i}.downsamples."
        for j in range(cfg.num_res_blocks):
            res(f"{pre}{j}.", ci if j == 0 else co, co)
        if i != len(cfg.dim_mult) - 1:
            s.update({f"{pre}{cfg.num_res_blocks}.resample.1.weight": (co, co, 3, 3),
                      f"{pre}{cfg.num_res_blocks}.resample.1.bias": (co,)})
    c = d[-1]
    res("encoder.middle.0.", c, c)
    s.update({"encoder.middle.1.norm.gamma": (c, 1, 1), "encoder.middle.1.to_qkv.weight": (3 * c, c, 1, 1),
              "encoder.middle.1.to_qkv.bias": (3 * c,), "encoder.middle.1.proj.weight": (c, c, 1, 1),
              "encoder.middle.1.proj.bias": (c,)})
    res("encoder.middle.2.", c, c)
    s.update({"encoder.head.0.gamma": (c, 1, 1, 1), "encoder.head.2.weight": (2 * cfg.z_dim, c, 3, 3, 3),
              "encoder.head.2.bias": (2 * cfg.z_dim,), "conv1.weight": (2 * cfg.z_dim, 2 * cfg.z_dim, 1, 1, 1),
              "conv1.bias": (2 * cfg.z_dim,)})
    return s


class FusedWanVAEEncoder:
    """VideoVAE38_.encode of one image [1, 3, H, W] (H, W multiples of 16) -> latent
    [1, z_dim, 1, H/16, W/16], bf16.

    params: the VAE's state dict under the reference's names ("encoder.*", "conv1.*"; the
    decoder's entries are ignored).  mean / std: the latent statistics (WanVideoVAE38.scale);
    defaults are the published Wan2.2 ones when z_dim is 48.
    """

    def __init__(self, cfg: WanVaeConfig, params: Dict[str, torch.Tensor], *, height: int, width: int,
                 mean: Optional[torch.Tensor] = None, std: Optional[torch.Tensor] = None, device="cuda"):
        if height % 16 or width % 16 or height < 16 or width < 16:
            raise ValueError(f"image size ({height}, {width}) must be positive multiples of 16")
        dev = torch.device(device)
        self.cfg, self.device, self.H, self.W = cfg, dev, height, width
        self.lib = lib = _capi.load()
        d = cfg.dims()
        z = cfg.z_dim
        if mean is None or std is None:
            if z != len(WAN22_LATENT_MEAN):
                raise ValueError("mean / std required for z_dim != 48")
            mean, std = torch.tensor(WAN22_LATENT_MEAN), torch.tensor(WAN22_LATENT_STD)
        self.mean = mean.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        self.inv_std = (1.0 / std.to(dtype=torch.float64)).to(device=dev, dtype=torch.float32).reshape(-1).contiguous()

        def P(n):
            if n not in params:
                raise KeyError(f"missing VAE parameter {n}")
            return params[n].to(device=dev)

        def conv3(wn, bn):
            # [Co, Ci, (3,) 3, 3] -> last temporal tap -> [Co, (kh, kw, Ci)] zero-padded to kpad
            w = P(wn).float()
            if w.dim() == 5:
                w = w[:, :, -1]
            co, ci = w.shape[:2]
            w = w.permute(0, 2, 3, 1).reshape(co, 9 * ci)
            out = torch.zeros(co, _kpad(9 * ci), dtype=_BF16, device=dev)
            out[:, :9 * ci] = w.to(_BF16)
            return out.contiguous(), P(bn).to(_BF16).contiguous()

        def conv1x1(wn, bn, rows=None):
            w = P(wn).float().reshape(P(wn).shape[0], -1)
            b = P(bn)
            if rows is not None:
                w, b = w[rows], b[rows]
            return w.to(_BF16).contiguous(), b.to(_BF16).contiguous()

        def gamma(n):
            return P(n).reshape(-1).to(_BF16).contiguous()

        self.steps: List = []
        self.meta: List[dict] = []
        self._descs: List = []
        self._keep: List[torch.Tensor] = []
        # channels-last stage outputs ([h*w, C] views), valid after a run
        self.stages: Dict[str, torch.Tensor] = {}
        z2 = self._buf

        h, w = height // 2, width // 2
        self.img = z2(3, height, width)
        a0 = z2(h * w, 128)
        self._add("patch_im2col", "fam_vae_patch_im2col", (self.img.data_ptr(), height, width, a0.data_ptr(), 128),
                  "im2col", 2 * (self.img.numel() + a0.numel()))
        wc, bc = conv3("encoder.conv1.weight", "encoder.conv1.bias")
        x = z2(h * w, d[0])
        self._gemm("conv1", a0, wc, bc, x)
        self.stages["conv1"] = x

        nlev = len(cfg.dim_mult)
        for i, (ci, co) in enumerate(zip(d[:-1], d[1:])):
            pre = f"encoder.downsamples.{i}.downsamples."
            x_copy = x
            down = i != nlev - 1
            t_down = cfg.temporal_downsample[i] if i < len(cfg.temporal_downsample) else False
            for j in range(cfg.num_res_blocks):
                last_plain = (not down) and j == cfg.num_res_blocks - 1
                x = self._res_block(f"{pre}{j}.", x, h, w, ci if j == 0 else co, co, P, conv3, conv1x1, gamma,
                                    level_input=x_copy if last_plain else None, level_cin=ci)
            if down:
                avg = z2((h // 2) * (w // 2), co)
                self._add(f"l{i}.avgdown", "fam_vae_avgdown",
                          (x_copy.data_ptr(), x_copy.stride(0), h, w, ci, co, 2 if t_down else 1, 2, None, 0,
                           avg.data_ptr(), co), "avgdown", 2 * (x_copy.numel() + avg.numel()))
                self.stages[f"l{i}.avg"] = avg
                a = self._im2col(f"l{i}.down", x, h, w, co, 2)
                wr, br = conv3(f"{pre}{cfg.num_res_blocks}.resample.1.weight", f"{pre}{cfg.num_res_blocks}.resample.1.bias")
                h, w = h // 2, w // 2
                xn = z2(h * w, co)
                self._gemm(f"l{i}.down", a, wr, br, xn, res=avg)
                x = xn
            self.stages[f"level{i}"] = x

        c = d[-1]
        x = self.stages["middle0"] = self._res_block("encoder.middle.0.", x, h, w, c, c, P, conv3, conv1x1, gamma)
        x = self.stages["attention"] = self._attention("encoder.middle.1.", x, h * w, c, P, conv1x1, gamma)
        x = self.stages["middle2"] = self._res_block("encoder.middle.2.", x, h, w, c, c, P, conv3, conv1x1, gamma)
        t = z2(h * w, c)
        self._add("head.norm", "fam_chan_rmsnorm", (x.data_ptr(), c, h * w, c, self._k(gamma("encoder.head.0.gamma")),
                                                     _capi.FAM_ACT_SILU, t.data_ptr(), c), "norm", 4 * x.numel())
        a = self._im2col("head", t, h, w, c, 1)
        wh, bh = conv3("encoder.head.2.weight", "encoder.head.2.bias")
        hz = z2(h * w, 2 * z)
        self._gemm("head", a, wh, bh, hz)
        self.stages["head"] = hz
        wmu, bmu = conv1x1("conv1.weight", "conv1.bias", rows=slice(0, z))
        mu = z2(h * w, z)
        self._gemm("mu", hz, wmu, bmu, mu)
        self.out = z2(1, z, 1, h, w)
        self._add("normalise", "fam_chan_affine_nchw", (mu.data_ptr(), z, h * w, z, self.mean.data_ptr(),
                                                        self.inv_std.data_ptr(), self.out.data_ptr()),
                  "affine", 4 * mu.numel())
        self.latent_hw = (h, w)
        # one fp32 workspace for the split-K products (the deep levels: few pixels, long K)
        wsf = max([lib.fam_gemm_ws_floats(d.M, d.N, d.K) for d in self._descs] + [0])
        self.ws = torch.empty(max(wsf, 4), dtype=torch.float32, device=dev)
        self._ws_args = (self.ws.data_ptr(), wsf)
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    # ------------------------------------------------------------------ plan building
    def _buf(self, *shape, dtype=_BF16) -> torch.Tensor:
        """A zero-filled device buffer that lives as long as the plan (the launches hold raw
        pointers into it)."""
        t = torch.zeros(*shape, dtype=dtype, device=self.device)
        self._keep.append(t)
        return t

    def _k(self, t: torch.Tensor) -> int:
        self._keep.append(t)
        return t.data_ptr()

    def _add(self, name, fname, args, kind, nbytes=0):
        f, lib = getattr(self.lib, fname), self.lib

        def run(stream):
            rc = f(*args, stream)
            if rc != 0:
                raise _capi.FamError(f"{fname}[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.steps.append(run)
        self.meta.append({"name": name, "kernel": kind, "bytes": int(nbytes)})

    def _gemm(self, name, a, w, bias, out, *, M=None, K=None, lda=None, ldw=None, ldo=None, res=None,
              out_f32=False):
        self._keep += [a, w, out] + ([bias] if bias is not None else []) + ([res] if res is not None else [])
        d = _capi.GemmDesc()
        d.a, d.lda = a.data_ptr(), lda if lda is not None else a.stride(0)
        d.w, d.ldw = w.data_ptr(), ldw if ldw is not None else w.stride(0)
        d.bias = bias.data_ptr() if bias is not None else None
        d.out, d.ldo = out.data_ptr(), ldo if ldo is not None else out.stride(0)
        d.M = M if M is not None else a.shape[0]
        d.N = w.shape[0]
        d.K = K if K is not None else w.shape[1]
        d.act = _capi.FAM_ACT_NONE
        d.res, d.ldr = (res.data_ptr(), res.stride(0)) if res is not None else (None, 0)
        d.rows_per_batch = max(d.M, 1)
        d.out_f32 = int(out_f32)
        self._descs.append(d)
        f, lib = self.lib.fam_gemm_ws, self.lib

        def run(stream):
            rc = f(C.byref(d), *self._ws_args, stream)
            if rc != 0:
                raise _capi.FamError(f"fam_gemm_ws[{name}]", rc, lib.fam_last_error().decode(errors="replace"))
        self.steps.append(run)
        self.meta.append({"name": name, "kernel": "gemm", "bytes": 2 * (d.M * d.K + d.N * d.K + d.M * d.N)})

    def _im2col(self, name, x, h, w, c, stride):
        ho, wo = (h, w) if stride == 1 else (h // 2, w // 2)
        kp = _kpad(9 * c)
        a = self._buf(ho * wo, kp)
        self.stages[name + ".im2col"] = a
        self._add(f"{name}.im2col", "fam_im2col3x3", (x.data_ptr(), x.stride(0), h, w, c, stride, a.data_ptr(), kp, kp),
                  "im2col", 2 * (x.numel() + a.numel()))
        return a

    def _res_block(self, pre, x, h, w, ci, co, P, conv3, conv1x1, gamma, level_input=None, level_cin=None):
        """ResidualBlock (FB/wan_video_vae.py:267-301).  level_input: on a level without
        downsampling the block is the last of its Down_ResidualBlock, whose identity AvgDown3D
        shortcut (:474) is folded into this block's residual (shortcut + level input)."""
        n, z2 = h * w, self._buf
        if ci != co:
            ws, bs = conv1x1(pre + "shortcut.weight", pre + "shortcut.bias")
            hs = z2(n, co)
            self._gemm(pre + "shortcut", x, ws, bs, hs)
            self.stages[pre + "shortcut"] = hs
        else:
            hs = x
        if level_input is not None:
            s = z2(n, co)
            self._add(pre + "level_shortcut", "fam_vae_avgdown",
                      (level_input.data_ptr(), level_input.stride(0), h, w, level_cin, co, 1, 1, hs.data_ptr(),
                       hs.stride(0), s.data_ptr(), co), "avgdown", 6 * s.numel())
            hs = s
        t = z2(n, ci)
        self._add(pre + "norm0", "fam_chan_rmsnorm", (x.data_ptr(), x.stride(0), n, ci, self._k(gamma(pre + "residual.0.gamma")),
                                                      _capi.FAM_ACT_SILU, t.data_ptr(), ci), "norm", 4 * t.numel())
        a = self._im2col(pre + "conv2", t, h, w, ci, 1)
        w2, b2 = conv3(pre + "residual.2.weight", pre + "residual.2.bias")
        y = z2(n, co)
        self._gemm(pre + "conv2", a, w2, b2, y)
        self.stages[pre + "conv2"] = y
        t2 = z2(n, co)
        self._add(pre + "norm3", "fam_chan_rmsnorm", (y.data_ptr(), co, n, co, self._k(gamma(pre + "residual.3.gamma")),
                                                      _capi.FAM_ACT_SILU, t2.data_ptr(), co), "norm", 4 * t2.numel())
        a2 = self._im2col(pre + "conv6", t2, h, w, co, 1)
        w6, b6 = conv3(pre + "residual.6.weight", pre + "residual.6.bias")
        out = z2(n, co)
        self._gemm(pre + "conv6", a2, w6, b6, out, res=hs)
        self.stages[pre + "out"] = out
        return out

    def _attention(self, pre, x, n, c, P, conv1x1, gamma):
        """AttentionBlock (FB/wan_video_vae.py:304-342) on n tokens of width c."""
        z2 = self._buf
        npad = _kpad(n)
        y = z2(n, c)
        self._add(pre + "norm", "fam_chan_rmsnorm", (x.data_ptr(), x.stride(0), n, c, self._k(gamma(pre + "norm.gamma")),
                                                     _capi.FAM_ACT_NONE, y.data_ptr(), c), "norm", 4 * y.numel())
        wqkv, bqkv = conv1x1(pre + "to_qkv.weight", pre + "to_qkv.bias")
        qk = z2(n, 2 * c)
        self._gemm(pre + "qk", y, wqkv[:2 * c].contiguous(), bqkv[:2 * c].contiguous(), qk)
        s = self._buf(n, npad, dtype=torch.float32)
        self._gemm(pre + "scores", qk, qk[:, c:], None, s, lda=2 * c, ldw=2 * c, K=c, ldo=npad, out_f32=True)
        p = z2(n, npad)                       # columns n..npad-1 stay zero
        self._add(pre + "softmax", "fam_softmax_rows", (s.data_ptr(), npad, n, n, 1.0 / math.sqrt(c), p.data_ptr(), npad),
                  "softmax", 6 * n * n)
        vt = z2(c, npad)                      # v0^T = W_v y^T; columns n..npad-1 stay zero
        wv = wqkv[2 * c:].contiguous()
        self._gemm(pre + "v", wv, y, None, vt, ldo=npad)
        o = z2(n, c)
        self._gemm(pre + "pv", p, vt, bqkv[2 * c:].contiguous(), o, K=npad)
        wp, bp = conv1x1(pre + "proj.weight", pre + "proj.bias")
        out = z2(n, c)
        self._gemm(pre + "proj", o, wp, bp, out, res=x)
        return out

    # ------------------------------------------------------------------ execution
    def set_input(self, image: torch.Tensor) -> None:
        """image [1, 3, H, W] or [3, H, W] (any float dtype), copied into the static buffer as bf16."""
        if image.dim() == 4:
            if image.shape[0] != 1:
                raise ValueError(f"one image per call (the reference encodes [1, 3, H, W]), got {tuple(image.shape)}")
            image = image[0]
        if tuple(image.shape) != (3, self.H, self.W):
            raise ValueError(f"image must be [3, {self.H}, {self.W}], got {tuple(image.shape)}")
        self.img.copy_(image.to(device=self.device, dtype=_BF16))

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

    def encode(self, image: torch.Tensor) -> torch.Tensor:
        """The normalised latent mu [1, z_dim, 1, H/16, W/16] (bf16, a copy)."""
        self.set_input(image)
        self.run()
        return self.out.clone()

    @property
    def num_launches(self) -> int:
        return len(self.steps)

"""CAE-FastWAM action-VAE decoder on the library's fp32 kernels (fam_cae_decode).

`ActionAE.decode(z, suite_ids)` (CAm/action_ae.py:152-166, run in fp32 at
CA/fastwam.py:855-863): latent tokens [B, num_tokens, latent_dim] -> action chunk
[B, action_horizon, action_dim].  The parameters are the reference's `decoder.*` state-dict
keys; the suite embedding, when the model has one, is looked up on the host and passed as
rows.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, List, Optional

import torch

from . import _capi


def cae_strides(ratio: int) -> List[int]:
    """Upsampling strides of the decoder: the factorisation of horizon / num_tokens into 4s,
    then 2s, then 3s, then the remainder (CAm/action_ae.py:90-101)."""
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


class CaeDecoder:
    """ActionDecoder for a fixed batch size; fp32 weights on the device."""

    def __init__(self, params: Dict[str, torch.Tensor], *, latent_dim: int, num_tokens: int, action_horizon: int,
                 action_dim: int, decoder_hidden: int, batch: int, device="cuda", gn_eps: float = 1e-5):
        dev = torch.device(device)
        self.lib = _capi.load()
        self.B, self.T0, self.L, self.H, self.A, self.C = batch, num_tokens, latent_dim, action_horizon, action_dim, decoder_hidden
        self.strides = cae_strides(action_horizon // num_tokens)
        if len(self.strides) > 3:
            raise ValueError(f"at most 3 upsampling stages, got strides {self.strides}")
        self.w = {k: v.to(device=dev, dtype=torch.float32).contiguous() for k, v in params.items()
                  if k.startswith("decoder.") and "suite_embed" not in k}
        T = num_tokens
        for s in self.strides:
            T = (T - 1) * s - 2 * (s // 2) + 2 * s
        self.T = T
        self.z = torch.zeros(batch, num_tokens, latent_dim, dtype=torch.float32, device=dev)
        self.suite = torch.zeros(batch, decoder_hidden, dtype=torch.float32, device=dev)
        self.work = torch.zeros(3 * batch * decoder_hidden * T, dtype=torch.float32, device=dev)
        self.out = torch.zeros(batch, action_horizon, action_dim, dtype=torch.float32, device=dev)
        self.d = self._desc(gn_eps)

    def _desc(self, eps: float) -> _capi.CaeDesc:
        w, d = self.w, _capi.CaeDesc()
        d.z, d.batch, d.tokens, d.latent_dim = self.z.data_ptr(), self.B, self.T0, self.L
        d.hidden, d.horizon, d.action_dim, d.nstages = self.C, self.H, self.A, len(self.strides)
        d.in_w, d.in_b = w["decoder.input_proj.weight"].data_ptr(), w["decoder.input_proj.bias"].data_ptr()
        for j, s in enumerate(self.strides):
            d.strides[j] = s
            u, g, r = f"decoder.up.{4 * j}", f"decoder.up.{4 * j + 1}", f"decoder.up.{4 * j + 3}.net."
            d.up_w[j], d.up_b[j] = w[u + ".weight"].data_ptr(), w[u + ".bias"].data_ptr()
            d.gn_w[j], d.gn_b[j] = w[g + ".weight"].data_ptr(), w[g + ".bias"].data_ptr()
            d.r1_w[j], d.r1_b[j] = w[r + "0.weight"].data_ptr(), w[r + "0.bias"].data_ptr()
            d.rg1_w[j], d.rg1_b[j] = w[r + "1.weight"].data_ptr(), w[r + "1.bias"].data_ptr()
            d.r2_w[j], d.r2_b[j] = w[r + "3.weight"].data_ptr(), w[r + "3.bias"].data_ptr()
            d.rg2_w[j], d.rg2_b[j] = w[r + "4.weight"].data_ptr(), w[r + "4.bias"].data_ptr()
        d.out_w, d.out_b = w["decoder.output_proj.weight"].data_ptr(), w["decoder.output_proj.bias"].data_ptr()
        d.work, d.out = self.work.data_ptr(), self.out.data_ptr()
        d.gn_eps = float(eps)
        return d

    def launch(self, stream: Optional[int] = None, with_suite: bool = False) -> None:
        """Enqueue the decode of the static `z` (and `suite` rows) into `out`."""
        self.d.suite = self.suite.data_ptr() if with_suite else None
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        _capi.call("fam_cae_decode", C.byref(self.d), s)

    def decode(self, z: torch.Tensor, suite_rows: Optional[torch.Tensor] = None) -> torch.Tensor:
        """z [B, num_tokens, latent_dim] -> [B, action_horizon, action_dim] fp32 (a copy)."""
        self.z.copy_(z.reshape(self.z.shape))
        if suite_rows is not None:
            self.suite.copy_(suite_rows.reshape(self.suite.shape))
        self.launch(with_suite=suite_rows is not None)
        return self.out.clone()

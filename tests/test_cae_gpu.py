"""CAE-FastWAM action-VAE decoder (CAm/action_ae.py:123-166) on the GPU (fam_cae_decode, fp32)
against the reference module's golden outputs and the oracle.  Bar: normwise relative error
<= 1e-4 (fp32 kernels vs fp32 reference; only the summation order differs)."""
import os

import pytest
import torch

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu
CASES = {"base": (16, 8, 32, 7, 128, 0, 41), "two_stage_suite": (8, 4, 32, 7, 64, 3, 42),
         "stride3_pad": (6, 3, 10, 5, 32, 0, 43)}


@pytest.fixture(scope="module")
def golden():
    from safetensors.torch import load_file
    return load_file(os.path.join(os.path.dirname(__file__), "golden", "cae_decoder.safetensors"))


def _rel(y, ref):
    return ((y - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.parametrize("name", sorted(CASES))
def test_cae_decode_golden(golden, name):
    from fam.cae import CaeDecoder
    L, T0, hz, A, C, ns, seed = CASES[name]
    cfg = O.CaeDecoderConfig(latent_dim=L, num_tokens=T0, action_horizon=hz, action_dim=A, decoder_hidden=C)
    p = O.init_cae_decoder_params(cfg, seed)
    dec = CaeDecoder(p, latent_dim=L, num_tokens=T0, action_horizon=hz, action_dim=A, decoder_hidden=C, batch=2)
    suite = golden.get(f"{name}.suite_rows")
    y = dec.decode(golden[f"{name}.z"].cuda(), suite.cuda() if suite is not None else None).cpu()
    assert _rel(y, golden[f"{name}.out"]) <= 1e-4
    # a second, different batch through the same static buffers
    z2 = torch.randn(2, T0, L, generator=torch.Generator().manual_seed(seed + 7))
    y2 = dec.decode(z2.cuda(), suite.cuda() if suite is not None else None).cpu()
    assert _rel(y2, O.cae_decode(p, cfg, z2, suite)) <= 1e-4


def test_cae_decode_batch_256():
    """Config 3's throughput batch: 256 latents of 8 x 16 -> 256 chunks of 32 x 7."""
    from fam.cae import CaeDecoder
    cfg = O.CaeDecoderConfig()
    p = O.init_cae_decoder_params(cfg, 44)
    z = torch.randn(256, 8, 16, generator=torch.Generator().manual_seed(45))
    dec = CaeDecoder(p, latent_dim=16, num_tokens=8, action_horizon=32, action_dim=7, decoder_hidden=128, batch=256)
    assert _rel(dec.decode(z.cuda()).cpu(), O.cae_decode(p, cfg, z)) <= 1e-4

"""The Wan2.2 VAE38 first-frame encoder on the library (fam.vae.FusedWanVAEEncoder) against the
oracle's restatement of VideoVAE38_.encode, which the reference module pins
(tests/golden/wan_vae_tiny.safetensors): fp32 oracle on bf16-valued weights and image, normwise
relative error <= 3e-2 on the latent (about 25 bf16 layers deep).  Plus the non-GEMM kernels
(im2col, channel RMS_norm, AvgDown3D, row softmax, latent normalisation) against torch."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _rel(y, ref):
    y, ref = y.float().cpu(), ref.float().cpu()
    return ((y - ref).abs().max() / ref.abs().max()).item()


def _lib():
    from fam import _capi
    return _capi.load()


def _s():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("H,W,C,stride", [(6, 10, 16, 1), (8, 12, 24, 2), (5, 7, 8, 1)])
def test_im2col3x3(H, W, C, stride):
    x = torch.randn(H * W, C, generator=torch.Generator().manual_seed(1)).to(BF)
    kp = (9 * C + 63) // 64 * 64
    ho, wo = (H, W) if stride == 1 else (H // 2, W // 2)
    out = torch.full((ho * wo, kp), 7.0, dtype=BF, device="cuda")
    xd = x.cuda()
    assert _lib().fam_im2col3x3(xd.data_ptr(), C, H, W, C, stride, out.data_ptr(), kp, kp, _s()) == 0
    img = x.reshape(1, H, W, C).permute(0, 3, 1, 2).float()
    pad = (1, 1, 1, 1) if stride == 1 else (0, 1, 0, 1)
    cols = F.unfold(F.pad(img, pad), 3, stride=stride)                # [1, C*9, L], (c, kh, kw)
    ref = cols.reshape(C, 9, ho * wo).permute(2, 1, 0).reshape(ho * wo, 9 * C)
    got = out.float().cpu()
    assert torch.equal(got[:, :9 * C], ref)
    assert torch.equal(got[:, 9 * C:], torch.zeros_like(got[:, 9 * C:]))


def test_vae_patch_im2col():
    H, W = 12, 20
    img = torch.randn(1, 3, H, W, generator=torch.Generator().manual_seed(2)).to(BF)
    out = torch.empty((H // 2) * (W // 2), 128, dtype=BF, device="cuda")
    imgd = img.cuda()
    assert _lib().fam_vae_patch_im2col(imgd.data_ptr(), H, W, out.data_ptr(), 128, _s()) == 0
    pt = O.vae_patchify(img.float(), 2)                                 # [1, 12, 6, 10]
    cols = F.unfold(F.pad(pt, (1, 1, 1, 1)), 3)
    ref = cols.reshape(12, 9, -1).permute(2, 1, 0).reshape(-1, 108)
    got = out.float().cpu()
    assert torch.equal(got[:, :108], ref)
    assert torch.equal(got[:, 108:], torch.zeros_like(got[:, 108:]))


@pytest.mark.parametrize("C,act", [(160, True), (640, False), (8, True)])
def test_chan_rmsnorm(C, act):
    from fam import _capi
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(37, C, generator=g) * 3).to(BF)
    gamma = (1 + 0.2 * torch.randn(C, generator=g)).to(BF)
    y = torch.empty(37, C, dtype=BF, device="cuda")
    xd, gd = x.cuda(), gamma.cuda()   # (device copies held for the launch)
    rc = _lib().fam_chan_rmsnorm(xd.data_ptr(), C, 37, C, gd.data_ptr(),
                                 _capi.FAM_ACT_SILU if act else _capi.FAM_ACT_NONE, y.data_ptr(), C, _s())
    assert rc == 0
    ref = O.vae_rms_norm(x.float().t().reshape(1, C, 37, 1), gamma.float()).reshape(C, 37).t()
    if act:
        ref = F.silu(ref)
    assert _rel(y, ref) <= 1e-2


@pytest.mark.parametrize("Cin,Cout,ft,fs", [(16, 16, 1, 2), (16, 32, 2, 2), (24, 24, 1, 1)])
def test_vae_avgdown(Cin, Cout, ft, fs):
    H, W = 6, 8
    g = torch.Generator().manual_seed(4)
    x = torch.randn(H * W, Cin, generator=g).to(BF)
    add = torch.randn((H // fs) * (W // fs), Cout, generator=g).to(BF)
    out = torch.empty((H // fs) * (W // fs), Cout, dtype=BF, device="cuda")
    xd = x.cuda()
    for a in (None, add.cuda()):
        assert _lib().fam_vae_avgdown(xd.data_ptr(), Cin, H, W, Cin, Cout, ft, fs,
                                      a.data_ptr() if a is not None else None, Cout, out.data_ptr(), Cout, _s()) == 0
        ref = O.vae_avg_down(x.float().t().reshape(1, Cin, H, W), Cout, ft, fs).reshape(Cout, -1).t()
        if a is not None:
            ref = ref + add.float()
        assert _rel(out, ref) <= 1e-2


def test_softmax_rows_and_affine():
    g = torch.Generator().manual_seed(5)
    s = torch.randn(9, 70, generator=g) * 4
    p = torch.zeros(9, 128, dtype=BF, device="cuda")
    sd = s.cuda()
    assert _lib().fam_softmax_rows(sd.data_ptr(), 70, 9, 70, 0.3, p.data_ptr(), 128, _s()) == 0
    assert _rel(p[:, :70], torch.softmax(s * 0.3, -1)) <= 1e-2
    assert torch.count_nonzero(p[:, 70:]).item() == 0
    x = torch.randn(12, 5, generator=g).to(BF)
    mean, std = torch.randn(5, generator=g), 0.5 + torch.rand(5, generator=g)
    out = torch.empty(5, 12, dtype=BF, device="cuda")
    inv = (1 / std).float().cuda()
    xd, md = x.cuda(), mean.cuda()
    assert _lib().fam_chan_affine_nchw(xd.data_ptr(), 5, 12, 5, md.data_ptr(), inv.data_ptr(), out.data_ptr(),
                                       _s()) == 0
    assert _rel(out, ((x.float() - mean) / std).t()) <= 1e-2


def _encoder_case(cfg, H, W, seed):
    from fam.vae import FusedWanVAEEncoder
    p = {k: v.to(BF) for k, v in O.init_wan_vae_params(cfg, seed).items()}
    g = torch.Generator().manual_seed(seed + 1)
    img = torch.randn(1, 3, H, W, generator=g).clamp(-1, 1).to(BF)
    mean = 0.3 * torch.randn(cfg.z_dim, generator=g)
    std = 0.5 + torch.rand(cfg.z_dim, generator=g)
    enc = FusedWanVAEEncoder(cfg, p, height=H, width=W, mean=mean, std=std)
    y = enc.encode(img.cuda())
    ref = O.wan_vae_encode_first_frame({k: v.float() for k, v in p.items()}, cfg, img.float(), mean, std)
    return enc, img, y, ref


@pytest.mark.parametrize("H,W", [(64, 128), (48, 80)])
def test_vae_encoder_tiny_matches_oracle(H, W):
    """The golden config (dim 16, z 8) at both golden image sizes."""
    cfg = O.WanVaeConfig(dim=16, z_dim=8)
    enc, img, y, ref = _encoder_case(cfg, H, W, 2468)
    err = _rel(y, ref)
    print(f"vae tiny {H}x{W}: {enc.num_launches} launches, relerr {err:.3e}")
    assert y.shape == ref.shape == (1, 8, 1, H // 16, W // 16)
    assert err <= 3e-2
    enc.capture()
    assert torch.equal(enc.encode(img.cuda()), y)


def test_vae_encoder_wan22_shape():
    """The Wan2.2 VAE38 encoder (dim 160, z 48, widths 160-160-320-640-640) on FastWAM's first
    frame, 224 x 448 (latent 14 x 28 -> 7 x 14 video patches)."""
    cfg = O.WanVaeConfig()
    enc, img, y, ref = _encoder_case(cfg, 224, 448, 97)
    err = _rel(y, ref)
    print(f"vae wan2.2 224x448: {enc.num_launches} launches, relerr {err:.3e}")
    assert y.shape == (1, 48, 1, 14, 28)
    assert err <= 3e-2

"""Per-kernel parity of the HIP library against the CPU oracle (bf16 kernels vs fp32 oracle).

Bar (from the task's north star): normwise max relative error
||y - y_ref||_inf / ||y_ref||_inf <= 2e-2 for every kernel; mean |d| is reported as well.
Inputs are seeded on the CPU in fp32, rounded to bf16, and the oracle runs on the
bf16-rounded values in fp32.
"""
import math

import pytest
import torch

from oracle import fam_oracle as O

pytestmark = pytest.mark.gpu
TOL = 2e-2


def ops():
    from fam import ops as _ops
    return _ops


def rnd(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def dev(t):
    return t.to("cuda")


def relerr(y, ref):
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert torch.isfinite(y).all(), "non-finite output"
    den = ref.abs().max().clamp_min(1e-6)
    return ((y - ref).abs().max() / den).item()


# --------------------------------------------------------------------------- AdaLN / LayerNorm
@pytest.mark.parametrize("B,S,D,per_token", [(1, 32, 1024, False), (2, 7, 3072, True), (1, 5, 32, False),
                                              (3, 17, 2048, False), (1, 3, 8192, False), (2, 4, 6144, True),
                                              (2, 64, 3072, False), (2, 33, 4096, False)])
def test_adaln(B, S, D, per_token):
    x = rnd(B, S, D, seed=1, scale=2.0) + 0.3
    Sm = S if per_token else 1
    shift, scale = rnd(B, Sm, D, seed=2, scale=0.1), rnd(B, Sm, D, seed=3, scale=0.1)
    ref = O.adaln(x.float(), shift.float(), scale.float(), 1e-6)
    norm = torch.nn.LayerNorm(D, eps=1e-6, elementwise_affine=False)
    y = ops().adaln_forward(dev(x), norm, dev(shift), dev(scale))
    assert relerr(y, ref) <= TOL


def test_adaln_chunk_views():
    """shift/scale as chunk views of (modulation + t_mod) [B, 6, D] (FB/wan_video_dit.py:273-274)."""
    B, S, D = 2, 32, 1024
    x = rnd(B, S, D, seed=4)
    mod = rnd(B, 6, D, seed=5, scale=0.1)
    sh, sc = dev(mod).chunk(6, dim=1)[0], dev(mod).chunk(6, dim=1)[1]
    ref = O.adaln(x.float(), mod[:, 0:1].float(), mod[:, 1:2].float(), 1e-6)
    norm = torch.nn.LayerNorm(D, eps=1e-6, elementwise_affine=False)
    assert relerr(ops().adaln_forward(dev(x), norm, sh, sc), ref) <= TOL


def test_layer_norm_affine():
    x = rnd(3, 11, 1024, seed=6)
    w, b = rnd(1024, seed=7, scale=0.5) + 1, rnd(1024, seed=8, scale=0.5)
    ref = O.layer_norm(x.float(), w.float(), b.float(), 1e-6)
    assert relerr(ops().layer_norm(dev(x), dev(w), dev(b), 1e-6), ref) <= TOL


# --------------------------------------------------------------------------- RMSNorm / RoPE
@pytest.mark.parametrize("R,D", [(32, 1024), (97, 3072), (4, 8)])
def test_rms_norm(R, D):
    x = rnd(1, R, D, seed=9, scale=3.0)
    w = rnd(D, seed=10, scale=0.2) + 1
    ref = O.rms_norm(x.float(), w.float(), 1e-6)
    assert relerr(ops().rms_norm(dev(x), dev(w), 1e-6), ref) <= TOL


@pytest.mark.parametrize("Lc,nb,A", [(129, 29, 3072), (7, 3, 64), (40, 5, 5000)])
def test_rms_norm_grouped_context_keys(Lc, nb, A):
    """Every block's context keys in one launch (rows (context row, block), block keys 2A
    apart, block b's weight): the oracle per block, and bit-identical to one fam_rmsnorm_rope
    per block; the v columns between the keys are untouched (A = 5000: the out-of-place
    wide-row kernel on a copy)."""
    from fam import _capi
    kv = rnd(Lc, nb * 2 * A, seed=95, scale=2.0)
    ws = rnd(nb, A, seed=96, scale=0.2) + 1
    lib, eps = _capi.lib(), 1e-6
    src = dev(kv)
    got = src.clone() if A <= 4096 else torch.zeros_like(src)
    out_p = got.data_ptr()
    wd = dev(ws)
    _capi.call("fam_rmsnorm_grouped", src.data_ptr() if A > 4096 else out_p, 2 * A, out_p, 2 * A, Lc * nb, A,
               wd.data_ptr(), nb, eps, None)
    per = src.clone()
    for b in range(nb):
        p = per.data_ptr() + 2 * (b * 2 * A)
        out = p if A <= 4096 else torch.zeros(Lc, A, dtype=torch.bfloat16, device="cuda")
        if A <= 4096:
            _capi.call("fam_rmsnorm_rope", p, nb * 2 * A, p, nb * 2 * A, Lc, Lc, A, wd[b].data_ptr(), eps, None, None,
                       0, 0, 0, None)
        else:
            _capi.call("fam_rmsnorm_rope", p, nb * 2 * A, out.data_ptr(), A, Lc, Lc, A, wd[b].data_ptr(), eps, None,
                       None, 0, 0, 0, None)
            per[:, b * 2 * A:b * 2 * A + A] = out
    torch.cuda.synchronize()
    g3 = got.reshape(Lc, nb, 2 * A)
    for b in range(nb):
        ref = O.rms_norm(kv.reshape(Lc, nb, 2 * A)[:, b, :A].float(), ws[b].float(), eps)
        assert relerr(g3[:, b, :A], ref) <= TOL
    assert torch.equal(g3[..., :A], per.reshape(Lc, nb, 2 * A)[..., :A])
    if A <= 4096:
        assert torch.equal(g3[..., A:].cpu(), kv.reshape(Lc, nb, 2 * A)[..., A:])
    with pytest.raises(_capi.FamError):
        _capi.call("fam_rmsnorm_grouped", out_p, 2 * A, out_p, 2 * A, Lc * nb + 1, A, wd.data_ptr(), nb, eps, None)


@pytest.mark.parametrize("B,S,H,Dh", [(1, 32, 16, 64), (2, 9, 24, 128), (1, 8, 4, 8), (1, 5, 4, 24)])
@pytest.mark.parametrize("layout", ["complex", "cat", "interleaved"])
def test_rope(B, S, H, Dh, layout):
    x = rnd(B, S, H * Dh, seed=11)
    fr = O.action_freqs(Dh, S)
    ref = O.rope_apply(x.float(), fr, H)
    if layout == "complex":
        y = ops().rope_apply(dev(x), fr, H)
    elif layout == "cat":
        packed = torch.cat([fr.real, fr.imag], dim=-1).float()
        y = ops().rope_apply(dev(x), dev(packed), H)
    else:
        inter = torch.view_as_real(fr).reshape(S, 1, Dh).double()
        y = ops().rope_apply_cae(dev(x), dev(inter), H)
    assert relerr(y, ref) <= TOL


@pytest.mark.parametrize("layout", ["complex", "interleaved"])
def test_rms_norm_rope_many_rows(layout):
    """4099 rows (two rows per wave, odd tail) of a 3-D-style per-row table, with the weight."""
    B, S, H, Dh = 1, 4099, 8, 64
    x = rnd(B, S, H * Dh, seed=73, scale=2.0)
    w = rnd(H * Dh, seed=74, scale=0.2) + 1
    ang = torch.rand(S, 1, Dh // 2, generator=torch.Generator().manual_seed(75), dtype=torch.float64) * 6.0
    fr = torch.polar(torch.ones_like(ang), ang)
    ref = O.rope_apply(O.rms_norm(x.float(), w.float(), 1e-6), fr, H)
    if layout == "complex":
        y = ops().rms_norm_rope(dev(x), dev(w), 1e-6, fr, H)
    else:
        inter = dev(torch.view_as_real(fr).reshape(S, 1, Dh).double())
        y = ops().rms_norm_rope(dev(x), dev(w), 1e-6, inter, H, layout="interleaved")
    assert relerr(y, ref) <= TOL


def test_rope_scalar_table_path():
    """Tables whose rows are not 16-byte multiples take the per-element table reads."""
    from fam import _capi
    B, S, H, Dh = 1, 6, 4, 16
    x = rnd(B, S, H * Dh, seed=12)
    fr = O.action_freqs(Dh, S)
    ref = O.rope_apply(x.float(), fr, H)
    half = Dh // 2
    tab = torch.zeros(S, 2 * half + 1, dtype=torch.float32)   # row stride 17 floats: (cos | sin | pad)
    tab[:, :half], tab[:, half:2 * half] = fr.real.reshape(S, half), fr.imag.reshape(S, half)
    t = dev(tab)
    xd = dev(x).reshape(S, H * Dh)
    y = torch.empty_like(xd)
    _capi.call("fam_rmsnorm_rope", xd.data_ptr(), H * Dh, y.data_ptr(), H * Dh, S, S, H * Dh, None, 0.0,
               t.data_ptr(), t.data_ptr() + 4 * half, 2 * half + 1, 1, Dh, 0)
    assert relerr(y.reshape(B, S, H * Dh), ref) <= TOL


def test_rope_3d_video_table():
    """3-D (f, h, w) table of a video grid (FB/wan_video_dit.py:620-624)."""
    f, h, w, H, Dh = 2, 5, 6, 4, 128
    fr = O.video_freqs(O.precompute_freqs_cis_3d(Dh), f, h, w)
    x = rnd(1, f * h * w, H * Dh, seed=12)
    ref = O.rope_apply(x.float(), fr, H)
    assert relerr(ops().rope_apply(dev(x), fr, H), ref) <= TOL


def test_rms_norm_rope_fused():
    B, S, H, Dh = 2, 32, 16, 64
    x = rnd(B, S, H * Dh, seed=13, scale=2.0)
    w = rnd(H * Dh, seed=14, scale=0.2) + 1
    fr = O.action_freqs(Dh, S)
    ref = O.rope_apply(O.rms_norm(x.float(), w.float(), 1e-6), fr, H)
    assert relerr(ops().rms_norm_rope(dev(x), dev(w), 1e-6, fr, H), ref) <= TOL


# --------------------------------------------------------------------------- attention
@pytest.mark.parametrize("B,H,Sq,Sk,Dh", [(1, 16, 32, 32, 64), (1, 16, 32, 1560, 64), (2, 24, 32, 130, 128),
                                           (2, 3, 17, 1001, 128), (1, 2, 5, 300, 64), (2, 2, 9, 700, 64),
                                           (1, 4, 32, 2048, 64), (1, 2, 32, 2049, 64), (1, 2, 16, 1024, 128),
                                           (1, 4, 8, 1560, 8), (1, 2, 100, 77, 32), (3, 3, 1, 5, 16),
                                           (1, 4, 300, 300, 128)])
def test_attention(B, H, Sq, Sk, Dh):
    q, k, v = rnd(B, Sq, H * Dh, seed=15), rnd(B, Sk, H * Dh, seed=16), rnd(B, Sk, H * Dh, seed=17)
    ref = O.flash_attention(q.float(), k.float(), v.float(), H)
    y = ops().flash_attention(dev(q), dev(k), dev(v), H)
    assert relerr(y, ref) <= TOL


@pytest.mark.parametrize("Sq,Sk", [(32, 1560), (64, 1000), (16, 129), (32, 130)])
def test_attention_short_deterministic(Sq, Sk):
    """Short-query attention (keys divided among the waves of a workgroup): matches the
    oracle and is bit-identical from run to run (fixed merge order)."""
    B, H, Dh = 1, 16, 64
    q, k, v = rnd(B, Sq, H * Dh, seed=18), rnd(B, Sk, H * Dh, seed=19), rnd(B, Sk, H * Dh, seed=20)
    ref = O.flash_attention(q.float(), k.float(), v.float(), H)
    y1 = ops().attention_bshd(dev(q), dev(k), dev(v), H)
    y2 = ops().attention_bshd(dev(q), dev(k), dev(v), H)
    assert relerr(y1, ref) <= TOL
    assert torch.equal(y1, y2), "wave merge must be deterministic"


@pytest.mark.parametrize("kind", ["bool", "f32", "bf16"])
def test_attention_masks(kind):
    B, H, Sq, Sk, Dh = 2, 4, 20, 70, 64
    q, k, v = rnd(B, Sq, H * Dh, seed=21), rnd(B, Sk, H * Dh, seed=22), rnd(B, Sk, H * Dh, seed=23)
    g = torch.Generator().manual_seed(24)
    m = torch.rand(B, 1, Sq, Sk, generator=g) > 0.4
    m[:, :, 3] = False            # fully masked row -> zeros
    m[1, :, 5, :] = True
    ref = O.flash_attention(q.float(), k.float(), v.float(), H, m)
    if kind == "bool":
        mm = dev(m)
    else:
        add = torch.where(m, 0.0, float("-inf"))
        mm = dev(add if kind == "f32" else add.to(torch.bfloat16))
    y = ops().flash_attention(dev(q), dev(k), dev(v), H, mm)
    assert relerr(y, ref) <= TOL
    assert torch.all(y[:, 3] == 0)


@pytest.mark.parametrize("B,H,Sq,Sk,Dh,mask", [(1, 24, 98, 98, 128, None), (1, 24, 98, 129, 128, "keys"),
                                                (2, 4, 98, 98, 64, None), (2, 3, 70, 200, 128, "rows"),
                                                (1, 24, 98, 129, 64, "keys"), (1, 40, 70, 98, 128, "rows"),
                                                (1, 2, 128, 256, 64, "rows"), (1, 2, 33, 31, 128, "rows")])
def test_attention_small_query_chunks(B, H, Sq, Sk, Dh, mask):
    """33-128 queries over <= 256 keys run the small kernel in chunks of 32 queries (grid.z): the
    video prefill's 98 tokens over their own 98 keys and over 129 context keys with the text mask
    ("keys": [B, Sk], shared by the queries), and a per-query bool mask ("rows": [B, 1, Sq, Sk],
    whose rows each chunk must take from its own offset, with a fully masked row), ragged last
    chunks (98 = 3 x 32 + 2, 70, 33) and a full 128."""
    q, k, v = rnd(B, Sq, H * Dh, seed=31), rnd(B, Sk, H * Dh, seed=32), rnd(B, Sk, H * Dh, seed=33)
    g = torch.Generator().manual_seed(34)
    m = None
    if mask == "keys":
        m = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
        m[..., Sk - 29:] = False
    elif mask == "rows":
        m = torch.rand(B, 1, Sq, Sk, generator=g) > 0.4
        m[:, :, Sq - 1] = False    # a fully masked row in the last chunk -> zeros
    ref = O.flash_attention(q.float(), k.float(), v.float(), H, m)
    if mask == "keys":
        y = ops().flash_attention(dev(q), dev(k), dev(v), H, ctx_mask=dev(m))
    else:
        y = ops().flash_attention(dev(q), dev(k), dev(v), H, None if m is None else dev(m))
    assert relerr(y, ref) <= TOL
    if mask == "rows":
        assert torch.all(y[:, Sq - 1] == 0)


def test_attention_two_segments_joint_mask():
    """Joint attention over a cached video prefix + action tokens with the MoT mask (FB/mot.py:446-478)."""
    Sv, Sa, H, Dh, tpf = 98, 32, 24, 128, 98
    q = rnd(1, Sa, H * Dh, seed=25)
    kv_, vv_ = rnd(1, Sv, H * Dh, seed=26), rnd(1, Sv, H * Dh, seed=27)
    ka, va = rnd(1, Sa, H * Dh, seed=28), rnd(1, Sa, H * Dh, seed=29)
    jm = O.mot_joint_mask(Sv, Sa, 49)
    amask = jm[Sv:, :]
    ref = O.flash_attention(q.float(), torch.cat([kv_, ka], 1).float(), torch.cat([vv_, va], 1).float(), H, amask)
    y = ops().attention_bshd(dev(q), dev(ka), dev(va), H, mask=dev(amask), k_prefix=dev(kv_), v_prefix=dev(vv_))
    assert relerr(y, ref) <= TOL


def test_attention_bhsd_layout_and_broadcast_kv():
    """[B,H,S,Dh] strides through attention_bshd's descriptor and a batch-broadcast context."""
    B, H, Sq, Sk, Dh = 4, 16, 32, 200, 64
    q = rnd(B, Sq, H * Dh, seed=30)
    k, v = rnd(1, Sk, H * Dh, seed=31), rnd(1, Sk, H * Dh, seed=32)
    ref = O.flash_attention(q.float(), k.float().expand(B, -1, -1), v.float().expand(B, -1, -1), H)
    y = ops().attention_bshd(dev(q), dev(k), dev(v), H)
    assert relerr(y, ref) <= TOL


# --------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(32, 3072, 1024), (32, 1024, 4096), (32, 7, 1024), (1, 64, 8), (7, 1000, 256),
                                    (100, 4096, 1024), (1024, 1024, 1024), (1560, 2048, 1024), (16, 29, 1024),
                                    (10, 6144, 1024), (256, 32, 256)])
def test_linear(M, N, K):
    x = rnd(M, K, seed=33)
    w = rnd(N, K, seed=34, scale=0.02)
    b = rnd(N, seed=35, scale=0.02)
    ref = O.linear(x.float(), w.float(), b.float())
    assert relerr(ops().linear(dev(x), dev(w), dev(b)), ref) <= TOL


def test_linear_small_k():
    x, w, b = rnd(2, 32, 7, seed=36), rnd(1024, 7, seed=37, scale=0.02), rnd(1024, seed=38, scale=0.02)
    ref = O.linear(x.float(), w.float(), b.float())
    assert relerr(ops().linear(dev(x), dev(w), dev(b)), ref) <= TOL


@pytest.mark.parametrize("M,N,K", [(32, 1024, 4096), (64, 3072, 1024), (2048, 1024, 1024)])
def test_gemm_deterministic(M, N, K):
    """Both GEMM kernels (waves share K for M <= 64, output tiles above) reduce in a fixed
    order: two runs are bit-identical."""
    x, w, b = rnd(M, K, seed=39), rnd(N, K, seed=40, scale=0.02), rnd(N, seed=41, scale=0.02)
    ref = O.linear(x.float(), w.float(), b.float())
    outs = []
    for _ in range(2):
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        ops().gemm(dev(x), dev(w), dev(b), y)
        outs.append(y)
    assert relerr(outs[0], ref) <= TOL
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 128), (3900, 3900, 128), (2600, 3000, 192), (300, 520, 320),
                                   (1000, 1500, 640), (1000, 1500, 576), (1560, 3072, 1024), (588, 2048, 2048),
                                   (588, 2048, 128), (130, 200, 192)])
def test_gemm_large_tiles_epilogue(M, N, K):
    """Large-M products on the big-tile kernel (256 x 256 tiles for the first two shapes,
    128 x 128 for the third, 64 x 64 for the fourth; ragged M and N): bias + GELU, then
    gate * y + residual with a per-row gate, then an fp32 residual output; and a shape off its
    envelope (N % 4 != 0) on the tiled kernel.  1000 x 1500 runs 96 tiles of 128 x 128 (at most
    one workgroup per CU): with 10 K blocks as two K groups per workgroup whose sums meet in
    LDS, with 9 (odd) as one group.  1560 x 3072 (config 2's o-projection rows and columns) runs
    416 tiles of 128 x 96.  The 64 x 64 grids of at most two workgroups per CU keep three K
    blocks in flight through four LDS slots: 300 x 520 (5 blocks), the DiT4DiT call's
    588 x 2048 x 2048 (320 tiles, 32 blocks), fewer blocks than slots (588 x 2048 x 128: 2) and a
    ragged 130 x 200 grid (3 blocks)."""
    from fam import _capi
    x, w, b = rnd(M, K, seed=65), rnd(N, K, seed=66, scale=0.05), rnd(N, seed=67, scale=0.05)
    lin = O.linear(x.float(), w.float(), b.float())
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops().gemm(dev(x), dev(w), dev(b), y, act=_capi.FAM_ACT_GELU_TANH)
    assert relerr(y, O.gelu_tanh(lin)) <= TOL
    res, gate = rnd(M, N, seed=68), rnd(M, N, seed=69, scale=0.3)
    out = dev(res.clone())
    ops().gemm(dev(x), dev(w), dev(b), out, res=out, gate=dev(gate), gate_bs=0, gate_rs=N, gate_ns=1,
               rows_per_batch=M)
    assert relerr(out, res.float() + gate.float() * lin) <= TOL
    resf = torch.randn(M, N, generator=torch.Generator().manual_seed(70))
    outf = dev(resf.clone())
    ops().gemm(dev(x), dev(w), dev(b), outf, res=outf, out_f32=True)
    assert (outf.cpu() - (resf + lin)).abs().max().item() <= 2e-2 * lin.abs().max().item()
    if M == 300:
        w3, b3 = rnd(N - 1, K, seed=71, scale=0.05), rnd(N - 1, seed=72, scale=0.05)
        assert relerr(ops().linear(dev(x), dev(w3), dev(b3)), O.linear(x.float(), w3.float(), b3.float())) <= TOL


@pytest.mark.parametrize("M,N,K", [(129, 36864, 768), (98, 32768, 1024), (120, 33000, 768)])
def test_gemm_streaming_single_split(M, N, K):
    """fam_gemm at 64 < M <= 144 rows against N >= 32768 columns (the stacked context K/V of every
    block) runs the streaming split-K kernel in one split, which adds the bias and stores bf16
    rows itself: against the oracle, and bit-identical to that kernel's fp32 plane + the row
    kernel's bias (both round sum + bias once).  7, 8 and 9 m-tiles; a ragged last column block."""
    from fam import _capi
    assert _capi.lib().fam_gemm_partial_splits(M, N, K) == 1
    x, w, b = rnd(M, K, seed=81), rnd(N, K, seed=82, scale=0.05), rnd(N, seed=83, scale=0.05)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops().gemm(dev(x), dev(w), dev(b), y)
    assert relerr(y, O.linear(x.float(), w.float(), b.float())) <= TOL
    part, S = ops().gemm_partial(dev(x), dev(w))
    y2 = torch.empty_like(y)
    ops().rowop(y2, partials=part, bias=dev(b))
    assert S == 1 and torch.equal(y, y2)


@pytest.mark.parametrize("M,N,K,epi", [(392, 640, 5760, "bias_res"), (1568, 640, 2880, "gelu"), (392, 392, 640, "f32"),
                                       (200, 96, 1024, "gate_res"), (4096, 4096, 128, "bias_res")])
def test_gemm_ws_split_k(M, N, K, epi):
    """fam_gemm_ws: few output tiles over a long K split over workgroups (the VAE encoder's deep
    levels), the fp32 planes summed in split order with the epilogue; deterministic; the same
    product as fam_gemm within bf16 rounding; a workspace too small for two planes is fam_gemm."""
    from fam import _capi
    x, w, b = rnd(M, K, seed=91), rnd(N, K, seed=92, scale=0.05), rnd(N, seed=93, scale=0.05)
    res, gate = rnd(M, N, seed=94), rnd(M, N, seed=95, scale=0.3)
    lin = O.linear(x.float(), w.float(), b.float())
    kw, ref = {}, lin
    if epi == "bias_res":
        kw, ref = dict(res=dev(res)), res.float() + lin
    elif epi == "gelu":
        kw, ref = dict(act=_capi.FAM_ACT_GELU_TANH), O.gelu_tanh(lin)
    elif epi == "gate_res":
        kw = dict(res=dev(res), gate=dev(gate), gate_bs=0, gate_rs=N, gate_ns=1, rows_per_batch=M)
        ref = res.float() + gate.float() * lin
    dt = torch.float32 if epi == "f32" else torch.bfloat16
    ws = torch.empty(ops().gemm_ws_floats(M, N, K) or 4, dtype=torch.float32, device="cuda")
    outs = []
    for _ in range(2):
        y = torch.empty(M, N, dtype=dt, device="cuda")
        ops().gemm(dev(x), dev(w), dev(b), y, out_f32=(epi == "f32"), ws=ws, **kw)
        outs.append(y)
    assert relerr(outs[0], ref) <= TOL
    assert torch.equal(outs[0], outs[1])
    y1 = torch.empty(M, N, dtype=dt, device="cuda")
    ops().gemm(dev(x), dev(w), dev(b), y1, out_f32=(epi == "f32"), **kw)
    y2 = torch.empty(M, N, dtype=dt, device="cuda")
    ops().gemm(dev(x), dev(w), dev(b), y2, out_f32=(epi == "f32"), ws=ws[:M * N - 1], **kw)
    assert torch.equal(y1, y2)
    assert relerr(outs[0], y1.float().cpu()) <= TOL


def test_gemm_fp32_residual_out():
    """out_f32: fp32 residual and output (the fused Euler update of fp32 latents)."""
    M, N, K = 32, 7, 1024
    x, w, b = rnd(M, K, seed=61), rnd(N, K, seed=62, scale=0.02), rnd(N, seed=63, scale=0.02)
    lat = torch.randn(M, N, generator=torch.Generator().manual_seed(64))
    delta = torch.tensor([-0.0217], dtype=torch.bfloat16)
    ref = lat + delta.float() * O.linear(x.float(), w.float(), b.float())
    out = dev(lat.clone())
    d_d = dev(delta)
    ops().gemm(dev(x), dev(w), dev(b), out, res=out, gate=d_d, gate_bs=0, gate_rs=0, gate_ns=0, out_f32=True)
    assert (out.cpu() - ref).abs().max().item() <= 1e-4


@pytest.mark.parametrize("M,rpb", [(32, 32), (96, 32)])
def test_gemm_adaln_prologue_gate_residual(M, rpb):
    """[AdaLN + GEMM] and [GEMM + gate * y + residual] as used by the block (FB/wan_video_dit.py:281-285)."""
    from fam import _capi
    K, N = 1024, 3072
    B = M // rpb
    x = rnd(M, K, seed=42, scale=1.5)
    sh, sc = rnd(B, K, seed=43, scale=0.1), rnd(B, K, seed=44, scale=0.1)
    w, b = rnd(N, K, seed=45, scale=0.02), rnd(N, seed=46, scale=0.02)
    xb = x.float().reshape(B, rpb, K)
    h = O.adaln(xb, sh.float()[:, None], sc.float()[:, None], 1e-6).reshape(M, K)
    ref = O.linear(h, w.float(), b.float())
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops().gemm(dev(x), dev(w), dev(b), y, prologue=_capi.FAM_PRO_ADALN, pro_shift=dev(sh), pro_scale=dev(sc),
               pro_mod_bs=K, pro_mod_rs=0, rows_per_batch=rpb)
    assert relerr(y, ref) <= TOL

    # epilogue: out = res + gate[b] * gelu(a w^T + b)
    N2 = K
    w2, b2 = rnd(N2, N, seed=47, scale=0.02), rnd(N2, seed=48, scale=0.02)
    a2 = rnd(M, N, seed=49)
    res, gate = rnd(M, N2, seed=50), rnd(B, N2, seed=51, scale=0.2)
    v = O.gelu_tanh(O.linear(a2.float(), w2.float(), b2.float()))
    ref2 = res.float() + gate.float().repeat_interleave(rpb, 0) * v
    out = dev(res.clone())
    ops().gemm(dev(a2), dev(w2), dev(b2), out, act=_capi.FAM_ACT_GELU_TANH, res=out, gate=dev(gate),
               gate_bs=N2, gate_rs=0, gate_ns=1, rows_per_batch=rpb)
    assert relerr(out, ref2) <= TOL


@pytest.mark.parametrize("M,K,N,kind", [(1, 768, 768, "adaln"), (17, 768, 2304, "adaln"), (17, 768, 3072, "ln_gelu"),
                                         (33, 1000, 520, "affine_res"), (64, 3072, 768, "adaln"), (16, 4096, 256, "ln_gelu")])
def test_gemm_folded_layernorm(M, K, N, kind):
    """FAM_PRO_LN_FOLDED: rstd (x w'^T - mean colsum) + bias' with the affine / modulation folded by
    fam.ops.fold_layernorm, against LN -> (affine | AdaLN) -> linear (-> GELU, + residual) in fp32.
    Rows carry a mean offset of several standard deviations (the pivoted row sums keep the
    variance exact enough); K = 3072 / 4096 run in several chunks per wave."""
    from fam import _capi
    x = rnd(M, K, seed=60, scale=1.0)
    x = (x.float() + 4.0 * rnd(M, 1, seed=61).float()).to(torch.bfloat16)
    w, b = rnd(N, K, seed=62, scale=0.02), rnd(N, seed=63, scale=0.02)
    lw, lb = rnd(K, seed=64, scale=0.3).float() + 1, rnd(K, seed=65, scale=0.3).float()
    sc, sh = rnd(K, seed=66, scale=0.1), rnd(K, seed=67, scale=0.1)
    res = rnd(M, N, seed=68)
    eps = 1e-5
    if kind == "adaln":
        h = O.adaln(x.float()[None], sh.float()[None, None], sc.float()[None, None], eps)[0]
        fold = dict(scale=dev(sc), shift=dev(sh))
    elif kind == "affine_res":
        h = O.layer_norm(x.float(), lw, lb, eps)
        fold = dict(ln_weight=dev(lw), ln_bias=dev(lb))
    else:
        h = O.layer_norm(x.float(), None, None, eps)
        fold = {}
    ref = O.linear(h, w.float(), b.float())
    if kind == "ln_gelu":
        ref = O.gelu_tanh(ref)
    if kind == "affine_res":
        ref = res.float() + ref
    w2, b2, cs = ops().fold_layernorm(dev(w), dev(b), **fold)
    y = dev(res.clone()) if kind == "affine_res" else torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops().gemm(dev(x), w2, b2, y, prologue=_capi.FAM_PRO_LN_FOLDED, pro_w=cs, pro_eps=eps,
               act=_capi.FAM_ACT_GELU_TANH if kind == "ln_gelu" else _capi.FAM_ACT_NONE,
               res=y if kind == "affine_res" else None)
    err = relerr(y, ref)
    print(f"folded LN M={M} K={K} N={N} {kind}: relerr {err:.3e}")
    assert err <= TOL


def test_gemm_folded_layernorm_rejects():
    from fam import _capi
    x = torch.zeros(65, 64, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(16, 64, dtype=torch.bfloat16, device="cuda")
    cs = torch.zeros(16, dtype=torch.float32, device="cuda")
    y = torch.empty(65, 16, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_capi.FamError):
        ops().gemm(x, w, None, y, prologue=_capi.FAM_PRO_LN_FOLDED, pro_w=cs)   # M > 64
    with pytest.raises(ValueError):
        ops().gemm(x[:8], w, None, y[:8], prologue=_capi.FAM_PRO_LN_FOLDED, pro_w=cs.to(torch.bfloat16))


def test_gemm_layernorm_affine_prologue():
    from fam import _capi
    M, K, N = 64, 1024, 1024
    x = rnd(M, K, seed=52)
    lw, lb = rnd(K, seed=53, scale=0.3) + 1, rnd(K, seed=54, scale=0.3)
    w, b = rnd(N, K, seed=55, scale=0.02), rnd(N, seed=56, scale=0.02)
    ref = O.linear(O.layer_norm(x.float(), lw.float(), lb.float(), 1e-6), w.float(), b.float())
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops().gemm(dev(x), dev(w), dev(b), y, prologue=_capi.FAM_PRO_LAYERNORM, pro_w=dev(lw), pro_b=dev(lb))
    assert relerr(y, ref) <= TOL


# --------------------------------------------------------------------------- sampler and small kernels
def test_euler_step():
    x, v = rnd(4, 32, 7, seed=57), rnd(4, 32, 7, seed=58)
    d = torch.tensor(-0.0217, dtype=torch.bfloat16)
    ref = O.scheduler_step(v, d, x)   # bf16 eager arithmetic: exact match expected
    y = ops().euler_step(dev(v), dev(d), dev(x))
    assert torch.equal(y.cpu(), ref)
    dB = torch.tensor([-0.1, -0.2, -0.3, -0.4], dtype=torch.bfloat16)
    refB = O.scheduler_step(v, dB, x)
    assert torch.equal(ops().euler_step(dev(v), dev(dB), dev(x)).cpu(), refB)
    # element counts off the 8-element vector path (scalar kernel) and a many-block vector case
    for shape, nb in (((3, 5, 7), 3), ((8, 129, 64), 8)):
        xs, vs = rnd(*shape, seed=59), rnd(*shape, seed=60)
        dd = (torch.arange(nb, dtype=torch.float32) * -0.05 - 0.01).to(torch.bfloat16)
        assert torch.equal(ops().euler_step(dev(vs), dev(dd), dev(xs)).cpu(), O.scheduler_step(vs, dd, xs))
    sched = ops().WanContinuousFlowMatchScheduler(shift=5.0)
    ts, ds = sched.build_inference_schedule(10, "cuda", torch.bfloat16)
    ots, ods = O.build_inference_schedule(10, 5.0, torch.bfloat16)
    assert torch.equal(ts.cpu(), ots) and torch.equal(ds.cpu(), ods)


def test_sinusoid_and_modulation():
    from fam import _capi
    ts, _ = O.build_inference_schedule(10, 5.0, torch.bfloat16)
    ts_d = dev(ts)  # device copies stay referenced until the launches have run
    out = torch.empty(10, 256, dtype=torch.bfloat16, device="cuda")
    _capi.call("fam_sinusoid", ts_d.data_ptr(), out.data_ptr(), 10, 256, torch.cuda.current_stream().cuda_stream)
    ref = O.sinusoidal_embedding_1d(256, ts)
    assert (out.cpu().float() - ref.float()).abs().max().item() <= 2 ** -8
    tm, mod = rnd(3, 48, seed=59), rnd(5, 48, seed=60)
    tm_d, mod_d = dev(tm), dev(mod)
    o = torch.empty(3, 5, 48, dtype=torch.bfloat16, device="cuda")
    _capi.call("fam_add_modulation", tm_d.data_ptr(), mod_d.data_ptr(), o.data_ptr(), 3, 5, 48,
               torch.cuda.current_stream().cuda_stream)
    assert torch.equal(o.cpu(), mod[None] + tm[:, None])


# --------------------------------------------------------------------------- split-K partials + row kernel
@pytest.mark.parametrize("M,N,K", [(32, 3072, 1024), (32, 1024, 4096), (32, 7, 1024), (1, 64, 8), (7, 1000, 256),
                                    (64, 4096, 1024), (17, 2048, 1000), (33, 96, 64), (98, 3072, 3072),
                                    (98, 3072, 14336), (128, 4090, 3000), (65, 1000, 1024), (100, 4096, 520),
                                    (98, 14336, 3072), (128, 9216, 3072), (77, 6004, 4104), (77, 4094, 4104),
                                    (98, 3000, 3072), (128, 3072, 3080), (129, 12288, 3072), (140, 20000, 1600),
                                    (32, 9216, 1024), (32, 1024, 3072), (16, 6000, 1000), (64, 4100, 1048),
                                    (40, 2048, 2056), (16, 4002, 1000),
                                    (1024, 1024, 4096), (1024, 3072, 1024), (200, 68, 192), (1560, 3072, 14336)])
def test_gemm_partial_rowop(M, N, K):
    """Split-K partials summed in split order by the row kernel = linear; bit-identical reruns.
    Above 64 rows: the streaming kernel where a one-round grid gives every workgroup >= 3
    chunks of 256 along K ((98, 3072, 14336): 10 planes; FFN up (98, 14336, 3072) with a
    14336-wide row finished over several row-kernel workgroups; 8 m-tiles at 128 rows; a
    ragged last column block and a K tail at (77, 6004 / 4094, 4104); 64-column workgroups for
    the 3072 x 3072 projections, with a ragged block at N=3000 and a K tail at 128 rows; 9
    m-tiles for 129-144 rows, ragged and with a K tail at (140, 20000, 1600)), the
    wide kernel (a
    512-wide K slice per workgroup, activations staged in LDS) and the 8-m-tile register
    kernel where neither fills the chip.  At <= 64 rows the wide kernel with two strips per
    workgroup for the large action projections (the real model's 9216 x 1024 q|k|v and
    1024 x 3072 o), with 1, 2 and 4 m-tiles, rows past M in a tile, ragged N (also N % 4 != 0)
    and K tails.  Above 144 rows the large-M tile kernel writes the planes: 2 K splits at config
    1's B=32 FFN down (1024 x 1024 x 4096), one plain fp32 plane at its q|k|v (1024 x 3072 x 1024),
    a ragged 200 x 68 product, 3 splits at config 2's FFN down."""
    x, w, b = rnd(M, K, seed=70), rnd(N, K, seed=71, scale=0.02), rnd(N, seed=72, scale=0.02)
    ref = O.linear(x.float(), w.float(), b.float())
    xd, wd, bd = dev(x), dev(w), dev(b)
    outs = []
    for _ in range(2):
        part, S = ops().gemm_partial(xd, wd)
        assert S >= 1 and part.shape == (S, M, N)
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        ops().rowop(y, partials=part, bias=bd)
        outs.append(y)
    assert relerr(outs[0], ref) <= TOL
    assert torch.equal(outs[0], outs[1])
    # the partials alone add up to the product (fp32 sum of the split planes)
    assert relerr(part.sum(0), O.linear(x.float(), w.float(), None)) <= 1e-3


@pytest.mark.parametrize("M,H", [(98, 24), (40, 4)])
def test_gemm_partial_qkv_windows(M, H):
    """One split-K product for q|k|v finished by three row-kernel windows of its planes (rows
    3A wide): q and k RMS-normalised over their A columns and rotated, v with its bias only
    (FB/wan_video_dit.py:116-131 on the fused projection, rope_apply :49-55)."""
    from fam import _capi
    Dh = 128
    A, K = H * Dh, 3072 if H == 24 else 512
    x, w, b = rnd(M, K, seed=90), rnd(3 * A, K, seed=91, scale=0.02), rnd(3 * A, seed=92, scale=0.02)
    wq, wk = rnd(A, seed=93, scale=0.2) + 1, rnd(A, seed=94, scale=0.2) + 1
    fr = O.action_freqs(Dh, M)
    cs, sn, trs, tes = ops().rope_tables(fr, "complex", torch.device("cuda"))
    part, _ = ops().gemm_partial(dev(x), dev(w))
    qkv = torch.empty(M, 3 * A, dtype=torch.bfloat16, device="cuda")
    bd = dev(b)
    for i, nw in ((1, dev(wk)), (2, None), (0, dev(wq))):
        o = qkv[:, i * A:(i + 1) * A]
        if nw is None:
            ops().rowop(o, partials=part, bias=bd[i * A:], col0=i * A)
        else:
            ops().rowop(o, partials=part, bias=bd[i * A:], col0=i * A, norm=_capi.FAM_ROWNORM_RMS, eps=1e-6,
                        segs=[(0, nw)], seg_width=A, rope=(cs, sn, trs, tes, Dh, M), nout=o)
    lin = O.linear(x.float(), w.float(), b.float()).to(torch.bfloat16).float()
    qr = O.rope_apply(O.rms_norm(lin[None, :, :A], wq.float(), 1e-6), fr, H)[0]
    kr = O.rope_apply(O.rms_norm(lin[None, :, A:2 * A], wk.float(), 1e-6), fr, H)[0]
    y = qkv.cpu()
    assert relerr(y[:, :A], qr) <= TOL
    assert relerr(y[:, A:2 * A], kr) <= TOL
    assert relerr(y[:, 2 * A:], lin[:, 2 * A:]) <= TOL
    with pytest.raises(ValueError):
        ops().rowop(qkv[:, :A], partials=part, bias=bd, col0=2 * A + 1)


@pytest.mark.parametrize("M,rpb", [(32, 32), (96, 32)])
def test_rowop_gelu_gate_residual_adaln(M, rpb):
    """out = res + gate[b] * gelu(a w^T + b), then AdaLN(out) for the next block (FB/wan_video_dit.py:281-288)."""
    from fam import _capi
    K, N = 4096, 1024
    B = M // rpb
    a, w, b = rnd(M, K, seed=73), rnd(N, K, seed=74, scale=0.02), rnd(N, seed=75, scale=0.02)
    res, gate = rnd(M, N, seed=76), rnd(B, N, seed=77, scale=0.2)
    sh, sc = rnd(B, N, seed=78, scale=0.1), rnd(B, N, seed=79, scale=0.1)
    ref = res.float() + gate.float().repeat_interleave(rpb, 0) * O.gelu_tanh(O.linear(a.float(), w.float(), b.float()))
    ad, wd = dev(a), dev(w)
    out, h = dev(res.clone()), torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    bd, gd, shd, scd = dev(b), dev(gate), dev(sh), dev(sc)
    for m0 in range(0, M, 64):  # partials cover <= 64 rows per call
        m1 = min(M, m0 + 64)
        part, _ = ops().gemm_partial(ad[m0:m1], wd)
        ops().rowop(out[m0:m1], partials=part, bias=bd, act=_capi.FAM_ACT_GELU_TANH, res=out[m0:m1],
                    gate=gd[m0 // rpb:], gate_strides=(N, 0, 1), rows_per_batch=rpb,
                    norm=_capi.FAM_ROWNORM_ADALN, eps=1e-6, shift=shd[m0 // rpb:], scale=scd[m0 // rpb:],
                    mod_strides=(N, 0), nout=h[m0:m1])
    assert relerr(out, ref) <= TOL
    ob = out.float().cpu().reshape(B, rpb, N)  # the norm reads the stored bf16 row
    href = O.adaln(ob, sh.float()[:, None], sc.float()[:, None], 1e-6).reshape(M, N)
    assert relerr(h, href) <= TOL


def test_rowop_layernorm_affine():
    from fam import _capi
    M, K, N = 32, 1024, 1024
    a, w, b = rnd(M, K, seed=80), rnd(N, K, seed=81, scale=0.02), rnd(N, seed=82, scale=0.02)
    lw, lb = rnd(N, seed=83, scale=0.3) + 1, rnd(N, seed=84, scale=0.3)
    part, _ = ops().gemm_partial(dev(a), dev(w))
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(out)
    lwd, lbd, bd = dev(lw), dev(lb), dev(b)
    ops().rowop(out, partials=part, bias=bd, norm=_capi.FAM_ROWNORM_LAYERNORM, eps=1e-6, ln_w=lwd, ln_b=lbd, nout=h)
    assert relerr(out, O.linear(a.float(), w.float(), b.float())) <= TOL
    assert relerr(h, O.layer_norm(out.float().cpu(), lw.float(), lb.float(), 1e-6)) <= TOL


def test_rowop_rms_segments_rope():
    """Fused QKV row: q and k segments RMS-normalised and rotated, v passed through
    (FB/wan_video_dit.py:116-131 with rope_apply :49-55)."""
    from fam import _capi
    S, H, Dh, K = 32, 16, 64, 1024
    A = H * Dh
    a, w, b = rnd(S, K, seed=85), rnd(3 * A, K, seed=86, scale=0.02), rnd(3 * A, seed=87, scale=0.02)
    wq, wk = rnd(A, seed=88, scale=0.2) + 1, rnd(A, seed=89, scale=0.2) + 1
    fr = O.action_freqs(Dh, S)
    cs, sn, trs, tes = ops().rope_tables(fr, "complex", torch.device("cuda"))
    part, _ = ops().gemm_partial(dev(a), dev(w))
    qkv = torch.empty(S, 3 * A, dtype=torch.bfloat16, device="cuda")
    wqd, wkd, bd = dev(wq), dev(wk), dev(b)
    ops().rowop(qkv, partials=part, bias=bd, norm=_capi.FAM_ROWNORM_RMS, eps=1e-6, segs=[(0, wqd), (A, wkd)],
                seg_width=A, rope=(cs, sn, trs, tes, Dh, S), nout=qkv)
    lin = O.linear(a.float(), w.float(), b.float()).to(torch.bfloat16).float()
    qr = O.rope_apply(O.rms_norm(lin[None, :, :A], wq.float(), 1e-6), fr, H)[0]
    kr = O.rope_apply(O.rms_norm(lin[None, :, A:2 * A], wk.float(), 1e-6), fr, H)[0]
    y = qkv.cpu()
    assert relerr(y[:, :A], qr) <= TOL
    assert relerr(y[:, A:2 * A], kr) <= TOL
    assert relerr(y[:, 2 * A:], lin[:, 2 * A:]) <= TOL


def test_rowop_smallk_source_fp32_input():
    """Small-K source (the 7-wide action encoder on fp32 latents) + AdaLN of the result."""
    from fam import _capi
    M, K, N = 32, 7, 1024
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(90))
    w, b = rnd(N, K, seed=91, scale=0.3), rnd(N, seed=92, scale=0.02)
    sh, sc = rnd(1, N, seed=93, scale=0.1), rnd(1, N, seed=94, scale=0.1)
    xd, wd, bd, shd, scd = dev(x), dev(w), dev(b), dev(sh), dev(sc)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(out)
    ops().rowop(out, x_in=xd, w_in=wd, bias=bd, norm=_capi.FAM_ROWNORM_ADALN, eps=1e-6, shift=shd, scale=scd,
                mod_strides=(N, 0), nout=h)
    assert relerr(out, O.linear(x, w.float(), b.float())) <= TOL
    assert relerr(h, O.adaln(out.float().cpu(), sh.float(), sc.float(), 1e-6)) <= TOL


def test_rowop_fp32_euler_update():
    """Head projection + Euler step on fp32 latents: lat += delta * (a w^T + b)."""
    M, N, K = 32, 7, 1024
    a, w, b = rnd(M, K, seed=95), rnd(N, K, seed=96, scale=0.02), rnd(N, seed=97, scale=0.02)
    lat = torch.randn(M, N, generator=torch.Generator().manual_seed(98))
    delta = torch.tensor([-0.0217], dtype=torch.bfloat16)
    ref = lat + delta.float() * O.linear(a.float(), w.float(), b.float())
    part, _ = ops().gemm_partial(dev(a), dev(w))
    out, dd, bd = dev(lat.clone()), dev(delta), dev(b)
    ops().rowop(out, partials=part, bias=bd, res=out, gate=dd, gate_strides=(0, 0, 0))
    assert (out.cpu() - ref).abs().max().item() <= 1e-4


# --------------------------------------------------------------------------- attention key splits
@pytest.mark.parametrize("Sq,Sk,splits", [(32, 1560, 13), (32, 1560, 4), (16, 129, 2), (32, 100, 8), (1, 77, 3)])
def test_attention_key_splits(Sq, Sk, splits):
    """Keys divided among workgroups, partials merged by the combine kernel in split order:
    matches the oracle, the unsplit kernel and itself bit for bit."""
    B, H, Dh = 1, 16, 64
    q, k, v = rnd(B, Sq, H * Dh, seed=99), rnd(B, Sk, H * Dh, seed=100), rnd(B, Sk, H * Dh, seed=101)
    ref = O.flash_attention(q.float(), k.float(), v.float(), H)
    qd, kd, vd = dev(q), dev(k), dev(v)
    y1 = ops().attention_bshd(qd, kd, vd, H, num_splits=splits)
    y2 = ops().attention_bshd(qd, kd, vd, H, num_splits=splits)
    y0 = ops().attention_bshd(qd, kd, vd, H)
    assert relerr(y1, ref) <= TOL
    assert torch.equal(y1, y2)
    assert relerr(y1, y0.float().cpu()) <= TOL


def test_attention_key_splits_masked_rows():
    """A split whose keys are all masked contributes nothing; a fully masked row stays 0."""
    B, H, Sq, Sk, Dh = 2, 4, 8, 300, 128
    q, k, v = rnd(B, Sq, H * Dh, seed=102), rnd(B, Sk, H * Dh, seed=103), rnd(B, Sk, H * Dh, seed=104)
    m = torch.ones(B, 1, Sq, Sk, dtype=torch.bool)
    m[:, :, :, 100:] = False      # splits past key 100 are fully masked
    m[:, :, 2] = False            # fully masked row
    ref = O.flash_attention(q.float(), k.float(), v.float(), H, m)
    y = ops().attention_bshd(dev(q), dev(k), dev(v), H, mask=dev(m), num_splits=3)
    assert relerr(y, ref) <= TOL
    assert torch.all(y[:, 2] == 0)


def test_rowop_generic_path_matches_vector_path():
    """Rows that do not start on a 4-column boundary take the per-element kernel: same
    stored row (same split order), same normalised row within rounding."""
    from fam import _capi
    M, K, N = 32, 1024, 1024
    a, w, b = rnd(M, K, seed=105), rnd(N, K, seed=106, scale=0.02), rnd(N, seed=107, scale=0.02)
    res = rnd(M, N, seed=108)
    sh, sc = rnd(1, N, seed=109, scale=0.1), rnd(1, N, seed=110, scale=0.1)
    part, _ = ops().gemm_partial(dev(a), dev(w))
    bd, shd, scd = dev(b), dev(sh), dev(sc)
    outs = []
    for pad in (0, 2):   # pad 2: row pitch N + 2 is not a multiple of 4 columns
        buf = torch.zeros(M, N + pad, dtype=torch.bfloat16, device="cuda")
        out = buf[:, :N]
        out.copy_(dev(res))
        h = torch.zeros(M, N + pad, dtype=torch.bfloat16, device="cuda")[:, :N]
        ops().rowop(out, partials=part, bias=bd, res=out, norm=_capi.FAM_ROWNORM_ADALN, eps=1e-6,
                    shift=shd, scale=scd, mod_strides=(N, 0), nout=h)
        outs.append((out.cpu(), h.cpu()))
    assert torch.equal(outs[0][0], outs[1][0])
    assert relerr(outs[1][1], outs[0][1].float()) <= 1e-2


def test_launch_events_time_the_kernel():
    """fam_set_launch_events arms a start/stop pair recorded at a kernel's own begin and end."""
    from fam import _capi
    lib = _capi.lib()
    x, w = dev(rnd(32, 1024, seed=111)), dev(rnd(1024, 1024, seed=112))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st = torch.cuda.current_stream()
    e0.record(st)
    e1.record(st)
    torch.cuda.synchronize()
    assert lib.fam_set_launch_events(e0.cuda_event, e1.cuda_event) == 0
    try:
        part, _ = ops().gemm_partial(x, w)
    finally:
        lib.fam_set_launch_events(None, None)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3
    assert 0.0 < us < 1e4
    assert relerr(part.sum(0), O.linear(x.float().cpu(), w.float().cpu(), None)) <= 1e-3


@pytest.mark.parametrize("M,N,K,act", [(32, 4096, 1024, 1), (32, 3072, 1024, 0), (32, 1024, 4096, 0), (7, 1000, 256, 2),
                                        (64, 96, 2048, 1), (1, 16, 8, 0), (17, 30, 4000, 0), (33, 1024, 3000, 1)])
def test_gemm_final(M, N, K, act):
    """Whole-K projection with bias/activation epilogue and per-16-column sums of squares."""
    x, w, b = rnd(M, K, seed=113), rnd(N, K, seed=114, scale=0.02), rnd(N, seed=115, scale=0.02)
    ref = O.linear(x.float(), w.float(), b.float())
    ref = O.gelu_tanh(ref) if act == 1 else (O.silu(ref) if act == 2 else ref)
    xd, wd, bd = dev(x), dev(w), dev(b)
    y, ss = ops().gemm_final(xd, wd, bd, act, want_sumsq=True)
    y2, ss2 = ops().gemm_final(xd, wd, bd, act, want_sumsq=True)
    assert relerr(y, ref) <= TOL
    assert torch.equal(y, y2) and torch.equal(ss, ss2)
    yf = y.float().cpu()
    G = (N + 15) // 16
    pad = torch.zeros(M, G * 16)
    pad[:, :N] = yf
    ss_ref = (pad * pad).reshape(M, G, 16).sum(-1)
    assert torch.allclose(ss.cpu(), ss_ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B", [1, 2])
def test_attention_qk_norm_on_load(B):
    """Raw q/k from fam_gemm_final + its sums of squares; attention applies RMSNorm (bf16
    before the weight) and RoPE to q and k as it loads them (FB/wan_video_dit.py:193-196)."""
    S, H, Dh, Kd = 32, 16, 64, 1024
    A = H * Dh
    x, w, bb = rnd(B * S, Kd, seed=116), rnd(3 * A, Kd, seed=117, scale=0.02), rnd(3 * A, seed=118, scale=0.02)
    wq, wk = rnd(A, seed=119, scale=0.2) + 1, rnd(A, seed=120, scale=0.2) + 1
    fr = O.action_freqs(Dh, S)
    qkv, ss = ops().gemm_final(dev(x), dev(w), dev(bb), want_sumsq=True)
    cs, sn, trs, _ = ops().rope_tables(fr, "complex", torch.device("cuda"))
    wqd, wkd = dev(wq), dev(wk)
    q3 = qkv.view(B, S, 3 * A)
    y = ops().attention_bshd(q3[:, :, :A], q3[:, :, A:2 * A], q3[:, :, 2 * A:], H,
                             qk_norm=dict(q_sumsq=ss, k_sumsq=ss, ss_batch_rows=S, q_group0=0, k_group0=A // 16,
                                          norm_width=A, q_norm_w=wqd, k_norm_w=wkd, eps=1e-6, rope=(cs, sn, trs)))
    raw = qkv.float().cpu().view(B, S, 3 * A)
    q = O.rope_apply(O.rms_norm(raw[..., :A].to(torch.bfloat16), wq, 1e-6).float(), fr, H)
    k = O.rope_apply(O.rms_norm(raw[..., A:2 * A].to(torch.bfloat16), wk, 1e-6).float(), fr, H)
    ref = O.flash_attention(q, k, raw[..., 2 * A:], H)
    assert relerr(y, ref) <= TOL


@pytest.mark.parametrize("S,H,Dh,Lc,splits", [(32, 16, 64, 1560, 13), (32, 16, 64, 1560, 1), (20, 8, 128, 777, 1)])
def test_attention_q_norm_cross_with_splits(S, H, Dh, Lc, splits):
    """Cross attention with the query normalised on load (no RoPE): 13 key splits + combine, or
    none (a head's output dims split over workgroups that each score every key)."""
    Kd = 1024
    A = H * Dh
    x, w, bb = rnd(S, Kd, seed=121), rnd(A, Kd, seed=122, scale=0.02), rnd(A, seed=123, scale=0.02)
    wq = rnd(A, seed=124, scale=0.2) + 1
    k, v = rnd(1, Lc, A, seed=125), rnd(1, Lc, A, seed=126)
    q_raw, ss = ops().gemm_final(dev(x), dev(w), dev(bb), want_sumsq=True)
    wqd, kd, vd = dev(wq), dev(k), dev(v)
    y = ops().attention_bshd(q_raw.view(1, S, A), kd, vd, H, num_splits=splits,
                             qk_norm=dict(q_sumsq=ss, ss_batch_rows=S, norm_width=A, q_norm_w=wqd, eps=1e-6))
    q = O.rms_norm(q_raw.cpu().view(1, S, A), wq, 1e-6).float()
    ref = O.flash_attention(q, k.float(), v.float(), H)
    assert relerr(y, ref) <= TOL


@pytest.mark.parametrize("B,Sq,Sk,H,Dh", [(1, 32, 32, 16, 64), (2, 20, 27, 4, 64), (1, 32, 32, 24, 128), (3, 7, 1, 2, 128)])
def test_attention_self_small(B, Sq, Sk, H, Dh):
    """The action tokens' own attention (Sq, Sk <= 32, no mask): the LDS-staged kernel."""
    q, k, v = rnd(B, Sq, H * Dh, seed=127), rnd(B, Sk, H * Dh, seed=128), rnd(B, Sk, H * Dh, seed=129)
    ref = O.flash_attention(q.float(), k.float(), v.float(), H)
    y = ops().attention_bshd(dev(q), dev(k), dev(v), H)
    assert relerr(y, ref) <= TOL


def test_attention_qk_norm_on_load_wide_heads():
    """Real FastWAM action-expert attention width (24 x 128 = 3072) with q/k norm + RoPE on load."""
    S, H, Dh, Kd = 32, 24, 128, 1024
    A = H * Dh
    x, w, bb = rnd(S, Kd, seed=130), rnd(3 * A, Kd, seed=131, scale=0.02), rnd(3 * A, seed=132, scale=0.02)
    wq, wk = rnd(A, seed=133, scale=0.2) + 1, rnd(A, seed=134, scale=0.2) + 1
    fr = O.action_freqs(Dh, S)
    qkv, ss = ops().gemm_final(dev(x), dev(w), dev(bb), want_sumsq=True)
    cs, sn, trs, _ = ops().rope_tables(fr, "complex", torch.device("cuda"))
    wqd, wkd = dev(wq), dev(wk)
    q3 = qkv.view(1, S, 3 * A)
    y = ops().attention_bshd(q3[:, :, :A], q3[:, :, A:2 * A], q3[:, :, 2 * A:], H,
                             qk_norm=dict(q_sumsq=ss, k_sumsq=ss, ss_batch_rows=S, q_group0=0, k_group0=A // 16,
                                          norm_width=A, q_norm_w=wqd, k_norm_w=wkd, eps=1e-6, rope=(cs, sn, trs)))
    raw = qkv.float().cpu().view(1, S, 3 * A)
    q = O.rope_apply(O.rms_norm(raw[..., :A].to(torch.bfloat16), wq, 1e-6).float(), fr, H)
    k = O.rope_apply(O.rms_norm(raw[..., A:2 * A].to(torch.bfloat16), wk, 1e-6).float(), fr, H)
    ref = O.flash_attention(q, k, raw[..., 2 * A:], H)
    assert relerr(y, ref) <= TOL


@pytest.mark.parametrize("B,H,Sq,Sk,Dh,kind", [(2, 4, 200, 333, 64, "random"), (1, 24, 1560, 512, 128, "tail"),
                                                (2, 3, 129, 300, 128, "head"), (2, 4, 200, 333, 128, "random")])
def test_attention_long_key_mask(B, H, Sq, Sk, Dh, kind):
    """Video tokens over a padded context: a bool key mask shared by the queries ([B, 1, 1, Sk],
    the cross-attention's text mask) on the long kernel.  "head" masks the first 70 keys of the
    second sample, so its first 64-key tile is all masked (running max still -inf).  At head dim
    128 a grid of at most one workgroup per CU (every case here but the 1560-query one) runs two
    key groups per workgroup whose softmax states merge at the end."""
    q, k, v = rnd(B, Sq, H * Dh, seed=138), rnd(B, Sk, H * Dh, seed=139), rnd(B, Sk, H * Dh, seed=140)
    g = torch.Generator().manual_seed(141)
    mask = torch.ones(B, 1, 1, Sk, dtype=torch.bool)
    if kind == "random":
        mask = torch.rand(B, 1, 1, Sk, generator=g) > 0.3
    elif kind == "tail":
        mask[..., Sk - 37:] = False
    else:
        mask[1, ..., :70] = False
    ref = O.flash_attention(q.float(), k.float(), v.float(), H, mask)
    y = ops().flash_attention(dev(q), dev(k), dev(v), H, ctx_mask=dev(mask))
    assert relerr(y, ref) <= TOL


@pytest.mark.parametrize("B,H,Sq,Sk,Dh", [(1, 8, 1560, 1560, 128), (2, 4, 200, 333, 64), (1, 2, 129, 512, 128),
                                           (1, 3, 65, 1, 128), (1, 2, 129, 192, 128), (2, 3, 130, 330, 128),
                                           (1, 1, 300, 64, 128), (1, 24, 1560, 200, 128)])
def test_attention_long_sequences(B, H, Sq, Sk, Dh):
    """Video-token attention (Sq > 64, no mask): 128-query workgroups, 64-key LDS tiles, 32x32 MFMA.
    The loop takes two tiles per iteration with the partial last tile separate, so the cases cover
    an even and an odd number of full tiles, each with and without a partial tile, a partial tile
    alone (Sk = 1) and a single full tile.  At head dim 128 grids of at most one workgroup per CU
    split each workgroup's tiles between two key groups (odd tile counts leave the second group a
    stage without a tile; Sk <= 64 leaves it none); 24 heads x 1560 queries (312 workgroups)
    takes the one-group kernel."""
    q, k, v = rnd(B, Sq, H * Dh, seed=135), rnd(B, Sk, H * Dh, seed=136), rnd(B, Sk, H * Dh, seed=137)
    ref = O.flash_attention(q.float(), k.float(), v.float(), H)
    y = ops().flash_attention(dev(q), dev(k), dev(v), H)
    assert relerr(y, ref) <= TOL


# --------------------------------------------------------------------------- rows past the end
def _nan_tailed(rows, cols, pad, seed, scale=1.0):
    """[rows + pad, cols] bf16 whose first `rows` rows are N(0, scale) and the rest NaN: a view of
    the first rows has NaN right after its last row, inside the same allocation."""
    buf = torch.full((rows + pad, cols), float("nan"), dtype=torch.bfloat16)
    buf[:rows] = rnd(rows, cols, seed=seed, scale=scale)
    return buf


@pytest.mark.parametrize("B,H,Sq,Sk,Dh,masked", [(1, 4, 200, 333, 128, False), (1, 4, 200, 333, 64, False),
                                                  (1, 24, 1560, 200, 128, False), (1, 4, 200, 333, 128, True)])
def test_attention_long_keys_past_the_end_read_as_zero(B, H, Sq, Sk, Dh, masked):
    """K and V are column windows of one [Sk + 64, 3A] q|k|v buffer whose rows past Sk are NaN (as
    config 2's self attention reads them from its projection output).  The partial last 64-key
    tile must not read those rows: 0 x NaN from a masked key's V would reach the stored output,
    and a NaN score stays NaN under the key mask."""
    A = H * Dh
    qkv = _nan_tailed(Sk, 3 * A, 64, seed=150).reshape(1, Sk + 64, 3 * A)
    q = rnd(B, Sq, A, seed=151)
    k, v = qkv[:, :Sk, A:2 * A], qkv[:, :Sk, 2 * A:]
    mask = None
    if masked:
        mask = torch.ones(1, 1, 1, Sk, dtype=torch.bool)
        mask[..., Sk - 29:] = False
    ref = O.flash_attention(q.float(), k.float(), v.float(), H, mask)
    qkv_d = dev(qkv)
    y = ops().flash_attention(dev(q), qkv_d[:, :Sk, A:2 * A], qkv_d[:, :Sk, 2 * A:], H,
                              ctx_mask=None if mask is None else dev(mask))
    assert relerr(y, ref) <= TOL   # relerr asserts the output is finite


@pytest.mark.parametrize("M,N,K", [(300, 520, 320), (1560, 3072, 1024), (98, 3072, 3072), (99, 4096, 1024)])
def test_gemm_rows_past_the_end_read_as_zero(M, N, K):
    """The activation and weight operands are views of the first M / N rows of buffers with NaN rows
    after them: the large-M tile kernel (tiles past M and N) and the 98-row streaming split-K kernel
    (row pairs, an odd M) must read zeros there, so every output is finite and equals the product."""
    a = _nan_tailed(M, K, 256, seed=152)
    w = _nan_tailed(N, K, 256, seed=153, scale=0.02)
    b = rnd(N, seed=154, scale=0.02)
    ref = O.linear(a[:M].float(), w[:N].float(), b.float())
    ad, wd, bd = dev(a), dev(w), dev(b)
    assert relerr(ops().linear(ad[:M], wd[:N], bd), ref) <= TOL
    part, _ = ops().gemm_partial(ad[:M], wd[:N])
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops().rowop(y, partials=part, bias=bd)
    assert relerr(y, ref) <= TOL

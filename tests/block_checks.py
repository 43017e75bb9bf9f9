"""Branch-level parity metrics for a video DiT block (FB/wan_video_dit.py:267-286).

A block's output is dominated by its residual stream and by the cross-attention and FFN
branches: on the config-2 shape, dropping the 3-D RoPE moves the whole output only 1.8e-2 and
the output minus the input 1.9e-2, both under the 2e-2 bar.  These metrics look inside the
block instead -- the rotated q and k, the v, each attention's output before its o projection,
and the output minus the input -- so that a dropped or transposed RoPE, a mis-strided head or a
zeroed self-attention fails (tests/test_oracle.py::test_block_branch_metrics_catch_planted_slips
shows each such slip moving one of them past the bar)."""
import torch

BAR = 2e-2


def rel(y, ref):
    """Normwise max relative error ||y - ref||_inf / ||ref||_inf (fp32, on the CPU)."""
    y, ref = y.detach().float().cpu(), ref.detach().float().cpu()
    assert y.shape == ref.shape, (tuple(y.shape), tuple(ref.shape))
    assert torch.isfinite(y).all(), "non-finite values"
    return ((y - ref).abs().max() / ref.abs().max().clamp_min(1e-12)).item()


def delta_rel(y, x, ref):
    """Normwise error of what the block adds: (y - x) against (ref - x)."""
    x = x.detach().float().cpu()
    return rel(y.detach().float().cpu() - x, ref.detach().float().cpu() - x)


def delta_bar(x, ref):
    """The bar for delta_rel: 2e-2 plus one bf16 rounding of the stored output (2^-8 of its
    largest magnitude) relative to the largest change.  The output is stored in bf16, so where a
    block adds little to a large residual stream, that rounding alone is a sizeable fraction of
    what it adds; where it adds as much as it carries (config 2) the bar stays near 2e-2."""
    x, ref = x.detach().float().cpu(), ref.detach().float().cpu()
    return BAR + 2.0 ** -8 * ref.abs().max().item() / (ref - x).abs().max().item()


def qkv_errors(qkv, trace, S, A):
    """Errors of a block's q | k | v buffer [B*S, 3A] (q and k normalised and rotated) against
    an oracle trace (fam_oracle.dit_block(..., trace=...))."""
    t = qkv.detach().float().cpu().reshape(-1, S, 3 * A)
    return {"q": rel(t[..., :A], trace["q"]), "k": rel(t[..., A:2 * A], trace["k"]),
            "v": rel(t[..., 2 * A:], trace["v"])}


def trace_errors(trace, ref_trace, x, y, ref):
    """The same metrics between two oracle traces (for planted-slip checks on the CPU)."""
    return {"q": rel(trace["q"], ref_trace["q"]), "k": rel(trace["k"], ref_trace["k"]),
            "v": rel(trace["v"], ref_trace["v"]), "self_attn": rel(trace["self_attn"], ref_trace["self_attn"]),
            "cross_attn": rel(trace["cross_attn"], ref_trace["cross_attn"]),
            "delta": delta_rel(y, x, ref) * BAR / delta_bar(x, ref)}


def gpu_block_errors(blk, x, t_mod, ctx, trace, y, ref):
    """The metrics of a fam.video_dit.FusedVideoDiTBlock whose forward(x, t_mod, ctx) gave y:
    what it adds (delta_rel scaled so that its own bar, delta_bar, reads as BAR), its q | k | v
    buffer after that run, then each attention's output before its o projection (eager launches
    up to that step, from the same inputs)."""
    S, A = blk.S, blk.A
    errs = {"delta": delta_rel(y, x, ref) * BAR / delta_bar(x, ref), **qkv_errors(blk.qkv, trace, S, A)}
    for name in ("self_attn", "cross_attn"):
        blk.set_inputs(x.cuda(), t_mod.cuda(), ctx.cuda())
        blk.run_until(name)
        errs[name] = rel(blk.attn.view(-1, S, A), trace[name])
    return errs

"""fam -- MI355X (gfx950) kernels for the FastWAM / DiT4DiT action-DiT denoising hot path.

`fam.ops` holds the drop-in operators with the reference's call signatures; `fam.action_dit`
the fused action expert and its denoise loop.  Both call the HIP library libfam_hip.so
through `fam._capi`; importing an operator module loads the library and fails loudly when
it has not been built.
"""
from ._capi import FamError, LIB_PATH, load  # noqa: F401

__all__ = ["FamError", "LIB_PATH", "load"]

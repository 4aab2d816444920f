"""Drop-in 3D convolution for AMD MI355X (gfx950) on hand-written HIP MFMA kernels.

Conv3d k=1 / k=3 (stride 1) and ConvTranspose3d k=2 s=2 run forward, dW and dX
on CDNA4 bf16/fp16 MFMA (fp32 accumulate) through the C-ABI library
librdna4_conv3d_hip.so.  Unsupported geometries, CPU tensors and non-gfx950
devices take the stock PyTorch path (F.conv3d).

The public names are those of the reference package
(src/rdna4_conv3d/__init__.py:10-37).
"""

from rdna4_conv3d.conv3d_wmma import (
    Conv3dWmma,
    ConvTranspose3dWmma,
    conv3d_plan,
    conv3d_wmma,
    swap_conv3d,
    wmma_dw,
    wmma_dx,
    wmma_fwd,
    wmma_ok_dw,
    wmma_ok_dx,
    wmma_ok_fwd,
)

__version__ = "0.1.0"
__all__ = [
    "Conv3dWmma",
    "ConvTranspose3dWmma",
    "conv3d_plan",
    "conv3d_wmma",
    "swap_conv3d",
    "wmma_dw",
    "wmma_dx",
    "wmma_fwd",
    "wmma_ok_dw",
    "wmma_ok_dx",
    "wmma_ok_fwd",
]

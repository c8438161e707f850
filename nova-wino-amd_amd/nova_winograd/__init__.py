"""
NOVA Winograd F(6,3) -- drop-in FP16 Winograd convolution for AMD Instinct
MI355X (gfx950), with hand-written HIP kernels behind the reference package's
Python surface (/root/reference/nova_winograd/__init__.py:20-36).

Quick start:
    from nova_winograd import NovaWinogradConv2d, replace_conv2d_with_nova

    conv = NovaWinogradConv2d(64, 128, kernel_size=3, padding=1).cuda()
    output = conv(input_fp16)

    replace_conv2d_with_nova(model)      # all eligible 3x3 stride-1 convs
    output = model(input_fp16)
"""

from nova_winograd.conv2d import (
    NovaWinogradConv2d,
    NovaWinogradConv2dTrainable,
    NovaWinogradConv2dCompilable,
)
from nova_winograd.ops import nova_forward, compute_tiling
from nova_winograd.surgery import replace_conv2d_with_nova

__version__ = "1.0.0"
__all__ = [
    "NovaWinogradConv2d",
    "NovaWinogradConv2dTrainable",
    "NovaWinogradConv2dCompilable",
    "nova_forward",
    "compute_tiling",
    "replace_conv2d_with_nova",
]

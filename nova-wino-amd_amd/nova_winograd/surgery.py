"""Model surgery: replace eligible nn.Conv2d layers with NOVA Winograd modules
(mirrors /root/reference/nova_winograd/surgery.py:9-53)."""

import torch.nn as nn

from nova_winograd.conv2d import NovaWinogradConv2d, NovaWinogradConv2dTrainable


def is_eligible(module):
    """3x3, stride 1, dilation 1, groups 1 (/root/reference/nova_winograd/surgery.py:33-40),
    plus what the reference does not check but its kernels assume: numeric,
    symmetric, zero padding."""
    if module.kernel_size != (3, 3) or module.stride != (1, 1):
        return False
    if module.dilation != (1, 1) or module.groups != 1:
        return False
    if isinstance(module.padding, str) or module.padding[0] != module.padding[1]:
        return False
    return module.padding_mode == "zeros"


def replace_conv2d_with_nova(model, trainable=False, verbose=True):
    """Replace all eligible nn.Conv2d layers with NovaWinogradConv2d, in place.

    Eligible layers: kernel_size=3, stride=1, dilation=1, groups=1 and
    symmetric zero padding. Other convolutions are skipped.

    Args:
        model:     nn.Module to modify (in-place).
        trainable: If True, use NovaWinogradConv2dTrainable (supports backward).
        verbose:   Print replacement summary.

    Returns:
        Number of layers replaced.
    """
    cls = NovaWinogradConv2dTrainable if trainable else NovaWinogradConv2d
    replaced = 0
    skipped = 0

    for name, module in list(model.named_modules()):
        if not isinstance(module, nn.Conv2d):
            continue
        if not is_eligible(module):
            skipped += 1
            continue

        nova_conv = cls.from_conv2d(module)
        parts = name.split(".")
        parent = model
        for p in parts[:-1]:
            parent = getattr(parent, p)
        setattr(parent, parts[-1], nova_conv)
        replaced += 1

    if verbose:
        print(f"NOVA: replaced {replaced} Conv2d layers, skipped {skipped} ineligible")

    return replaced

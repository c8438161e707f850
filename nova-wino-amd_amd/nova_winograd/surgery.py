"""In-place conversion of a model's eligible ``nn.Conv2d`` layers to NOVA
Winograd modules.

Interface kept from /root/reference/nova_winograd/surgery.py:9-53: the
function name, its arguments, the returned count and the one-line summary it
prints. The selection rule is stricter (see ``is_eligible``).
"""

import torch.nn as nn

from nova_winograd.conv2d import NovaWinogradConv2d, NovaWinogradConv2dTrainable


def is_eligible(conv):
    """Whether the NOVA kernels compute exactly what ``conv`` computes: a 3x3
    kernel at stride 1 without dilation or groups (the reference's test,
    /root/reference/nova_winograd/surgery.py:33-40), and -- which the
    reference leaves unchecked although its kernels assume it -- numeric,
    equal, zero-valued padding on both axes."""
    geometry = (conv.kernel_size, conv.stride, conv.dilation, conv.groups)
    if geometry != ((3, 3), (1, 1), (1, 1), 1):
        return False
    pad = conv.padding
    return (not isinstance(pad, str) and pad[0] == pad[1]
            and conv.padding_mode == "zeros")


def replace_conv2d_with_nova(model, trainable=False, verbose=True):
    """Swap, inside ``model``, every ``nn.Conv2d`` that ``is_eligible``
    accepts for a NOVA module built from it (same parameters, same device).

    ``trainable`` selects ``NovaWinogradConv2dTrainable`` (forward and
    backward) instead of the inference module ``NovaWinogradConv2d``. With
    ``verbose`` the numbers of swapped and skipped layers are printed.
    Returns the number of swapped layers. A model that is itself a single
    ``nn.Conv2d`` has no parent to hold a replacement and is left unchanged.
    """
    make = (NovaWinogradConv2dTrainable if trainable else NovaWinogradConv2d).from_conv2d
    # Decide everything before the first swap: the module tree is then not
    # mutated while it is being walked.
    convs = [(path, m) for path, m in model.named_modules()
             if path and isinstance(m, nn.Conv2d)]
    chosen = [(path, m) for path, m in convs if is_eligible(m)]
    for path, conv in chosen:
        owner_path, _, attr = path.rpartition(".")
        setattr(model.get_submodule(owner_path), attr, make(conv))
    if verbose:
        print(f"NOVA: replaced {len(chosen)} Conv2d layers, "
              f"skipped {len(convs) - len(chosen)} ineligible")
    return len(chosen)

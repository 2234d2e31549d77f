"""wrap_with_flashdp_layers: put DP layers in place of a model's Linear,
LayerNorm and HF Conv1D modules.

The call keeps the reference's signature, argument meanings, error types and
messages (flashdp/api/wrap_model.py:17-68, 71-76), so that existing training
scripts run unchanged.  How a module is chosen:

  * candidates are the submodules whose type is one of ``target_modules``
    exactly (a subclass of nn.Linear that is not nn.Linear itself, such as an
    already wrapped DPLinear or nn.MultiheadAttention's out_proj, is left as
    it is);
  * a candidate is replaced when its dotted name is in ``target_layers`` (all
    names when that is empty) and not in ``skip_layers``.  Names match
    exactly, as in the reference (flashdp/api/wrap_model.py:169-182): skipping
    "h.0" does not skip "h.0.fc".  ``priority_to_target`` is accepted; with
    exact names both of the reference's orders give the same set difference.

The DP module gets the replaced module's weights, training mode, device and
dtype (the reference moves it to the device only, so a bf16 model would get
fp32 DP layers).  A LayerNorm without a bias or over more than one trailing
axis gets the non-fused DPLayerNorm (the fused one requires a bias and one
axis; both compute the same per-sample math here).  With ``feedback`` the
names of the layers actually replaced are printed, and the skip list.  A
module type in ``target_modules`` that the model does not use draws a
warning; skip names are checked only after their expansion to the model's own
names, as in the reference, so an unknown skip name draws none.
"""
from __future__ import annotations

from typing import Iterator, List, Tuple, Type

import torch.nn as nn

from ..layers.layernorm import DPLayerNorm
from ..layers.linear import DPLinear
from ..layers.transformers_conv1d import DPConv1D, _HFConv1D

dp_supported_modules = {
    nn.Linear: DPLinear,
    nn.LayerNorm: DPLayerNorm,
}
if _HFConv1D is not None:
    dp_supported_modules[_HFConv1D] = DPConv1D


def _walk(module: nn.Module, prefix: str = "") -> Iterator[Tuple[nn.Module, str, nn.Module, str]]:
    """(parent, attribute name, child, dotted name) of every submodule, a parent
    before its children (every path, also of a module reachable by two)."""
    for attr, child in module.named_children():
        path = prefix + attr
        yield module, attr, child, path
        yield from _walk(child, path + ".")


def _dp_twin(child: nn.Module, dp_options: dict) -> nn.Module:
    """The DP module standing in for `child`, with its hyper-parameters."""
    kind = type(child)
    if kind is nn.Linear:
        twin = DPLinear(child.in_features, child.out_features, bias=child.bias is not None,
                        **dp_options)
    elif kind is nn.LayerNorm:
        # the fused mode needs a bias and a 1-D normalized_shape; the non-fused
        # mode computes the same per-sample math for the others
        no_bias = child.elementwise_affine and child.bias is None
        fused = not no_bias and len(child.normalized_shape) == 1
        twin = DPLayerNorm(child.normalized_shape, eps=child.eps,
                           elementwise_affine=child.elementwise_affine, bias=not no_bias,
                           use_fused=fused, **dp_options)
    else:  # HF Conv1D: weight [nx, nf]
        twin = DPConv1D(child.nf, child.weight.shape[0], **dp_options)
    ref = next(child.parameters(), None)
    if ref is not None:
        twin = twin.to(device=ref.device, dtype=ref.dtype)
    twin.load_state_dict(child.state_dict())
    twin.train(child.training)
    return twin


def wrap_with_flashdp_layers(
        model,
        target_modules: List[Type[nn.Module]] = None,
        target_layers: List[str] = None,
        skip_layers: List[str] = None,
        priority_to_target: bool = False,
        feedback: bool = True,
        C=1.0,
        noise_multiplier=1.0,
        clamp_value=1.0,
) -> nn.Module:
    """Replace the selected modules of ``model`` in place and return it.

    target_modules: types among nn.Linear, nn.LayerNorm and transformers'
    Conv1D (required, non-empty); target_layers: dotted names to consider
    (default: all); skip_layers: dotted names to leave alone; C,
    noise_multiplier, clamp_value: the DP layers' clipping bound, noise
    multiplier and clip factor cap.  Raises ValueError for a missing, empty or
    unsupported target_modules.
    """
    print("Wrapping the model with FlashDP...")
    if target_modules is None and target_layers is None:
        raise ValueError("Either target_modules or target_layers must be specified.")
    if target_modules is None or len(target_modules) == 0:
        raise ValueError("target_modules cannot be empty and must be list of torch.nn.Module.")
    supported = dp_supported_modules.keys()
    if any(kind not in supported for kind in target_modules):
        raise ValueError(f"target_modules must be among {supported}, got {target_modules}")
    del priority_to_target  # exact-name selection: the same set either way

    entries = list(_walk(model))
    present = {type(child) for _, _, child, _ in entries}
    for kind in target_modules:
        if kind not in present:
            print(f"Warning: Module type '{kind.__name__}' specified in target_modules is not "
                  "used in the model.")

    wanted = set(target_layers) if target_layers else {path for *_, path in entries}
    wanted -= set(skip_layers or [])
    kinds = set(target_modules)
    dp_options = dict(C=C, clamp_value=clamp_value, noise_multiplier=noise_multiplier)
    replaced, gone = [], set()
    for parent, attr, child, path in entries:
        if id(parent) in gone:  # inside a module replaced above
            gone.add(id(child))
            continue
        if type(child) in kinds and path in wanted:
            setattr(parent, attr, _dp_twin(child, dp_options))
            gone.add(id(child))
            replaced.append(path)

    if feedback:
        print(f"Layers Wrapped: {', '.join(replaced)}" if replaced else "No layers Wrapped.")
        skipped = list(skip_layers or [])
        print(f"Layers Skipped: {', '.join(skipped)}" if skipped else "No layers Skipped.")
    print("Model wrapped with FlashDP.")
    return model

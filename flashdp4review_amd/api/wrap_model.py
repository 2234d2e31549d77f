"""wrap_with_flashdp_layers: swap supported modules for their DP counterparts.

Reference: flashdp/api/wrap_model.py:11-276.  Same arguments, selection rules
and messages.  Selection keeps the reference's behaviour exactly: the
prefix-expanded groups of _process_layer_groups only drive the skip-name
validation, and the layers actually wrapped are chosen by _select_layers,
which matches names exactly (wrap_model.py:83-86,169-182), so skipping a parent
name does not skip its children.  One deliberate difference: the new module is
moved to the replaced module's device AND dtype (the reference moves it to the
device only, wrap_model.py:204-205, so a bf16 model would get fp32 DP layers).
"""
from __future__ import annotations

from typing import List, Type

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

    Args mirror the reference (flashdp/api/wrap_model.py:17-68): target_modules
    (types among nn.Linear, nn.LayerNorm, transformers Conv1D), target_layers
    (names; default all), skip_layers (exact names), priority_to_target,
    feedback (print wrapped/skipped), C, noise_multiplier, clamp_value.
    Raises ValueError for missing/empty/unsupported target_modules.
    """
    print("Wrapping the model with FlashDP...")
    if target_modules is None and target_layers is None:
        raise ValueError("Either target_modules or target_layers must be specified.")
    if target_modules is None or len(target_modules) == 0:
        raise ValueError("target_modules cannot be empty and must be list of torch.nn.Module.")
    supported_modules = dp_supported_modules.keys()
    if not all(m in supported_modules for m in target_modules):
        raise ValueError(f"target_modules must be among {supported_modules}, got {target_modules}")

    target_layers = target_layers if target_layers is not None else []
    skip_layers = skip_layers if skip_layers is not None else []

    _, skipped_layers = _process_layer_groups(model, target_layers, skip_layers,
                                              priority_to_target)
    selected_layers = _select_layers(model, target_layers, skip_layers, priority_to_target)

    if target_modules:
        _validate_target_modules(model, target_modules)
    if skip_layers:
        _validate_skip_layers(model, skipped_layers)

    _wrap_selected_layers(model, selected_layers, target_modules, C, clamp_value,
                          noise_multiplier)

    if feedback:
        _print_layer_feedback(selected_layers, "Wrapped")
        _print_layer_feedback(skip_layers, "Skipped")
    print("Model wrapped with FlashDP.")
    return model


def _get_init_args(module):
    if isinstance(module, nn.Linear):
        return {"in_features": module.in_features, "out_features": module.out_features,
                "bias": module.bias}
    if isinstance(module, nn.LayerNorm):
        return {"normalized_shape": module.normalized_shape, "eps": module.eps,
                "elementwise_affine": module.elementwise_affine}
    if _HFConv1D is not None and isinstance(module, _HFConv1D):
        return {"nf": module.nf, "nx": module.weight.shape[0]}
    raise NotImplementedError(f"Unsupported module type: {type(module)}")


def _collect_all_layer_names(model):
    names = []

    def collect(module, prefix=""):
        for name, child in module.named_children():
            path = f"{prefix}.{name}" if prefix else name
            names.append(path)
            collect(child, path)

    collect(model)
    return names


def _expand_submodules(layers, all_layers):
    out = []
    for layer in layers:
        out.extend(l for l in all_layers if l.startswith(layer + ".") or l == layer)
    return out


def _process_layer_groups(model, target_layers, skip_layers, priority_to_target):
    all_layers = _collect_all_layer_names(model)
    t = set(_expand_submodules(target_layers, all_layers))
    s = set(_expand_submodules(skip_layers, all_layers))
    if priority_to_target:
        return list(t - s), list(s - t)
    return list(t - t.intersection(s)), list(s)


def _select_layers(model, target_layers, skip_layers, priority_to_target):
    all_layers = set(_collect_all_layer_names(model))
    selected = set(target_layers) if target_layers else all_layers
    skip = set(skip_layers) if skip_layers else set()
    if priority_to_target:
        return selected - skip
    return selected.difference(selected.intersection(skip))


def _wrap_selected_layers(model, selected_layers, target_modules, C, clamp_value,
                          noise_multiplier):
    targets = tuple(target_modules)

    def replace(module, path=""):
        for child_name, child in module.named_children():
            full_name = f"{path}.{child_name}" if path else child_name
            if isinstance(child, targets) and full_name in selected_layers:
                dp_cls = dp_supported_modules[type(child)]
                new_module = dp_cls(**_get_init_args(child), C=C, clamp_value=clamp_value,
                                    noise_multiplier=noise_multiplier)
                p = next(child.parameters(), None)
                if p is not None:
                    new_module = new_module.to(device=p.device, dtype=p.dtype)
                new_module.load_state_dict(child.state_dict())
                new_module.train(child.training)
                setattr(module, child_name, new_module)
            else:
                replace(child, full_name)

    replace(model)


def _validate_target_modules(model, target_modules):
    used = set()

    def collect(module):
        for child in module.children():
            used.add(type(child))
            collect(child)

    collect(model)
    for tm in target_modules:
        if tm not in used:
            print(f"Warning: Module type '{tm.__name__}' specified in target_modules is not used "
                  "in the model.")


def _validate_skip_layers(model, skip_layers):
    names = set(_collect_all_layer_names(model))
    for s in skip_layers:
        if s not in names:
            print(f"Warning: '{s}' specified in skip_layers does not exist in the model.")


def _print_layer_feedback(layers, action):
    if layers:
        print(f"Layers {action}: {', '.join(layers)}")
    else:
        print(f"No layers {action}.")

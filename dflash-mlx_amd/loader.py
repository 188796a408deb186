"""MLX quantized safetensors checkpoints -> QuantizedLinear / VerifyQuantizedLinear.

The reference loads its targets through mlx-lm (dflash_mlx/runtime/loading.py:183),
which reads MLX-format quantized checkpoints: every quantized linear is stored
as ``<path>.weight`` (uint32 ``[N, K*bits/32]``, word j of row n holding
k = 8j .. 8j+7 at bits 4i for 4-bit), ``<path>.scales`` and ``<path>.biases``
(``[N, K/group_size]`` in the activation dtype) and an optional
``<path>.bias``; ``config.json`` carries ``"quantization"`` (or
``"quantization_config"``) with the default ``group_size`` / ``bits`` (and
``mode``), optionally overridden per module path by a nested dict, or
``false`` for a module left unquantized.

The packed words are exactly what the verify kernels consume, so the tensors
are moved to the device as stored: no repacking, no dequantisation.  Weight
files are found the way the reference inspects them
(dflash_mlx/runtime/loading.py:124-158): ``model.safetensors.index.json``'s
``weight_map`` when present, else every ``model*.safetensors``.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, List, Optional, Tuple, Union

import torch
from torch import nn

from .verify_linear import (QuantizedLinear, VerifyQuantizedLinear, _set_module,
                            is_verify_eligible)

PathLike = Union[str, Path]


def read_config(model_dir: PathLike) -> dict:
    """``config.json`` of a checkpoint directory ({} when absent)."""
    path = Path(model_dir) / "config.json"
    if not path.exists():
        return {}
    try:
        payload = json.loads(path.read_text())
    except json.JSONDecodeError as exc:
        raise ValueError(f"Invalid config JSON: {path}") from exc
    if not isinstance(payload, dict):
        raise ValueError(f"Invalid config payload: {path}")
    return payload


def quantization_for(config: dict, module_path: str) -> Optional[Tuple[int, int, str]]:
    """(group_size, bits, mode) of ``module_path``, or None if it is not quantized.

    A per-module entry (a dict, or ``false``) overrides the defaults."""
    q = config.get("quantization", config.get("quantization_config"))
    if not isinstance(q, dict):
        return None
    entry = q.get(module_path, None)
    if entry is False:
        return None
    gs, bits, mode = q.get("group_size", 64), q.get("bits", 4), q.get("mode", "affine")
    if isinstance(entry, dict):
        gs = entry.get("group_size", gs)
        bits = entry.get("bits", bits)
        mode = entry.get("mode", mode)
    return int(gs), int(bits), str(mode)


def weight_files(model_dir: PathLike) -> List[Path]:
    """The checkpoint's safetensors files (index weight_map first)."""
    model_path = Path(model_dir)
    index_path = model_path / "model.safetensors.index.json"
    if index_path.exists():
        try:
            payload = json.loads(index_path.read_text())
        except json.JSONDecodeError as exc:
            raise ValueError(f"Invalid safetensors index JSON: {index_path}") from exc
        if not isinstance(payload, dict):
            raise ValueError(f"Invalid safetensors index payload: {index_path}")
        weight_map = payload.get("weight_map")
        if not isinstance(weight_map, dict):
            raise ValueError(f"Invalid safetensors index weight_map: {index_path}")
        return [model_path / name for name in sorted(set(str(v) for v in weight_map.values()))]
    return sorted(model_path.glob("model*.safetensors"))


def _quantized_prefixes(names: List[str]) -> List[str]:
    have = set(names)
    return sorted(n[: -len(".scales")] for n in names
                  if n.endswith(".scales") and n[: -len(".scales")] + ".weight" in have)


def load_quantized_linears(model_dir: PathLike, *, device: Union[str, torch.device] = "cuda",
                           verify: bool = True, enable_qmm: Optional[bool] = None,
                           include: Optional[List[str]] = None) -> Dict[str, nn.Module]:
    """Every quantized linear of a checkpoint, keyed by module path.

    Eligible modules (``is_verify_eligible``, i.e. the reference's rules,
    dflash_mlx/verify_linear.py:54-87) become ``VerifyQuantizedLinear`` when
    ``verify`` is true; the rest stay ``QuantizedLinear``.  ``include``
    restricts loading to paths starting with one of the given prefixes."""
    from safetensors import safe_open

    config = read_config(model_dir)
    files = weight_files(model_dir)
    if not files:
        raise FileNotFoundError(f"no model*.safetensors under {model_dir}")
    located: Dict[str, Path] = {}
    for f in files:
        with safe_open(str(f), framework="pt") as handle:
            for name in handle.keys():
                located[str(name)] = f
    modules: Dict[str, nn.Module] = {}
    for prefix in _quantized_prefixes(list(located)):
        if include is not None and not any(prefix.startswith(p) for p in include):
            continue
        if not isinstance(config.get("quantization", config.get("quantization_config")), dict):
            raise ValueError(f"{prefix}: quantized tensors but config.json of {model_dir} "
                             "has no quantization entry")
        q = quantization_for(config, prefix)
        if q is None:  # marked unquantized: not a quantized linear
            continue
        gs, bits, mode = q
        tensors = {}
        for part in ("weight", "scales", "biases", "bias"):
            name = f"{prefix}.{part}"
            if name not in located:
                continue
            with safe_open(str(located[name]), framework="pt") as handle:
                tensors[part] = handle.get_tensor(name)
        if "biases" not in tensors:
            raise ValueError(f"{prefix}: affine quantized weights need '.biases'")
        w = tensors["weight"]
        if w.dtype not in (torch.uint32, torch.int32):
            raise ValueError(f"{prefix}.weight: packed words must be uint32, got {w.dtype}")
        s, b = tensors["scales"], tensors["biases"]
        K = int(w.shape[1]) * (32 // bits)
        if tuple(s.shape) != (int(w.shape[0]), K // gs) or tuple(b.shape) != tuple(s.shape):
            raise ValueError(f"{prefix}: scales / biases {tuple(s.shape)} do not match "
                             f"weight {tuple(w.shape)} at bits={bits}, group_size={gs}")
        ql = QuantizedLinear(w.to(device), s.to(device), b.to(device),
                             tensors["bias"].to(device) if "bias" in tensors else None,
                             group_size=gs, bits=bits, mode=mode)
        if verify and is_verify_eligible(ql, path=prefix):
            ql = VerifyQuantizedLinear.from_quantized(ql, enable_qmm=enable_qmm)
        modules[prefix] = ql
    return modules


def install_quantized_linears(model: nn.Module, modules: Dict[str, nn.Module]) -> int:
    """Put loaded modules into ``model`` at their paths (where the path
    exists); returns the number installed."""
    existing = {name for name, _ in model.named_modules()}
    count = 0
    for path, module in modules.items():
        if path in existing:
            _set_module(model, path, module)
            count += 1
    return count


__all__ = ["install_quantized_linears", "load_quantized_linears", "quantization_for",
           "read_config", "weight_files"]

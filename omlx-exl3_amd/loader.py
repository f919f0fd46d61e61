# SPDX-License-Identifier: Apache-2.0
"""Load ExLlamaV3 (EXL3) checkpoint tensors into PyTorch models with EXL3Linear layers (mirrors the
EXL3-specific part of src/omlx/exl3/loader.py of the reference).

The checkpoint's EXL3 tensors (<prefix>.trellis / suh / svh / su / sv / mul1 / mcg / bias) are
inventoried from the safetensors headers (no tensor data is read for that); each nn.Linear whose module
path has an inventory entry is replaced by an EXL3Linear declaring exactly those tensors; the tensors are
then read with safetensors (which executes nothing from the file) straight into the layers' buffers on
the target device. Afterwards same-input siblings with equal K and codebook are grouped into
single-launch EXL3SiblingGroups, and the decode-path rotation fusions are installed (fusion.py).

Supported: integer bitrates 1..8, codebooks 3inst / mcg / mul1, legacy packed su / sv signs, bias. Not
supported (as in the reference): half-integer bitrates, MoE expert tensors. Building the model graph of a
particular architecture (the reference patches mlx-vlm's Qwen3.5 class) is the caller's part: pass any
torch module tree whose nn.Linear leaves carry the checkpoint's names.
"""
from __future__ import annotations

import json
import os
import struct
from pathlib import Path
from typing import Any, Callable

import torch
from torch import nn

from .fusion import fuse_decode
from .linear import EXL3_PARTS, EXL3Linear, EXL3SiblingGroup, RowExactLinear, _DTYPE_NAMES

SIBLINGS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"), ("in_proj_qkv", "in_proj_z"))


def is_exl3_config(config: dict[str, Any]) -> bool:
    """True when a model config declares EXL3 quantization (loader.py:45-47)."""
    qc = config.get("quantization_config") or {}
    return str(qc.get("quant_method", "")).lower() == "exl3"


def _read_header(path: Path) -> dict[str, Any]:
    """The JSON header of one safetensors file (8-byte little-endian length, then JSON)."""
    with open(path, "rb") as fh:
        raw = fh.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file")
        n = struct.unpack("<Q", raw)[0]
        header = json.loads(fh.read(n))
    header.pop("__metadata__", None)
    return header


def _files(model_path: Path) -> list[str]:
    index = model_path / "model.safetensors.index.json"
    if index.exists():
        return sorted(set(json.loads(index.read_text())["weight_map"].values()))
    return ["model.safetensors"]


def inventory(model_path) -> dict[str, dict[str, tuple[tuple[int, ...], torch.dtype]]]:
    """EXL3 linear prefix (checkpoint naming) -> {part: (shape, dtype)} (loader.py:58-72)."""
    model_path = Path(model_path)
    headers: dict[str, Any] = {}
    for f in _files(model_path):
        headers.update(_read_header(model_path / f))
    inv: dict[str, dict[str, tuple[tuple[int, ...], torch.dtype]]] = {}
    for key in headers:
        if key.endswith(".trellis"):
            prefix = key[: -len(".trellis")]
            inv[prefix] = {part: (tuple(headers[f"{prefix}.{part}"]["shape"]),
                                  _DTYPE_NAMES[headers[f"{prefix}.{part}"]["dtype"]])
                           for part in EXL3_PARTS if f"{prefix}.{part}" in headers}
    return inv


def swap_linears(model: nn.Module, inv: dict, sanitize_key: Callable[[str], str] = lambda k: k,
                 device=None) -> int:
    """Replace every nn.Linear whose (sanitized) path has an inventory entry with an EXL3Linear declaring
    exactly those tensors (loader.py:90-104). A non-Linear target raises TypeError."""
    by_path = {sanitize_key(prefix): parts for prefix, parts in inv.items()}
    swapped = 0
    for path, module in list(model.named_modules()):
        parts = by_path.get(path)
        if parts is None:
            continue
        if not isinstance(module, nn.Linear):
            raise TypeError(f"EXL3 tensor at {path} targets a {type(module).__name__}, expected Linear")
        dev = device if device is not None else module.weight.device
        new = EXL3Linear(module.in_features, module.out_features, parts, device=dev)
        parent_path, _, name = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        setattr(parent, name, new)
        swapped += 1
    return swapped


def load_exl3_tensors(model: nn.Module, model_path, sanitize_key: Callable[[str], str] = lambda k: k,
                      strict: bool = True) -> int:
    """Copy every EXL3 part of the checkpoint into the matching EXL3Linear buffers. With `strict`, a
    declared buffer the checkpoint lacks, or a shape / dtype mismatch, raises."""
    from safetensors import safe_open

    model_path = Path(model_path)
    layers = {path: m for path, m in model.named_modules() if isinstance(m, EXL3Linear)}
    filled = {path: set() for path in layers}
    loaded = 0
    for f in _files(model_path):
        with safe_open(str(model_path / f), framework="pt") as fh:
            for key in fh.keys():
                prefix, _, part = key.rpartition(".")
                if part not in EXL3_PARTS:
                    continue
                m = layers.get(sanitize_key(prefix))
                if m is None or part not in m:
                    continue
                t = fh.get_tensor(key)
                dst = getattr(m, part)
                if tuple(t.shape) != tuple(dst.shape) or t.dtype != dst.dtype:
                    raise ValueError(f"{key}: checkpoint {tuple(t.shape)} {t.dtype} does not match the layer's "
                                     f"{tuple(dst.shape)} {dst.dtype}")
                dst.copy_(t)
                filled[sanitize_key(prefix)].add(part)
                loaded += 1
    if strict:
        for path, m in layers.items():
            missing = set(m._parts) - filled[path]
            if missing:
                raise ValueError(f"{path}: checkpoint lacks {sorted(missing)}")
    for m in layers.values():
        m._ready = False
    return loaded


def group_siblings(model: nn.Module) -> int:
    """Group same-input EXL3 siblings (q/k/v, gate/up, in_proj_qkv/z) into single-launch groups, partitioned
    by codebook (loader.py:137-156 partitions by (K, codebook); here one launch also serves members of
    different K)."""
    groups = 0
    for _, module in model.named_modules():
        for names in SIBLINGS:
            members = [getattr(module, n, None) for n in names]
            if not all(isinstance(m, EXL3Linear) for m in members):
                continue
            for m in members:
                m._prepare()
            by_rate: dict = {}
            for m in members:
                by_rate.setdefault(m._cb, []).append(m)
            for subset in by_rate.values():
                if EXL3SiblingGroup.fusable(subset):
                    EXL3SiblingGroup(subset)
                    groups += 1
    return groups


def row_exact_dense(model: nn.Module, prefix: str = "") -> int:
    """Wrap every plain nn.Linear left in the model (the layers the checkpoint does not quantize) whose
    path starts with `prefix` in RowExactLinear, so speculative-verify rows give the bits of single-row
    decoding (loader.py:123-134). Returns how many were wrapped."""
    wrapped = 0
    for path, module in list(model.named_modules()):
        if type(module) is not nn.Linear or not path.startswith(prefix):
            continue
        parent_path, _, name = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        setattr(parent, name, RowExactLinear(module))
        wrapped += 1
    return wrapped


def load_exl3(model: nn.Module, model_path, *, sanitize_key: Callable[[str], str] = lambda k: k,
              device=None) -> dict[str, Any]:
    """Bind an EXL3 checkpoint to a torch model (the EXL3 part of loader.py:183-223): swap the linears,
    load their tensors, group siblings, wrap the remaining dense linears for row-exact verify when
    OMLX_EXL3_ROW_EXACT_DENSE=1 (off by default, as in the reference, loader.py:214-216), and install the
    decode fusions (OMLX_EXL3_FUSE=0 disables them). Non-EXL3 tensors of the checkpoint are the caller's to
    load. Returns what was done."""
    inv = inventory(model_path)
    if not inv:
        raise ValueError(f"no EXL3 trellis tensors found in {model_path}")
    swapped = swap_linears(model, inv, sanitize_key, device)
    loaded = load_exl3_tensors(model, model_path, sanitize_key)
    groups = group_siblings(model)
    dense = row_exact_dense(model) if os.environ.get("OMLX_EXL3_ROW_EXACT_DENSE") == "1" else 0
    fused = fuse_decode(model) if os.environ.get("OMLX_EXL3_FUSE", "1") != "0" else {}
    return {"linears": swapped, "tensors": loaded, "groups": groups, "row_exact_dense": dense, "fused": fused}


__all__ = ["is_exl3_config", "inventory", "swap_linears", "load_exl3_tensors", "group_siblings", "row_exact_dense",
           "load_exl3", "SIBLINGS"]

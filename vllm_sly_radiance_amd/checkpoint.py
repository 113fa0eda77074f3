"""MXFP4 checkpoint ingestion for the W4A8 linears (safetensors, read tensor by tensor).

Quark / compressed-tensors MXFP4 checkpoints store each linear as packed e2m1 codes [N, K/2] uint8
(low nibble = even k) under ``<prefix>.weight_packed`` (compressed-tensors) or ``<prefix>.weight``
(Quark), and e8m0 block exponents [N, K/32] uint8 under ``<prefix>.weight_scale``. vLLM's merged
linears (gate_up, qkv, qkvz) hold their parts concatenated along N, in the order the model lists
them; the reference's benches build the same tensors with ``torch.cat([...], 0)``
(ci/bench_at_psw.py:55-67, ci/check_psw_all_paths.py:59). The loaded pair is what
``process_weights_after_loading`` repacks, in place when N % 16 == 0 and K % 512 == 0 (the memory
discipline of sly/mxfp4/radiance_mxfp4.py:1140-1145: the granules go back into the checkpoint
tensor's storage, so loading a model leaves no per-layer holes).

Sharded checkpoints are read through ``model.safetensors.index.json``; each tensor is opened on its
own (``safe_open``), so a layer never needs more host memory than its own tensors.
"""
from __future__ import annotations

import glob
import json
import os

import torch

PACKED_NAMES = ("weight_packed", "weight")       # compressed-tensors, Quark


class CheckpointIndex:
    """Tensor name -> safetensors file, for a directory (with or without an index) or one file."""

    def __init__(self, path: str):
        self.path = path
        self.files: dict[str, str] = {}
        if os.path.isfile(path):
            self._add_file(path)
        else:
            idx = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(idx):
                with open(idx) as f:
                    wm = json.load(f)["weight_map"]
                self.files = {k: os.path.join(path, v) for k, v in wm.items()}
            else:
                for fn in sorted(glob.glob(os.path.join(path, "*.safetensors"))):
                    self._add_file(fn)
        if not self.files:
            raise RuntimeError(f"[radiance.mxfp4] no safetensors tensors under {path}")

    def _add_file(self, fn: str) -> None:
        from safetensors import safe_open
        with safe_open(fn, framework="pt", device="cpu") as f:
            for k in f.keys():
                self.files[k] = fn

    def __contains__(self, name: str) -> bool:
        return name in self.files

    def get(self, name: str) -> torch.Tensor:
        from safetensors import safe_open
        if name not in self.files:
            raise KeyError(f"[radiance.mxfp4] tensor {name} not in the checkpoint {self.path}")
        with safe_open(self.files[name], framework="pt", device="cpu") as f:
            return f.get_tensor(name)


def _packed_name(index: CheckpointIndex, prefix: str) -> str:
    for n in PACKED_NAMES:
        if f"{prefix}.{n}" in index:
            return f"{prefix}.{n}"
    raise KeyError(f"[radiance.mxfp4] no packed MXFP4 weight for {prefix} "
                   f"(looked for {', '.join(PACKED_NAMES)})")


def read_mxfp4_linear(index: CheckpointIndex, prefix: str, parts=None, device="cpu"):
    """The packed codes and block exponents of one linear, parts concatenated along N.

    prefix: the module path, e.g. ``model.layers.3.mlp``; parts: the sub-module names of a merged
    linear, e.g. ``["gate_proj", "up_proj"]`` (None: ``prefix`` is the linear itself).
    Returns (weight uint8 [N, K/2], weight_scale uint8 [N, K/32]) on `device`. Shapes are checked:
    every part must share K, and weight_scale must be [N_part, K/32]."""
    names = [prefix] if not parts else [f"{prefix}.{p}" for p in parts]
    ws, ss, K = [], [], None
    for n in names:
        w = index.get(_packed_name(index, n))
        s = index.get(f"{n}.weight_scale")
        if w.dtype not in (torch.uint8, torch.int8) or s.dtype not in (torch.uint8, torch.int8):
            raise RuntimeError(f"[radiance.mxfp4] {n}: expected uint8 packed codes and e8m0 "
                               f"scales, got {w.dtype} / {s.dtype}")
        w, s = w.view(torch.uint8), s.view(torch.uint8)
        if w.dim() != 2 or s.dim() != 2:
            raise RuntimeError(f"[radiance.mxfp4] {n}: expected 2-D tensors, got "
                               f"{tuple(w.shape)} / {tuple(s.shape)}")
        k = w.shape[1] * 2
        if K is None:
            K = k
        if k != K:
            raise RuntimeError(f"[radiance.mxfp4] {n}: K={k} differs from the other parts (K={K})")
        if s.shape[0] != w.shape[0] or s.shape[1] * 32 != K:
            raise RuntimeError(f"[radiance.mxfp4] {n}: weight_scale {tuple(s.shape)} does not "
                               f"match weight {tuple(w.shape)} (expected [{w.shape[0]}, {K // 32}])")
        ws.append(w)
        ss.append(s)
    w = ws[0] if len(ws) == 1 else torch.cat(ws, 0)
    s = ss[0] if len(ss) == 1 else torch.cat(ss, 0)
    return w.contiguous().to(device), s.contiguous().to(device)


def load_linear(layer: torch.nn.Module, index: CheckpointIndex, prefix: str, parts=None,
                device="cuda") -> torch.nn.Module:
    """Attach a checkpoint linear to `layer` as the parameters the plugin's
    process_weights_after_loading expects (``weight`` [N, K/2], ``weight_scale`` [N, K/32])."""
    w, s = read_mxfp4_linear(index, prefix, parts, device)
    layer.weight = torch.nn.Parameter(w, requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(s, requires_grad=False)
    return layer

"""Seeded inputs shared by the CPU and GPU tests and the golden generator's
conventions: params from torch.Generator().manual_seed(0), grads for step t
from torch.Generator().manual_seed(1000 + t), drawn param by param in order,
N(0, scale^2), with an optional Bernoulli outlier mask (x50)."""

from __future__ import annotations

import json
import os

import torch
from safetensors.torch import load_file

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def make_params(shapes: dict, dtype=torch.float32, scale=0.02, device="cpu"):
    g = torch.Generator().manual_seed(0)
    return {k: torch.nn.Parameter((torch.randn(s, generator=g) * scale).to(dtype).to(device))
            for k, s in shapes.items()}


def grads_for_step(t: int, shapes: dict, dtype=torch.float32, scale=0.02, outliers=0.0):
    g = torch.Generator().manual_seed(1000 + t)
    out = {}
    for k, s in shapes.items():
        x = torch.randn(s, generator=g) * scale
        if outliers > 0:
            mask = torch.rand(s, generator=g) < outliers
            x = torch.where(mask, x * 50.0, x)
        out[k] = x.to(dtype)
    return out


def load_golden(name: str):
    tensors = load_file(os.path.join(GOLDEN, f"{name}.safetensors"))
    with open(os.path.join(GOLDEN, f"{name}.json")) as f:
        meta = json.load(f)
    return tensors, meta


def config_from_meta(meta: dict) -> dict:
    cfg = dict(meta["config"])
    if "betas" in cfg:
        cfg["betas"] = tuple(cfg["betas"])
    return cfg

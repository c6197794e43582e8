"""Loader of the static query metric M_st shipped with the reference for real-weight runs.

Format (assets/restore_query_metric.py:18-27 of the reference): a torch-serialised dict with
  M_triu  (L, H, d (d + 1) / 2) fp32  upper triangle (torch.triu_indices order) of each symmetric
          (d, d) metric, per layer and query head, pre-RoPE;
  dim     d (128);
  inv_freq (d / 2,) fp32 RoPE frequencies, attention_scaling float, and descriptive fields
  (space, source, n_requests).
The file is read with torch.load(weights_only=True): tensors and plain values only, nothing in
it is executed.  The result is the `static` dict OursHIP takes: M (L, H, d, d) fp32, inv_freq,
attention_scaling (plus the descriptive fields).
"""
from __future__ import annotations

import torch


def unpack_triu(tri: torch.Tensor, d: int) -> torch.Tensor:
    """(..., d (d + 1) / 2) upper triangles -> (..., d, d) symmetric matrices."""
    if tri.shape[-1] != d * (d + 1) // 2:
        raise ValueError(f"packed metric has {tri.shape[-1]} entries per matrix, expected {d * (d + 1) // 2}")
    iu = torch.triu_indices(d, d)
    M = torch.zeros(*tri.shape[:-1], d, d, dtype=tri.dtype)
    M[..., iu[0], iu[1]] = tri
    M[..., iu[1], iu[0]] = tri
    return M


def pack_triu(M: torch.Tensor) -> torch.Tensor:
    """(..., d, d) symmetric matrices -> (..., d (d + 1) / 2) upper triangles."""
    d = M.shape[-1]
    iu = torch.triu_indices(d, d)
    return M[..., iu[0], iu[1]].contiguous()


def load_static_metric(path: str, head_dim: int = 128) -> dict:
    packed = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(packed, dict) or "M_triu" not in packed or "dim" not in packed:
        raise ValueError(f"{path}: not a packed query metric (expected keys M_triu, dim)")
    d = int(packed["dim"])
    if d != head_dim:
        raise ValueError(f"{path}: head dim {d}, expected {head_dim}")
    if packed.get("space", "pre-rope") != "pre-rope":
        raise ValueError(f"{path}: metric space {packed['space']!r}, expected 'pre-rope'")
    tri = packed["M_triu"].float()
    if tri.dim() != 3:
        raise ValueError(f"{path}: M_triu must be (layers, heads, d(d+1)/2), got {tuple(tri.shape)}")
    out = {k: v for k, v in packed.items() if k not in ("M_triu", "dim")}
    out["M"] = unpack_triu(tri, d)
    out["inv_freq"] = packed["inv_freq"].float()
    if out["inv_freq"].shape != (d // 2,):
        raise ValueError(f"{path}: inv_freq must be ({d // 2},)")
    out["attention_scaling"] = float(packed.get("attention_scaling", 1.0))
    return out

"""float64 oracle for the block's SwiGLU activation and weightless RMSNorm -- TEST
INFRASTRUCTURE.

Only tests may import this module, as the checker; the product path never calls it.

* ``swiglu_fwd``: ``F.silu(gate) * up`` with ``gate, up = gu.chunk(2, dim=-1)``
  (reference models/layers.py:167-168); silu(g) = g * sigmoid(g).
* ``swiglu_bwd``: its gradient with respect to gu, [dy * u * s * (1 + g (1 - s)),
  dy * g * s] with s = sigmoid(g).
* ``rms_norm_fwd``: ``F.rms_norm(x, (N,), eps)`` without a weight (reference
  models/transformer.py:87): y = x * r, r = (mean(x^2) + eps)^(-1/2) per row.
* ``rms_norm_bwd``: dx = r * dy - x * r^3 * mean(dy * x).

Pinned by tests/test_norm_mlp_cpu.py: the forwards against PyTorch's own CPU
``F.silu`` and ``F.rms_norm`` in float64 (library routines), the backwards against
PyTorch autograd of those and against central finite differences, plus closed forms
(silu(0) = 0 with slope u/2; a constant row normalises to +-1/sqrt(1 + eps/c^2)).
"""
from __future__ import annotations

import numpy as np

__all__ = ["swiglu_fwd", "swiglu_bwd", "rms_norm_fwd", "rms_norm_bwd"]


def _sigmoid(g):
    # split by sign so that exp never overflows
    out = np.empty_like(g)
    pos = g >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-g[pos]))
    e = np.exp(g[~pos])
    out[~pos] = e / (1.0 + e)
    return out


def swiglu_fwd(gu):
    gu = np.asarray(gu, dtype=np.float64)
    F = gu.shape[-1] // 2
    g, u = gu[..., :F], gu[..., F:]
    return g * _sigmoid(g) * u


def swiglu_bwd(gu, dy):
    gu = np.asarray(gu, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    F = gu.shape[-1] // 2
    g, u = gu[..., :F], gu[..., F:]
    s = _sigmoid(g)
    return np.concatenate([dy * u * s * (1.0 + g * (1.0 - s)), dy * g * s], axis=-1)


def rms_norm_fwd(x, eps):
    x = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r, r[..., 0]


def rms_norm_bwd(x, rstd, dy):
    x = np.asarray(x, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    r = np.asarray(rstd, dtype=np.float64)[..., None]
    return r * dy - x * r ** 3 * np.mean(dy * x, axis=-1, keepdims=True)

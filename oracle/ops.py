"""Oracle: CPU PyTorch restatement of the reference ops on the hot path.

TEST INFRASTRUCTURE ONLY (checker and CPU baseline), never imported by flashcart_amd.
Every function runs on CPU tensors of any float dtype and is differentiable with
torch autograd, which is how the reference obtains its backward on CPU.

Function -> reference it restates:
  irreps            src/flashcart/o3/_irreps.py:50-67 (py_irreps), Eq. (1) _codegen_irreps.py:147-164
  chebyshev         src/flashcart/nn/radial.py:98-121
  bessel            src/flashcart/nn/radial.py:44-54
  cutoff            src/flashcart/nn/radial.py:181-242
  edge_vectors      src/flashcart/utils/geometry.py:25-53
  tensor_product    src/flashcart/o3/_codegen_tensor_product.py:833-1012 (py_tensor_product:
                    index_select -> per-path polynomials -> weights -> stack/cat -> scatter_sum)
  linear            src/flashcart/o3/_linear.py:64-110 (py_linear)
  dense / silu      src/flashcart/nn/layers.py:84-145, :12-45
  scatter_sum       src/flashcart/utils/scatter.py:33-68
"""

from __future__ import annotations

import math
from functools import lru_cache
from typing import List, Optional, Sequence

import numpy as np
import torch

from oracle.cartesian import STORED, dfact, enumerate_paths, full_index, path_tensor, sym_projector

SILU_SCALE = 1.6765324703310907
SIGMOID_SCALE = 1.8462285453386054
MIN_EDGE_LENGTH = 1.0e-4


def stored(x: float) -> float:
    """A constant as the reference's modules hold it: in a buffer made under torch's default dtype,
    float32 (nn/layers.py:24-27, :60-63, :106-110; o3/_linear.py:148-164 via o3/linear.py:68-79),
    so a model cast to float64 still multiplies by the float32 rounding of the constant."""
    return float(torch.tensor(x, dtype=torch.float32))


def _t(a: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    return torch.as_tensor(a, dtype=like.dtype, device=like.device)


def _outer_power(r: torch.Tensor, p: int, m: int) -> torch.Tensor:
    """(n, 3^(p+2m)) flattened r^(x)p (x) delta^(x)m (r first, deltas last)."""
    n = r.shape[0]
    out = torch.ones(n, 1, dtype=r.dtype)
    for _ in range(p):
        out = (out.unsqueeze(-1) * r.unsqueeze(1)).reshape(n, -1)
    eye = torch.eye(3, dtype=r.dtype).reshape(1, 1, 9)
    for _ in range(m):
        out = (out.unsqueeze(-1) * eye).reshape(n, -1)
    return out


def irreps(x: torch.Tensor, l_max: int) -> torch.Tensor:
    """Eq. (1) stored components of ranks 0..l_max, as a polynomial in the given vectors."""
    cols = [torch.ones(x.shape[0], 1, dtype=x.dtype)]
    for l in range(1, l_max + 1):
        S = _t(sym_projector(l), x)
        full = torch.zeros(x.shape[0], 3 ** l, dtype=x.dtype)
        for m in range(l // 2 + 1):
            coef = (dfact(2 * l - 1) / math.factorial(l)) * ((-1) ** m) * dfact(2 * l - 2 * m - 1) / dfact(2 * l - 1)
            placements = math.factorial(l) / (math.factorial(l - 2 * m) * math.factorial(m) * 2 ** m)
            full = full + coef * placements * (_outer_power(x, l - 2 * m, m) @ S.T)
        sel = [full_index(abc) for abc in STORED[l]]
        cols.append(full[:, sel])
    return torch.cat(cols, dim=1)


def chebyshev(d: torch.Tensor, n_radial: int, r_max: float, r_min: float = 0.0, mapping: str = "affine"):
    t = (d - r_min) / (r_max - r_min)
    x = torch.cos(t * math.pi) if mapping == "cosine" else 2.0 * t - 1.0
    if n_radial == 1:
        return torch.ones_like(x).unsqueeze(-1)
    T = [torch.ones_like(x), x]
    for _ in range(2, n_radial):
        T.append(2.0 * x * T[-1] - T[-2])
    return torch.stack(T, dim=-1)


def bessel(d: torch.Tensor, n_radial: int, r_max: float) -> torch.Tensor:
    w = (math.pi / r_max) * torch.arange(1, n_radial + 1, dtype=d.dtype)
    x = d.unsqueeze(-1) * w
    return math.sqrt(2.0 / r_max) * w * torch.sinc(x / math.pi)


def cutoff(d: torch.Tensor, r_max: float, p: int = 6) -> torch.Tensor:
    d = torch.clamp(d, min=0.0)
    t = d / r_max
    tp = t.clone()
    for _ in range(p - 1):
        tp = tp * t
    tp1 = tp * t
    tp2 = tp1 * t
    c1, c2, c3 = (p + 1.0) * (p + 2.0) / 2.0, p * (p + 2.0), p * (p + 1.0) / 2.0
    env = 1.0 - c1 * tp + c2 * tp1 - c3 * tp2
    return torch.clamp(env * (d < r_max).to(env.dtype), min=0.0, max=1.0)


def edge_vectors(positions, cell, shifts, edge_index, batch, use_shifts=True):
    i, j = edge_index[0], edge_index[1]
    if not use_shifts:
        return positions[j] - positions[i]
    sv = (shifts.to(cell.dtype).unsqueeze(-2) @ cell[batch[i]]).squeeze(-2)
    return positions[j] - positions[i] + sv


def scatter_sum(src: torch.Tensor, index: torch.Tensor, dim_size: int) -> torch.Tensor:
    out = torch.zeros((dim_size,) + tuple(src.shape[1:]), dtype=src.dtype)
    return out.index_add(0, index, src)


@lru_cache(maxsize=None)
def _path_tensor_t(l1, l2, lo, dtype):
    return torch.as_tensor(path_tensor(l1, l2, lo), dtype=dtype)


# How tensor_product evaluates each path: "einsum" contracts the dense path tensor in one call;
# "components" follows the op sequence of the reference's generated CPU module
# (src/flashcart/o3/_codegen_tensor_product.py:833-1012): every output component as a sum of
# products of input component columns, then stack, path weight, cat and scatter_sum. Both give
# the same values; the CPU baseline times the second. Set with components_form().
TP_FORM = "einsum"


class components_form:
    """Context manager: tensor_product evaluates per output component (the reference's CPU
    op sequence) inside the block."""

    def __enter__(self):
        global TP_FORM
        self._prev, TP_FORM = TP_FORM, "components"
        return self

    def __exit__(self, *exc):
        global TP_FORM
        TP_FORM = self._prev


@lru_cache(maxsize=None)
def _path_terms(l1, l2, lo):
    """Nonzero coefficients of the path tensor, per output component: [(b, c, coeff), ...]."""
    B = path_tensor(l1, l2, lo)
    return tuple(tuple((int(b), int(c), float(B[a, b, c])) for b, c in zip(*np.nonzero(np.abs(B[a]) > 1e-14)))
                 for a in range(B.shape[0]))


def _path_components(x, y, l1, l2, lo):
    """out_a = sum over (b, c) of B[a, b, c] * x[:, b] * y[:, c], column by column: x (n, 2l1+1, C),
    y (n, 2l2+1, C or 1) -> (n, 2lo+1, C)."""
    xs = [x[:, b] for b in range(x.shape[1])]
    ys = [y[:, c] for c in range(y.shape[1])]
    comps = []
    for terms in _path_terms(l1, l2, lo):
        acc = None
        for b, c, k in terms:
            t = k * xs[b] * ys[c]
            acc = t if acc is None else acc + t
        comps.append(acc if acc is not None else torch.zeros_like(xs[0] * ys[0]))
    return torch.stack(comps, dim=1)


def tensor_product(in1, in2, weights, idx_i, idx_j, in1_l_max, in2_l_max, out_l_max, in1_features,
                   in2_features, symmetric_product=False, shared_weights=False, reduce_paths=False, out_rows=None):
    """``out_rows``: rows of a convolution's output (default: the rows of in1)."""
    rows = in1.shape[0] if out_rows is None else out_rows
    conv = idx_i is not None and idx_j is not None
    if conv:
        in1 = in1.index_select(0, idx_j)
    n = in1.shape[0]
    C = max(in1_features, in2_features)

    components = TP_FORM == "components"

    def blocks(x, lmax, f):
        return [x[:, l * l * f:(l + 1) * (l + 1) * f].reshape(n, 2 * l + 1, f) if components else
                x[:, l * l * f:(l + 1) * (l + 1) * f].reshape(n, 2 * l + 1, f).expand(n, 2 * l + 1, C)
                for l in range(lmax + 1)]

    b1, b2 = blocks(in1, in1_l_max, in1_features), blocks(in2, in2_l_max, in2_features)
    buckets: List[List[torch.Tensor]] = [[] for _ in range(out_l_max + 1)]
    for p, (l1, l2, lo, swap) in enumerate(enumerate_paths(in1_l_max, in2_l_max, out_l_max, symmetric_product)):
        x, y = (b2[l1], b1[l2]) if swap else (b1[l1], b2[l2])
        if components:
            out = _path_components(x, y, l1, l2, lo)
            out = out.expand(n, 2 * lo + 1, C) if out.shape[-1] != C else out
        else:
            B = _path_tensor_t(l1, l2, lo, in1.dtype)
            out = torch.einsum("abc,nbf,ncf->naf", B, x, y)
        w = weights[p * C:(p + 1) * C] if shared_weights else weights[:, p * C:(p + 1) * C].unsqueeze(1)
        buckets[lo].append(out * w)
    flats = []
    for lo, bucket in enumerate(buckets):
        if not bucket:
            continue
        if reduce_paths:
            flats.append(sum(bucket).reshape(n, -1))
        else:
            flats.append(torch.stack(bucket, dim=2).reshape(n, -1))
    out = torch.cat(flats, dim=-1)
    if conv:
        out = scatter_sum(out, idx_i, rows)
    return out


def linear(x: torch.Tensor, weights: Sequence[torch.Tensor], in_l_max: int, out_l_max: int, in_features: int,
           out_features: int, in_paths: Optional[Sequence[int]] = None, weight_scale: Optional[float] = None):
    in_paths = [1] * (in_l_max + 1) if in_paths is None else list(in_paths)
    common = min(in_l_max, out_l_max)
    n = x.shape[0]
    outs, off = [], 0
    for l in range(in_l_max + 1):
        k = in_features * in_paths[l]
        size = (2 * l + 1) * k
        if l <= common:
            s = stored(float(weight_scale) if weight_scale is not None else float(k) ** -0.5)
            xl = x[:, off:off + size].reshape(n, 2 * l + 1, k)
            outs.append(torch.nn.functional.linear(xl, weights[l] * s).reshape(n, -1))
        off += size
    pad = sum((2 * l + 1) * out_features for l in range(common + 1, out_l_max + 1))
    if pad:
        outs.append(x.new_zeros(n, pad))
    return torch.cat(outs, dim=-1)


def dense(x, weight, bias=None, weight_scale=None):
    s = stored(float(weight.shape[1]) ** -0.5 if weight_scale is None else weight_scale)
    return torch.nn.functional.linear(x, weight * s, bias)


def silu(x):
    return stored(SILU_SCALE) * torch.nn.functional.silu(x)

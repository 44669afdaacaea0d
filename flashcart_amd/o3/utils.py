"""Layout helpers of the Cartesian feature format (reference src/flashcart/o3/utils.py).

These describe where rank blocks and paths live in a flattened feature row and
convert between stored (2l+1) and full (3^l) Cartesian components. They are layout
utilities (device-agnostic torch), not part of the kernel path.
"""

from __future__ import annotations

import functools
import itertools
from typing import List, Literal, Optional, Sequence, Tuple

import torch

from flashcart_amd.codegen.cartesian import count_output_paths as _count_output_paths
from flashcart_amd.codegen.cartesian import reconstruction, stored_basis

ShapeMode = Literal["flattened", "factorized"]


def count_output_paths(in1_l_max: int, in2_l_max: int, out_l_max: int,
                       symmetric_product: bool = False) -> Tuple[List[int], int]:
    """Per-output-rank path counts and their total (reference ``o3/utils.py:157-203``)."""
    return _count_output_paths(in1_l_max, in2_l_max, out_l_max, symmetric_product)


def get_irreps_slices(l_max: int, n_features: int, n_paths: Optional[List[int]] = None) -> list:
    """(start, stop) of each rank block in the stored layout (reference ``o3/utils.py:206-227``)."""
    n_paths = [1] * (l_max + 1) if n_paths is None else n_paths
    out, start = [], 0
    for l in range(l_max + 1):
        size = (2 * l + 1) * n_features * n_paths[l]
        out.append((start, start + size))
        start += size
    return out


def get_irreps_shapes(l_max: int, n_features: int, n_paths: Optional[List[int]] = None,
                      mode: ShapeMode = "flattened") -> list:
    """Block shapes per rank (reference ``o3/utils.py:233-263``)."""
    n_paths = [1] * (l_max + 1) if n_paths is None else n_paths
    if mode == "factorized":
        return [(2 * l + 1, n_features, n_paths[l]) for l in range(l_max + 1)]
    return [(2 * l + 1, n_features * n_paths[l]) for l in range(l_max + 1)]


def get_cartesian_slices(l_max: int, n_features: int, n_paths: Optional[List[int]] = None) -> list:
    n_paths = [1] * (l_max + 1) if n_paths is None else n_paths
    out, start = [], 0
    for l in range(l_max + 1):
        size = (3 ** l) * n_features * n_paths[l]
        out.append((start, start + size))
        start += size
    return out


def apply_path_weight(x: torch.Tensor, weights: torch.Tensor, path_idx: int, out_features: int,
                      shared: bool) -> torch.Tensor:
    """Scale one path block by its per-feature weights (reference ``o3/utils.py:127-154``)."""
    start = path_idx * out_features
    if shared:
        w = weights[start:start + out_features]
    else:
        w = weights[:, start:start + out_features]
        w = w.reshape(w.shape[0], *([1] * (x.dim() - 2)), w.shape[1])
    return x * w


@functools.lru_cache(maxsize=None)
def _reconstruction_matrix(l: int) -> torch.Tensor:
    """(3^l, 2l+1) matrix mapping stored components to full Cartesian components."""
    if l == 0:
        return torch.ones(1, 1, dtype=torch.float64)
    rec = reconstruction(l)
    M = torch.zeros(3 ** l, 2 * l + 1, dtype=torch.float64)
    for flat, idx in enumerate(itertools.product(range(3), repeat=l)):
        for pos, w in rec[idx].items():
            M[flat, pos] = w
    return M


@functools.lru_cache(maxsize=None)
def _stored_full_indices(l: int) -> Tuple[int, ...]:
    if l == 0:
        return (0,)
    out = []
    for a, b, c in stored_basis(l):
        flat = 0
        for d in (0,) * a + (1,) * b + (2,) * c:
            flat = flat * 3 + d
        out.append(flat)
    return tuple(out)


def _n_features(total: int, per_feature: int, l_max: int) -> int:
    if total % per_feature != 0:
        raise ValueError(f"Tensor size {total} incompatible with l_max={l_max}.")
    return total // per_feature


def irreps_to_cartesian(irreps: torch.Tensor, l_max: int, n_paths: Optional[List[int]] = None) -> torch.Tensor:
    """Reconstruct full Cartesian tensors from stored components (reference ``o3/utils.py:289-342``)."""
    n_paths = [1] * (l_max + 1) if n_paths is None else list(n_paths)
    b = irreps.shape[0]
    nf = _n_features(irreps.shape[1], sum((2 * l + 1) * n_paths[l] for l in range(l_max + 1)), l_max)
    parts, off = [], 0
    for l in range(l_max + 1):
        size = (2 * l + 1) * nf * n_paths[l]
        block = irreps[:, off:off + size]
        off += size
        if l == 0:
            parts.append(block)
            continue
        M = _reconstruction_matrix(l).to(device=block.device, dtype=block.dtype)
        full = torch.einsum("fk,bku->bfu", M, block.reshape(b, 2 * l + 1, nf * n_paths[l]))
        parts.append(full.reshape(b, -1))
    return torch.cat(parts, dim=-1)


def cartesian_to_irreps(tensors: torch.Tensor, l_max: int, n_paths: Optional[List[int]] = None) -> torch.Tensor:
    """Select the stored components of symmetric traceless tensors (reference ``o3/utils.py:345-393``)."""
    n_paths = [1] * (l_max + 1) if n_paths is None else list(n_paths)
    b = tensors.shape[0]
    nf = _n_features(tensors.shape[1], sum((3 ** l) * n_paths[l] for l in range(l_max + 1)), l_max)
    parts, off = [], 0
    for l in range(l_max + 1):
        size = (3 ** l) * nf * n_paths[l]
        block = tensors[:, off:off + size]
        off += size
        if l == 0:
            parts.append(block)
            continue
        idx = torch.as_tensor(_stored_full_indices(l), device=block.device, dtype=torch.long)
        parts.append(block.reshape(b, 3 ** l, nf * n_paths[l]).index_select(1, idx).reshape(b, -1))
    return torch.cat(parts, dim=1)


def _rotate_full(T: torch.Tensor, R: torch.Tensor, l: int) -> torch.Tensor:
    for axis in range(1, l + 1):
        T = torch.movedim(torch.tensordot(T, R, dims=([axis], [1])), -1, axis)
    return T


def rotate_irreps(irreps: torch.Tensor, rot_matrix: torch.Tensor, l_max: int,
                  n_paths: Optional[List[int]] = None) -> torch.Tensor:
    """Apply an orthogonal 3x3 transformation to stored components (reference ``o3/utils.py:400-468``)."""
    if rot_matrix.dim() != 2 or tuple(rot_matrix.shape) != (3, 3):
        raise ValueError(f"Rotation matrix must be of shape [3, 3]. Provided shape: {rot_matrix.shape}.")
    n_paths = [1] * (l_max + 1) if n_paths is None else list(n_paths)
    b = irreps.shape[0]
    nf = _n_features(irreps.shape[1], sum((2 * l + 1) * n_paths[l] for l in range(l_max + 1)), l_max)
    cart = irreps_to_cartesian(irreps, l_max, n_paths)
    parts, off = [], 0
    for l in range(l_max + 1):
        size = (3 ** l) * nf * n_paths[l]
        block = cart[:, off:off + size]
        off += size
        if l == 0:
            parts.append(block)
            continue
        T = block.reshape(b, *([3] * l), nf * n_paths[l])
        parts.append(_rotate_full(T, rot_matrix, l).reshape(b, -1))
    return cartesian_to_irreps(torch.cat(parts, dim=1), l_max, n_paths)


def get_triton_dot_input_precision() -> str:
    """Matrix-core input precision of the linear kernels: always IEEE fp32 here (no TF32 inputs)."""
    return "ieee"

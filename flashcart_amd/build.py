"""Build ``libflashcart_hip.so`` in-tree for gfx950.

Steps: regenerate the HIP headers from the exact derivation (codegen), compile
every ``csrc/*.hip`` translation unit with hipcc in parallel, link one shared
library next to this file. Usage: ``python -m flashcart_amd.build [-j N]``.

Tensor ranks: the default library holds the kernels of ranks 0..3 (the reference's default
``FLASHCART_KERNEL_L_MAX``). ``FLASHCART_KERNEL_L_MAX=4 python -m flashcart_amd.build`` (or
``--l-max 4``) builds ``libflashcart_hip_l4.so`` with ranks 0..4 beside it, from headers generated
into ``_build_l4/generated`` (several minutes: the rank-4 products are long unrolled kernels);
``flashcart_amd._lib`` loads it when ``FLASHCART_KERNEL_L_MAX=4`` is set.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libflashcart_hip.so")
ROOT = os.path.dirname(HERE)
_ENV_L_MAX = "FLASHCART_KERNEL_L_MAX"


def _variant(l_max: int):
    """(generated-header directory, object directory, library) of the build for ranks <= l_max."""
    if l_max <= 3:
        return os.path.join(CSRC, "generated"), BUILD, LIB
    if l_max == 4:
        b = os.path.join(HERE, "_build_l4")
        return os.path.join(b, "generated"), b, os.path.join(HERE, "libflashcart_hip_l4.so")
    raise ValueError(f"the kernels can be built for ranks up to 4, not {l_max}.")
ARCH = os.environ.get("FLASHCART_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=fast",
    # Packed FP32 (v_pk_*_f32) stays disabled in every kernel of this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{CSRC}",
    f"-I{os.path.join(ROOT, 'include')}",
]


# The device neighbour list must reproduce the host list's float64 distance tests bit for
# bit, so its products and sums stay separate roundings (no fused multiply-add), like the
# host build's.
NO_CONTRACT = {"fc_neighbors_dev.hip": ["-ffp-contract=off"]}


def _sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _deps_digest(gen: str) -> str:
    h = hashlib.sha256()
    for d in (CSRC, gen, os.path.join(ROOT, "include")):
        for f in sorted(os.listdir(d)):
            if f.endswith((".h", ".hip", ".cpp")):
                with open(os.path.join(d, f), "rb") as fh:
                    h.update(f.encode() + fh.read())
    h.update(" ".join(CFLAGS).encode() + repr(sorted(NO_CONTRACT.items())).encode())
    return h.hexdigest()


def _compile(src: str, gen: str, build_dir: str) -> str:
    obj = os.path.join(build_dir, os.path.basename(src).rsplit(".", 1)[0] + ".o")
    if src.endswith(".cpp"):  # host-only code
        cmd = ["g++", "-O3", "-fPIC", "-std=c++17", "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *CFLAGS, f"-I{gen}", *NO_CONTRACT.get(os.path.basename(src), []), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, force: bool = True, verbose: bool = False, l_max: int | None = None) -> str:
    """Compile the library (always recompiles when ``force``) and return its path. ``l_max``
    (default: ``FLASHCART_KERNEL_L_MAX``, else 3) selects the rank-3 or the rank-4 library."""
    sys.path.insert(0, ROOT)
    from flashcart_amd.codegen.emit_hip import write_all

    if l_max is None:
        l_max = int(os.environ.get(_ENV_L_MAX, "3"))
    gen, build_dir, lib_path = _variant(l_max)
    write_all(gen, 3 if l_max <= 3 else l_max)
    os.makedirs(build_dir, exist_ok=True)
    digest = _deps_digest(gen)
    stamp = os.path.join(build_dir, "stamp")
    if not force and os.path.exists(lib_path) and os.path.exists(stamp) and open(stamp).read() == digest:
        return lib_path
    srcs = _sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    # the longest units (the products of the highest in1 rank) first
    srcs.sort(key=lambda p: (not os.path.basename(p).startswith("fc_tp_l"), -ord(os.path.basename(p)[-5])))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda p: _compile(p, gen, build_dir), srcs))
    tmp = lib_path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, lib_path)
    with open(stamp, "w") as fh:
        fh.write(digest)
    if verbose:
        print(f"built {lib_path}")
    return lib_path


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--if-stale", action="store_true", help="skip when sources are unchanged")
    ap.add_argument("--l-max", type=int, default=None,
                    help="highest tensor rank of the kernels: 3 (default) or 4 (libflashcart_hip_l4.so)")
    a = ap.parse_args()
    build(a.jobs, force=not a.if_stale, verbose=True, l_max=a.l_max)

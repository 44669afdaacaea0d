"""Build ``libflashcart_hip.so`` in-tree for gfx950.

Steps: regenerate the HIP headers from the exact derivation (codegen), compile
every ``csrc/*.hip`` translation unit with hipcc in parallel, link one shared
library next to this file. Usage: ``python -m flashcart_amd.build [-j N]``.
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


def _deps_digest() -> str:
    h = hashlib.sha256()
    for d in (CSRC, os.path.join(CSRC, "generated"), os.path.join(ROOT, "include")):
        for f in sorted(os.listdir(d)):
            if f.endswith((".h", ".hip", ".cpp")):
                with open(os.path.join(d, f), "rb") as fh:
                    h.update(f.encode() + fh.read())
    h.update(" ".join(CFLAGS).encode() + repr(sorted(NO_CONTRACT.items())).encode())
    return h.hexdigest()


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).rsplit(".", 1)[0] + ".o")
    if src.endswith(".cpp"):  # host-only code
        cmd = ["g++", "-O3", "-fPIC", "-std=c++17", "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *CFLAGS, *NO_CONTRACT.get(os.path.basename(src), []), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, force: bool = True, verbose: bool = False) -> str:
    """Compile the library (always recompiles when ``force``) and return its path."""
    sys.path.insert(0, ROOT)
    from flashcart_amd.codegen.emit_hip import write_all

    write_all(os.path.join(CSRC, "generated"))
    os.makedirs(BUILD, exist_ok=True)
    digest = _deps_digest()
    stamp = os.path.join(BUILD, "stamp")
    if not force and os.path.exists(LIB) and os.path.exists(stamp) and open(stamp).read() == digest:
        return LIB
    srcs = _sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB)
    with open(stamp, "w") as fh:
        fh.write(digest)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--if-stale", action="store_true", help="skip when sources are unchanged")
    a = ap.parse_args()
    build(a.jobs, force=not a.if_stale, verbose=True)

"""Rank-4 parity checks, run in a process of its own with FLASHCART_KERNEL_L_MAX=4 (the variable
selects libflashcart_hip_l4.so at import, as the reference generates its kernels for the limit
it reads at import; tests/test_gpu_rank4.py starts this script). Each check is one of the GPU
parity tests of this directory at rank 4: the expansion, convolution and node-wise products with
rank-4 operands and outputs, the linear maps, RMS norm and gate at l_max = 4, and a model with
l_max_edge_attrs = 4 (per edge and frozen, fused) against the float64 oracle. Prints one line per
check; exits non-zero at the first failure.
"""

import os
import sys
import traceback

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def main() -> int:
    assert os.environ.get("FLASHCART_KERNEL_L_MAX") == "4", "run with FLASHCART_KERNEL_L_MAX=4"
    from flashcart_amd import _lib
    lib = _lib.load()
    assert os.path.basename(_lib.LIB_PATH) == "libflashcart_hip_l4.so"
    assert lib.fc_kernel_l_max() == 4, lib.fc_kernel_l_max()
    from tests import test_gpu_model as M
    from tests import test_gpu_ops as T
    from flashcart_amd.data import AtomicGraph
    from flashcart_amd.data.synthetic import fcc_alloy, model_config

    def model_l4(frozen):
        numbers, pos, cell, pbc = fcc_alloy(2, 2, 2, seed=5)
        cfg = model_config(["Cu", "Ni", "Fe", "Cr"], 16, 4, avg_neighbors=42.0)
        g = AtomicGraph.from_arrays(numbers, pos, cfg["elements"], 5.0, cell=cell, pbc=pbc)
        M._check(M._model(cfg), g, cfg, frozen)

    checks = [
        ("irreps l_max=4", lambda: T.test_irreps_fwd_bwd(4)),
        ("conv TP 4x4->4, C=8", lambda: T._tp_case(4, 4, 4, 8, 1, conv=True)),
        ("conv TP 2x4->4, C=32 (specialised backward)", lambda: T._tp_case(2, 4, 4, 32, 1, conv=True, seed=1)),
        ("conv TP 0x4->4, C=16", lambda: T._tp_case(0, 4, 4, 16, 1, conv=True, seed=2)),
        ("conv TP 4x2->3, C=8", lambda: T._tp_case(4, 2, 3, 8, 1, conv=True, seed=3)),
        ("rows TP 4x4->4 shared", lambda: T._tp_case(conv=False, n=120, l1=4, l2=4, lo=4, f1=8, f2=8, shared=True)),
        ("rows TP 4x4->0 symmetric", lambda: T._tp_case(conv=False, n=120, l1=4, l2=4, lo=0, f1=8, f2=8, sym=True,
                                                        shared=True)),
        ("linear 4->4 with paths", lambda: T.test_linear((4, 4, 16, 8, [1, 2, 3, 2, 1]))),
        ("linear 4->2", lambda: T.test_linear((4, 2, 32, 16, None))),
        ("rms norm l_max=4", lambda: T.test_rms_norm(4, 16)),
        ("gate l_max=4", lambda: T.test_gate(4, 1)),
        ("model L=4 per edge", lambda: model_l4(False)),
        ("model L=4 frozen (pairs, species density, fused blocks)", lambda: model_l4(True)),
    ]
    for name, fn in checks:
        print(f"-- {name}", flush=True)
        try:
            fn()
        except Exception:
            traceback.print_exc()
            print(f"FAILED {name}", flush=True)
            return 1
        print(f"ok {name}", flush=True)
    print("all rank-4 checks passed", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""The golden fixtures catch plausible slips in the oracle (CPU).

Each case plants one mistake in a copy of oracle/ (never in the repository's files) — a dropped
term, a wrong normalisation, a wrong slice or operand order — and runs tests/test_golden.py
against the copy in a subprocess. The reference-generated fixtures must fail every one of them;
a slip they let through would leave that part of the oracle unpinned.
"""

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (file, exact text, replacement, what the slip is)
SLIPS = [
    ("oracle/model.py", 'agg = agg / sd[f"{prefix}.sqrt_avg_neighbors"].to(agg.dtype)', "agg = agg",
     "interaction: missing 1/sqrt(avg_neighbors)"),
    ("oracle/model.py", 'out = out + _o3_linear(sd, f"{prefix}.skip_projection", residual, lin, lout, C, C)', "out = out",
     "dropped skip projection"),
    ("oracle/model.py", "lw = torch.tensor([1.0 / ((2 * l + 1) * (l_max + 1))",
     "lw = torch.tensor([1.0 / ((2 * l + 1) * (l_max + 2))", "RMS norm: wrong rank weights"),
    ("oracle/model.py", "x = torch.cat([o[:, :C] for o in outs], dim=1)",
     "x = torch.cat([o[:, C:2*C] if o.shape[1] > C else o[:, :C] for o in outs], dim=1)",
     "readout: wrong scalar slice"),
    ("oracle/model.py", "if reduced or per_row:", "if per_row:", "product: step-0 weights skipped when path-reduced"),
    ("oracle/model.py", "output = output + feats[:, :out_dim]", "output = output + feats[:, -out_dim:]",
     "product: wrong output selector"),
    ("oracle/ops.py", "x, y = (b2[l1], b1[l2]) if swap else (b1[l1], b2[l2])",
     "x, y = (b1[l1], b2[l2]) if swap else (b1[l1], b2[l2])", "tensor product: swapped paths not swapped"),
]


def _copy_tree(tmp):
    shutil.copytree(os.path.join(ROOT, "oracle"), os.path.join(tmp, "oracle"),
                    ignore=shutil.ignore_patterns("_ref", "__pycache__", "*.so", "*.o"))
    tests = os.path.join(tmp, "tests")
    os.makedirs(os.path.join(tests, "golden"))
    for f in ("__init__.py", "conftest.py", "helpers.py", "test_golden.py"):
        shutil.copy(os.path.join(ROOT, "tests", f), tests)
    shutil.copy(os.path.join(ROOT, "tests", "golden", "__init__.py"), os.path.join(tests, "golden"))
    for f in os.listdir(os.path.join(ROOT, "tests", "golden")):
        if f.endswith(".npz") and not f.startswith("fcc25k"):
            shutil.copy(os.path.join(ROOT, "tests", "golden", f), os.path.join(tests, "golden"))


def _run(tmp):
    env = dict(os.environ, PYTHONPATH=ROOT, OMP_NUM_THREADS="2")
    return subprocess.run([sys.executable, "-m", "pytest", "tests/test_golden.py", "-q", "-x", "-p", "no:cacheprovider",
                           "-k", "not fullsize"], cwd=tmp, env=env, capture_output=True, text=True, timeout=600)


def test_unmodified_copy_passes(tmp_path):
    _copy_tree(str(tmp_path))
    r = _run(str(tmp_path))
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]


@pytest.mark.parametrize("slip", SLIPS, ids=[s[3] for s in SLIPS])
def test_fixtures_catch_slip(tmp_path, slip):
    f, old, new, what = slip
    _copy_tree(str(tmp_path))
    path = os.path.join(str(tmp_path), f)
    src = open(path).read()
    assert src.count(old) == 1, f"slip site not found: {old}"
    with open(path, "w") as fh:
        fh.write(src.replace(old, new))
    r = _run(str(tmp_path))
    assert r.returncode == 1 and " failed" in r.stdout, f"golden tests did not catch: {what}\n{r.stdout[-1500:]}"

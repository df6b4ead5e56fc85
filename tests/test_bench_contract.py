"""bench.py's arithmetic and contract, without a GPU: the no-reuse gather
model reproduces the per-mode and per-iteration bytes quoted for config 3
(12092 x 9184 x 28818, 76 879 419 nonzeros, R = 128: 158.999 / 158.996 /
159.016 GB per mode, 477.01 GB per iteration), and a multi-GPU request
exits with a message (every GPU box here has one GPU)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_gather_model_config3():
    import bench
    dims, nnz, R = (12092, 9184, 28818), 76879419, 128
    per_mode = [bench.gather_bytes(nnz, dims[m], R) / 1e9 for m in range(3)]
    assert [round(x, 3) for x in per_mode] == [158.999, 158.996, 159.016]
    assert round(sum(per_mode), 2) == 477.01
    # 2068 bytes per nonzero per mode: 20 B of COO + two 1 KB factor rows
    assert bench.gather_bytes(1, 0, R) == 2068
    # N-order form: (4N + 8) + (N - 1) R 8 per nonzero
    assert bench.gather_bytes(1, 0, 32, N=5) == 28 + 4 * 32 * 8


@pytest.mark.parametrize("n", ["2", "8"])
def test_multi_gpu_request_exits(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", n],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""

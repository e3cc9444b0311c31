"""bench.py's contract on the CPU: a run asked for more than one GPU exits with a message (this
build measures one GPU), and the algorithmic bytes behind `value` and `roofline.achieved` are the
sizes of the tensors one launch must move -- the int4 codes, the 16-bit scale and min per group of
128, the bf16 activations and the output (bf16, or fp32 per partial slot)."""
import os
import subprocess
import sys

import pytest

from oracle import int4 as o

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


@pytest.mark.parametrize("N,K,M,slots", [(256, 1024, 8, None), (512, 2048, 1, None), (256, 1024, 8, 3),
                                         (128, 640, 32, 2)])
def test_algorithmic_bytes_are_the_tensor_sizes(N, K, M, slots):
    sys.path.insert(0, ROOT)
    import bench
    p, s, m = o.make_weights(N, K, seed=3, dtype="fp16")
    x = o.make_x(M, K, seed=4)
    moved = p.nbytes + 2 * (s.size + m.size) + 2 * x.size   # fp16 scale / min, bf16 x on the device
    moved += 4 * slots * M * N if slots else 2 * M * N         # fp32 partial slots, or the bf16 product
    assert bench.algo_bytes(N, K, M, slots) == moved

"""The product path has no CPU fallback: without the built library every entry fails loudly, and
host tensors are refused before anything runs (no compute on the CPU, no GPU needed here)."""
import os
import subprocess
import sys

import pytest
import torch

from conftest import ROOT

NO_CPU = "no CPU path"


def test_missing_library_raises():
    code = ("import sys; sys.path.insert(0, 'token-rush_amd'); from tokenrush_amd import gfx950; gfx950.ext()")
    env = dict(os.environ, TOKENRUSH_HIP_LIB=os.path.join(ROOT, "_no_such_dir", "libtrhip.so"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300, cwd=ROOT, env=env)
    assert r.returncode != 0
    assert "is not built" in r.stderr


def test_gemm_entries_refuse_host_tensors():
    from tokenrush_amd import gfx950
    N, K = 32, 256
    q = torch.zeros(N, K // 2, dtype=torch.uint8)
    s = torch.ones(N, K // 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match=NO_CPU):
        gfx950.pack(q, s, s.clone())
    B = torch.zeros(N // 16, 1, gfx950.QUAD, dtype=torch.uint8)
    x = torch.zeros(8, K, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match=NO_CPU):
        gfx950.mul(x, B, s)


def test_row_kernels_refuse_host_tensors():
    from tokenrush_amd import fused
    x = torch.zeros(2, 512, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match=NO_CPU):
        fused.add_rmsnorm(x, None, torch.zeros(512, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(RuntimeError, match=NO_CPU):
        fused.silu_mul(x)


def test_accept_and_sample_refuse_host_tensors():
    from tokenrush_amd.accept import AcceptState, accept_greedy
    from tokenrush_amd.sample import SamplingParams, sample
    logits = torch.zeros(4, 4096, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match=NO_CPU):
        accept_greedy(logits, torch.zeros(4, dtype=torch.long), AcceptState(4, "cpu"))
    with pytest.raises(RuntimeError, match=NO_CPU):
        sample(logits, SamplingParams("cpu"))

"""tr_int4_gemm_noalloc (the int4 verify GEMM with its workspace in the library's fixed device
scratch) against tr_int4_gemm with a caller's workspace, through the C-ABI: bit-identical outputs
on consecutive calls (each later call smaller than the one before, so stale partials or counters
left by a larger call would show), and the size limit reported as an error code."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import int4 as o

pytestmark = pytest.mark.gpu


def _weights(N, K, seed):
    from tokenrush_amd import gfx950
    p, s, m = o.make_weights(N, K, seed=seed, dtype="fp16")
    d = torch.device("cuda:0")
    B, sv, _ = gfx950.pack(torch.from_numpy(p).to(d), torch.from_numpy(s).half().to(d), torch.from_numpy(m).half().to(d))
    return B


def _x(M, K, seed):
    return torch.from_numpy(o.make_x(M, K, seed=seed)).to(torch.bfloat16).to("cuda:0")


def test_noalloc_matches_workspace_entry_point(dev):
    from tokenrush_amd import _lib, gfx950
    lib = _lib.lib()
    # (N, K, M): K slots summed in the kernel (the scratch in use), largest first; then a one-slot plan
    cases = [(5120, 17408, 8), (2048, 6144, 24), (1024, 17408, 3), (5120, 5120, 1)]
    for i, (N, K, M) in enumerate(cases):
        print(f"noalloc call {i}: N={N} K={K} M={M} (workspace {gfx950.workspace_bytes(N, K, M)} B)", flush=True)
        assert gfx950.workspace_bytes(N, K, M) <= 16 << 20
        B, x = _weights(N, K, 60 + i), _x(M, K, 70 + i)
        ws, nbytes = gfx950.workspaces(N, dev, K, M)
        st = _lib.stream_of(x)
        want = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        _lib.check(lib.tr_int4_gemm(_lib.ptr(x), _lib.ptr(B), _lib.ptr(want), None, _lib.ptr(ws), nbytes, M, N, K, 128,
                                    1, 0, st), "tr_int4_gemm")
        _lib.check(lib.tr_int4_gemm_noalloc(_lib.ptr(x), _lib.ptr(B), _lib.ptr(got), M, N, K, 128, 1, st),
                   "tr_int4_gemm_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want), (N, K, M)
        # and the same call again: the counters the previous call used read zero again
        got.fill_(float("nan"))
        _lib.check(lib.tr_int4_gemm_noalloc(_lib.ptr(x), _lib.ptr(B), _lib.ptr(got), M, N, K, 128, 1, st),
                   "tr_int4_gemm_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want), (N, K, M, "repeat")


def test_noalloc_rejects_sizes_beyond_its_scratch(dev):
    from tokenrush_amd import _lib, gfx950
    lib = _lib.lib()
    N, K, M = 65536, 17408, 32                     # 6 K slots x 32 x 65536 fp32 partials: 48 MiB
    assert gfx950.workspace_bytes(N, K, M) > 16 << 20
    # rejected on the host before any pointer is used or any kernel is launched
    assert lib.tr_int4_gemm_noalloc(None, None, None, M, N, K, 128, 1, None) == _lib.ERR_SCRATCH
    assert lib.tr_int4_gemm_noalloc(None, None, None, 8, 100, K, 128, 1, None) == _lib.ERR_SHAPE
    with pytest.raises(RuntimeError, match="16 MiB"):
        _lib.check(_lib.ERR_SCRATCH, "tr_int4_gemm_noalloc")

"""Loader for the gfx950 C-ABI library (libtrhip.so, built from ../csrc).

Every GPU operation of this package goes through this library. There is no other
compute path: when the library is missing or cannot load, `lib()` raises, and so does
every caller. Arguments are plain device pointers, sizes and the current HIP stream,
so launches are recorded by hipGraph capture like any other kernel on that stream.
"""
import ctypes
import os

import torch  # loads torch's HIP runtime first; the library binds to the same libamdhip64.so.7

_HERE = os.path.dirname(os.path.abspath(__file__))
# TOKENRUSH_HIP_LIB names another build of the same library (e.g. an instrumented one)
LIB_PATH = os.environ.get("TOKENRUSH_HIP_LIB") or os.path.join(_HERE, "libtrhip.so")

# Error codes (tr_common.h). 1 and 2 mean what the reference's Marlin launcher means by
# them (marlin_bf16.cu:627-669, marlin_bf16.cpp:41-43).
OK, ERR_SHAPE, ERR_CONFIG, ERR_ARG, ERR_LAUNCH, ERR_SCRATCH = 0, 1, 2, 3, 4, 5
_ERRORS = {ERR_SHAPE: "problem shape not supported", ERR_CONFIG: "no kernel configuration",
           ERR_ARG: "bad argument", ERR_LAUNCH: "kernel launch failed",
           ERR_SCRATCH: "needs more than the 16 MiB device scratch of the no-allocation entry point"}

_P, _I = ctypes.c_void_p, ctypes.c_int
# name -> (restype, argtypes); the signatures of include/tokenrush_hip.h
_S = ctypes.c_size_t
SIGNATURES = {
    "tr_gemm_plan": (_I, [_I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "tr_partial_slots": (_I, [_I, _I, _I]),
    "tr_gemm_workspace_bytes": (_S, [_I, _I, _I]),
    "tr_packed_bytes": (_S, [_I, _I]),
    "tr_int4_gemm": (_I, [_P, _P, _P, _P, _P, _S, _I, _I, _I, _I, _I, _I, _P]),
    "tr_int4_gemm_ex": (_I, [_P, _P, _P, _P, _P, _S, _I, _I, _I, _I, _I, _I, _I, _P]),
    "tr_int4_gemm_noalloc": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "tr_int4_gemm_silu": (_I, [_P, _P, _P, _P, _S, _I, _I, _I, _I, _I, _P]),
    "tr_pack_int4": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "tr_unpack_int4": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "tr_pack_int4_pairs": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "tr_unpack_int4_pairs": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "tr_dequant_int4": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "tr_accept_workspace_bytes": (_S, [_I, _I]),
    "tr_lm_head_workspace_bytes": (_S, [_I, _I, _I]),
    "tr_lm_head_greedy": (_I, [_P, _P, _P, _P, _S, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tr_argmax_rows": (_I, [_P, _I, _I, _P, _S, _P, _P]),
    "tr_accept_greedy": (_I, [_P, _I, _I, _P, _P, _S, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tr_accept_tree": (_I, [_P, _I, _I, _P, _P, _P, _S, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tr_sample": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _S, _P, _P]),
    "tr_accept_sample": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _S, _P, _P, _P, _P, _P, _P, _P, _P]),
    "tr_accept_residual": (_I, [_P, _I, _I, _P, _P, _P, _P, _S, _P, _P, _P, _P, _P, _P, _P]),
    "tr_commit_rows": (_I, [_P, _I, ctypes.c_long, _I, _P, _P, _P, _I, _P, _P]),
    "tr_add_rmsnorm": (_I, [_P, _P, _I, _I, _P, _P, _P, _I, _I, ctypes.c_float, _I, _P]),
    "tr_silu_mul": (_I, [_P, ctypes.c_long, _P, _I, _I, _P]),
    "tr_embed_rows": (_I, [_P, _P, _P, _I, _I, ctypes.c_long, _P, _P]),
    "tr_gdn_workspace_bytes": (_S, [_I, _I, _I]),
    "tr_attn_workspace_bytes": (_S, [_I, _I, _I]),
    "tr_attn_prep": (_I, [_P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, ctypes.c_float, _P]),
    "tr_attn_decode": (_I, [_P, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _S, _I, _I, _I, _I, _I, _P]),
    "tr_gdn_step": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, ctypes.c_long, _P, _P, _P, _P, _P, _S, _I, _I, _I, _I,
                         _I, _I, _I, ctypes.c_float, _P]),
    "tr_gdn_tree_step": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, ctypes.c_long, _P, _P, _P, _P, _P, _P, _P, _S, _I,
                              _I, _I, _I, _I, _I, _I, ctypes.c_float, _P]),
    "tr_gdn_tree_commit": (_I, [_P, ctypes.c_long, _P, ctypes.c_long, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "tr_attn_prep_tree": (_I, [_P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I,
                               ctypes.c_float, _P]),
    "tr_attn_decode_tree": (_I, [_P, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _S, _I, _I, _I, _I, _I, _P]),
}

_lib = None


def lib():
    """The loaded library (raises RuntimeError if it is not built or does not load)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C token-rush_amd/csrc)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def check(rc: int, what: str):
    if rc != OK:
        raise RuntimeError(f"{what}: {_ERRORS.get(rc, 'error')} (code {rc})")


def stream_of(t: torch.Tensor):
    """The current HIP stream of t's device, as a raw handle."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("tokenrush_amd kernels take device tensors (no CPU path)")


# Workspaces replaced by larger ones. They stay allocated until the process ends: a hipGraph
# captured earlier still holds their addresses, and freeing them would let the caching
# allocator hand that memory to other tensors which a later replay would then overwrite.
_retired = []


def grown_workspace(registry: dict, key, need: int, device, zero: bool = True) -> torch.Tensor:
    """registry[key], replaced by a new uint8 buffer of at least `need` bytes (zero-filled when
    `zero`) if it is missing or smaller; the buffer it replaces is kept alive."""
    ws = registry.get(key)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _retired.append(ws)
        ws = (torch.zeros if zero else torch.empty)(max(need, 256), dtype=torch.uint8, device=device)
        registry[key] = ws
    return ws

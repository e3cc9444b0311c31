"""The C-ABI library loads and exports every symbol include/*.h declares (no GPU calls)."""
import ctypes
import glob
import os
import re

from conftest import ROOT


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names |= set(re.findall(r"\b(?:int|size_t)\s+(tr_\w+)\s*\(", src))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert {"tr_int4_gemm", "tr_pack_int4", "tr_partial_slots"} <= names


def test_library_exports_every_declared_symbol():
    from tokenrush_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from tokenrush_amd import _lib
    assert _declared() == set(_lib.SIGNATURES), set(_lib.SIGNATURES) ^ _declared()


def test_plan_is_host_only_and_independent_of_m():
    from tokenrush_amd import gfx950
    for N, K in [(5120, 5120), (7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408), (248320, 5120), (16, 128)]:
        for M in (1, 8, 16, 17, 32):
            S, W, R = gfx950.plan(N, K, M)
            assert 1 <= W <= 12 and S >= 1 and R >= 1, (N, K, M, S, W, R)
            assert gfx950.plan(N, K, 1 if M <= 16 else 32) == (S, W, R)     # depends on M only via M > 16
            ws = gfx950.ext().tr_gemm_workspace_bytes(N, K, M)
            assert (ws == 0) == (S == 1)


def test_shape_errors_are_codes_not_crashes():
    from tokenrush_amd import _lib
    lib = _lib.lib()
    # rejected before any HIP call: null pointers / bad shapes
    assert lib.tr_int4_gemm(None, None, None, None, None, 0, 8, 100, 5120, 128, 0, 0, None) == _lib.ERR_SHAPE
    assert lib.tr_int4_gemm(None, None, None, None, None, 0, 33, 128, 5120, 128, 0, 0, None) == _lib.ERR_SHAPE
    assert lib.tr_int4_gemm(None, None, None, None, None, 0, 8, 128, 5120, 64, 0, 0, None) == _lib.ERR_CONFIG
    assert lib.tr_int4_gemm(None, None, None, None, None, 0, 8, 128, 5120, 128, 0, 0, None) == _lib.ERR_ARG
    assert lib.tr_pack_int4(None, None, None, None, 16, 128, None) == _lib.ERR_ARG
    assert lib.tr_partial_slots(100, 128, 1) == -1


def test_packed_bytes():
    from tokenrush_amd import _lib
    lib = _lib.lib()
    assert lib.tr_packed_bytes(34816, 5120) == 34816 // 16 * 10 * 4352 == 34816 * 5120 // 2 + 4 * 34816 * 5120 // 128
    assert lib.tr_packed_bytes(16, 384) == 4352                       # 3 groups padded to one quad
    assert lib.tr_packed_bytes(100, 5120) == 0 and lib.tr_packed_bytes(16, 100) == 0
    assert lib.tr_packed_bytes(1 << 20, 1 << 15) == 0                 # 2 GiB or more: unsupported


def test_ext_module_surface():
    """ext() answers the reference extension module's partial_slots (marlin_bf16.cpp:45-56) with
    the binding's positional arguments, and still exposes every C-ABI entry point."""
    from tokenrush_amd import gfx950
    e = gfx950.ext()
    for N, K in [(5120, 17408), (5120, 6144), (34816, 5120)]:
        assert e.partial_slots(N, K) == gfx950.partial_slots(N, K) == e.partial_slots(N, K, -1, -1, -1)
    assert e.tr_packed_bytes(5120, 5120) == gfx950.ext().tr_packed_bytes(5120, 5120) > 0


def test_tree_split_count_fits_one_pass():
    """A draft tree's flash-decoding grid (kv heads x splits x 64-row groups) fits the split
    kernel's resident slots in one pass; chains and small trees keep NSPLIT."""
    from tokenrush_amd import attn
    cfg = attn.AttnConfig()
    assert attn.tree_splits(32, cfg) == 42                     # 4 x 42 x 3 = 504 <= 512
    assert attn.tree_splits(10, cfg) == attn.NSPLIT            # 60 rows: one group
    for M in range(1, 33):
        s = attn.tree_splits(M, cfg)
        groups = -(-6 * M // 64)
        assert 1 <= s <= attn.NSPLIT and cfg.n_kv_heads * s * groups <= attn.SPLIT_SLOTS


def test_partial_plan_is_host_only_and_independent_of_m():
    """The partial-mode plan (the caller sums the slots): between the out-mode plan's slot
    count and 6, depending on M only through the kernel's row range (1-8 staged, 9-16, 17-32),
    and the slot counts measured fastest for the o and down projections (3 at every M; down 5
    up to 8 rows, 4 at 9-16, 6 above)."""
    from tokenrush_amd import gfx950
    for N, K in [(5120, 5120), (7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408), (16, 128), (512, 17408)]:
        for M in (1, 8, 9, 16, 17, 32):
            S = gfx950.partial_slots(N, K, M)
            S0 = gfx950.plan(N, K, M)[0]
            assert S0 <= S <= max(S0, 6), (N, K, M, S, S0)
            assert gfx950.partial_slots(N, K, 1 if M <= 8 else (16 if M <= 16 else 32)) == S
    assert [gfx950.partial_slots(5120, 6144, M) for M in (1, 8, 16, 32)] == [3, 3, 3, 3]
    assert [gfx950.partial_slots(5120, 17408, M) for M in (1, 8, 16, 32)] == [5, 5, 4, 6]
    assert gfx950.partial_slots(5120, 17408, 32) == gfx950.plan(5120, 17408, 32)[0] == 6

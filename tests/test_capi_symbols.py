"""The HIP library loads and exports every entry point declared in include/*.h.

No compute call is made (this runs without a GPU)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "jakal-net_amd" / "lib" / "libjakal_net_hip.so"


def _declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(jn_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared_symbols()
    assert "jn_propagation_topk_forward" in names
    assert "jn_last_error" in names


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), f"{LIB} is not built (run __graft_entry__.build())"
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in _declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"undeclared exports missing from the library: {missing}"


def test_error_channel_and_abi_version_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    lib.jn_abi_version.restype = ctypes.c_int
    assert lib.jn_abi_version() >= 1
    lib.jn_last_error.restype = ctypes.c_char_p
    # argument validation runs on the host before any device call
    P, I64, I32, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
    fn = lib.jn_lowrank_topk_select
    fn.argtypes = [P, I64, I64, P, I64, I64, P, I32, P, F, I64, I64, I64, I64, I64, P, P, P, ctypes.c_size_t, P]
    fn.restype = ctypes.c_int
    rc = fn(None, 4, 0, None, 4, 0, None, 0, None, 1.0, 1, 8, 8, 4, 2, None, None, None, 0, None)
    assert rc != 0
    assert b"null" in lib.jn_last_error()
    ws = lib.jn_propagation_topk_workspace_bytes
    ws.argtypes = [I64] * 6
    ws.restype = ctypes.c_size_t
    # dP [M, 2r] alone is 33.5 MB at B=16, N=4096, r=64
    assert ws(16, 4096, 512, 512, 64, 32) > 16 * 4096 * 128 * 4


def test_select_workspace_is_mode_independent_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    I64 = ctypes.c_int64
    lib.jn_set_select_mode.argtypes = [ctypes.c_int32]
    for name in ("jn_propagation_topk_forward_workspace_bytes", "jn_lowrank_topk_select_workspace_bytes"):
        getattr(lib, name).argtypes = [I64] * 3
        getattr(lib, name).restype = ctypes.c_size_t
    fwd = lib.jn_propagation_topk_forward_workspace_bytes
    try:
        assert lib.jn_set_select_mode(0) == 0
        # split key rows: hi and lo fp16 planes of the rank rounded up to 32
        assert fwd(16, 4096, 64) >= 16 * 4096 * 2 * 64 * 2
        assert fwd(2, 100, 20) >= 2 * 100 * 2 * 32 * 2
        assert lib.jn_lowrank_topk_select_workspace_bytes(16, 4096, 64) == fwd(16, 4096, 64)
        # the size does not depend on the mode: a query and a launch agree whatever mode is set in between
        split_size = fwd(16, 4096, 64)
        for mode in (1, 2, 4, 5, 6):
            assert lib.jn_set_select_mode(mode) == 0
            assert fwd(16, 4096, 64) == split_size
        assert lib.jn_set_select_mode(3) != 0  # retired
        assert lib.jn_set_select_mode(7) != 0
    finally:
        lib.jn_set_select_mode(0)


def test_dense_backward_workspace_without_the_score_matrix():
    """A softsign dense backward that may overwrite the edge matrix needs no
    [B, N, N] workspace; the row-normalising kinds (and softsign without
    reuse) keep one."""
    lib = ctypes.CDLL(str(LIB))
    I64, I32 = ctypes.c_int64, ctypes.c_int32
    ws = lib.jn_propagation_dense_workspace_bytes
    ws.argtypes = [I64] * 5 + [I32, I32]
    ws.restype = ctypes.c_size_t
    square = 16 * 4096 * 4096 * 4
    assert ws(16, 4096, 512, 512, 64, 0, 1) < 100 << 20
    assert ws(16, 4096, 512, 512, 64, 0, 0) > square
    assert ws(16, 4096, 512, 512, 64, 1, 1) > square


def _declared_parameter_counts():
    counts = {}
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for m in re.finditer(r"\b(jn_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
            params = m.group(2).strip()
            counts[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return counts


def test_python_bindings_match_the_header_arity():
    import jakal_net_native as JN  # loads the library; no device call

    counts = _declared_parameter_counts()
    bound = {name: getattr(JN._LIB, name).argtypes for name in counts if getattr(JN._LIB, name).argtypes is not None}
    assert len(bound) >= 30
    wrong = {n: (len(a), counts[n]) for n, a in bound.items() if len(a) != counts[n]}
    assert not wrong, f"ctypes argtypes disagree with include/*.h (bound, declared): {wrong}"


def test_multihead_workspace_queries_without_gpu():
    lib = ctypes.CDLL(str(LIB))
    I64 = ctypes.c_int64
    fwd = lib.jn_propagation_topk_forward_multihead_workspace_bytes
    fwd.argtypes, fwd.restype = [I64] * 4, ctypes.c_size_t
    one = lib.jn_propagation_topk_forward_workspace_bytes
    one.argtypes, one.restype = [I64] * 3, ctypes.c_size_t
    # each head's ranks are padded to 32: 2 heads of rank 20 take the split rows of rank 64
    assert fwd(2, 100, 20, 2) == one(2, 100, 64)
    assert fwd(2, 100, 64, 2) == one(2, 100, 128)
    assert fwd(2, 100, 64, 3) == 0  # 3 x 64 ranks exceed the 128 ranks of a score
    # 3 heads of rank 40 pad to 3 x 64 split ranks, beyond the register select's
    # four K-steps: the scored-rows select takes them, in the same workspace size
    assert fwd(2, 100, 40, 3) == one(2, 100, 192)
    bwd = lib.jn_propagation_topk_multihead_workspace_bytes
    bwd.argtypes, bwd.restype = [I64] * 7, ctypes.c_size_t
    single = lib.jn_propagation_topk_workspace_bytes
    single.argtypes, single.restype = [I64] * 6, ctypes.c_size_t
    # one more bias column per extra head in the row sums and the reduction stage
    assert bwd(2, 100, 16, 16, 8, 4, 5) > single(2, 100, 16, 16, 32, 5)
    tr = lib.jn_transition_topk_multihead_workspace_bytes
    tr.argtypes, tr.restype = [I64] * 9, ctypes.c_size_t
    assert tr(2, 50, 40, 8, 8, 8, 16, 2, 4) > 0
    assert tr(2, 50, 40, 8, 8, 8, 64, 3, 4) == 0
    assert tr(2, 50, 40, 8, 8, 8, 40, 3, 4) > 0  # scored-rows select of 3 heads of rank 40
    assert tr(2, 50, 40, 8, 8, 8, 40, 3, 40) > 0  # every destination: no select, 3 x 40 <= 128 ranks


def test_edge_grouping_beyond_its_size_limit_is_rejected():
    """The top-k backward groups edges by key with per-tile key counts (B x
    (tiles + 1) x N int32, tiles of up to 1024 rows); the workspace and layout
    queries return 0 (unsupported) where that table would exceed 2^28 entries,
    and stay positive below it."""
    lib = ctypes.CDLL(str(LIB))
    I64 = ctypes.c_int64
    lay = lib.jn_propagation_topk_layout_bytes
    lay.argtypes, lay.restype = [I64] * 3, ctypes.c_size_t
    ws = lib.jn_propagation_topk_workspace_bytes
    ws.argtypes, ws.restype = [I64] * 6, ctypes.c_size_t
    tr = lib.jn_transition_topk_workspace_bytes
    tr.argtypes, tr.restype = [I64] * 8, ctypes.c_size_t
    assert lay(1, 70000, 8) > 0 and ws(1, 70000, 16, 16, 8, 8) > 0
    assert lay(1, 500000, 8) > 0  # (489 tiles + the degree row) x 500,000 keys: below the 2^28 entries
    assert lay(1, 1 << 20, 32) == 0 and ws(1, 1 << 20, 16, 16, 8, 32) == 0
    assert tr(1, 1 << 20, 1 << 20, 8, 8, 8, 8, 4) == 0 and tr(1, 4096, 1 << 20, 8, 8, 8, 8, 4) > 0
    # windows need no grouping: their workspace stays linear in N
    win = lib.jn_propagation_window_workspace_bytes
    win.argtypes, win.restype = [I64] * 6, ctypes.c_size_t
    assert 0 < win(1, 1 << 20, 16, 16, 8, 31) < 1 << 31

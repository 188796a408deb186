"""The C ABI (include/dfmi.h) without a GPU: libdfmi.so loads, exports every
declared function, the ctypes table binds exactly that set, and the host-side
argument checks answer without touching the device."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from dflash_mlx_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "dfmi.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dfmi_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        import __graft_entry__

        __graft_entry__.build()
    return _lib.load()


def test_header_declares_the_bound_set():
    declared = _declared()
    assert declared, "no declarations parsed"
    assert declared == sorted(_lib.EXPORTED_SYMBOLS)


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [name for name in _declared() if not hasattr(raw, name)]
    assert not missing, missing
    assert _lib.missing_symbols() == []


def test_version_and_error_string(lib):
    assert lib.dfmi_version().decode().startswith("dfmi ")
    assert isinstance(lib.dfmi_last_error(), bytes)


def test_host_side_validation_without_gpu(lib):
    # bits, group size, dtype and shape checks return DFMI_EINVAL before any device call
    assert lib.dfmi_qmm_affine(None, _lib.DFMI_BF16, None, None, None, None, 16, 4096, 4096, 64, 3,
                               None, 0, None) == _lib.DFMI_EINVAL
    assert b"bits=3" in lib.dfmi_last_error()
    assert lib.dfmi_qmm_affine(None, _lib.DFMI_BF16, None, None, None, None, 16, 4096, 4096, 48, 4,
                               None, 0, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_qmm_affine(None, _lib.DFMI_F32, None, None, None, None, 16, 4096, 4096, 64, 4,
                               None, 0, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_qmm_affine(None, _lib.DFMI_BF16, None, None, None, None, 16, 4100, 4096, 64, 4,
                               None, 0, None) == _lib.DFMI_EINVAL
    # null pointers with a valid shape
    assert lib.dfmi_qmm_affine(None, _lib.DFMI_BF16, None, None, None, None, 16, 4096, 4096, 64, 4,
                               None, 0, None) == _lib.DFMI_EINVAL
    assert b"null" in lib.dfmi_last_error()
    # empty problems are a no-op
    assert lib.dfmi_qmm_affine(None, _lib.DFMI_BF16, None, None, None, None, 0, 4096, 4096, 64, 4,
                               None, 0, None) == _lib.DFMI_OK
    # a forced streaming plan outside the streaming kernel is an error for
    # both weight widths (M > 32; K not whole 256-k steps), and so is an
    # unknown path
    for bits in (4, 8):
        for (M, K) in ((40, 1024), (16, 96)):
            t = _lib.QmmTuning(2, 0, 0, 0)
            assert lib.dfmi_qmm_affine_ex(None, _lib.DFMI_BF16, None, None, None, None, M, K, 64,
                                          32, bits, None, 0, ctypes.byref(t), None) \
                == _lib.DFMI_EINVAL
            assert b"outside the streaming kernel" in lib.dfmi_last_error()
    # path 3 and above are unknown paths
    t3 = _lib.QmmTuning(3, 0, 0, 0)
    assert lib.dfmi_qmm_affine_ex(None, _lib.DFMI_BF16, None, None, None, None, 16, 4096, 4096,
                                  64, 4, None, 0, ctypes.byref(t3), None) == _lib.DFMI_EINVAL
    assert lib.dfmi_qmm_kernel_name(16, 4096, 4096, 64, 4, ctypes.byref(t3)) is None
    # the shared-activation launch: segment count and per-segment checks
    seg = (_lib.QmmSegment * 5)()
    assert lib.dfmi_qmm_affine_multi(None, _lib.DFMI_BF16, seg, 5, 16, 1024, 64, 4, None, 0,
                                     None) == _lib.DFMI_EINVAL
    assert lib.dfmi_qmm_affine_multi(None, _lib.DFMI_BF16, seg, 0, 16, 1024, 64, 4, None, 0,
                                     None) == _lib.DFMI_EINVAL
    seg[0].N, seg[1].N = 64, 64
    assert lib.dfmi_qmm_affine_multi(None, _lib.DFMI_BF16, seg, 2, 16, 1024, 64, 4, None, 0,
                                     None) == _lib.DFMI_EINVAL
    assert lib.dfmi_qmm_affine_multi(None, _lib.DFMI_BF16, seg, 2, 0, 1024, 64, 4, None, 0,
                                     None) == _lib.DFMI_OK
    # its plan: one streaming grid over the matrices' blocks, or one call per
    # matrix outside the streaming kernel
    ns = (ctypes.c_int64 * 3)(5120, 1024, 1024)
    assert lib.dfmi_qmm_multi_kernel_name(16, 5120, ns, 3, 64, 4) == b"qmm_stream_multi_kernel"
    assert lib.dfmi_qmm_multi_kernel_name(16, 5120, ns, 1, 64, 4) == b"qmm_stream_kernel"
    assert lib.dfmi_qmm_multi_kernel_name(16, 5120, ns, 2, 64, 8) == b"qmm_stream_multi_kernel"
    assert lib.dfmi_qmm_multi_kernel_name(40, 5120, ns, 3, 64, 4) is None      # M > 32
    assert lib.dfmi_qmm_multi_kernel_name(16, 1088, ns, 3, 64, 4) is None      # K % 256
    assert lib.dfmi_qmm_multi_kernel_name(16, 5120, ns, 5, 64, 4) is None
    # the grid's split partials cover 64 columns per block of every matrix
    ws = lib.dfmi_qmm_multi_workspace_bytes(16, 5120, ns, 3, 64, 4)
    assert ws == 0 or (ws - 65536) % (16 * 4 * 64 * (80 + 16 + 16)) == 0
    for path in (4, -1):
        t = _lib.QmmTuning(path, 0, 0, 0)
        assert lib.dfmi_qmm_affine_ex(None, _lib.DFMI_BF16, None, None, None, None, 16, 4096,
                                      4096, 64, 4, None, 0, ctypes.byref(t), None) \
            == _lib.DFMI_EINVAL
        assert lib.dfmi_qmm_kernel_name(16, 4096, 4096, 64, 4, ctypes.byref(t)) is None
    assert lib.dfmi_gather_qmm_affine(None, _lib.DFMI_BF16, 4, None, None, None, None, None, None,
                                      8, 256, 64, 4, 64, 8, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_moe_combine(None, _lib.DFMI_F32, None, None, None, 4, 2, 8, None) == _lib.DFMI_EINVAL
    # no routed pairs (zero tokens, so no activation rows either) and no tokens are no-ops
    assert lib.dfmi_gather_qmm_affine(None, _lib.DFMI_BF16, 0, None, None, None, None, None, None,
                                      0, 256, 64, 4, 64, 4, None) == _lib.DFMI_OK
    assert lib.dfmi_gather_qmm_affine(None, _lib.DFMI_BF16, 0, None, None, None, None, None, None,
                                      3, 256, 64, 4, 64, 4, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_moe_combine(None, _lib.DFMI_BF16, None, None, None, 0, 2, 8, None) == _lib.DFMI_OK
    # GDN pair: Dk must be 32 * {1, 2, 4, 8, 16}, Hv a multiple of Hk, float dtypes
    bf, f32 = _lib.DFMI_BF16, _lib.DFMI_F32
    gdn = [None] * 10
    assert lib.dfmi_gated_delta_tape(*gdn, 1, 4, 2, 4, 48, 8, bf, f32, bf, f32, 0, None) == _lib.DFMI_EINVAL
    assert b"Dk" in lib.dfmi_last_error()
    assert lib.dfmi_gated_delta_tape(*gdn, 1, 4, 3, 4, 64, 8, bf, f32, bf, f32, 0, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_gated_delta_tape(*gdn, 1, 4, 2, 4, 64, 8, 7, f32, bf, f32, 0, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_gated_delta_tape(*gdn, 1, 4, 2, 4, 64, 8, bf, f32, bf, f32, 0, None) == _lib.DFMI_EINVAL
    assert b"null" in lib.dfmi_last_error()
    assert lib.dfmi_gated_delta_tape(*gdn, 0, 4, 2, 4, 64, 8, bf, f32, bf, f32, 0, None) == _lib.DFMI_OK
    assert lib.dfmi_tape_replay(*([None] * 6), 1, 4, 2, 4, 640, 8, bf, f32, f32, 0, None) == _lib.DFMI_EINVAL
    assert lib.dfmi_tape_replay(*([None] * 6), 1, 4, 2, 4, 128, 8, bf, f32, f32, 0, None) == _lib.DFMI_EINVAL


def test_workspace_queries(lib):
    # split-K plans need a counter region plus fp32 partials; unsplit plans none
    assert lib.dfmi_qmm_workspace_bytes(16, 4096, 4096, 64, 4) >= 0
    big = lib.dfmi_qmm_workspace_bytes(16, 12288, 4096, 64, 4)
    assert big == 0 or big >= 65536 + 16 * 4096 * 4 * 2
    assert lib.dfmi_qmm_workspace_bytes(16, 4096, 4096, 64, 3) == 0
    assert lib.dfmi_greedy_workspace_bytes(16) >= 256 + 8 * 16
    assert lib.dfmi_lmhead_workspace_bytes(16) >= 256 + 8 * 16


def _plan(lib, M, K, Ns, bits=4, gs=64, tuning=None):
    """(waves, k_splits, whole_blocks, workgroups, pair_streaming, rows_per_block)
    of the streaming launch, checked against the workspace query."""
    from dflash_mlx_amd import _lib
    ns = (ctypes.c_int64 * len(Ns))(*Ns)
    info = _lib.QmmPlanInfo()
    tptr = ctypes.byref(tuning) if tuning is not None else None
    assert lib.dfmi_qmm_plan(M, K, ns, len(Ns), gs, bits, tptr, ctypes.byref(info)) == 0
    assert info.streaming == 1
    if len(Ns) == 1:
        ws = lib.dfmi_qmm_workspace_bytes_ex(M, K, Ns[0], gs, bits, tptr)
    else:
        ws = lib.dfmi_qmm_multi_workspace_bytes(M, K, ns, len(Ns), gs, bits)
    # counters + kp fp32 partials of the split blocks' rows
    split_rows = info.rows_per_block * (info.blocks - info.whole_blocks)
    assert ws == (65536 + info.k_splits * M * split_rows * 4 if info.k_splits > 1 else 0)
    assert info.workgroups == info.whole_blocks + (info.blocks - info.whole_blocks) * info.k_splits
    return (info.waves, info.k_splits, info.whole_blocks, info.workgroups, info.pair_streaming,
            info.rows_per_block)


def test_streaming_split_plans(lib):
    """The streaming matmul's launch plans, read back through the plan query
    (and checked against the workspace query)."""
    # M <= 16, 4-bit, gs 64: pair-streaming plans.  Fewer than 256 blocks:
    # K split so that one workgroup per CU runs (kp = 256 / blocks).  128-row
    # blocks (8 wavefronts, two per CU) where every matrix is a multiple of
    # 128 rows and a workgroup streams >= 8 steps on average, else 64-row
    # blocks (4 wavefronts, three per CU).
    assert _plan(lib, 16, 4096, [4096]) == (4, 4, 0, 256, 1, 64)
    assert _plan(lib, 16, 5120, [5120]) == (4, 3, 0, 240, 1, 64)
    assert _plan(lib, 16, 5120, [5120, 1024, 1024]) == (4, 2, 0, 224, 1, 64)  # 27B q/k/v
    assert _plan(lib, 16, 17408, [5120]) == (8, 6, 0, 240, 1, 128)      # 27B down
    assert _plan(lib, 8, 12288, [4096]) == (4, 4, 0, 256, 1, 64)        # any M <= 16
    assert _plan(lib, 16, 4096, [12288, 12288]) == (8, 1, 0, 192, 1, 128)  # 9B gate/up
    # a split's K range stays within one scale window (120 groups): 68 steps
    # of 4 groups need at least 3 splits, whatever the grid
    assert _plan(lib, 16, 17408, [40960])[1:3] == (3, 0)
    # 256..511 blocks of 128 rows: one whole block per CU and the rest split
    # into one piece per CU; 512..767 blocks of 64 rows: two whole per CU and
    # one piece; whole rounds beyond
    assert _plan(lib, 16, 5120, [32768]) == (8, 1, 0, 256, 1, 128)
    assert _plan(lib, 16, 5120, [17408, 17408]) == (8, 16, 256, 256 + 16 * 16, 1, 128)  # 27B gate/up
    assert _plan(lib, 16, 5120, [40960]) == (8, 4, 256, 256 + 64 * 4, 1, 128)
    assert _plan(lib, 16, 5120, [151936]) == (8, 1, 0, 1187, 1, 128)   # lm_head rows
    # N not a multiple of 128: 64-row blocks
    assert _plan(lib, 16, 5120, [518 * 64 - 51]) == (4, 20, 512, 512 + 6 * 20, 1, 64)
    assert _plan(lib, 16, 5120, [5120, 1000]) == (4, 2, 0, 2 * 96, 1, 64)
    # the 64-row plans on request
    r64 = _lib_tuning(0, 0, 0, 0, 64)
    assert _plan(lib, 16, 17408, [5120], tuning=r64) == (4, 3, 0, 240, 1, 64)
    assert _plan(lib, 16, 5120, [34816], tuning=r64) == (4, 8, 512, 512 + 32 * 8, 1, 64)
    assert _plan(lib, 16, 5120, [40960], tuning=r64) == (4, 2, 512, 512 + 128 * 2, 1, 64)
    assert _plan(lib, 16, 5120, [5120], tuning=_lib_tuning(0, 0, 0, 5, 64)) == \
        (4, 5, 0, 400, 1, 64)
    # 128-row blocks with explicit splits
    assert _plan(lib, 16, 5120, [5120], tuning=_lib_tuning(0, 0, 0, 3, 128)) == \
        (8, 3, 0, 120, 1, 128)
    # gs 128 too; gs 32 and 8-bit weights keep the window plans
    assert _plan(lib, 16, 5120, [17408, 17408], gs=128)[4:] == (1, 128)
    assert _plan(lib, 16, 5120, [5120], gs=128)[4:] == (1, 64)
    assert _plan(lib, 16, 5120, [5120], gs=32)[4:] == (0, 64)
    # M = 17..32, 4-bit gs 64: pair streaming with two activation blocks in
    # 64-row blocks (two stages, three workgroups per CU), the M = 16 rules,
    # and for fewer blocks than CUs splits toward two workgroups per CU while
    # each keeps >= 8 steps of 256 k
    assert _plan(lib, 32, 17408, [5120]) == (4, 6, 0, 480, 1, 64)
    assert _plan(lib, 32, 5120, [5120]) == (4, 3, 0, 240, 1, 64)
    assert _plan(lib, 32, 5120, [17408])[:3] == (4, 20, 256)
    assert _plan(lib, 32, 5120, [34816]) == (4, 8, 512, 512 + 32 * 8, 1, 64)
    # 8-bit, M = 16: the unsplit 192-block grid runs as 4 wavefronts, 2 splits
    assert _plan(lib, 16, 4096, [12288], bits=8)[:2] == (4, 2)
    assert _plan(lib, 16, 4096, [4096], bits=8)[:2] == (8, 4)
    # explicit splits / wavefronts take the window planner; the plan still
    # runs on the pair kernel when it has 4 wavefronts and one activation block
    assert _plan(lib, 16, 5120, [5120], tuning=_lib_tuning(0, 0, 4, 2)) == (4, 2, 0, 160, 1, 64)
    assert _plan(lib, 16, 5120, [5120], tuning=_lib_tuning(0, 0, 8, 2)) == (8, 2, 0, 160, 0, 64)
    # 128-row blocks need a pair-streaming shape with N a multiple of 128
    from dflash_mlx_amd import _lib
    for (M, K, N, gs, bits) in ((16, 5120, 5000, 64, 4), (32, 5120, 5120, 64, 4),
                                (16, 5120, 5120, 32, 4), (16, 5120, 5120, 64, 8)):
        ns = (ctypes.c_int64 * 1)(N)
        info = _lib.QmmPlanInfo()
        t = _lib_tuning(0, 0, 0, 0, 128)
        assert lib.dfmi_qmm_plan(M, K, ns, 1, gs, bits, ctypes.byref(t), ctypes.byref(info)) == \
            _lib.DFMI_EINVAL


def _lib_tuning(path, tiles, waves, splits, rows=0):
    from dflash_mlx_amd import _lib
    return _lib.QmmTuning(path, tiles, waves, splits, rows)

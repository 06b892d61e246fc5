"""The C ABI without a GPU: the library loads, exports every declared symbol,
rejects bad arguments with its status codes before touching a device, and its
planner makes the documented dispatch decisions."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest
import torch

from switchyard import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "switchyard.h"
OK, NULL, SHAPE, DTYPE, WORKSPACE, STRIDE, DEVICE, OP = 0, -1, -2, -3, -4, -5, -6, -7
BF16, F16, F32 = 2, 1, 0


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(sy_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 24, names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in switchyard.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_abi_version_and_error_strings():
    lib = _lib.lib()
    assert lib.sy_abi_version() == 4
    for code in (OK, NULL, SHAPE, DTYPE, WORKSPACE, STRIDE, DEVICE, OP):
        assert lib.sy_strerror(code)
    assert b"NULL" in lib.sy_strerror(NULL)
    assert b"unknown" in lib.sy_strerror(-99)


def _p(x: int | None):
    return None if x is None else ctypes.c_void_p(x)


FAKE = 0x1000  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize(
    "args,code",
    [
        ((None, FAKE, FAKE, None, 9, 16, 2048, 16 * 2048, BF16, BF16), NULL),
        ((FAKE, FAKE, FAKE, None, 0, 16, 2048, 16 * 2048, BF16, BF16), SHAPE),
        ((FAKE, FAKE, FAKE, None, 9, 16, 0, 0, BF16, BF16), SHAPE),
        ((FAKE, FAKE, FAKE, None, 9, -1, 2048, 0, BF16, BF16), SHAPE),
        ((FAKE, FAKE, FAKE, None, 9, 16, 2048, 16 * 2048, 7, BF16), DTYPE),
        ((FAKE, FAKE, FAKE, None, 9, 16, 2048, 16 * 2048, BF16, -1), DTYPE),
        ((FAKE, FAKE, FAKE, None, 9, 16, 2048, 100, BF16, BF16), STRIDE),
    ],
)
def test_forward_rejects_bad_arguments_before_device_work(args, code):
    v, w, out, stats, n, t, d, stride, vt, wt = args
    rc = _lib.lib().sy_fwd(_p(v), _p(w), _p(out), _p(stats), n, t, d, stride, vt, wt, 1e-6, None)
    assert rc == code


def test_forward_with_no_tokens_is_a_no_op():
    # Empty tensors have NULL data pointers; nothing is launched.
    assert _lib.lib().sy_fwd(None, None, None, None, 9, 0, 2048, 0, BF16, BF16, 1e-6, None) == OK


def test_backward_and_batched_reject_bad_arguments():
    lib = _lib.lib()
    # dw is always written, so it is required even with no tokens
    assert lib.sy_bwd(None, None, None, None, None, None, None, 0, 9, 0, 2048, 0, BF16, BF16, 1e-6, None) == NULL
    assert lib.sy_bwd(_p(FAKE), _p(FAKE), None, None, _p(FAKE), _p(FAKE), _p(FAKE), 1 << 20,
                      9, 16, 2048, 16 * 2048, BF16, BF16, 1e-6, None) == NULL
    assert lib.sy_bwd_main(_p(FAKE), _p(FAKE), _p(FAKE), None, _p(FAKE), _p(FAKE), 1 << 20,
                           0, 16, 2048, 16 * 2048, BF16, BF16, 1e-6, None) == SHAPE
    assert lib.sy_fwd_batched(_p(FAKE), _p(FAKE), _p(FAKE), 9, 0, 16, 2048, 16 * 2048, BF16, 1e-6, None) == SHAPE
    assert lib.sy_fwd_batched(None, _p(FAKE), _p(FAKE), 9, 4, 16, 2048, 16 * 2048, BF16, 1e-6, None) == NULL
    assert lib.sy_sol(_p(FAKE), _p(FAKE), 9, 16, 2048, 16 * 2048, 9, None) == DTYPE
    assert lib.sy_dw_reduce(None, 4, 2048, _p(FAKE), BF16, None) == NULL
    assert lib.sy_dw_reduce(_p(FAKE), 4, 0, _p(FAKE), BF16, None) == SHAPE
    assert lib.sy_bw_probe(4, _p(FAKE), _p(FAKE), 1024, None) == OP
    assert lib.sy_bw_probe(3, _p(FAKE), _p(FAKE), 1024, None) == SHAPE  # the mix probe reads 144-byte units
    assert lib.sy_bw_probe(0, _p(FAKE), _p(FAKE), 1000, None) == SHAPE
    assert lib.sy_bw_probe(2, None, _p(FAKE), 1024, None) == NULL
    assert lib.sy_bwd_workspace_bytes(0, 16, 2048, BF16, BF16) == SHAPE
    assert lib.sy_bwd_workspace_bytes(9, 16, 2048, 5, BF16) == DTYPE
    assert lib.sy_bwd_workspace_bytes(9, 0, 2048, BF16, BF16) == 0
    assert lib.sy_bwd_partial_rows(9, 0, 2048, BF16, BF16, 1, 1) == 0


def _table(*ptrs):
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def test_pointer_table_entry_points_reject_bad_arguments():
    lib = _lib.lib()
    rows = _table(FAKE, FAKE)
    # NULL table, NULL row, too many rows, bad dtype, bad size
    assert lib.sy_fwd_table(None, _p(FAKE), _p(FAKE), None, 2, 16, 2048, BF16, BF16, 1e-6, None) == NULL
    assert lib.sy_fwd_table(_table(FAKE, None), _p(FAKE), _p(FAKE), None, 2, 16, 2048, BF16, BF16,
                            1e-6, None) == NULL
    big = _table(*([FAKE] * 17))
    assert lib.sy_fwd_table(big, _p(FAKE), _p(FAKE), None, 17, 16, 2048, BF16, BF16, 1e-6, None) == SHAPE
    assert lib.sy_fwd_table(rows, _p(FAKE), _p(FAKE), None, 2, 16, 2048, 9, BF16, 1e-6, None) == DTYPE
    assert lib.sy_fwd_table(rows, _p(FAKE), _p(FAKE), None, 2, 16, 0, BF16, BF16, 1e-6, None) == SHAPE
    assert lib.sy_fwd_table(None, None, None, None, 2, 0, 2048, BF16, BF16, 1e-6, None) == OK
    assert lib.sy_bwd_table(rows, _p(FAKE), _p(FAKE), None, rows, None, _p(FAKE), 1 << 20, 2, 16, 2048,
                            BF16, BF16, 1e-6, None) == NULL
    assert lib.sy_bwd_table(rows, _p(FAKE), _p(FAKE), None, _table(FAKE, None), _p(FAKE), _p(FAKE),
                            1 << 20, 2, 16, 2048, BF16, BF16, 1e-6, None) == NULL
    assert lib.sy_fwd_batched_table(rows, _p(FAKE), _p(FAKE), 2, 0, 16, 2048, BF16, 1e-6, None) == SHAPE


def test_statistics_and_merge_entry_points_reject_bad_arguments():
    lib = _lib.lib()
    f = _p(FAKE)
    assert lib.sy_attn_with_stats(f, f, f, None, f, None, 9, 16, 2048, 16 * 2048, BF16, BF16, 1e-6,
                                  None) == NULL
    assert lib.sy_attn_with_stats(f, f, f, f, f, None, 9, 16, 2048, 100, BF16, BF16, 1e-6, None) == STRIDE
    assert lib.sy_attn_with_stats_bwd(f, f, f, None, f, None, f, f, f, 1 << 20, 9, 16, 2048, 16 * 2048,
                                      BF16, BF16, 1e-6, None) == NULL
    assert lib.sy_batched_with_stats(f, f, f, f, f, 9, 0, 16, 2048, 16 * 2048, BF16, 1e-6, None) == SHAPE
    assert lib.sy_merge_stats(f, f, f, f, f, f, f, f, f, 16, 2048, 7, None) == DTYPE
    assert lib.sy_merge_stats(f, f, f, f, f, f, f, f, f, 16, 0, BF16, None) == SHAPE
    assert lib.sy_merge_stats(f, f, None, f, f, f, f, f, f, 16, 2048, BF16, None) == NULL
    assert lib.sy_merge_stats(None, None, None, None, None, None, None, None, None, 0, 2048, BF16,
                              None) == OK
    assert lib.sy_merge_stats_bwd(*([f] * 14), None, 16, 2048, BF16, None) == NULL
    # the fused phase 2: every pointer is required (m and l carry the merged
    # statistics), normalize is 0 or 1, and nothing runs without tokens
    assert lib.sy_attn_with_stats_merge(f, f, f, f, None, f, f, f, 5, 16, 2048, 16 * 2048, BF16, BF16,
                                        1e-6, 1, None) == NULL
    assert lib.sy_attn_with_stats_merge(f, f, f, f, f, f, None, f, 5, 16, 2048, 16 * 2048, BF16, BF16,
                                        1e-6, 1, None) == NULL
    assert lib.sy_attn_with_stats_merge(f, f, f, f, f, f, f, f, 5, 16, 2048, 100, BF16, BF16, 1e-6, 1,
                                        None) == STRIDE
    assert lib.sy_attn_with_stats_merge(f, f, f, f, f, f, f, f, 5, 16, 2048, 16 * 2048, BF16, BF16, 1e-6,
                                        2, None) == OP
    assert lib.sy_attn_with_stats_merge(None, None, None, None, None, None, None, None, 5, 0, 2048, 0, BF16,
                                        BF16, 1e-6, 1, None) == OK


def test_batched_backward_rejects_bad_arguments():
    lib = _lib.lib()
    f = _p(FAKE)
    assert lib.sy_bwd_batched(f, f, f, f, None, f, 1 << 20, 9, 8, 16, 2048, 16 * 2048, BF16, 1e-6,
                              None) == NULL
    assert lib.sy_bwd_batched(f, f, f, f, f, f, 1 << 20, 9, 0, 16, 2048, 16 * 2048, BF16, 1e-6,
                              None) == SHAPE
    assert lib.sy_bwd_batched(f, f, f, f, f, f, 1 << 20, 9, 8, 16, 2048, 100, BF16, 1e-6, None) == STRIDE
    assert lib.sy_bwd_batched_workspace_bytes(9, 0, 16, 2048, BF16) == SHAPE
    assert lib.sy_bwd_batched_workspace_bytes(9, 8, 0, 2048, BF16) == 0


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device status")
def test_device_queries_report_missing_device():
    lib = _lib.lib()
    assert lib.sy_bwd_workspace_bytes(9, 4096, 2048, BF16, BF16) == DEVICE
    info = (ctypes.c_int32 * 4)()
    assert lib.sy_kernel_info(0, 9, 4096, 2048, BF16, BF16, info) in (DEVICE, OK)


def test_probe_grid_is_bounded():
    lib = _lib.lib()
    assert lib.sy_probe_grid(16) == 1
    assert lib.sy_probe_grid(1 << 30) == 32768
    assert lib.sy_probe_grid(1 << 20) == 64
    assert lib.sy_probe_grid(0) == 1


# --------------------------------------------------------------------------
# Planner (pure host arithmetic)
# --------------------------------------------------------------------------


def plan(op, n, d, dt=torch.bfloat16, **kw):
    return _lib.plan(op, n, d, dt, **kw)


def test_representative_shape_is_register_resident_everywhere():
    for op in (_lib.OP_FWD, _lib.OP_BWD, _lib.OP_SOL):
        assert plan(op, 9, 2048)["family_name"] == "resident"
    assert plan(_lib.OP_BATCHED, 9, 2048, n_q=8)["family_name"] == "matrix"
    assert plan(_lib.OP_BATCHED, 9, 2048, torch.float32, n_q=8)["family_name"] == "resident"


@pytest.mark.parametrize("n,d", [(9, 4096), (16, 2048), (9, 8192), (16, 4096), (4, 1024), (1, 256)])
def test_sweep_shapes_stay_resident_in_both_directions(n, d):
    """Every sweep shape's backward holds all rows in registers; so does the
    forward up to 9 rows. Past 9 rows the forward keeps one wave's four chunks
    per lane and runs online-softmax chunks of 4 rows instead of spreading the
    token over more waves."""
    f = plan(_lib.OP_FWD, n, d)
    if n <= 9:
        assert f["family_name"] == "resident"
    else:
        assert f["family_name"] == "chunked" and f["chunks_per_lane"] == 4
        assert f["rows_per_tile"] == 4 and f["n_chunks"] == (n + 3) // 4
        assert f["waves_per_token"] == d // 2048
    assert plan(_lib.OP_BWD, n, d)["family_name"] == "resident"


def test_tiles_cover_the_row_exactly_once():
    for n in (1, 2, 9, 16):
        for d in (64, 128, 512, 1024, 1536, 2048, 4096, 8192):
            for dt, ce in ((torch.bfloat16, 8), (torch.float16, 8), (torch.float32, 4)):
                for op in (_lib.OP_FWD, _lib.OP_BWD):
                    p = plan(op, n, d, dt)
                    if p["family_name"] in ("resident", "chunked"):
                        assert p["elems_per_chunk"] == ce
                        cover = 64 * p["waves_per_token"] * p["chunks_per_lane"] * ce
                        assert cover >= d and cover < 2 * d + 64 * ce, (n, d, dt, op, p)
                        if p["family_name"] == "resident":
                            assert p["rows_per_tile"] >= n


def test_large_n_forward_uses_online_chunks_and_backward_the_32_row_tile():
    f = plan(_lib.OP_FWD, 33, 512)
    assert f["family_name"] == "chunked" and f["n_chunks"] == 3
    assert plan(_lib.OP_FWD, 17, 2048)["family_name"] == "chunked"
    # 16 < N <= 32 (with the forward's stats): 32 rows resident
    for n, d, dt, tile in ((17, 2048, torch.bfloat16, (2, 2, 32)), (32, 2048, torch.bfloat16, (2, 2, 32)),
                           (24, 1024, torch.float16, (2, 1, 32)), (32, 4096, torch.bfloat16, (4, 2, 32)),
                           (32, 2048, torch.float32, (4, 2, 32)), (20, 1024, torch.float32, (2, 2, 32))):
        p = plan(_lib.OP_BWD, n, d, dt)
        assert p["family_name"] == "resident", (n, d)
        assert (p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]) == tile
        assert p["block_threads"] == (512 if tile[1] == 1 else 256)  # two waves per SIMD, or one
    # 32 < N <= 64: 64 rows of one chunk a lane on two or four waves, one wave
    # per SIMD (rows of at most 256 chunks)
    for n, d, dt, tile in ((33, 2048, torch.bfloat16, (4, 1, 64)), (64, 1024, torch.float16, (2, 1, 64)),
                           (48, 1024, torch.float32, (4, 1, 64)), (40, 512, torch.float32, (2, 1, 64))):
        p = plan(_lib.OP_BWD, n, d, dt)
        assert (p["family_name"], p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]) == \
            ("resident",) + tile, (n, d, dt)
        assert p["block_threads"] == 256
    # beyond 64 rows, above 4096 bf16 columns (2048 past 32 rows) or below 128: generic
    for n, d in ((65, 2048), (32, 8192), (33, 4096), (20, 512), (40, 512)):
        assert plan(_lib.OP_BWD, n, d)["family_name"] == "generic", (n, d)


def test_unaligned_rows_and_mixed_dtypes_take_the_generic_kernels():
    assert plan(_lib.OP_FWD, 3, 777)["family_name"] == "generic"
    assert plan(_lib.OP_BWD, 5, 63)["family_name"] == "generic"
    assert plan(_lib.OP_FWD, 9, 2048, aligned=False)["family_name"] == "generic"
    assert plan(_lib.OP_FWD, 9, 2048, w_dtype=torch.float32)["family_name"] == "generic"
    assert plan(_lib.OP_BATCHED, 3, 777, n_q=2)["family_name"] == "per_query"


def test_batched_query_cap():
    assert plan(_lib.OP_BATCHED, 9, 2048, n_q=16)["family_name"] == "matrix"
    assert plan(_lib.OP_BATCHED, 9, 2048, torch.float32, n_q=16)["family_name"] == "resident"
    assert plan(_lib.OP_BATCHED, 9, 2048, n_q=17)["family_name"] == "per_query"


def test_batched_matrix_core_plan_bounds():
    """16-bit inputs with N <= 16, S <= 16 and D in {512, 1024, 1536, 2048}
    (and N <= 9 at D = 4096) take the matrix-core kernel; anything else keeps
    the register tiles."""
    fam = lambda n, d, s, dt=torch.bfloat16: plan(_lib.OP_BATCHED, n, d, dt, n_q=s)["family_name"]
    for dt in (torch.bfloat16, torch.float16):
        for d in (512, 1024, 1536, 2048):
            assert fam(1, d, 4, dt) == "matrix"
            assert fam(16, d, 16, dt) == "matrix"
    assert fam(9, 2048, 3) == "resident"  # few queries: the register tile is faster
    assert fam(17, 2048, 8) != "matrix"
    # D = 4096: eight waves of 512 columns share a token, up to 9 rows
    assert fam(9, 4096, 8) == "matrix" and fam(1, 4096, 16) == "matrix"
    assert fam(10, 4096, 8) == "resident" and fam(9, 4096, 3) == "resident"
    p4 = plan(_lib.OP_BATCHED, 9, 4096, n_q=8)
    assert (p4["waves_per_token"], p4["block_threads"]) == (8, 512)
    assert fam(9, 8192, 8) != "matrix"
    assert fam(9, 256, 8) == "resident"
    assert fam(9, 1000, 8) != "matrix"
    assert fam(9, 2048, 8, torch.float32) == "resident"
    assert plan(_lib.OP_BATCHED, 9, 2048, n_q=8, aligned=False)["family_name"] == "per_query"
    p = plan(_lib.OP_BATCHED, 9, 2048, n_q=8)
    assert (p["waves_per_token"], p["block_threads"], p["tokens_per_block"]) == (4, 256, 1)


def test_backward_takes_four_chunks_only_with_one_wave_per_simd():
    """Four chunks per lane run one wave per SIMD (256-thread workgroups, 512
    registers, at most 4 waves per token), except on rows of 1025-2048 chunks,
    which only eight such waves cover (two a SIMD, 256 registers; up to 9
    rows); every other backward tile runs two waves per SIMD (512 threads)."""
    for n in (1, 2, 4, 5, 9, 12, 16):
        for d in (512, 1024, 1536, 2048, 4096, 8192, 16384):
            for dt in (torch.bfloat16, torch.float32):
                p = plan(_lib.OP_BWD, n, d, dt)
                if p["family_name"] != "resident":
                    continue
                if p["chunks_per_lane"] == 4 and p["waves_per_token"] == 8:
                    assert 1024 < d // (4 if dt == torch.float32 else 8) <= 2048, (n, d, dt, p)
                    assert 2 <= n <= 9, (n, d, dt, p)
                    assert p["rows_per_tile"] == (4 if n <= 4 else 9), (n, d, dt, p)
                    assert (p["block_threads"], p["tokens_per_block"]) == (512, 1), (n, d, dt, p)
                elif p["chunks_per_lane"] == 4:
                    assert 5 <= n <= 16 or (n >= 2 and dt != torch.float32), (n, d, dt, p)
                    assert p["rows_per_tile"] == (4 if n <= 4 else 9 if n <= 9 else 16), (n, d, dt, p)
                    assert p["waves_per_token"] <= (4 if n <= 9 else 2), (n, d, dt, p)
                    assert p["block_threads"] == 256, (n, d, dt, p)
                    assert p["tokens_per_block"] * p["waves_per_token"] == 4
                else:
                    assert p["chunks_per_lane"] <= 2 and p["block_threads"] == 512, (n, d, dt, p)
                    assert p["tokens_per_block"] * p["waves_per_token"] == 8
    tile = lambda p: (p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"])
    assert tile(plan(_lib.OP_BWD, 9, 2048)) == (1, 4, 9)
    assert tile(plan(_lib.OP_BWD, 9, 4096)) == (2, 4, 9)
    assert tile(plan(_lib.OP_BWD, 9, 2048, torch.float32)) == (2, 4, 9)
    assert tile(plan(_lib.OP_BWD, 9, 8192)) == (4, 4, 9)
    assert tile(plan(_lib.OP_BWD, 9, 16384)) == (8, 4, 9)  # two waves a SIMD: spills, still 6x generic
    assert tile(plan(_lib.OP_BWD, 10, 16384))[1] <= 2
    assert tile(plan(_lib.OP_BWD, 9, 8192, torch.float32)) == (8, 4, 9)
    assert tile(plan(_lib.OP_BWD, 4, 8192, torch.float32)) == (8, 4, 4)
    assert tile(plan(_lib.OP_BWD, 3, 16384)) == (8, 4, 4)
    assert tile(plan(_lib.OP_BWD, 4, 2048)) == (1, 4, 4)  # few rows, 16-bit: still four chunks
    assert tile(plan(_lib.OP_BWD, 2, 8192)) == (4, 4, 4)
    assert tile(plan(_lib.OP_BWD, 4, 2048, torch.float32)) == (4, 2, 4)  # fp32: two chunks
    assert tile(plan(_lib.OP_BWD, 1, 2048))[1] <= 2
    assert tile(plan(_lib.OP_BWD, 16, 2048)) == (1, 4, 16)
    assert tile(plan(_lib.OP_BWD, 12, 2048)) == (1, 4, 16)
    assert tile(plan(_lib.OP_BWD, 16, 4096)) == (2, 4, 16)
    # No four-chunk 16-row tile on four waves: 16 rows x 2 chunks on eight,
    # which the with-stats variant (what the plan reports) fits.
    assert tile(plan(_lib.OP_BWD, 16, 8192)) == (8, 2, 16)
    assert tile(plan(_lib.OP_BWD, 16, 1024)) == (1, 2, 16)


def test_batched_backward_plan():
    # matrix cores: 16-bit, S <= 8, D in {512, 1024, 1536, 2048}, N <= 16 (N <= 9 at 2048)
    for dt in (torch.bfloat16, torch.float16):
        for n, s, d in ((9, 8, 2048), (1, 1, 512), (16, 8, 1536), (12, 3, 1024), (4, 3, 512)):
            p = plan(_lib.OP_BWD_BATCHED, n, d, dt, n_q=s)
            assert (p["family_name"], p["waves_per_token"], p["rows_per_tile"]) == \
                ("matrix", 4, 9 if n <= 9 else 16), (n, s, d, dt)
    # else one chunk per lane on the fewest waves that cover the row; N <= 9, S <= 8
    p = plan(_lib.OP_BWD_BATCHED, 9, 2048, torch.float32, n_q=8)
    assert (p["family_name"], p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]) == \
        ("resident", 8, 1, 9)
    assert plan(_lib.OP_BWD_BATCHED, 4, 4096, n_q=3)["waves_per_token"] == 8
    assert plan(_lib.OP_BWD_BATCHED, 4, 1024, torch.float32, n_q=3)["rows_per_tile"] == 4
    assert plan(_lib.OP_BWD_BATCHED, 9, 2048, torch.float32, n_q=2)["waves_per_token"] == 8
    for n, s, d in ((10, 8, 2048), (9, 9, 2048), (9, 8, 8192), (5, 3, 777)):
        assert plan(_lib.OP_BWD_BATCHED, n, d, n_q=s)["family_name"] == "generic", (n, s, d)
    assert plan(_lib.OP_BWD_BATCHED, 9, 2048, n_q=8, aligned=False)["family_name"] == "generic"
    p = _lib.Plan()
    # the generic kernel's per-(query, source) scalars must fit its LDS
    assert _lib.lib().sy_plan_for(4, 4096, 8, 2048, BF16, BF16, 1, ctypes.byref(p)) == SHAPE
    assert _lib.lib().sy_plan_for(4, 9, 0, 2048, BF16, BF16, 1, ctypes.byref(p)) == SHAPE


def test_planner_rejects_bad_input():
    p = _lib.Plan()
    lib = _lib.lib()
    assert lib.sy_plan_for(9, 9, 0, 2048, BF16, BF16, 1, ctypes.byref(p)) == OP
    assert lib.sy_plan_for(5, 9, 1, 2048, BF16, BF16, 1, ctypes.byref(p)) == OP
    assert lib.sy_plan_for(0, 0, 0, 2048, BF16, BF16, 1, ctypes.byref(p)) == SHAPE
    assert lib.sy_plan_for(2, 9, 0, 2048, BF16, BF16, 1, ctypes.byref(p)) == SHAPE
    assert lib.sy_plan_for(0, 9, 0, 2048, 3, BF16, 1, ctypes.byref(p)) == DTYPE
    assert lib.sy_plan_for(0, 9, 0, 2048, BF16, BF16, 1, None) == NULL
    assert lib.sy_plan_for(0, 5000, 0, 7, BF16, BF16, 1, ctypes.byref(p)) == SHAPE


def test_plan_for_tokens_checks_input_and_matches_the_plan_without_a_device():
    """Without a device the token-count rule is skipped, so the plan for a
    launch equals sy_plan_for; bad arguments are rejected the same way."""
    lib = _lib.lib()
    p, q = _lib.Plan(), _lib.Plan()
    assert lib.sy_plan_for_tokens(0, 9, 0, 512, 2048, BF16, BF16, 1, None) == NULL
    assert lib.sy_plan_for_tokens(0, 9, 0, -1, 2048, BF16, BF16, 1, ctypes.byref(p)) == SHAPE
    assert lib.sy_plan_for_tokens(9, 9, 0, 512, 2048, BF16, BF16, 1, ctypes.byref(p)) == OP
    for op in (0, 1, 3):
        assert lib.sy_plan_for_tokens(op, 9, 0, 512, 2048, BF16, BF16, 1, ctypes.byref(p)) == OK
        assert lib.sy_plan_for(op, 9, 0, 2048, BF16, BF16, 1, ctypes.byref(q)) == OK
        assert p.as_dict() == q.as_dict()


# -- measurement overrides ---------------------------------------------------


def test_no_overrides_are_installed_by_default():
    t = _lib.Tuning()
    assert _lib.lib().sy_tuning_get(ctypes.byref(t)) == OK
    assert all(getattr(t, f)[k] == 0 for f in ("fwd_tile", "bwd_tile", "batched_tile", "sol_tile")
               for k in range(3))
    assert (t.bwd_blocks_per_cu, t.mx_slots, t.bmx_waves) == (0, 0, 0)


def test_environment_does_not_change_the_launch(monkeypatch):
    """The library reads no environment variables: the names round one used
    for its measurement knobs are inert now."""
    base = _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096)
    for name, val in (("SY_TILE_FWD", "2,2,9"), ("SY_TILE_BWD", "2,2,9"), ("SY_BWD_BLOCKS_PER_CU", "3"),
                      ("SY_MX_SLOTS", "1"), ("SY_BMX_WAVES", "4")):
        monkeypatch.setenv(name, val)
    assert _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096) == base


def test_tuning_overrides_the_launched_tile_and_restores():
    base = _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096)
    with _lib.tuning(fwd_tile=(2, 2, 9)):
        p = _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096)
        assert (p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]) == (2, 2, 9)
        # a tile that does not cover the row is ignored
        with _lib.tuning(fwd_tile=(1, 1, 9)):
            assert _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096) == base
        p = _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096)
        assert p["waves_per_token"] == 2
        # sy_plan_for never applies overrides
        assert _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16)["waves_per_token"] == 1
    assert _lib.plan(_lib.OP_FWD, 9, 2048, torch.bfloat16, n_tok=4096) == base


@pytest.mark.parametrize("field,val", [("bwd_blocks_per_cu", 65), ("mx_slots", 3), ("bmx_waves", 8),
                                       ("bwd_blocks_per_cu", -1)])
def test_tuning_rejects_out_of_range_values(field, val):
    t = _lib.Tuning()
    setattr(t, field, val)
    assert _lib.lib().sy_tuning_set(ctypes.byref(t)) == SHAPE
    got = _lib.Tuning()
    assert _lib.lib().sy_tuning_get(ctypes.byref(got)) == OK
    assert getattr(got, field) == 0
    assert _lib.lib().sy_tuning_get(None) == NULL

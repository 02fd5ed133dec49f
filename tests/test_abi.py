"""The C ABI library loads, exports every declared entry point, and its
host-only logic (plan validation, row-index division) is correct. No call
here touches a GPU."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from stagehand_amd import _native
from stagehand_amd._native import DESC_DTYPE, PLAN_INFO_DTYPE
from stagehand_amd.unpack import (
    KIND_BF16_F32,
    KIND_COPY_BYTES,
    KIND_F32_BF16,
    KIND_I8_ROWSCALE_BF16,
    KIND_I8_ROWSCALE_F32,
    KIND_ZERO_BYTES,
    make_descs,
)

HEADER = Path(__file__).resolve().parent.parent / "include" / "stagehand_native.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(sh_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.exported_symbols())


def test_abi_version_and_last_error():
    lib = _native.lib()
    assert lib.sh_abi_version() == _native.ABI_VERSION
    st = lib.sh_plan_describe(None, 1, None)
    assert st == _native.SH_ERR_INVALID
    assert "info is NULL" in _native.last_error()


def test_struct_sizes_match_header():
    assert DESC_DTYPE.itemsize == 64
    assert PLAN_INFO_DTYPE.itemsize == 56


def test_struct_mirrors_match_the_c_layout(tmp_path):
    """Every numpy mirror of a header struct has the C compiler's size and field offsets
    (compiled against include/stagehand_native.h with gcc)."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    mirrors = {
        "sh_unpack_desc": _native.DESC_DTYPE,
        "sh_plan_info": _native.PLAN_INFO_DTYPE,
        "sh_load_request": _native.LOAD_REQUEST_DTYPE,
        "sh_copy_item": _native.COPY_ITEM_DTYPE,
        "sh_file_range": _native.FILE_RANGE_DTYPE,
        "sh_file_info": _native.FILE_INFO_DTYPE,
        "sh_pool_stats": _native.POOL_STATS_DTYPE,
        "sh_vmm_stats": _native.VMM_STATS_DTYPE,
        "sh_vmm_region_stats": _native.VMM_REGION_DTYPE,
        "sh_turbo_span": _native.TURBO_SPAN_DTYPE,
    }
    lines = ['#include <stdio.h>', f'#include "{HEADER}"', "int main(void) {"]
    for struct, dt in mirrors.items():
        lines.append(f'  printf("{struct} (sizeof) %zu\\n", sizeof({struct}));')
        for name in dt.names:
            lines.append(f'  printf("{struct} {name} %zu\\n", offsetof({struct}, {name}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-o", str(exe), str(src)], check=True, capture_output=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        struct, field, value = line.split()
        got[(struct, field)] = int(value)
    for struct, dt in mirrors.items():
        assert got[(struct, "(sizeof)")] == dt.itemsize, struct
        for name in dt.names:
            assert got[(struct, name)] == dt.fields[name][1], (struct, name)


def describe(rows) -> dict:
    table = make_descs(rows)
    info = np.zeros(1, dtype=PLAN_INFO_DTYPE)
    _native.call("sh_plan_describe", table.ctypes.data, len(table), info.ctypes.data)
    return {k: int(info[0][k]) for k in PLAN_INFO_DTYPE.names}


def test_plan_describe_counts_and_extents():
    info = describe([
        (KIND_I8_ROWSCALE_BF16, 8, 0, 3072, 3072, 0, 0),
        (KIND_I8_ROWSCALE_BF16, 8 + 3072 * 3072, 2 * 3072 * 3072, 1000, 77, 0, 3072),
    ])
    n = 3072 * 3072 + 77000
    assert info["elements"] == n
    assert info["algo_bytes"] == n * 3 + 4 * (3072 + 1000)
    assert info["src_extent"] == 8 + n
    assert info["dst_extent"] == 2 * n
    assert info["scale_extent"] == 4072
    t = info["tile_elems"]
    assert t % 16 == 0 and t >= 256
    assert info["n_tiles"] == -(-3072 * 3072 // t) + -(-77000 // t)
    assert info["kind_mask"] == 1 << KIND_I8_ROWSCALE_BF16


def test_plan_tiles_start_on_destination_lines():
    """A region whose destination starts off a 4 KiB boundary gets a lead of elements before its
    element 0, so the tiles' destination spans start on such boundaries; the lead is a whole number
    of chunks (8 int8, 4 fp32, 16 bytes of copy, 32 of zero fill) or nothing."""
    t_i8 = describe([(KIND_I8_ROWSCALE_BF16, 0, 0, 1, 1 << 16, 0, 0)])["tile_elems"]
    t_f32 = (1 << 20) // describe([(KIND_F32_BF16, 0, 0, 1, 1 << 20, 0, 0)])["n_tiles"]
    t_copy = (1 << 20) // describe([(KIND_COPY_BYTES, 0, 0, 1, 1 << 20, 0, 0)])["n_tiles"]
    t_zero = (1 << 20) // describe([(KIND_ZERO_BYTES, 0, 0, 1, 1 << 20, 0, 0)])["n_tiles"]

    def tiles(kind, dst_off, numel):
        return describe([(kind, 0, dst_off, 1, numel, 0, 0)])["n_tiles"]

    # exactly one tile of elements: a lead adds a tile, no lead keeps one
    assert tiles(KIND_I8_ROWSCALE_BF16, 16, t_i8) == 2      # lead 8 elements (16 B)
    assert tiles(KIND_I8_ROWSCALE_BF16, 48, t_i8) == 2      # lead 24
    assert tiles(KIND_I8_ROWSCALE_BF16, 4096, t_i8) == 1    # on a boundary already
    assert tiles(KIND_I8_ROWSCALE_BF16, 3 * 4096, t_i8) == 1
    assert tiles(KIND_I8_ROWSCALE_BF16, 64, t_i8) == 2      # lead 32: on a line, not on a boundary
    assert tiles(KIND_I8_ROWSCALE_BF16, 4096 + 4080, t_i8) == 2   # lead 2040, below one tile
    assert tiles(KIND_I8_ROWSCALE_BF16, 4096 + 4080, t_i8 - 2040) == 1
    assert tiles(KIND_I8_ROWSCALE_BF16, 4096 + 4080, t_i8 - 2039) == 2
    assert tiles(KIND_F32_BF16, 4088, t_f32) == 2           # lead 2044 of a 2048-element tile
    assert tiles(KIND_F32_BF16, 4088, 4) == 1
    assert tiles(KIND_F32_BF16, 4088, 5) == 2
    assert tiles(KIND_F32_BF16, 8192, t_f32) == 1
    assert tiles(KIND_I8_ROWSCALE_BF16, 18, t_i8) == 1      # 9 elements: not whole chunks
    assert tiles(KIND_I8_ROWSCALE_BF16, 8, t_i8) == 1       # 4 elements: not whole chunks
    assert tiles(KIND_F32_BF16, 8, t_f32) == 2              # lead 4
    assert tiles(KIND_F32_BF16, 4, t_f32) == 1              # 2 elements
    assert tiles(KIND_COPY_BYTES, 16, t_copy) == 2
    assert tiles(KIND_COPY_BYTES, 8, t_copy) == 1
    assert tiles(KIND_ZERO_BYTES, 32, t_zero) == 2
    assert tiles(KIND_ZERO_BYTES, 16, t_zero) == 1
    assert tiles(KIND_BF16_F32, 16, 1 << 16) == tiles(KIND_BF16_F32, 0, 1 << 16)  # 16-element chunks: never
    # the lead is counted in the last tile too: numel + lead elements
    assert tiles(KIND_I8_ROWSCALE_BF16, 16, t_i8 - 8) == 1
    assert tiles(KIND_I8_ROWSCALE_BF16, 16, t_i8 - 7) == 2


def test_plan_describe_padded_source_extent():
    info = describe([(KIND_I8_ROWSCALE_BF16, 0, 0, 6, 10, 16, 0)])
    assert info["src_extent"] == 5 * 16 + 10
    assert info["dst_extent"] == 6 * 10 * 2


def test_plan_describe_splits_oversize_regions():
    # 2^31 + 2^20 fp32 elements → more than one descriptor, same totals
    n = (1 << 31) + (1 << 20)
    info = describe([(KIND_F32_BF16, 0, 0, 1, n, 0, 0)])
    assert info["n_desc"] == 3
    assert info["elements"] == n
    assert info["src_extent"] == 4 * n and info["dst_extent"] == 2 * n
    info = describe([(KIND_I8_ROWSCALE_BF16, 0, 0, 300000, 12288, 0, 0)])
    assert info["n_desc"] == 2
    assert info["scale_extent"] == 300000


def test_plan_describe_all_kinds_and_empty_regions():
    info = describe([
        (KIND_I8_ROWSCALE_F32, 0, 0, 2, 16, 0, 0),
        (KIND_F32_BF16, 32, 128, 1, 5, 0, 0),
        (KIND_BF16_F32, 52, 138, 1, 3, 0, 0),
        (KIND_COPY_BYTES, 58, 150, 1, 7, 0, 0),
        (KIND_ZERO_BYTES, 0, 157, 1, 9, 0, 0),
        (KIND_F32_BF16, 0, 0, 0, 5, 0, 0),  # empty: dropped
    ])
    assert info["n_desc"] == 5
    assert info["dst_extent"] == 166
    assert info["src_extent"] == 65


@pytest.mark.parametrize("bad", [
    (9, 0, 0, 1, 4, 0, 0),                        # unknown kind
    (KIND_I8_ROWSCALE_BF16, 0, 0, 4, 16, 8, 0),   # src_ld < cols
    (KIND_F32_BF16, 0, 0, 2, 16, 32, 0),          # strided non-int8 region
])
def test_plan_describe_rejects_bad_descriptors(bad):
    with pytest.raises(ValueError):
        describe([bad])


def _div(d: int, n: np.ndarray) -> np.ndarray:
    n = np.ascontiguousarray(n, dtype=np.uint32)
    q = np.zeros_like(n)
    _native.call("sh_index_div", d, n.ctypes.data, q.ctypes.data, n.size)
    return q


def test_index_division_is_exact():
    rng = np.random.default_rng(0)
    divisors = [1, 2, 3, 7, 16, 77, 1000, 3072, 12288, 65535, 65536, 65537, 2**31 - 1, 2**31, 2**32 - 1]
    divisors += [int(x) for x in rng.integers(1, 2**32, 20, dtype=np.uint64)]
    for d in divisors:
        n = np.concatenate([
            rng.integers(0, 2**32, 20000, dtype=np.uint64),
            np.array([0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, 2**32 - 1, 2**32 - 2], dtype=np.uint64) % 2**32,
            (np.arange(1, 2000, dtype=np.uint64) * d) % 2**32,
            (np.arange(1, 2000, dtype=np.uint64) * d - 1) % 2**32,
        ]).astype(np.uint32)
        np.testing.assert_array_equal(_div(d, n), n // np.uint32(d), err_msg=f"d={d}")


def test_index_division_rejects_zero():
    with pytest.raises(ValueError):
        _div(0, np.array([1], np.uint32))


def test_plan_describe_refuses_plans_beyond_the_launch_limit():
    """A plan launches one workgroup of SH_UNPACK_THREADS (512) work-items per tile in a 1-D grid,
    which must stay under 2^32 work-items: the largest plan has (2^32 - 1) // 512 tiles, and one
    tile more is refused at validation instead of failing at launch."""
    max_tiles = (2**32 - 1) // 512
    per_tile = (1 << 20) // describe([(KIND_F32_BF16, 0, 0, 1, 1 << 20, 0, 0)])["n_tiles"]
    info = describe([(KIND_F32_BF16, 0, 0, max_tiles, per_tile, 0, 0)])
    assert info["n_tiles"] == max_tiles
    table = make_descs([(KIND_F32_BF16, 0, 0, max_tiles + 1, per_tile, 0, 0)])
    out = np.zeros(1, dtype=PLAN_INFO_DTYPE)
    assert _native.lib().sh_plan_describe(table.ctypes.data, len(table), out.ctypes.data) == _native.SH_ERR_INVALID
    assert b"tiles" in _native.lib().sh_last_error()


def test_noalloc_entry_point_refuses_tables_beyond_its_scratch():
    """``sh_unpack_noalloc`` checks its static scratch's limits on the host, before any device call:
    at most SH_UNPACK_NOALLOC_MAX_DESCS descriptors and SH_UNPACK_NOALLOC_MAX_TILES tiles."""
    header = (Path(__file__).resolve().parent.parent / "include" / "stagehand_native.h").read_text()
    max_descs = int(re.search(r"#define SH_UNPACK_NOALLOC_MAX_DESCS (\d+)u", header).group(1))
    max_tiles = int(re.search(r"#define SH_UNPACK_NOALLOC_MAX_TILES (\d+)u", header).group(1))
    assert max_descs * 64 + max_tiles * 4 == 8 << 20  # the scratch: table, then one uint32 per tile
    lib = _native.lib()
    per_tile = (1 << 20) // describe([(KIND_F32_BF16, 0, 0, 1, 1 << 20, 0, 0)])["n_tiles"]
    tiles = make_descs([(KIND_F32_BF16, 0, 0, max_tiles + 1, per_tile, 0, 0)])
    assert lib.sh_unpack_noalloc(tiles.ctypes.data, 1, None, 0, None, None, 0, None, 0, None) == _native.SH_ERR_INVALID
    assert b"tiles" in lib.sh_last_error()
    many = make_descs([(KIND_ZERO_BYTES, 0, 16 * i, 1, 16, 0, 0) for i in range(max_descs + 1)])
    assert lib.sh_unpack_noalloc(many.ctypes.data, len(many), None, 0, None, None, 0, None, 0,
                                 None) == _native.SH_ERR_INVALID
    assert b"descriptors" in lib.sh_last_error()


def test_vmm_python_binding_loads_and_reports_statuses():
    """The compiled VMM hot-path binding (``_lib/_sh_vmm``) links the same library as the ctypes
    handle: a NULL allocator or handle comes back as the negated SH_ERR_INVALID, with the message in
    the library's thread-local last error; 64-bit ids are refused before the call."""
    from stagehand_amd import vmm

    m = vmm._fast()
    assert m.ensure(0, 1, 2, 0) == -_native.SH_ERR_INVALID
    assert "sh_vmm_ensure_resident" in _native.last_error()
    assert m.export(0, 4, 16, [3, 4]) == -_native.SH_ERR_INVALID
    assert "sh_vmm_handle_export" in _native.last_error()
    with pytest.raises(ValueError):
        m.ensure(0, 1 << 40, 2, 0)
    with pytest.raises(ValueError):
        m.export(0, 4, 16, [1] * 17)

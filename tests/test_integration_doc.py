"""INTEGRATION.md's binding agrees with the product (CPU only).

The reference-side ctypes sample in INTEGRATION.md maps native statuses to Python exceptions, and
the table at the top of that file says the same in prose. Both must raise what
``stagehand_amd._native.check`` raises, for every status the header declares: the reference's
callers catch these types (``vmm_src/error.rs:30-53``, ``src/stagehand/pool.py:133-139``,
``src/stagehand/errors.py:13-30``).
"""
from __future__ import annotations

import ast
import re
from pathlib import Path

import pytest

from stagehand_amd import _native
from stagehand_amd.errors import StagehandError, StagehandOOMError

REPO = Path(__file__).resolve().parent.parent
DOC = (REPO / "INTEGRATION.md").read_text()
HEADER = (REPO / "include" / "stagehand_native.h").read_text()
NAMES = {"ValueError": ValueError, "StagehandOOMError": StagehandOOMError, "MemoryError": MemoryError,
         "TimeoutError": TimeoutError, "OSError": OSError, "RuntimeError": RuntimeError}


def _statuses() -> dict[str, int]:
    body = re.search(r"enum\s+sh_status\s*\{(.*?)\}", HEADER, re.S)
    assert body, "status enum not found in the header"
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"(SH_\w+)\s*=\s*(\d+)", body.group(1))}


def _sample_map() -> tuple[dict[int, type], type]:
    """The status map and the fallback of the sample's ``check``."""
    code = re.search(r"```python\n(# src/stagehand/_hip.py.*?)```", DOC, re.S)
    assert code, "the ctypes sample is missing from INTEGRATION.md"
    tree = ast.parse(code.group(1))
    mapping, default = None, None
    for node in ast.walk(tree):
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "STATUS_ERRORS" for t in node.targets):
            mapping = {ast.literal_eval(k): NAMES[v.id] for k, v in zip(node.value.keys, node.value.values)}
        if isinstance(node, ast.Call) and getattr(node.func, "attr", None) == "get" and len(node.args) == 2:
            default = NAMES[node.args[1].id]
    assert mapping is not None and default is not None, "STATUS_ERRORS / .get(rc, default) not found in the sample"
    return mapping, default


def _table() -> dict[str, str]:
    return dict(re.findall(r"^\| `(SH_\w+)` \| `?(\w+)`?", DOC, re.M))


def _raised(status: int) -> type | None:
    try:
        _native.check(status, "probe")
    except Exception as exc:  # noqa: BLE001
        return type(exc)
    return None


@pytest.mark.parametrize("name", sorted(_statuses()))
def test_sample_and_table_raise_what_check_raises(name):
    status = _statuses()[name]
    mapping, default = _sample_map()
    got = _raised(status)
    if name in ("SH_OK", "SH_ERR_NOT_READY"):
        assert got is None
        return
    assert got is not None
    sample = mapping.get(status, default)
    assert sample is got, f"{name}: the sample raises {sample.__name__}, check raises {got.__name__}"
    table = _table()
    assert NAMES[table.get(name, "RuntimeError")] is got, f"{name}: INTEGRATION.md's table disagrees"


def test_oom_error_is_a_stagehand_error_not_a_runtime_error():
    assert issubclass(StagehandOOMError, StagehandError)
    assert not issubclass(StagehandOOMError, RuntimeError)
    assert "a `RuntimeError`" not in DOC

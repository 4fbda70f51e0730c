"""Host-side guard: a device pointer handed to the C ABI must come from a
tensor that is still referenced when the launch is enqueued.  `_lib.ptr(f(t))`
takes the address of a temporary (a dtype conversion or contiguous copy) that
CPython frees as soon as `ptr` returns; the caching allocator can then give
the same memory to the next temporary of the same argument list, and the
kernel reads one buffer twice.  Every such argument is bound to a name first.
"""

from __future__ import annotations

import ast
from pathlib import Path

PKG = Path(__file__).resolve().parents[1] / "metal-marlin_amd" / "mmfp4"


def _offenders(root: Path = PKG):
    out = []
    for f in sorted(root.rglob("*.py")):
        tree = ast.parse(f.read_text(), filename=str(f))
        for node in ast.walk(tree):
            if not isinstance(node, ast.Call):
                continue
            fn = node.func
            name = fn.attr if isinstance(fn, ast.Attribute) else getattr(fn, "id", "")
            if name == "ptr" and node.args and isinstance(node.args[0], ast.Call):
                out.append(f"{f.relative_to(root.parent)}:{node.lineno}: {ast.unparse(node)}")
    return out


def test_no_pointer_to_a_temporary():
    assert _offenders() == []


def test_guard_sees_the_pattern(tmp_path):
    """The scan flags a pointer to a converted copy and passes a named one."""
    pkg = tmp_path / "pkg"
    pkg.mkdir()
    (pkg / "bad.py").write_text("def f(_lib, s):\n    return _lib.ptr(s.contiguous())\n")
    (pkg / "good.py").write_text("def f(_lib, s):\n    c = s.contiguous()\n"
                                 "    return _lib.ptr(c)\n")
    found = _offenders(pkg)
    assert len(found) == 1 and "bad.py:2" in found[0]

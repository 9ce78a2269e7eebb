"""bench.py runs only on a GPU box; this CPU test reads it statically so that
a name a function uses but never binds (a NameError at round end) shows up
here: every name read inside a function must be bound in that function or an
enclosing one, at module level, or be a builtin."""
from __future__ import annotations

import ast
import builtins
from pathlib import Path

BENCH = Path(__file__).resolve().parent.parent / "bench.py"


def _bound(node: ast.AST) -> set[str]:
    names: set[str] = set()
    for n in ast.walk(node):
        if isinstance(n, ast.Name) and isinstance(n.ctx, (ast.Store, ast.Del)):
            names.add(n.id)
        elif isinstance(n, (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef)):
            names.add(n.name)
        elif isinstance(n, ast.arg):
            names.add(n.arg)
        elif isinstance(n, (ast.Import, ast.ImportFrom)):
            for a in n.names:
                names.add((a.asname or a.name).split(".")[0])
        elif isinstance(n, ast.ExceptHandler) and n.name:
            names.add(n.name)
        elif isinstance(n, (ast.Global, ast.Nonlocal)):
            names.update(n.names)
    return names


def test_bench_functions_bind_every_name_they_read():
    tree = ast.parse(BENCH.read_text())
    module = {"__file__", "__name__", "__doc__"}
    for s in tree.body:
        if isinstance(s, (ast.FunctionDef, ast.ClassDef)):
            module.add(s.name)
        else:
            module |= _bound(s)
    known = module | set(dir(builtins))
    missing = []
    for fn in [s for s in tree.body if isinstance(s, ast.FunctionDef)]:
        local = _bound(fn)
        for n in ast.walk(fn):
            if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load) and n.id not in local and n.id not in known:
                missing.append(f"{fn.name}:{n.lineno}: {n.id}")
    assert not missing, missing

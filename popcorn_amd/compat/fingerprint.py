"""Code digests that tie a stored record to the code that produced it.

Popcorn hashes an AST-normalised form of the reference, the adapter and the
source module, plus the bytes of sibling CUDA files (core/fingerprint.py:24,
80-87, 163-202), so that editing any of them makes old records stale. This
restatement keeps that contract with a simpler normalisation:

  * a Python callable is hashed by `ast.dump` of its source with docstrings
    removed (comments and formatting never reach the AST);
  * a `source=` dotted path is hashed by the text of the module file it names
    (only its parent packages are imported) and, when that module's package has a
    `csrc/` directory, by the bytes of every file in it -- the HIP kernels of
    this backend;
  * anything whose source cannot be read yields None, which disables the
    staleness check for that record (store.matching).
"""

from __future__ import annotations

import ast
import hashlib
import importlib.util
import inspect
import textwrap
from pathlib import Path
from typing import Any


def _strip_docstrings(tree: ast.AST) -> ast.AST:
    for node in ast.walk(tree):
        if isinstance(node, (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef, ast.Module)):
            body = getattr(node, "body", [])
            if body and isinstance(body[0], ast.Expr) and isinstance(getattr(body[0], "value", None), ast.Constant):
                if isinstance(body[0].value.value, str):
                    node.body = body[1:] or [ast.Pass()]
    return tree


def _callable_text(obj: Any) -> str | None:
    target = inspect.unwrap(obj) if callable(obj) else obj
    try:
        source = textwrap.dedent(inspect.getsource(target))
    except (OSError, TypeError):
        return None
    try:
        tree = ast.parse(source)
    except SyntaxError:
        # lambdas inside a larger expression: hash the raw line
        return source
    return ast.dump(_strip_docstrings(tree), include_attributes=False)


def _module_files(dotted: str) -> list[Path]:
    """The module file a dotted source path lives in (only parent packages are imported)."""
    parts = dotted.split(".")
    spec = None
    for cut in range(1, len(parts) + 1):
        try:
            found = importlib.util.find_spec(".".join(parts[:cut]))
        except (ImportError, ValueError):
            found = None
        if found is None:
            break
        spec = found
        if found.submodule_search_locations is None:
            break  # a plain module: the remaining parts are attributes
    if spec is None or not spec.origin or spec.origin in ("built-in", "frozen"):
        return []
    origin = Path(spec.origin)
    files = [origin]
    csrc = origin.parent / "csrc"
    if csrc.is_dir():
        files += sorted(p for p in csrc.rglob("*") if p.is_file())
    return files


def fingerprint(*parts: Any, source: str | None = None) -> str | None:
    digest = hashlib.sha1()
    for part in parts:
        text = _callable_text(part)
        if text is None:
            return None
        digest.update(text.encode())
    if source is not None:
        files = _module_files(source)
        if not files:
            return None
        digest.update(source.encode())
        for path in files:
            digest.update(path.name.encode())
            digest.update(path.read_bytes())
    return digest.hexdigest()[:16]

"""Operator discovery for the package namespace.

The public contract is the reference's (src/flaggems_sglang/__init__.py:34-55,
runtime/op_registrar.py:116): each public module of ``flaggems_sglang.ops``
exposes its operators through ``__all__``, and only plain Python functions
(``inspect.isfunction``) are taken. The reference layers vendor and
architecture overrides on top of the generic modules; this package has a
single implementation (gfx950 HIP kernels), so discovery is one pass.

``discover_operators`` returns a fresh name -> function table; the package
``__init__`` publishes it and answers ``all_registered_ops`` / ``get_op``
from it.
"""

from __future__ import annotations

import importlib
import inspect
import pkgutil
from types import ModuleType
from typing import Callable, Dict, Iterator

OPS_PACKAGE = "flaggems_sglang.ops"


def _operator_modules(package: str) -> Iterator[ModuleType]:
    """Import and yield the package's public leaf modules (sub-packages and
    names with a leading underscore are private)."""
    root = importlib.import_module(package)
    for info in pkgutil.iter_modules(root.__path__):
        if info.ispkg or info.name[:1] == "_":
            continue
        yield importlib.import_module(package + "." + info.name)


def discover_operators(package: str = OPS_PACKAGE) -> Dict[str, Callable]:
    """Map every function named in a public module's ``__all__`` to itself.

    Names that a module lists but does not define, and listed objects that
    are not plain functions (classes, constants, builtins), are skipped.
    A later module wins when two export the same name.
    """
    table: Dict[str, Callable] = {}
    for module in _operator_modules(package):
        for name in getattr(module, "__all__", None) or ():
            candidate = getattr(module, name, None)
            if inspect.isfunction(candidate):
                table[name] = candidate
    return table


__all__ = ["discover_operators", "OPS_PACKAGE"]

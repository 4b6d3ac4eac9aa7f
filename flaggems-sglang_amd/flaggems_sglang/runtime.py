"""Operator registry of the package.

Same contract as the reference's ``OpRegistrar``
(src/flaggems_sglang/runtime/op_registrar.py:42-118): walk the
``flaggems_sglang.ops`` package, import each public module and merge every
plain function its ``__all__`` lists (``inspect.isfunction`` filter, :116).
The reference's vendor and architecture tiers (:79-94) do not exist here:
the only implementation is the gfx950 one.
"""

from __future__ import annotations

import importlib
import inspect
import pkgutil
from typing import Callable, Dict, List, Optional


class OpRegistrar:
    """Collect operators from the ``ops`` package."""

    def __init__(self, generic_pkg: str = "flaggems_sglang.ops"):
        self._generic_pkg = generic_pkg
        self._resolved: Dict[str, Callable] = {}

    def apply(self, target_globals: Optional[Dict] = None) -> Dict[str, Callable]:
        self._resolved.clear()
        pkg = importlib.import_module(self._generic_pkg)
        for mod_info in pkgutil.iter_modules(pkg.__path__):
            if mod_info.ispkg or mod_info.name.startswith("_"):
                continue
            mod = importlib.import_module(f"{self._generic_pkg}.{mod_info.name}")
            for name in getattr(mod, "__all__", ()):
                fn = getattr(mod, name, None)
                if fn is not None and inspect.isfunction(fn):
                    self._resolved[name] = fn
        if target_globals is not None:
            target_globals.update(self._resolved)
        return dict(self._resolved)

    @property
    def resolved(self) -> Dict[str, Callable]:
        return dict(self._resolved)

    def names(self) -> List[str]:
        return sorted(self._resolved)

    def get(self, name: str) -> Optional[Callable]:
        return self._resolved.get(name)


__all__ = ["OpRegistrar"]

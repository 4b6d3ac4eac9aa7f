"""flaggems_sglang -- fused-MoE operator for AMD Instinct MI355X (gfx950).

Public surface of the reference package (src/flaggems_sglang/__init__.py:
34-55): the operators of ``flaggems_sglang.ops`` are published as package
attributes, listed by ``all_registered_ops()`` and looked up with
``get_op(name)``; ``device`` and ``vendor_name`` name the hardware. All
operators run hand-written HIP kernels for gfx950 (``libfgs_moe.so``); there
is no vendor or architecture dispatch.
"""

from typing import Callable, List, Optional

from flaggems_sglang.runtime import discover_operators

_OPERATORS = discover_operators()
globals().update(_OPERATORS)


def all_registered_ops() -> List[str]:
    """Sorted names of the operators published on this package."""
    return sorted(_OPERATORS)


def get_op(name: str) -> Optional[Callable]:
    """The operator published as ``name``, or ``None`` for unknown names."""
    return _OPERATORS.get(name)


device = "cuda"  # torch's device type for HIP GPUs
vendor_name = "amd"

__version__ = "0.2.0"

__all__ = ["all_registered_ops", "get_op", "device", "vendor_name",
           *sorted(_OPERATORS)]

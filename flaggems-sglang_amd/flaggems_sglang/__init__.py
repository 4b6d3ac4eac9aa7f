"""flaggems_sglang -- fused-MoE operator for AMD Instinct MI355X (gfx950).

The package keeps the reference's public surface
(src/flaggems_sglang/__init__.py:34-55): every function listed in an
``ops`` module's ``__all__`` is resolved into the package namespace by
:class:`OpRegistrar`, and ``all_registered_ops()``, ``get_op()``,
``device`` and ``vendor_name`` are exported. There is one tier only: the ops
run on hand-written HIP kernels for gfx950 (``libfgs_moe.so``); no vendor or
architecture dispatch exists.
"""

from typing import Callable, List, Optional

from flaggems_sglang.runtime import OpRegistrar

_op_registrar = OpRegistrar()
_op_registrar.apply(globals())


def all_registered_ops() -> List[str]:
    """Names of all operators resolved on the package."""
    return _op_registrar.names()


def get_op(name: str) -> Optional[Callable]:
    """Look up a resolved operator by name; ``None`` if not registered."""
    return _op_registrar.get(name)


device = "cuda"  # torch's device type for HIP GPUs
vendor_name = "amd"

__version__ = "0.1.0"

__all__ = ["all_registered_ops", "get_op", "device", "vendor_name"] + list(
    _op_registrar.names()
)

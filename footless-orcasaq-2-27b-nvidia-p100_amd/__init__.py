"""MI355X (gfx950) implementation of the footless attention / Gated DeltaNet
hot path: hand-written HIP kernels behind a C ABI (include/fl355.h, built into
libfl355.so next to this file) and a PyTorch-ROCm op layer that keeps the
reference kernels' names and argument meanings.

The directory name is not a Python identifier; load it with
``load_package()`` from ``__graft_entry__`` (or importlib), which registers it
as the module ``footless_amd``.
"""
from . import geometry  # noqa: F401
from . import ops  # noqa: F401
from . import state_blob  # noqa: F401
from . import runtime  # noqa: F401
from . import backend  # noqa: F401
from ._lib import FlError, LIB_PATH  # noqa: F401

__all__ = ["geometry", "ops", "runtime", "backend", "state_blob", "FlError", "LIB_PATH"]

"""PokitLMs routed-MoE K-quant path on AMD Instinct MI355X (gfx950).

The compute is hand-written HIP in ``csrc/`` built into ``libpokit_hip.so``
(C ABI: ``include/pokit_hip.h``).  ``backend.HipBackend`` is the Python host
API over it; ``synth`` generates seeded GGUF-compatible inputs.
"""
from . import synth  # noqa: F401

__version__ = "0.1.0"


def library_path() -> str:
    from . import _abi
    return _abi.LIB_PATH


def load():
    """Load libpokit_hip.so (raises ImportError when it has not been built)."""
    from . import _abi
    return _abi.lib()

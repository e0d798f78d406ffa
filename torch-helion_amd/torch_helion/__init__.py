"""torch-helion on MI355X: PyTorch model -> OpIR -> hand-written gfx950 HIP kernels.

Drop-in for the reference package's public API (reference:
src/torch_helion/__init__.py): ``compile_model``, ``CompileConfig``,
``CompileResult``.
"""

from .config import CompileConfig
from .pipeline import CompileResult, compile_model

__version__ = "0.1.0.dev0"

__all__ = ["CompileConfig", "CompileResult", "compile_model", "__version__"]

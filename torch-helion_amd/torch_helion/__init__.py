"""torch-helion on MI355X: PyTorch model -> OpIR -> hand-written gfx950 HIP kernels."""

__version__ = "0.1.0.dev0"

"""Backends for the OpIR: the HIP launch-plan emitter and the CPU interpreter."""

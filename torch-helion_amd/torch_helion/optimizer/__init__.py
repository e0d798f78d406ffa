"""Optimizer: canonicalisation passes, partitioning, legality, planning, OpIR."""

"""The MI355X (gfx950) backend: C-ABI binding, OpIR lowering and runtime."""

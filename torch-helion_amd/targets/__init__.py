"""Eager target models (the parity definitions): llama_block, llama_decode, mamba."""

"""Kernel entry points of the Llama-3 attention path (gfx950 HIP behind a C ABI)."""

"""Entry points kept at the reference's import paths (src/llm_cuda/kernels/triton/).

The module names are kept so that callers written against the reference import
them unchanged; the implementation is hand-written HIP for gfx950, not Triton.
"""

"""Extension-style wrappers (reference: src/llm_cuda/kernels/cuda/), backed by liblcuda_hip.so."""

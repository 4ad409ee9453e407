"""The workload kernels, written against the unchanged user surface.

Kernel bodies are the reference's example kernels (the north-star configs run exactly
these user programs; reference: examples/01-10_*.py); host wrappers here are this
repository's own. They import `enceladus` and `enceladus.language as tl` exactly as
drop-in user code does.
"""

"""The workload kernels, written against the unchanged user surface.

Kernel bodies are the reference's example kernels, kept as written: the north-star configs
are defined as these user programs (reference: examples/01-10_*.py). The host wrappers
(`add`, `softmax`, `matmul_desc`, `matmul_tuned`, `attention`, `attention_tuned`, ...)
follow the reference's wrappers too: same names, arguments and launch grids, so code
written against the reference's examples calls them unchanged. They import `enceladus`
and `enceladus.language as tl` exactly as drop-in user code does. `workloads.py` is this
repository's: the BASELINE configs at full size and the specializations the benchmark
times, shared with the GPU parity tests.
"""

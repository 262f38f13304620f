"""hsd on MI355X: the hot path of mlx-heimr-sparse-down ("hsd") as gfx950 HIP kernels.

Modules keep the reference's names: layout (neuron-major permutation), decode (sparse
down projection), prefill (tile order, union, MFMA grouped GEMM), mamba (multi-row
verify with per-row checkpoints and rollback), mtp (device-side greedy acceptance and
the drafter call surface), synth (seeded synthetic workloads). Tensors are torch
tensors on a ROCm device; every kernel is in libhsd.so (`_native`).
"""
__version__ = "0.1.0"

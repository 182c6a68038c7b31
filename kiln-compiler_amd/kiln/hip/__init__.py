"""Kiln's MI355X backend: lowering to HIP kernel families, ctypes binding,
runtime (plans + hipGraph) and the GEMM tile tuner."""

"""Host launchers for the HIP kernels (one module per kernel family)."""

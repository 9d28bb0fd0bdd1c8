"""Host wrappers of the gfx950 HIP kernels (decode, prefill)."""

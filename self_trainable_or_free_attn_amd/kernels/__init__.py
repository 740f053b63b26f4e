"""Attention kernel sets. `gfx950` holds the MI355X set (HIP kernels behind the C ABI of libechosparse_hip.so)."""

"""Drop-in replacement of the reference's ``kernels`` package (FP8 hot path on gfx950)."""

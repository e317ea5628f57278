"""Library baselines the matrix runner times beside the gfx950 kernels."""

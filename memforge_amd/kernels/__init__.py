"""Device operators of the data path (the reference's memforge_ml.kernels)."""

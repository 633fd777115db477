"""The standalone PagedAttention operator (the reference's memforge_ml.models)."""

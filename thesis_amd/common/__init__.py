"""Model, engines and method registry (the reference's common/ surface)."""

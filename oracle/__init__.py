"""CPU oracle of the GDN decode step (test infrastructure, never the product path)."""

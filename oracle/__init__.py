"""CPU oracle package (test infrastructure; not imported by the product)."""

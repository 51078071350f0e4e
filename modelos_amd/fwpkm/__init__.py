"""Drop-ins for the reference's fwpkm/ package (fast-weight product-key memory)."""

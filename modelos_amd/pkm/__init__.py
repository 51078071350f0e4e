"""Drop-ins for the reference's pkm/ package (slow-weight product-key memory)."""

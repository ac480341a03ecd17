"""Decorated solver loops (the loops of the reference's README and demos)."""

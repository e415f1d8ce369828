"""Python helpers over the tile-IR builder (python/frisk/common in the reference)."""

"""HIP sources (gfx950) and their in-tree build."""

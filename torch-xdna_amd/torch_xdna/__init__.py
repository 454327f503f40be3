"""torch_xdna for MI355X (placeholder while the host layer is written)."""

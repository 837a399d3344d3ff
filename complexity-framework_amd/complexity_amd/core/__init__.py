"""Plug-in layer (mirror of the parts of complexity/core the TR-MoE path uses)."""

"""Quantized-linear provider (mirror of the reference's ``minisgl.quant`` W4A8 surface)."""

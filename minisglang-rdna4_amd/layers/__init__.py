"""Layer-side mirror of the reference's W4A8 MoE expert storage and quant methods."""

"""Inference-side quantized-linear interface (mirror of taomate_h3.inference / digitalhuman_h3.inference)."""

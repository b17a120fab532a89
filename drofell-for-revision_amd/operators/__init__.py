"""Operator layer: the quantized-Linear API of the reference's ``operators/``."""

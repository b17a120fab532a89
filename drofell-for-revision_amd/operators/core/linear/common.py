"""Quantisation config (reference ``operators/core/linear/common.py:4-13``)."""
from dataclasses import dataclass


@dataclass
class QuantizationConfig:
    bits: int
    group_size: int
    desc_act: bool
    quant_method: str

    def __post_init__(self):
        # AssertionError, as the reference's asserts raise
        if self.quant_method != "gptq":
            raise AssertionError("only GPTQ checkpoints are supported")
        if self.bits != 4:
            raise AssertionError("only 4-bit GPTQ is supported")

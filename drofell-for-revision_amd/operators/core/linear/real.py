"""Abstract Linear / LinearMaker contract.

Interface kept identical to the reference's
``operators/core/linear/real.py:6-15``: a Linear is an ``nn.Module`` with
``forward(x)``; a maker builds Linears from (in_features, out_features,
bias) and owns their post-load initialisation.
"""
from abc import ABC, abstractmethod

import torch
from torch import nn


class Linear(ABC, nn.Module):
    @abstractmethod
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class LinearMaker(ABC):
    @abstractmethod
    def make_linear(self, in_features: int, out_features: int, bias: bool) -> Linear:
        raise NotImplementedError

"""Host-side behaviour of the Marlin-backend mirror (no GPU needed)."""
from __future__ import annotations

import pytest
import torch

from hip_extends.marlin import MarlinDenseCache, MarlinTuningParams, make_marlin_workspace
from operators.core.linear.real_marlin import MarlinQuantLinear, MarlinQuantLinearMaker


def test_tuning_params_dispatch_rule():
    tp = MarlinTuningParams(reconstruct_threshold=768, grad_reconstruct_threshold=128)
    assert not tp.use_reconstructed_forward(767, cache_weight=False)
    assert tp.use_reconstructed_forward(768, cache_weight=False)
    assert not tp.use_reconstructed_forward(127, cache_weight=True)
    assert tp.use_reconstructed_forward(128, cache_weight=True)
    assert tp.direct_max_m() == 767
    off = MarlinTuningParams(reconstruct_threshold=None)
    assert not off.use_reconstructed_forward(10 ** 6, cache_weight=False)
    assert off.direct_max_m() == 4096
    assert tp.reuse_reconstruct_cache(True) is True
    assert MarlinTuningParams(reuse_reconstruct_cache_when_grad=False).reuse_reconstruct_cache(True) is False
    with pytest.raises(ValueError):
        MarlinTuningParams(reconstruct_threshold=0)
    with pytest.raises(ValueError):
        MarlinTuningParams(grad_reconstruct_threshold=-3)


def test_dense_cache_lifecycle():
    cache = MarlinDenseCache(torch.device("cpu"))
    with pytest.raises(RuntimeError):
        cache.weight(4, 4)
    cache.update(64, 32)
    cache.update(32, 32)
    cache.init_cache()
    assert tuple(cache.weight(64, 32).shape) == (64, 32)
    assert tuple(cache.weight(16, 8).shape) == (16, 8)
    with pytest.raises(RuntimeError):
        cache.weight(128, 32)
    with pytest.raises(RuntimeError):
        cache.update(128, 128)
    with pytest.raises(RuntimeError):
        cache.init_cache()


def test_workspace_and_linear_need_a_device():
    with pytest.raises(ValueError):
        make_marlin_workspace(torch.device("cpu"))
    with pytest.raises(ValueError):
        MarlinQuantLinear(128, 4096, 4096, bias=False, use_act_order=False)


def test_maker_rejects_empty_post_init():
    maker = MarlinQuantLinearMaker(quantization_group_size=128, use_act_order=False)
    with pytest.raises(RuntimeError):
        maker.post_init(MarlinTuningParams(), MarlinDenseCache(torch.device("cpu")))
    with pytest.raises(ValueError):
        maker.merge([])

"""Per-layer checkpoint loading for the quantized projections.

The reference splits a GPTQ checkpoint into one safetensors file per decoder
layer (``scripts/converts/model.py:13-61`` in
``/root/reference/After-Revision-DROFELL``) whose keys are the layer's module
paths: ``self_attn.q_proj.qweight``, ``mlp.down_proj.scales``,
``input_layernorm.weight`` ...  ``make_our_decoders_from_files``
(``operators/assemble/decoders/real_loader_our.py:15-61``) builds each layer
with a shared ``QuantLinearMaker``, loads the file through
``Decoder.load_parameters`` (``operators/assemble/decoder/real.py:201-212``:
biases must be zero and are dropped, the rotary ``inv_freq`` is checked and
dropped), then repacks every projection once (``post_init``) and allocates
the group's shared cache.

:class:`QuantDecoderLinears` holds the part of a layer on this path -- the
seven projections and the two RMSNorm weights under the same names -- and
:func:`make_quant_decoder_linears_from_files` follows the same steps.
:func:`make_marlin_decoder_linears_from_files` is the Marlin-path load
(``operators/assemble/decoders/real_loader_marlin.py:17-91``): the same
files, then q/k/v and gate/up merged before the repack.  Moving
a loaded layer to host memory and back (the swap of the reference's memory
planner) keeps the packed layout; see ``QuantLinear._apply``.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch
from safetensors import safe_open
from torch import nn

from hip_extends.marlin import MarlinDenseCache, MarlinTuningParams
from hip_extends.w4a16 import CacheV2, TuningParams

from .real import Linear, LinearMaker
from .real_marlin import MarlinQuantLinearMaker
from .real_quant import QuantLinearMaker


class _Attention(nn.Module):
    def __init__(self, maker: LinearMaker, hidden: int, kv_out: int) -> None:
        super().__init__()
        self.q_proj = maker.make_linear(hidden, hidden, False)
        self.k_proj = maker.make_linear(hidden, kv_out, False)
        self.v_proj = maker.make_linear(hidden, kv_out, False)
        self.o_proj = maker.make_linear(hidden, hidden, False)


class _MLP(nn.Module):
    def __init__(self, maker: LinearMaker, hidden: int, intermediate: int) -> None:
        super().__init__()
        self.gate_proj = maker.make_linear(hidden, intermediate, False)
        self.up_proj = maker.make_linear(hidden, intermediate, False)
        self.down_proj = maker.make_linear(intermediate, hidden, False)


class QuantDecoderLinears(nn.Module):
    """The quantized projections and RMSNorm weights of one decoder layer,
    under the reference's state-dict names."""

    def __init__(self, maker: LinearMaker, hidden: int, intermediate: int,
                 kv_out: Optional[int] = None) -> None:
        super().__init__()
        self.self_attn = _Attention(maker, hidden, hidden if kv_out is None else kv_out)
        self.mlp = _MLP(maker, hidden, intermediate)
        self.register_buffer("input_layernorm_weight", torch.ones(hidden, dtype=torch.float16))
        self.register_buffer("post_attention_layernorm_weight",
                             torch.ones(hidden, dtype=torch.float16))

    # the reference's key names for the two norms
    _NORM_KEYS = {"input_layernorm.weight": "input_layernorm_weight",
                  "post_attention_layernorm.weight": "post_attention_layernorm_weight"}

    def projections(self) -> Dict[str, Linear]:
        """Every projection by module path (merged ones under their merged
        names, ``self_attn.qkv_proj`` and ``mlp.gate_up_proj``)."""
        return {f"{part}.{name}": m for part in ("self_attn", "mlp")
                for name, m in getattr(self, part).named_children()}

    def load_parameters(self, state_dict: Dict[str, torch.Tensor]) -> None:
        """``Decoder.load_parameters`` for this layer's keys: biases must be
        all zero and are dropped, ``self_attn.rotary_emb.inv_freq`` is
        dropped; every other key must match a buffer exactly."""
        state: Dict[str, torch.Tensor] = {}
        for k, v in state_dict.items():
            if k.endswith(".bias"):
                if torch.count_nonzero(v).item() != 0:
                    raise AssertionError(f"{k}: the quantized path drops biases, which must be zero")
                continue
            if k == "self_attn.rotary_emb.inv_freq":
                continue
            state[self._NORM_KEYS.get(k, k)] = v
        # checkpoints store the norm weights in fp16 or fp32
        for name in self._NORM_KEYS.values():
            if name in state:
                state[name] = state[name].to(torch.float16)
        self.load_state_dict(state, strict=True)


def _load_layers(maker: LinearMaker, hidden: int, intermediate: int, device: torch.device,
                 state_files: Sequence[str], kv_out: Optional[int]) -> List[QuantDecoderLinears]:
    layers: List[QuantDecoderLinears] = []
    with torch.device(device):
        for state_file in state_files:
            layer = QuantDecoderLinears(maker, hidden, intermediate, kv_out)
            with safe_open(state_file, framework="pt") as f:
                with torch.device("cpu"):
                    raw = {k: f.get_tensor(k) for k in f.keys()}
            layer.load_parameters(raw)
            layers.append(layer)
    return layers


def make_quant_decoder_linears_from_files(
        hidden: int, intermediate: int, group_size: int, desc_act: bool,
        device: torch.device, state_files: Sequence[str],
        tunning_params: Optional[TuningParams] = None,
        linear_cache: Optional[CacheV2] = None,
        kv_out: Optional[int] = None) -> Tuple[List[QuantDecoderLinears], CacheV2]:
    """Build one :class:`QuantDecoderLinears` per layer file on ``device``,
    load it, repack every projection once and allocate the shared cache."""
    device = torch.device(device)
    if linear_cache is None:
        linear_cache = CacheV2(device)
    if tunning_params is None:
        tunning_params = TuningParams()
    maker = QuantLinearMaker(quantization_group_size=group_size, use_act_order=desc_act)
    layers = _load_layers(maker, hidden, intermediate, device, state_files, kv_out)
    maker.post_init(tunning_params, linear_cache)
    linear_cache.init_cache()
    return layers, linear_cache


def make_marlin_decoder_linears_from_files(
        hidden: int, intermediate: int, group_size: int, desc_act: bool,
        device: torch.device, state_files: Sequence[str],
        tuning_params: Optional[MarlinTuningParams] = None,
        linear_cache: Optional[MarlinDenseCache] = None,
        kv_out: Optional[int] = None, bits: int = 4,
) -> Tuple[List[QuantDecoderLinears], MarlinDenseCache, MarlinQuantLinearMaker]:
    """The Marlin-path load (the reference's default decoder backend,
    ``make_marlin_decoders_from_files``,
    ``operators/assemble/decoders/real_loader_marlin.py:17-91``): one layer
    per file on ``device`` with a shared :class:`MarlinQuantLinearMaker`,
    loaded through ``load_parameters``; then q/k/v are merged into
    ``self_attn.qkv_proj`` and gate/up into ``mlp.gate_up_proj`` (the
    separate modules become ``None``), every projection is repacked once
    (``post_init``) and the group's dense cache is allocated.  The maker is
    returned too: the reference keeps it alive with the group
    (``attached_no_gc``).  Checkpoints must be symmetric 4-bit GPTQ, as the
    reference's Marlin backend requires."""
    if bits != 4:
        raise ValueError("the Marlin decode backend requires 4-bit GPTQ weights")
    device = torch.device(device)
    if tuning_params is None:
        tuning_params = MarlinTuningParams()
    if linear_cache is None:
        linear_cache = MarlinDenseCache(device)
    maker = MarlinQuantLinearMaker(quantization_group_size=group_size, use_act_order=desc_act)
    layers = _load_layers(maker, hidden, intermediate, device, state_files, kv_out)
    for layer in layers:
        attn, mlp = layer.self_attn, layer.mlp
        attn.qkv_proj = maker.merge([attn.q_proj, attn.k_proj, attn.v_proj])
        attn.q_proj = attn.k_proj = attn.v_proj = None
        mlp.gate_up_proj = maker.merge([mlp.gate_proj, mlp.up_proj])
        mlp.gate_proj = mlp.up_proj = None
    maker.post_init(tuning_params, linear_cache)
    linear_cache.init_cache()
    return layers, linear_cache, maker

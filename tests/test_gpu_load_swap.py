"""Per-layer checkpoint loading, memory twins and swap-out/swap-in on the GPU.

Layer files are written in the reference's per-layer safetensors format
(keys ``self_attn.q_proj.qweight`` ... ``input_layernorm.weight``, zero
biases and a rotary ``inv_freq`` that the loader drops), loaded through
make_quant_decoder_linears_from_files, and then:
* every projection's product is checked against the oracle
  (max|y - y_ref| <= 2e-2 * ||y_ref row||_inf);
* the device bytes the modules and the shared cache hold equal the memory
  twins' total;
* a layer moved to host memory refuses products, and after moving back
  gives bit-identical products with no repack, with q/k/v (and gate/up)
  again sharing one act-order permutation tensor.
The Marlin-path load (the reference's default backend,
``operators/assemble/decoders/real_loader_marlin.py:17-91``) reads the same
files of symmetric checkpoints, merges q/k/v and gate/up, repacks and
allocates the dense cache; the merged products, the twin bytes and the swap
are checked the same way.
Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from gptq_synth import GPTQLayer, make_layer, make_x
from hip_extends.marlin import MarlinTuningParams
from hip_extends.w4a16 import TuningParams
from operators.core.linear.loader import (make_marlin_decoder_linears_from_files,
                                          make_quant_decoder_linears_from_files)
from operators.core.linear.memory import (CacheV2MemoryModel, MarlinQuantLinearMakerMemoryModel,
                                          QuantLinearMakerMemoryModel)
from operators.core.memory.static import MemoryModule, MemoryTensor
from oracle import gptq

pytestmark = pytest.mark.gpu

HIDDEN, INTER = 512, 1408
TOL = 2e-2


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _layer_file(path, seed: int, act: bool, symmetric: bool = False):
    """One layer's tensors under the reference's key names; returns the
    oracle's dequantised weight of every projection."""
    shapes = {"self_attn.q_proj": (HIDDEN, HIDDEN), "self_attn.k_proj": (HIDDEN, HIDDEN),
              "self_attn.v_proj": (HIDDEN, HIDDEN), "self_attn.o_proj": (HIDDEN, HIDDEN),
              "mlp.gate_proj": (HIDDEN, INTER), "mlp.up_proj": (HIDDEN, INTER),
              "mlp.down_proj": (INTER, HIDDEN)}
    state, dense = {}, {}
    shared = {}
    for i, (name, (k, n)) in enumerate(shapes.items()):
        lay = make_layer(k, n, 128, seed=seed + i, act_order=act, symmetric=symmetric)
        # q/k/v and gate/up are quantised against one input: equal g_idx
        share_key = "qkv" if name[-6:] in ("q_proj", "k_proj", "v_proj") else \
            "gu" if name.endswith(("gate_proj", "up_proj")) else None
        if act and share_key is not None:
            g_idx = shared.setdefault(share_key, lay.g_idx)
            lay = GPTQLayer(k, n, 128, lay.qweight, lay.qzeros, lay.scales, g_idx, True,
                            symmetric)
        for field in ("qweight", "qzeros", "scales", "g_idx"):
            state[f"{name}.{field}"] = getattr(lay, field).contiguous().clone()
        state[f"{name}.bias"] = torch.zeros(n, dtype=torch.float16)
        a = lay.numpy()
        dense[name] = gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], a["g_idx"])
    gen = torch.Generator().manual_seed(seed)
    state["input_layernorm.weight"] = torch.randn(HIDDEN, generator=gen).to(torch.float16)
    state["post_attention_layernorm.weight"] = torch.randn(HIDDEN, generator=gen)
    state["self_attn.rotary_emb.inv_freq"] = 1.0 / (10000 ** (torch.arange(0, 64, 2) / 64))
    save_file(state, str(path))
    return dense, state


def _device_bytes(layers, cache) -> int:
    seen = {}
    for layer in layers:
        for t in layer.buffers():
            if t.numel():
                seen[t.data_ptr()] = t.numel() * t.element_size()
    seen[cache.workspace.data_ptr()] = cache.workspace.numel()
    return sum(seen.values())


def _twin_bytes(n_layers: int, act: bool, max_m: int) -> int:
    maker = QuantLinearMakerMemoryModel(128, act)
    root = MemoryModule()
    per_layer = []
    for _ in range(n_layers):
        q, k, v, o = (maker.make_linear(HIDDEN, HIDDEN) for _ in range(4))
        gate, up = maker.make_linear(HIDDEN, INTER), maker.make_linear(HIDDEN, INTER)
        down = maker.make_linear(INTER, HIDDEN)
        per_layer.append((q, k, v, o, gate, up, down))
    cache = CacheV2MemoryModel()
    maker.post_init(TuningParams(MAX_M=max_m), cache)
    cache.init_cache()
    mods = []
    for i, (q, k, v, o, gate, up, down) in enumerate(per_layer):
        if act:
            maker.share_perm([q, k, v])
            maker.share_perm([gate, up])
        mods += [q, k, v, o, gate, up, down]
        setattr(root, f"norm_in_{i}", MemoryTensor((HIDDEN,), torch.float16))
        setattr(root, f"norm_post_{i}", MemoryTensor((HIDDEN,), torch.float16))
    root.mount_list(mods, "proj")
    root.workspace = cache.workspace
    return root.memory


@pytest.mark.parametrize("act", [False, True], ids=["plain", "act_order"])
def test_load_twin_and_swap(hip_device, tmp_path, act):
    files, denses, states = [], [], []
    for i in range(2):
        f = tmp_path / f"layer_{i}.safetensors"
        d, st = _layer_file(f, 500 + 10 * i, act)
        files.append(str(f))
        denses.append(d)
        states.append(st)
    say(f"load 2 layers act={act}")
    layers, cache = make_quant_decoder_linears_from_files(
        HIDDEN, INTER, 128, act, hip_device, files, TuningParams(MAX_M=64))
    torch.cuda.synchronize()
    assert torch.equal(layers[1].input_layernorm_weight.cpu(),
                       states[1]["input_layernorm.weight"])

    xs = {k: make_x(5, k, seed=77 + k) for k in (HIDDEN, INTER)}
    before = {}
    for li, layer in enumerate(layers):
        for name, proj in layer.projections().items():
            say(f"forward layer {li} {name}")
            x = xs[proj.infeatures]
            y = proj(x.to(hip_device))
            torch.cuda.synchronize()
            ref = x.numpy().astype(np.float64) @ denses[li][name].astype(np.float64)
            ok, worst = gptq.within_tolerance(y.float().cpu().numpy(), ref, TOL)
            assert ok, f"layer {li} {name}: worst error ratio {worst:.3f}"
            before[(li, name)] = y.clone()

    say("memory twin")
    assert _device_bytes(layers, cache) == _twin_bytes(2, act, 64)

    say("swap layer 0 out")
    layers[0].to("cpu")
    torch.cuda.synchronize()
    assert layers[0].self_attn.q_proj.qweight.device.type == "cpu"
    with pytest.raises(RuntimeError):
        layers[0].self_attn.q_proj(xs[HIDDEN].to(hip_device))
    say("swap layer 0 in")
    layers[0].to(hip_device)
    torch.cuda.synchronize()
    if act:
        a = layers[0].self_attn
        assert a.q_proj.perm.data_ptr() == a.k_proj.perm.data_ptr() == a.v_proj.perm.data_ptr()
        assert a.q_proj.q4_matrix.perm.data_ptr() == a.q_proj.perm.data_ptr()
        m = layers[0].mlp
        assert m.gate_proj.perm.data_ptr() == m.up_proj.perm.data_ptr()
    for li, layer in enumerate(layers):
        for name, proj in layer.projections().items():
            say(f"forward after swap layer {li} {name}")
            y = proj(xs[proj.infeatures].to(hip_device))
            torch.cuda.synchronize()
            assert torch.equal(y, before[(li, name)]), (li, name)
    assert _device_bytes(layers, cache) == _twin_bytes(2, act, 64)


MERGED = {"self_attn.qkv_proj": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
          "self_attn.o_proj": ("self_attn.o_proj",),
          "mlp.gate_up_proj": ("mlp.gate_proj", "mlp.up_proj"),
          "mlp.down_proj": ("mlp.down_proj",)}


def _marlin_twin_bytes(n_layers: int, act: bool) -> int:
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    maker = MarlinQuantLinearMakerMemoryModel(128, act, workspace_elements=4 * cus)
    root = MemoryModule()
    mods = []
    for i in range(n_layers):
        q, k, v, o = (maker.make_linear(HIDDEN, HIDDEN) for _ in range(4))
        gate, up = maker.make_linear(HIDDEN, INTER), maker.make_linear(HIDDEN, INTER)
        down = maker.make_linear(INTER, HIDDEN)
        mods += [maker.merge([q, k, v]), o, maker.merge([gate, up]), down]
        setattr(root, f"norm_in_{i}", MemoryTensor((HIDDEN,), torch.float16))
        setattr(root, f"norm_post_{i}", MemoryTensor((HIDDEN,), torch.float16))
    maker.post_init()
    root.mount_list(mods, "proj")
    root.dense_cache = maker.dense_cache
    return root.memory


def _marlin_device_bytes(layers, cache) -> int:
    seen = {}
    for layer in layers:
        for t in layer.buffers():
            if t.numel():
                seen[t.data_ptr()] = t.numel() * t.element_size()
    for t in (cache.weight(1, 1), cache.workspace):
        seen[t.data_ptr()] = t.untyped_storage().nbytes()
    return sum(seen.values())


@pytest.mark.parametrize("act", [False, True], ids=["plain", "act_order"])
def test_marlin_load_merge_twin_and_swap(hip_device, tmp_path, act):
    files, denses = [], []
    for i in range(2):
        f = tmp_path / f"layer_{i}.safetensors"
        d, _ = _layer_file(f, 900 + 10 * i, act, symmetric=True)
        files.append(str(f))
        denses.append(d)
    say(f"marlin load 2 layers act={act}")
    layers, cache, maker = make_marlin_decoder_linears_from_files(
        HIDDEN, INTER, 128, act, hip_device, files, MarlinTuningParams())
    torch.cuda.synchronize()
    assert len(maker.quant_linears) == 2 * 4
    for layer in layers:
        assert layer.self_attn.q_proj is None and layer.mlp.gate_proj is None
        assert sorted(layer.projections()) == sorted(MERGED)

    xs = {k: make_x(5, k, seed=91 + k) for k in (HIDDEN, INTER)}
    before = {}
    for li, layer in enumerate(layers):
        for name, proj in layer.projections().items():
            say(f"marlin forward layer {li} {name}")
            x = xs[proj.infeatures]
            y = proj(x.to(hip_device))
            torch.cuda.synchronize()
            w = np.concatenate([denses[li][part] for part in MERGED[name]], axis=1)
            assert y.shape == (5, w.shape[1])
            ref = x.numpy().astype(np.float64) @ w.astype(np.float64)
            ok, worst = gptq.within_tolerance(y.float().cpu().numpy(), ref, TOL)
            assert ok, f"layer {li} {name}: worst error ratio {worst:.3f}"
            before[(li, name)] = y.clone()

    say("marlin memory twin")
    assert _marlin_device_bytes(layers, cache) == _marlin_twin_bytes(2, act)

    say("marlin swap layer 0 out")
    qkv = layers[0].self_attn.qkv_proj
    packed = qkv.qweight.clone()
    layers[0].to("cpu")
    torch.cuda.synchronize()
    assert qkv.qweight.device.type == "cpu" and qkv.q4_matrix.qweight.device.type == "cpu"
    with pytest.raises(RuntimeError):
        qkv(xs[HIDDEN].to(hip_device))
    say("marlin swap layer 0 in")
    layers[0].to(hip_device)
    torch.cuda.synchronize()
    assert qkv.q4_matrix.qweight.data_ptr() == qkv.qweight.data_ptr()
    assert torch.equal(qkv.qweight, packed)  # the packed words, not a second repack
    for li, layer in enumerate(layers):
        for name, proj in layer.projections().items():
            say(f"marlin forward after swap layer {li} {name}")
            y = proj(xs[proj.infeatures].to(hip_device))
            torch.cuda.synchronize()
            assert torch.equal(y, before[(li, name)]), (li, name)
    assert _marlin_device_bytes(layers, cache) == _marlin_twin_bytes(2, act)

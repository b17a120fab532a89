"""GPU parity of the Marlin-backend mirror (merge, dispatch, gradients)."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from gptq_synth import make_layer, make_x
from hip_extends.marlin import MarlinDenseCache, MarlinTuningParams
from oracle import gptq
from operators.core.linear.real_marlin import MarlinQuantLinearMaker

pytestmark = pytest.mark.gpu
TOL = 2e-2


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def check_tol(y: torch.Tensor, ref: np.ndarray, what: str) -> None:
    yy = y.float().cpu().numpy()
    assert np.all(np.isfinite(yy)), what
    ok, worst = gptq.within_tolerance(yy, ref, TOL)
    assert ok, f"{what}: worst error ratio {worst:.4f} > 1"


def _load(lin, lay):
    lin.load_state_dict({"qweight": lay.qweight, "qzeros": lay.qzeros, "scales": lay.scales,
                         "g_idx": lay.g_idx}, strict=False)


def _w(lay):
    a = lay.numpy()
    return gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], a["g_idx"])


def test_marlin_linear_direct_and_dense(hip_device):
    k, n = 4096, 4096
    lay = make_layer(k, n, 128, seed=11, symmetric=True)
    w = _w(lay)
    maker = MarlinQuantLinearMaker(quantization_group_size=128, use_act_order=False)
    with torch.device(hip_device):
        lin = maker.make_linear(k, n, bias=False)
    _load(lin, lay)
    cache = MarlinDenseCache(hip_device)
    maker.post_init(MarlinTuningParams(), cache)
    cache.init_cache()
    say("marlin dequant bit-exact")
    out = torch.empty(k, n, dtype=torch.float16, device=hip_device)
    lin.reconstruct_weight(out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), w.view(np.uint16))
    at = MarlinTuningParams().reconstruct_threshold
    ms = (1, 8, 300, 800) + (() if at is None else (at - 1, at))
    for m in ms:  # the default crossover: packed kernel below it, dense route from it
        say(f"marlin forward M={m} (default crossover {at})")
        x = make_x(m, k, seed=m)
        y = lin(x.to(hip_device))
        torch.cuda.synchronize()
        check_tol(y, gptq.gemm_ref(x.numpy(), w), f"marlin M={m}")
    maker.set_tuning_param(MarlinTuningParams(reconstruct_threshold=600))
    for m in (599, 600):  # either side of an explicit crossover
        say(f"marlin forward M={m} (crossover 600)")
        assert lin.q4_matrix.use_reconstructed_forward(m, cache_weight=False) == (m >= 600)
        x = make_x(m, k, seed=m + 1)
        y = lin(x.to(hip_device))
        torch.cuda.synchronize()
        check_tol(y, gptq.gemm_ref(x.numpy(), w), f"marlin M={m} crossover 600")
    maker.set_tuning_param(MarlinTuningParams())
    say("marlin bf16 input keeps its dtype")
    yb = lin(make_x(4, k, seed=4).to(hip_device, torch.bfloat16))
    assert yb.dtype == torch.bfloat16
    with pytest.raises(RuntimeError):
        lin.post_init(MarlinTuningParams(), cache)


def test_marlin_kept_weight_crossover(hip_device):
    """Training with a grad-tracking input keeps the reconstructed weight
    from the default crossover on (dense forward, dense activation
    gradient); one row below it the packed forward and the reconstruct-then-
    dense gradient run.  Both sides match the fp64 reference."""
    k, n = 1024, 2048
    lay = make_layer(k, n, 128, seed=21, symmetric=True)
    w = _w(lay)
    maker = MarlinQuantLinearMaker(quantization_group_size=128, use_act_order=False)
    with torch.device(hip_device):
        lin = maker.make_linear(k, n, bias=False)
    _load(lin, lay)
    cache = MarlinDenseCache(hip_device)
    maker.post_init(MarlinTuningParams(), cache)
    cache.init_cache()
    at = MarlinTuningParams().grad_reconstruct_threshold
    assert at is not None
    for m in (at - 1, at):
        say(f"marlin kept-weight forward + gradient M={m} (default crossover {at})")
        assert lin.q4_matrix.use_reconstructed_forward(m, cache_weight=True) == (m >= at)
        xg = make_x(m, k, seed=300 + m).to(hip_device).requires_grad_(True)
        y = lin(xg)
        gout = make_x(m, n, seed=400 + m)
        y.backward(gout.to(hip_device))
        torch.cuda.synchronize()
        check_tol(y.detach(), gptq.gemm_ref(xg.detach().cpu().numpy(), w), f"forward M={m}")
        check_tol(xg.grad, gout.numpy().astype(np.float64) @ w.astype(np.float64).T,
                  f"grad M={m}")


def test_marlin_rejects_asymmetric_zeros(hip_device):
    lay = make_layer(256, 256, 128, seed=3, symmetric=False)
    maker = MarlinQuantLinearMaker(quantization_group_size=128, use_act_order=False)
    with torch.device(hip_device):
        lin = maker.make_linear(256, 256)
    _load(lin, lay)
    say("marlin asymmetric rejected")
    with pytest.raises(ValueError):
        maker.post_init(MarlinTuningParams(), MarlinDenseCache(hip_device))


def test_marlin_merge_qkv_act_order(hip_device):
    """merge(q, k, v) == concatenation of the three products (act-order)."""
    k, n = 5120, 1280
    lays = [make_layer(k, n, 128, seed=20 + i, symmetric=True, act_order=True) for i in range(3)]
    # merged linears must share g_idx: give all three the first one's
    g = lays[0].g_idx
    maker = MarlinQuantLinearMaker(quantization_group_size=128, use_act_order=True)
    with torch.device(hip_device):
        lins = [maker.make_linear(k, n) for _ in range(3)]
    for lin, lay in zip(lins, lays):
        lin.load_state_dict({"qweight": lay.qweight, "qzeros": lay.qzeros,
                             "scales": lay.scales, "g_idx": g}, strict=False)
    ws = []
    for lay in lays:
        a = lay.numpy()
        ws.append(gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], g.numpy()))
    merged = maker.merge(lins)
    assert merged.outfeatures == 3 * n and maker.quant_linears == [merged]
    with torch.device(hip_device):
        other = maker.make_linear(k // 2, n)
    with pytest.raises(ValueError):
        maker.merge([merged, other])
    maker.quant_linears.remove(other)
    cache = MarlinDenseCache(hip_device)
    maker.post_init(MarlinTuningParams(), cache)
    cache.init_cache()
    wcat = np.concatenate(ws, axis=1)
    for m in (1, 8, 64):
        say(f"marlin merged qkv act-order M={m}")
        x = make_x(m, k, seed=100 + m)
        y = merged(x.to(hip_device))
        torch.cuda.synchronize()
        check_tol(y, gptq.gemm_ref(x.numpy(), wcat), f"merged M={m}")
    for m in (16, 200):  # packed transposed kernel, then reconstruct + dense
        say(f"marlin merged input gradient M={m}")
        xg = make_x(m, k, seed=7).to(hip_device).requires_grad_(True)
        yg = merged(xg)
        gout = make_x(m, 3 * n, seed=8)
        yg.backward(gout.to(hip_device))
        torch.cuda.synchronize()
        check_tol(xg.grad, gout.numpy().astype(np.float64) @ wcat.astype(np.float64).T,
                  f"grad M={m}")

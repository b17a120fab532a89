"""GPU parity of the transposed W4A16 product (dw4_gemm_t, the PEFT
backward out = g @ W^T) against the oracle, through the C ABI and through
Q4MatrixV2.transpose_matmul / autograd.

Bar: max|out - out_ref| <= 2e-2 * ||out_ref row||_inf, out_ref = g @ W^T in
float64 with W the oracle's dequantised weight.  Covers Llama-2-7B shapes,
act-order 13B, group sizes 32/64/256/1024 and g = K, N-ranges that do not
divide the strips, M across one and several 64-row blocks, determinism and
the error statuses.  Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import ctypes
import functools
import sys

import numpy as np
import pytest
import torch

from gptq_synth import make_layer, make_x
from hip_extends import _lib
from hip_extends.w4a16 import CacheV2, Q4LinearFunction, Q4MatrixV2, TuningParams
from oracle import gptq

pytestmark = pytest.mark.gpu

TOL = 2e-2


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@functools.lru_cache(maxsize=16)
def _layer(k, n, g, seed, act):
    lay = make_layer(k, n, g, seed=seed, act_order=act)
    a = lay.numpy()
    return lay, gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], a["g_idx"])


def _matrix(lay, dev, max_m=256):
    cache = CacheV2(dev)
    d = lay.to(dev)
    q4 = Q4MatrixV2(d.qweight, d.qzeros, d.scales, d.in_features, d.out_features,
                    d.g_idx if d.act_order else None, d.act_order,
                    TuningParams(MAX_M=max_m, TRANSPOSE_MAX_M=4096), cache)
    cache.init_cache()
    return q4


def _gemm_t(q4, g2):
    m = g2.shape[0]
    out = torch.full((m, q4.height), float("nan"), dtype=torch.float16, device=g2.device)
    nbytes = _lib.gemm_t_workspace_size(m, q4.height, q4.width, q4.group_size)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=g2.device)
    _lib.call("dw4_gemm_t", m, q4.height, q4.width, q4.group_size, g2.data_ptr(), g2.stride(0),
              q4.qweight.data_ptr(), q4.qzeros.data_ptr(), q4.scales.data_ptr(),
              q4.perm.data_ptr() if q4.use_act else None, out.data_ptr(), out.stride(0),
              ws.data_ptr(), ws.numel(), torch.cuda.current_stream(g2.device).cuda_stream)
    return out


def _check(out, g, w, what):
    ref = g.numpy().astype(np.float64) @ w.astype(np.float64).T
    y = out.float().cpu().numpy()
    assert np.all(np.isfinite(y)), what
    ok, worst = gptq.within_tolerance(y, ref, TOL)
    assert ok, f"{what}: worst error ratio {worst:.4f} > 1"


@pytest.mark.parametrize("shape", [(4096, 4096), (4096, 11008), (11008, 4096)],
                         ids=["4096x4096", "4096x11008", "11008x4096"])
def test_transpose_7b(hip_device, shape):
    k, n = shape
    lay, w = _layer(k, n, 128, 3000 + k + n, False)
    q4 = _matrix(lay, hip_device)
    for m in (1, 5, 16, 33, 64, 65, 100, 256):
        say(f"gemm_t {k}x{n} M={m}")
        g = make_x(m, n, seed=4000 + m)
        out = _gemm_t(q4, g.to(hip_device))
        torch.cuda.synchronize()
        _check(out, g, w, f"{k}x{n} M={m}")


@pytest.mark.parametrize("k,n,gs,act", [(5120, 13824, 128, True), (1024, 512, 32, False),
                                        (1024, 512, 64, True), (2048, 272, 256, True),
                                        (1024, 80, 1024, False), (128, 4096, 128, True)])
def test_transpose_groups_and_act(hip_device, k, n, gs, act):
    lay, w = _layer(k, n, gs, 5000 + k + n + gs, act)
    q4 = _matrix(lay, hip_device)
    for m in (1, 8, 70):
        say(f"gemm_t {k}x{n} g={gs} act={act} M={m}")
        g = make_x(m, n, seed=6000 + m)
        out = _gemm_t(q4, g.to(hip_device))
        torch.cuda.synchronize()
        _check(out, g, w, f"{k}x{n} g={gs} act={act} M={m}")


def test_transpose_deterministic_and_routes(hip_device):
    lay, w = _layer(4096, 11008, 128, 7000, True)
    q4 = _matrix(lay, hip_device)
    g = make_x(24, 11008, seed=7001).to(hip_device)
    say("gemm_t determinism")
    a = _gemm_t(q4, g)
    b = _gemm_t(q4, g)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    say("transpose_matmul native vs dense route")
    native = q4.transpose_matmul(g.view(2, 12, 11008))
    q4.tuning_params = TuningParams(TRANSPOSE_MAX_M=0)
    dense = q4.transpose_matmul(g.view(2, 12, 11008))
    torch.cuda.synchronize()
    assert native.shape == dense.shape == (2, 12, 4096)
    _check(native.view(24, 4096), g.cpu(), w, "native route")
    _check(dense.view(24, 4096), g.cpu(), w, "dense route")
    say("autograd backward through the native kernel")
    q4.tuning_params = TuningParams(TRANSPOSE_MAX_M=256)
    x = make_x(24, 4096, seed=7002).to(hip_device).requires_grad_(True)
    y = Q4LinearFunction.apply(x, q4, None, False)
    y.backward(g)
    torch.cuda.synchronize()
    _check(x.grad, g.cpu(), w, "autograd grad_input")


def test_transpose_status(hip_device):
    lay, _ = _layer(1024, 512, 32, 8000, False)
    q4 = _matrix(lay, hip_device)
    lib = _lib.load()
    g = torch.zeros(4, 512, dtype=torch.float16, device=hip_device)
    out = torch.empty(4, 1024, dtype=torch.float16, device=hip_device)
    args = (q4.qweight.data_ptr(), q4.qzeros.data_ptr(), q4.scales.data_ptr(), None,
            out.data_ptr(), 1024)
    say("gemm_t statuses")
    assert lib.dw4_gemm_t(4, 1024, 500, 32, g.data_ptr(), 512, *args, None, 0, None) == \
        _lib.DW4_ERR_UNSUPPORTED
    assert lib.dw4_gemm_t(4, 1024, 512, 32, g.data_ptr() + 2, 512, *args, None, 0, None) == \
        _lib.DW4_ERR_MISALIGNED
    need = _lib.gemm_t_workspace_size(4, 1024, 512, 32)
    if need:
        assert lib.dw4_gemm_t(4, 1024, 512, 32, g.data_ptr(), 512, *args, None, 0, None) == \
            _lib.DW4_ERR_WORKSPACE
    assert lib.dw4_gemm_t(0, 1024, 512, 32, None, 512, *args, None, 0, None) == _lib.DW4_OK

"""The torch-CPU restatement used as the CPU baseline agrees with the oracle."""
import numpy as np
import torch

from gptq_synth import make_layer, make_x
from oracle import cpu_path, gptq


def test_cpu_path_dequant_bit_exact_with_oracle():
    for sym, act, g in ((True, False, 128), (False, False, 64), (False, True, 128)):
        lay = make_layer(512, 96, g, seed=31 + g, symmetric=sym, act_order=act)
        w = cpu_path.reconstruct_weights(lay.qweight, lay.qzeros, lay.scales, lay.g_idx)
        a = lay.numpy()
        ref = gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], a["g_idx"])
        assert w.dtype == torch.float16
        assert np.array_equal(w.numpy().view(np.uint16), ref.view(np.uint16))


def test_cpu_path_forward_within_tolerance():
    lay = make_layer(512, 96, 128, seed=5)
    x = make_x(4, 512, seed=6)
    y = cpu_path.forward(x, lay.qweight, lay.qzeros, lay.scales, lay.g_idx)
    a = lay.numpy()
    ref = gptq.gemm_ref(x.numpy(), gptq.dequantize(a["qweight"], a["qzeros"], a["scales"], a["g_idx"]))
    ok, worst = gptq.within_tolerance(y.float().numpy(), ref)
    # fp16 output rounding alone contributes up to 2**-11 / 2e-2 = 0.0244
    assert ok and worst < 0.03

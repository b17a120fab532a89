"""The decode chain (dw4_gemm_chain) against the oracle.

A chain runs the projections of whole decoder layers in one launch, each
projection reading its activations only after the projections it depends on
have completed on every workgroup.  The links here follow one decoder
layer's data flow with the attention left out: q, k, v read the layer input
h; o reads v's output (standing in for the attention output) with h as its
residual; gate and up read o's output h2; down reads up's output (standing in
for silu(gate) * up) with h2 as its residual and writes the next layer's
input.  Every buffer is its own tensor, so after a launch each link's output
can be checked against the oracle product of the inputs that link read:
max|y - y_ref| <= 2e-2 * ||y_ref row||_inf, y_ref = x @ W (+ bias)
(+ residual) in float64 with the oracle's bit-exact weights.  Before every
launch all intermediate buffers are filled with NaN, so a link that read its
input before the producing link had finished would fail.  Launches are
repeated eagerly and from a captured HIP graph (with other device work
between the replays); the launch counter must advance once per launch and
no dependency wait may give up.
Every case prints its name before touching the GPU.
"""
from __future__ import annotations

import sys
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from gptq_synth import make_layer
from hip_extends.chain import ChainStep, Q4Chain
from hip_extends.w4a16 import CacheV2, Q4MatrixV2, TuningParams
from oracle import gptq

pytestmark = pytest.mark.gpu

TOL = 2e-2


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _proj(hidden, inter):
    return (("q", hidden, hidden), ("k", hidden, hidden), ("v", hidden, hidden),
            ("o", hidden, hidden), ("gate", hidden, inter), ("up", hidden, inter),
            ("down", inter, hidden))


def _build_layer(args):
    li, hidden, inter, g, seed = args
    out = {}
    for pi, (name, k, n) in enumerate(_proj(hidden, inter)):
        lay = make_layer(k, n, g, seed=seed + 10 * li + pi, scale_mul=0.002, scale_add=2e-4)
        a = lay.numpy()
        out[name] = (lay, gptq.WideWeight(gptq.dequantize(a["qweight"], a["qzeros"],
                                                          a["scales"], a["g_idx"])))
    return out


def _chain_case(dev, hidden, inter, layers, m, g, seed):
    """Matrices, buffers and links of `layers` decoder layers' projections."""
    cache = CacheV2(dev)
    tp = TuningParams(MAX_M=8)
    with ThreadPoolExecutor(max_workers=min(layers, 4)) as pool:
        built = list(pool.map(_build_layer, [(li, hidden, inter, g, seed) for li in range(layers)]))
    mats, refs = [], []
    for lay_set in built:
        lm, lr = {}, {}
        for name, (lay, ww) in lay_set.items():
            d = lay.to(dev)
            lm[name] = Q4MatrixV2(d.qweight, d.qzeros, d.scales, lay.in_features,
                                  lay.out_features, None, False, tp, cache)
            lr[name] = ww
        mats.append(lm)
        refs.append(lr)
    cache.init_cache()
    f16 = dict(dtype=torch.float16, device=dev)
    gen = torch.Generator().manual_seed(seed)
    bias_q = (torch.randn(hidden, generator=gen) * 0.1).half().to(dev)
    hs = [torch.empty(m, hidden, **f16) for _ in range(layers + 1)]
    steps, checks = [], []
    down_idx = -1
    for li in range(layers):
        W, R = mats[li], refs[li]
        q, k, v, o = (torch.empty(m, hidden, **f16) for _ in range(4))
        gt, up = torch.empty(m, inter, **f16), torch.empty(m, inter, **f16)
        base = len(steps)
        steps += [ChainStep(W["q"], hs[li], q, down_idx, bias=bias_q),
                  ChainStep(W["k"], hs[li], k, down_idx),
                  ChainStep(W["v"], hs[li], v, down_idx),
                  ChainStep(W["o"], v, o, base + 2, residual=hs[li]),
                  ChainStep(W["gate"], o, gt, base + 3),
                  ChainStep(W["up"], o, up, base + 3),
                  ChainStep(W["down"], up, hs[li + 1], base + 5, residual=o)]
        down_idx = base + 6
        checks += [(hs[li], R["q"], q, bias_q, None), (hs[li], R["k"], k, None, None),
                   (hs[li], R["v"], v, None, None), (v, R["o"], o, None, hs[li]),
                   (o, R["gate"], gt, None, None), (o, R["up"], up, None, None),
                   (up, R["down"], hs[li + 1], None, o)]
    inter_bufs = [st.y for st in steps]
    return steps, checks, hs[0], inter_bufs


def _check_all(checks, what):
    worst = 0.0
    for i, (x, w, y, bias, res) in enumerate(checks):
        xv = x.float().cpu().numpy()
        assert np.all(np.isfinite(xv)), f"{what}: link {i} input not finite"
        ref = gptq.gemm_ref(xv.astype(np.float16), w)
        if bias is not None:
            ref = ref + bias.float().cpu().numpy()[None, :]
        if res is not None:
            ref = ref + res.float().cpu().numpy()
        got = y.float().cpu().numpy()
        assert np.all(np.isfinite(got)), f"{what}: link {i} output not finite"
        ok, r = gptq.within_tolerance(got, ref, TOL)
        assert ok, f"{what}: link {i} worst error ratio {r:.3f}"
        worst = max(worst, r)
    return worst


CASES = {
    "small_2layer_m1": (1024, 2816, 2, 1, 128),
    "7b_1layer_m1": (4096, 11008, 1, 1, 128),
    "m3_g256": (2048, 5632, 1, 3, 256),
}


@pytest.mark.parametrize("case", list(CASES))
def test_chain_matches_oracle_eager_and_graph(hip_device, case):
    hidden, inter, layers, m, g = CASES[case]
    say(f"chain {case}: building {layers} layer(s) {hidden}/{inter} M={m} g={g}")
    steps, checks, x0, bufs = _chain_case(hip_device, hidden, inter, layers, m, g, 4242)
    chain = Q4Chain(steps, m)
    say(f"chain {case}: plan ring={chain.plan.ring} workgroups={chain.plan.workgroups} "
        f"smem={chain.plan.smem_bytes}")
    gen = torch.Generator(device=hip_device).manual_seed(7)
    runs = 0
    first = None
    for r in range(3):
        say(f"chain {case}: eager launch {r}")
        x0.copy_(torch.randn(x0.shape, device=hip_device, generator=gen).half()
                 if r < 2 else first[0])
        for b in bufs:
            b.fill_(float("nan"))
        chain.run()
        runs += 1
        torch.cuda.synchronize()
        worst = _check_all(checks, f"{case} eager {r}")
        say(f"chain {case}: eager {r} worst error / tolerance = {worst:.3e}")
        if r == 0:
            first = (x0.clone(), [b.clone() for b in bufs])
        if r == 2:  # the same input as launch 0: the same bits (deterministic)
            for a, b in zip(first[1], bufs):
                assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    say(f"chain {case}: capture")
    side = torch.cuda.Stream(device=hip_device)
    side.wait_stream(torch.cuda.current_stream(hip_device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        chain.run(side.cuda_stream)
    for r in range(3):
        say(f"chain {case}: replay {r}")
        x0.copy_(torch.randn(x0.shape, device=hip_device, generator=gen).half())
        for b in bufs:
            b.fill_(float("nan"))
        _ = (x0.float() * 3).sum().item()  # other device work between replays
        graph.replay()
        runs += 1
        torch.cuda.synchronize()
        worst = _check_all(checks, f"{case} replay {r}")
        say(f"chain {case}: replay {r} worst error / tolerance = {worst:.3e}")
    assert not chain.timed_out()
    assert chain.launches() == runs
    del graph


def test_chain_matches_dw4_gemm(hip_device):
    """The chain's outputs against dw4_gemm's (the per-projection decode
    kernel) on the same inputs: both within the tolerance of each other."""
    hidden, inter = 4096, 11008
    say("chain vs dw4_gemm: one 7B layer M=1")
    steps, checks, x0, bufs = _chain_case(hip_device, hidden, inter, 1, 1, 128, 99)
    chain = Q4Chain(steps, 1)
    x0.copy_(torch.randn(x0.shape, device=hip_device).half())
    chain.run()
    torch.cuda.synchronize()
    for i, st in enumerate(steps):
        y = st.matrix.matmul(st.x.clone())
        if st.bias is not None:
            y = (y + st.bias).half()
        if st.residual is not None:
            y = (y + st.residual).half()
        torch.cuda.synchronize()
        ok, r = gptq.within_tolerance(st.y.float().cpu().numpy(),
                                      y.float().cpu().numpy().astype(np.float64), TOL)
        assert ok, f"link {i}: chain vs dw4_gemm ratio {r:.3f}"
    assert not chain.timed_out()

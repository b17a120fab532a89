"""dw4_gemm_noalloc (the entry point that allocates nothing) against dw4_gemm.

The no-allocation variant runs the same kernels with the same plan, its
split-K partials, arrival counters and gathered act-order activations in the
library's fixed per-GPU scratch array instead of a caller workspace, so its
output must equal dw4_gemm's bit for bit.  Two calls in a row, the second
smaller, check that what the first left in the shared array does not leak
into the second; a call needing more than the array is refused before any
launch.  The register-fed prefill kernel's in-kernel split-K (M of 33-128
rows) keeps per-tile arrival counters at the head of the array, which every
call must leave at zero: two such calls in a row check that.  A call
captured into a HIP graph (after one eager call has set the array up on the
device) replays to the same bits.
"""
from __future__ import annotations

import sys

import pytest
import torch

from gptq_synth import make_layer, make_x
from hip_extends import _lib
from hip_extends.w4a16 import CacheV2, Q4MatrixV2, TuningParams

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _matrix(dev, k, n, act, seed):
    lay = make_layer(k, n, 128, seed=seed, act_order=act).to(dev)
    cache = CacheV2(dev)
    q4 = Q4MatrixV2(lay.qweight, lay.qzeros, lay.scales, k, n, lay.g_idx if act else None, act,
                    TuningParams(MAX_M=512), cache)
    cache.init_cache()
    return q4


def _both(q4, m, seed):
    """(dw4_gemm output with its own zeroed workspace, dw4_gemm_noalloc output)."""
    lib = _lib.load()
    dev = q4.device
    k, n = q4.height, q4.width
    x = make_x(m, k, seed=seed).to(dev)
    perm = q4.perm.data_ptr() if q4.use_act else None
    ws = torch.zeros(max(16, _lib.workspace_size(m, k, n, 128, q4.use_act)), dtype=torch.uint8,
                     device=dev)
    y_ref = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    st = lib.dw4_gemm(m, k, n, 128, x.data_ptr(), k, q4.qweight.data_ptr(), q4.qzeros.data_ptr(),
                      q4.scales.data_ptr(), perm, None, y_ref.data_ptr(), n, ws.data_ptr(),
                      ws.numel(), stream)
    assert st == _lib.DW4_OK, _lib.strerror(st)
    st = lib.dw4_gemm_noalloc(m, k, n, 128, x.data_ptr(), k, q4.qweight.data_ptr(),
                              q4.qzeros.data_ptr(), q4.scales.data_ptr(), perm, None,
                              y.data_ptr(), n, stream)
    assert st == _lib.DW4_OK, _lib.strerror(st)
    torch.cuda.synchronize()
    return y_ref, y


@pytest.mark.parametrize("act", [False, True], ids=["plain", "act"])
def test_noalloc_matches_gemm_two_calls(hip_device, act):
    """First call: M=256 on 8192x4096 (the LDS-streamed prefill kernel split
    over K: fp32 partial planes in the scratch, summed by a second kernel;
    act-order also gathers x there).  Second call, smaller: M=40 on
    4096x2048, then M=1 decode."""
    big = _matrix(hip_device, 8192, 4096, act, 61)
    small = _matrix(hip_device, 4096, 2048, act, 62)
    assert _lib.workspace_size(256, 8192, 4096, 128, False) > 0  # the scratch is really used
    for q4, m in ((big, 256), (small, 40), (small, 1), (big, 256)):
        say(f"noalloc vs gemm {q4.height}x{q4.width} M={m} act={act}")
        y_ref, y = _both(q4, m, seed=m + 3 * act)
        assert not torch.isnan(y).any()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), f"M={m}"


def test_noalloc_split_counters_return_to_zero(hip_device):
    """M=96 on 4096x4096 runs the register-fed prefill kernel split over K,
    whose last-arriving split of each tile sums the partials and resets that
    tile's arrival counter at the head of the scratch.  Two calls in a row
    (then one with M=72) equal dw4_gemm bit for bit: a counter left non-zero
    by the first call would make the second call's sums start early."""
    q4 = _matrix(hip_device, 4096, 4096, False, 63)
    assert _lib.workspace_size(96, 4096, 4096, 128, False) > 0  # split: counters in use
    for m in (96, 96, 72):
        say(f"noalloc vs gemm split counters 4096x4096 M={m}")
        y_ref, y = _both(q4, m, seed=m)
        assert not torch.isnan(y).any()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), f"M={m}"


def test_noalloc_captured_in_graph(hip_device):
    """One eager call sets the scratch up on the device (address lookup and
    counter clear); a call captured into a HIP graph then replays three
    times, with other device work between the replays, each equal to
    dw4_gemm bit for bit."""
    lib = _lib.load()
    q4 = _matrix(hip_device, 4096, 4096, False, 64)
    k = n = 4096
    m = 96
    say("noalloc graph capture 4096x4096 M=96")
    y_ref, _ = _both(q4, m, seed=5)  # eager: also the first use on the device
    x = make_x(m, k, seed=5).to(hip_device)
    y = torch.zeros(m, n, dtype=torch.float16, device=hip_device)
    side = torch.cuda.Stream(device=hip_device)
    side.wait_stream(torch.cuda.current_stream(hip_device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        st = lib.dw4_gemm_noalloc(m, k, n, 128, x.data_ptr(), k, q4.qweight.data_ptr(),
                                  q4.qzeros.data_ptr(), q4.scales.data_ptr(), None, None,
                                  y.data_ptr(), n, side.cuda_stream)
        assert st == _lib.DW4_OK, _lib.strerror(st)
    for r in range(3):
        y.fill_(float("nan"))
        _ = torch.randn(1 << 20, device=hip_device).sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), f"replay {r}"


def test_noalloc_refuses_calls_beyond_its_scratch(hip_device):
    """M=4096 x K=13824 act-order gathers 113 MB of activations: more than the
    64 MiB array, refused with DW4_ERR_SCRATCH before any launch (y untouched)."""
    lib = _lib.load()
    m, k, n = 4096, 13824, 128
    need = _lib.workspace_size(m, k, n, 128, True)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    say("noalloc refuses a call beyond its scratch")
    x = torch.zeros(m, k, dtype=torch.float16, device=hip_device)
    pq = torch.zeros(k // 8 * n, dtype=torch.int32, device=hip_device)
    pz = torch.zeros(k // 128 * n // 8, dtype=torch.int32, device=hip_device)
    ps = torch.zeros(k // 128 * n, dtype=torch.float16, device=hip_device)
    perm = torch.arange(k, dtype=torch.int32, device=hip_device)
    y = torch.full((m, n), 7.0, dtype=torch.float16, device=hip_device)
    st = lib.dw4_gemm_noalloc(m, k, n, 128, x.data_ptr(), k, pq.data_ptr(), pz.data_ptr(),
                              ps.data_ptr(), perm.data_ptr(), None, y.data_ptr(), n,
                              torch.cuda.current_stream().cuda_stream)
    assert st == _lib.DW4_ERR_SCRATCH
    assert "scratch" in _lib.strerror(st)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())

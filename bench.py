#!/usr/bin/env python3
"""W4A16 GEMM benchmark on one MI355X: HBM GB/s at M=1, TFLOP/s at M=256, Llama-2-7B shapes.

Step = one M=1 decode token through the 7 GPTQ projections (q, k, v, o,
gate, up, down) of 8 Llama-2-7B layers -- one pipeline stage of the
reference's split model (8 of the 32 decoder layers) with the
GPTQ 4-bit quantisation (group 128, asymmetric zeros).  The 56 packed weight
matrices (842 MB) are distinct, four times the 256 MB Infinity Cache, so
every launch streams its weights from HBM.  The projections run in a
decoder layer's data-flow order with the fewest launches it allows: q, k, v
(same input) in one grouped launch, o, gate and up (same input) in one
grouped launch, down -- 32 launches per step; the 56-launch form (one per
projection) is reported beside it.  The step is captured once into a HIP
graph and replayed; timing uses HIP events on the replay stream.

Printed JSON line: ``value`` = algorithmic bytes moved per second (GB/s) at
M=1, ``roofline`` for the decode kernel (the only kernel in the step),
``prefill`` = the same 56 GEMMs at M=256 (the same launch grouping) in
TFLOP/s against the fp16 MFMA peak, ``cpu_baseline`` = the reference's CPU dequantise-then-matmul path
(restated with torch CPU ops) on a bounded sample, timed in its dequantise,
matmul and combined phases.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "drofell-for-revision_amd")
sys.path[:0] = [REPO, PKG]

METRIC = "W4A16 GEMM: HBM GB/s @M=1, TFLOP/s @M=256 (% MI355X roofline), 7B shapes"
HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0
GROUP = 128


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def build_matrices(dev, layers: int, max_m: int, seed0: int = 1234, shapes=None,
                   scale_mul: float = 0.01, act_order: bool = False, symmetric: bool = False):
    import torch
    from gptq_synth import LLAMA2_7B_SHAPES
    from hip_extends.w4a16 import CacheV2, Q4MatrixV2, TuningParams

    cache = CacheV2(dev)
    tp = TuningParams(MAX_M=max_m)
    gen = torch.Generator(device=dev)
    mats = []
    for layer in range(layers):
        for pi, (name, (k, n)) in enumerate((shapes or LLAMA2_7B_SHAPES).items()):
            gen.manual_seed(seed0 + 100 * layer + pi)
            groups = k // GROUP
            # uniform random words == every nibble uniform in 0..15
            qweight = torch.randint(-2 ** 31, 2 ** 31, (k // 8, n), dtype=torch.int32,
                                    device=dev, generator=gen)
            qzeros = torch.randint(-2 ** 31, 2 ** 31, (groups, n // 8), dtype=torch.int32,
                                   device=dev, generator=gen)
            if symmetric:  # config 1: every stored zero 7 (effective zero 8)
                qzeros.fill_(0x77777777)
            scales = (torch.randn(groups, n, device=dev, generator=gen).abs() * scale_mul
                      + scale_mul / 10).to(torch.float16)
            g_idx = None
            if act_order:  # config 4: g_idx[k] = pi(k) // 128 for a seeded permutation pi
                g_idx = (torch.randperm(k, device=dev, generator=gen) // GROUP).to(torch.int32)
            q4 = Q4MatrixV2(qweight, qzeros, scales, k, n, g_idx, act_order, tp, cache)
            mats.append((name, k, n, q4))
            del qweight, qzeros, scales, g_idx
    cache.init_cache()
    torch.cuda.synchronize()
    return mats, cache


def time_graph(mats, m: int, steps: int, warmup: int, dev, select=None, per_replay=None):
    """Capture one pass over `mats` at M=m into a graph; return ms per pass.
    With a list `per_replay`, each replay is also timed on its own (appended, ms)."""
    import torch

    sel = [t for t in mats if select is None or select(t)]
    gen = torch.Generator(device=dev)
    gen.manual_seed(m)
    xs = {k: torch.randn(m, k, device=dev, generator=gen).to(torch.float16)
          for k in sorted({t[1] for t in sel})}
    ys = {n: torch.empty(m, n, dtype=torch.float16, device=dev) for n in sorted({t[2] for t in sel})}

    def one_pass():
        for _, k, n, q4 in sel:
            q4.matmul(xs[k], output=ys[n])

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        one_pass()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        one_pass()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(end) / steps
    if per_replay is not None:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        for a, b in evs:
            a.record(stream)
            graph.replay()
            b.record(stream)
        torch.cuda.synchronize(dev)
        per_replay.extend(a.elapsed_time(b) for a, b in evs)
    return ms, wall, sel


# The decode kernel's sources and the Makefile (whose flags for
# w4a16_decode.hip change the generated code).
DECODE_SOURCES = ("w4a16_decode.hip", "w4a16_internal.h", "w4a16_device.h", "Makefile")


def decode_source_sha256() -> str:
    """Digest of the sources the decode kernel is built from."""
    import hashlib

    h = hashlib.sha256()
    for name in DECODE_SOURCES:
        with open(os.path.join(REPO, "drofell-for-revision_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def time_callable(fn, steps: int, warmup: int, dev) -> float:
    """ms per call of `fn` (enqueues device work only), captured once into a
    HIP graph and replayed `steps` times between HIP events."""
    import torch

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize(dev)
    del graph
    return start.elapsed_time(end) / steps


# (label, bytes, workgroups, threads): the weight bytes of a decode launch and
# the decode kernel's launch shape at M=1 (one workgroup per 16-column strip;
# 16 waves when strips <= CUs, 4 when strips >= 2 x CUs), plus two shapes with
# more, smaller workgroups for the 8 MiB case.
STREAM_SHAPES = (
    ("4096x4096", 8 << 20, 256, 1024),
    ("4096x4096 1024x256", 8 << 20, 1024, 256),
    ("4096x4096 2048x256", 8 << 20, 2048, 256),
    ("4096x11008", 4096 * 11008 // 2, 688, 256),
    ("11008x4096", 11008 * 4096 // 2, 256, 1024),
    ("4096x12288", 4096 * 12288 // 2, 768, 256),
    ("4096x22016", 4096 * 22016 // 2, 1376, 256),
)


def stream_ceiling(dev, steps: int) -> list:
    """Per-launch time of the library's calibration read (dw4_stream_read)
    in the decode launch shapes.  Each graph replay reads consecutive slices
    of a 1 GiB buffer, so no slice is read twice within 1 GiB (four times the
    Infinity Cache)."""
    import torch
    from hip_extends import _lib

    lib = _lib.load()
    pool_bytes = 1 << 30
    pool = torch.randint(-2 ** 31, 2 ** 31, (pool_bytes // 4,), dtype=torch.int32, device=dev)
    sink = torch.zeros(2048 * 1024, dtype=torch.int32, device=dev)
    out = []
    for label, nbytes, wgs, threads in STREAM_SHAPES:
        per = pool_bytes // nbytes
        stream = torch.cuda.current_stream(dev).cuda_stream

        def one_pass(nbytes=nbytes, wgs=wgs, threads=threads, per=per):
            st = torch.cuda.current_stream(dev).cuda_stream
            for i in range(per):
                _lib.check("dw4_stream_read", lib.dw4_stream_read(
                    pool.data_ptr() + i * nbytes, nbytes, wgs, threads, 0x9E3779B9,
                    sink.data_ptr(), st))
        del stream
        ms = time_callable(one_pass, max(3, steps // 10), 2, dev)
        us = ms * 1e3 / per
        rec = {"shape": label, "bytes": nbytes, "workgroups": wgs, "threads": threads,
               "us_per_launch": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
               "launches_per_pass": per}
        log(json.dumps({"stream_read": rec}))
        out.append(rec)
    del pool, sink
    torch.cuda.empty_cache()
    return out


def device_peaks(dev, steps: int) -> dict:
    """What this box reaches outside the W4A16 kernels, as context for the
    roofline fractions (which stay against the spec peaks): a large fp16
    library GEMM (torch.matmul, hipBLASLt), a 1 GiB device copy and the
    library's streaming read over 1 GiB, each captured in a HIP graph."""
    import torch
    from hip_extends import _lib

    props = torch.cuda.get_device_properties(dev)
    rec = {"device": props.name, "arch": getattr(props, "gcnArchName", ""),
           "cus": props.multi_processor_count, "hip": torch.version.hip, "torch": torch.__version__}
    gemm = {}
    for n in (4096, 8192, 16384):
        a = torch.randn(n, n, device=dev).to(torch.float16)
        b = torch.randn(n, n, device=dev).to(torch.float16)
        c = torch.empty(n, n, device=dev, dtype=torch.float16)
        ms = time_callable(lambda: torch.matmul(a, b, out=c), max(5, steps // 5), 3, dev)
        gemm[str(n)] = {"ms": round(ms, 4), "TFLOP/s": round(2 * n ** 3 / (ms * 1e-3) / 1e12, 1)}
        del a, b, c
    rec["fp16_gemm_square"] = gemm
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    ms = time_callable(lambda: dst.copy_(src), max(5, steps // 5), 3, dev)
    rec["copy_1GiB"] = {"ms": round(ms, 4), "GB/s (read + write)": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}
    del dst
    lib = _lib.load()
    sink = torch.zeros(2048 * 256, dtype=torch.int32, device=dev)
    ms = time_callable(lambda: _lib.check("dw4_stream_read", lib.dw4_stream_read(
        src.data_ptr(), nbytes, 2048, 256, 0x9E3779B9, sink.data_ptr(),
        torch.cuda.current_stream(dev).cuda_stream)), max(5, steps // 5), 3, dev)
    rec["stream_read_1GiB"] = {"ms": round(ms, 4), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    del src, sink
    torch.cuda.empty_cache()
    info = device_info(dev)  # current clock levels after the runs (informational)
    rec["clocks"] = {"sclk": info["sclk"], "mclk": info["mclk"]}
    log(json.dumps({"device_peaks": rec}))
    return rec


def crossover(mats, dev, steps: int, ms_list=(64, 128, 256, 512, 768, 1024, 2048, 4096, 8192)):
    """Per M: the 56-matrix pass through the native W4A16 kernel, through the
    reference's dense route (bit-exact dequantisation into one shared fp16
    buffer, then a library GEMM per matrix) and through a dense GEMM over an
    already-reconstructed weight.  For training with a kept weight (PEFT),
    also forward plus activation gradient: packed (the native forward, then
    ``transpose_matmul``, which runs the packed transposed kernel up to its
    row limit) against dense (dequantise once, then a library GEMM for the
    forward and one for the gradient over that weight)."""
    import torch

    kmax = max(k * n for _, k, n, _ in mats)
    temp = torch.empty(kmax, dtype=torch.float16, device=dev)
    shapes = sorted({(k, n) for _, k, n, _ in mats})
    kept = {kn: torch.empty(kn, dtype=torch.float16, device=dev) for kn in shapes}
    for (k, n), w in kept.items():
        q4 = next(q for _, kk, nn, q in mats if (kk, nn) == (k, n))
        q4.get_float16_weights_matrix_v2(w)
    rows = []
    for m in ms_list:
        gen = torch.Generator(device=dev)
        gen.manual_seed(m)
        xs = {k: torch.randn(m, k, device=dev, generator=gen).to(torch.float16)
              for k in sorted({k for k, _ in shapes})}
        ys = {n: torch.empty(m, n, dtype=torch.float16, device=dev)
              for n in sorted({n for _, n in shapes})}

        def native():
            for _, k, n, q4 in mats:
                q4.matmul(xs[k], output=ys[n])

        def dense():
            for _, k, n, q4 in mats:
                w = temp[: k * n].view(k, n)
                q4.get_float16_weights_matrix_v2(w)
                torch.matmul(xs[k], w, out=ys[n])

        def dense_kept():
            for _, k, n, q4 in mats:
                torch.matmul(xs[k], kept[(k, n)], out=ys[n])

        gs_ = {n: torch.randn(m, n, device=dev, generator=gen).to(torch.float16)
               for n in sorted({n for _, n in shapes})}
        gx = {k: torch.empty(m, k, dtype=torch.float16, device=dev)
              for k in sorted({k for k, _ in shapes})}

        def peft_packed():
            for _, k, n, q4 in mats:
                q4.matmul(xs[k], output=ys[n])
                q4.transpose_matmul(gs_[n], output=gx[k])

        def peft_dense():
            for _, k, n, q4 in mats:
                w = temp[: k * n].view(k, n)
                q4.get_float16_weights_matrix_v2(w)
                torch.matmul(xs[k], w, out=ys[n])
                torch.matmul(gs_[n], w.t(), out=gx[k])

        st = max(3, steps // 10)
        rec = {"m": m, "native_ms": round(time_callable(native, st, 2, dev), 4),
               "dense_ms": round(time_callable(dense, st, 2, dev), 4),
               "dense_kept_weight_ms": round(time_callable(dense_kept, st, 2, dev), 4),
               "peft_packed_ms": round(time_callable(peft_packed, st, 2, dev), 4),
               "peft_dense_ms": round(time_callable(peft_dense, st, 2, dev), 4)}
        log(json.dumps({"crossover": rec}))
        rows.append(rec)
        del xs, ys, gs_, gx
        torch.cuda.empty_cache()
    return rows


def stage_reference_fp32(x, layer_mats, norm, eps, kcaches, vcaches, tables, pos, sin, cos,
                         heads, hd, bs):
    """One decode step of the stage in float32 torch ops on the GPU, rounded
    to fp16 where the stage's tensors are fp16: the bench's own check of its
    stage leg (the weights come from the bit-exact dequantiser; the caches
    are copies taken before the step and are updated here)."""
    import torch
    import torch.nn.functional as F

    def rms_norm(t):
        t = t.float().clamp(-65504.0, 65504.0)
        r = torch.rsqrt(t.pow(2).mean(dim=-1, keepdim=True) + eps)
        return (t * norm.float() * r).half()

    def mm(a, q4):
        return (a.float() @ q4.get_float16_weights_matrix_v2().float()).half()

    def rope(t):  # t [b, heads, hd] fp16, rotate-half at pos[b]
        s_, c_ = sin[pos.long()].float()[:, None, :], cos[pos.long()].float()[:, None, :]
        tf = t.float()
        rot = torch.cat([-tf[..., hd // 2:], tf[..., :hd // 2]], dim=-1)
        return (tf * c_ + rot * s_).half()

    b = x.shape[0]
    ar = torch.arange(b, device=x.device)
    for li, w in enumerate(layer_mats):
        h = rms_norm(x)
        q = rope(mm(h, w["q_proj"]).view(b, heads, hd))
        k = rope(mm(h, w["k_proj"]).view(b, heads, hd))
        v = mm(h, w["v_proj"]).view(b, heads, hd)
        blk = tables[ar, pos.long() // bs].long()
        off = pos.long() % bs
        kc, vc = kcaches[li], vcaches[li]  # [blocks, heads, hd/8, bs, 8], [blocks, heads, hd, bs]
        kc[blk, :, :, off, :] = k.view(b, heads, hd // 8, 8)
        vc[blk, :, :, off] = v
        outs = []
        for s in range(b):
            n = int(pos[s]) + 1
            kb = kc[tables[s].long()].permute(0, 3, 1, 2, 4).reshape(-1, heads, hd)[:n]
            vb = vc[tables[s].long()].permute(0, 3, 1, 2).reshape(-1, heads, hd)[:n]
            kt = kb.float().permute(1, 2, 0).contiguous()  # [heads, hd, n]
            logits = torch.bmm(q[s].float().unsqueeze(1), kt) * hd ** -0.5  # [heads, 1, n]
            vt = vb.float().permute(1, 0, 2).contiguous()  # [heads, n, hd]
            outs.append(torch.bmm(F.softmax(logits, dim=-1), vt).squeeze(1))
        attn = torch.stack(outs).half().view(b, heads * hd)
        x2 = (x.float() + mm(attn, w["o_proj"]).float()).half()
        h2 = rms_norm(x2)
        g, u = mm(h2, w["gate_proj"]).float(), mm(h2, w["up_proj"]).float()
        act = (g / (1.0 + torch.exp(-g)) * u).half()
        x = (x2.float() + mm(act, w["down_proj"]).float()).half()
    return x


def stage_leg(dev, layers: int, batch: int, ctx0: int, decode_steps: int, block_size: int,
              warmup: int) -> dict:
    """The 8-layer Llama-2-7B decoder stage at decode: per layer the fused
    q/k/v stage (RMSNorm + grouped q/k/v), RoPE, the KV-cache write, paged
    attention and the after-attention stage (o_proj + residual, RMSNorm,
    gate/up with SiLU*mul, down + residual), for `batch` sequences whose
    cached context grows from `ctx0` by one token per step.  One step (all
    layers) is captured into a HIP graph; positions, slots and context
    lengths advance on the device inside it."""
    import torch
    from gptq_synth import LLAMA2_7B_SHAPES
    from hip_extends.w4a16 import attention_forward_qkv_stage_v2_py, decoder_after_stage_v2_py
    from operators import flags
    from operators.core.attention.common import AttentionConfig
    from operators.core.attention.real_page import PagedAttention
    from operators.core.block.common import BlockInfo
    from operators.core.block.real import LayerBlocksHolder

    hidden, inter, heads, hd = 4096, 11008, 32, 128
    flags.BLOCK_SIZE = block_size
    max_ctx = ctx0 + decode_steps
    mats, cache = build_matrices(dev, layers, batch, seed0=777, scale_mul=0.002)
    per = len(LLAMA2_7B_SHAPES)
    lay = [{name: q4 for name, _, _, q4 in mats[i * per:(i + 1) * per]} for i in range(layers)]
    info = BlockInfo(head_dim=hd, num_key_value_heads=heads)
    bps = (max_ctx + block_size - 1) // block_size  # blocks per sequence
    holders = []
    for _ in range(layers):
        h = LayerBlocksHolder.create_contigious_cacher(info, batch * bps, dev)
        kc, vc = h.contigious_kv_tenosr
        kc.normal_()
        vc.normal_()
        holders.append(h)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    tables = torch.randperm(batch * bps, device=dev, generator=gen).to(torch.int32).view(batch, bps)
    att = PagedAttention(AttentionConfig(hidden, hd, heads, heads, 1))
    att.workspace(batch, max_ctx, dev)
    inv = 1.0 / 10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd)
    ang = torch.outer(torch.arange(max_ctx + 1, dtype=torch.float64), inv)
    ang = torch.cat([ang, ang], dim=1)
    sin, cos = ang.sin().to(dev, torch.float16), ang.cos().to(dev, torch.float16)
    f16 = dict(dtype=torch.float16, device=dev)
    embed = (torch.randn(batch, hidden, device=dev, generator=gen)).to(torch.float16)
    xa, xb = torch.empty(batch, hidden, **f16), torch.empty(batch, hidden, **f16)
    rms, q, k, v = (torch.empty(batch, hidden, **f16) for _ in range(4))
    x2 = torch.empty(batch, hidden, **f16)
    hbuf, ubuf = torch.empty(batch, inter, **f16), torch.empty(batch, inter, **f16)
    norm = torch.ones(hidden, **f16)
    ctx = torch.full((batch,), ctx0, dtype=torch.int32, device=dev)

    lens = torch.empty(batch, dtype=torch.int32, device=dev)

    def step():
        xa.copy_(embed)  # each step's new tokens (synthetic embeddings)
        xin, xout = xa, xb
        for li in range(layers):
            w = lay[li]
            attention_forward_qkv_stage_v2_py(norm, 1e-5, w["q_proj"], w["k_proj"], w["v_proj"],
                                              rms, q, k, v, None, xin, 0, 0, 0, 1, batch)
            # RoPE on q and k at position ctx, k and v to their cache slots,
            # lens = ctx + 1: one launch
            holders[li].rope_and_cache(q.view(batch, heads, hd), k.view(batch, heads, hd),
                                       v.view(batch, heads, hd), sin, cos, ctx, tables, lens)
            o = att.forward(q.view(batch, heads, hd), max_ctx, lens, tables, holders[li])
            decoder_after_stage_v2_py(w["o_proj"], w["gate_proj"], w["up_proj"], w["down_proj"],
                                      norm, 1e-5, o.view(batch, hidden), xin, x2, rms, hbuf, ubuf,
                                      xout)
            xin, xout = xout, xin
        ctx.add_(1)

    # step 0 on fresh state, checked against the float32 composition
    kref = [h.contigious_kv_tenosr[0].clone() for h in holders]
    vref = [h.contigious_kv_tenosr[1].clone() for h in holders]
    pos0 = ctx.clone()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    got = (xa if layers % 2 == 0 else xb).float()
    want = stage_reference_fp32(embed, lay, norm, 1e-5, kref, vref, tables, pos0, sin, cos,
                                heads, hd, block_size).float()
    row_tol = 2e-2 * want.abs().amax(dim=1, keepdim=True)
    step0_ratio = float(((got - want).abs().amax(dim=1, keepdim=True) / row_tol).max())
    del kref, vref
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize(dev)
    ctx.fill_(ctx0)
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(decode_steps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize(dev)
    ms = start.elapsed_time(end) / decode_steps
    finite = bool(torch.isfinite(xa).all().item() and torch.isfinite(xb).all().item())
    kv_bytes = layers * batch * (ctx0 + decode_steps / 2) * heads * hd * 2 * 2
    wbytes = sum(q4.qweight.numel() * 4 + q4.scales.numel() * 2 + q4.qzeros.numel() * 4
                 for _, _, _, q4 in mats)
    del graph, holders, mats, cache
    torch.cuda.empty_cache()
    return {"tokens_per_s": round(batch / (ms * 1e-3), 1), "ms_per_step": round(ms, 4),
            "batch": batch, "layers": layers, "context": [ctx0, max_ctx],
            "decode_steps": decode_steps, "block_size": block_size,
            "weight_bytes": wbytes, "mean_kv_bytes_per_step": int(kv_bytes),
            "hbm_gbs": round((wbytes + kv_bytes) / (ms * 1e-3) / 1e9, 1), "finite": finite,
            "step0_error_over_tolerance": round(step0_ratio, 5),
            "step0_check": ("final hidden state of step 0 against a float32 torch composition "
                            "of the same stage (fp16 rounding at the stage's tensor "
                            "boundaries, bit-exact dequantised weights); per row "
                            "max|h - h_ref| / (2e-2 * ||h_ref row||_inf), <= 1 passes"),
            "workload": ("8 Llama-2-7B decoder layers (GPTQ g128 asymmetric), per layer: "
                         "RMSNorm+q/k/v (one launch), RoPE+KV-cache write (one launch), paged "
                         "attention (32 heads x 128, fp16 KV), o_proj+residual, RMSNorm, "
                         "gate/up+SiLU*mul (one launch), down+residual")}


def host_cpu() -> dict:
    """CPU model, physical cores (distinct (package, core) pairs) and the
    logical CPUs this process may run on, from /proc/cpuinfo."""
    model, cores, pkg, core = None, set(), None, None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model is None:
                    model = val
                elif key == "physical id":
                    pkg = val
                elif key == "core id":
                    core = val
                elif not key and pkg is not None and core is not None:
                    cores.add((pkg, core))
                    pkg = core = None
        if pkg is not None and core is not None:
            cores.add((pkg, core))
    except OSError:
        pass
    return {"cpu_model": model, "physical_cores": len(cores) or None,
            "logical_cpus_allowed": len(os.sched_getaffinity(0))}


def cpu_baseline(seconds: float) -> dict:
    """The reference's CPU dequantise-then-matmul on one 4096x4096 projection,
    timed in its three phases: dequantise (reconstruct the fp16 weight), the
    fp32 matmul against an already dequantised weight, and both back to back
    (the reference's forward).  ``value`` is the combined phase's rate."""
    import statistics

    import torch
    from gptq_synth import algorithmic_bytes, make_layer, make_x
    from oracle import cpu_path

    # at most 16 threads: the GPU box gives one GPU's job a 16-CPU share
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    lay = make_layer(4096, 4096, GROUP, seed=1000)
    x = make_x(1, 4096, seed=1)
    w = cpu_path.reconstruct_weights(lay.qweight, lay.qzeros, lay.scales, lay.g_idx)
    phases = {
        "dequantise": lambda: cpu_path.reconstruct_weights(lay.qweight, lay.qzeros, lay.scales,
                                                           lay.g_idx),
        "matmul": lambda: (x.float() @ w.float()).to(torch.float16),
        "both": lambda: cpu_path.forward(x, lay.qweight, lay.qzeros, lay.scales, lay.g_idx),
    }
    share = {"dequantise": 0.3, "matmul": 0.2, "both": 0.5}
    med, runs = {}, {}
    for name, fn in phases.items():
        fn()  # warm-up
        times = []
        t_end = time.perf_counter() + seconds * share[name]
        while len(times) < 3 or time.perf_counter() < t_end:
            t0 = time.perf_counter_ns()
            fn()
            times.append((time.perf_counter_ns() - t0) * 1e-9)
        med[name], runs[name] = statistics.median(times), len(times)
    nbytes = algorithmic_bytes(1, 4096, 4096, GROUP, False)
    return {"value": round(nbytes / med["both"] / 1e9, 4), "unit": "GB/s", "cores": threads,
            **host_cpu(), "kind": "port",
            "phases_ms": {k: round(v * 1e3, 3) for k, v in med.items()},
            "sample": (f"torch-CPU dequantise+matmul (real_quant.py:69-102 restated) of one "
                       f"4096x4096 g128 asymmetric projection at M=1; median of "
                       f"{runs['dequantise']} / {runs['matmul']} / {runs['both']} runs of the "
                       f"dequantise / matmul / combined phases; torch {torch.__version__}")}


def device_info(dev) -> dict:
    """GPU name, architecture, CU count, ROCm/HIP version and the current
    shader and memory clock levels (None where a field is not available).
    The clocks and the product name come from the amdgpu sysfs files of the
    card whose PCI address matches the device (no child process: this runs
    after the GPU is initialised)."""
    import glob

    import torch
    props = torch.cuda.get_device_properties(dev)
    info = {"gpu": props.name, "arch": getattr(props, "gcnArchName", None),
            "cus": props.multi_processor_count, "hip": torch.version.hip,
            "torch": torch.__version__, "rocm": None, "product": None, "pci": None,
            "sclk": None, "mclk": None}
    try:
        with open("/opt/rocm/.info/version") as f:
            info["rocm"] = f.read().strip()
    except OSError:
        pass
    bus = getattr(props, "pci_bus_id", None)
    dom = getattr(props, "pci_domain_id", 0) or 0
    devn = getattr(props, "pci_device_id", 0) or 0
    if bus is None:
        return info
    info["pci"] = f"{dom:04x}:{bus:02x}:{devn:02x}.0"

    def read(path):
        try:
            with open(path) as f:
                return f.read()
        except OSError:
            return None

    for card in glob.glob("/sys/class/drm/card*/device"):
        if not os.path.realpath(card).endswith(info["pci"]):
            continue
        name = read(os.path.join(card, "product_name"))
        info["product"] = name.strip() if name else None
        for key, fname in (("sclk", "pp_dpm_sclk"), ("mclk", "pp_dpm_mclk")):
            levels = read(os.path.join(card, fname)) or ""
            cur = [ln.split(":", 1)[-1].replace("*", "").strip()
                   for ln in levels.splitlines() if ln.rstrip().endswith("*")]
            info[key] = cur[0] if cur else None
        break
    return info


def grouped_leg(mats, dev, steps: int, warmup: int, m: int = 1) -> dict:
    """The 56 projections of the decode leg at M=m with the launches a
    decoder layer's data flow allows: q, k, v share the layer input (one
    dw4_gemm_group launch), o alone, gate and up share o's output (one
    launch), down alone -- 4 launches per layer instead of 7.  Same
    matrices, same bytes."""
    import torch
    from gptq_synth import algorithmic_bytes, flops
    from hip_extends.w4a16 import gemm_group

    gen = torch.Generator(device=dev)
    gen.manual_seed(13)
    xs = {k: torch.randn(m, k, device=dev, generator=gen).to(torch.float16)
          for k in sorted({t[1] for t in mats})}
    groups = []
    for li in range(len(mats) // 7):
        w = {name.split("_")[0]: (q4, k, n) for name, k, n, q4 in mats[7 * li:7 * li + 7]}
        for names in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
            k = w[names[0]][1]
            outs = [torch.empty(m, w[nm][2], dtype=torch.float16, device=dev) for nm in names]
            groups.append((xs[k], [w[nm][0] for nm in names], outs))

    def one_pass():
        for x, q4s, outs in groups:
            if len(q4s) == 1:
                q4s[0].matmul(x, output=outs[0])
            else:
                gemm_group(x, q4s, outs)

    ms = time_callable(one_pass, steps, warmup, dev)
    nbytes = sum(algorithmic_bytes(m, k, n, GROUP, False) for _, k, n, _ in mats)
    gbs = nbytes / (ms * 1e-3) / 1e9
    tf = sum(flops(m, k, n) for _, k, n, _ in mats) / (ms * 1e-3) / 1e12
    if m == 1:
        log(f"decode M=1: {ms * 1e3:.1f} us per step ({len(groups)} launches), {gbs:.1f} GB/s")
    else:
        log(f"prefill M={m}: {ms * 1e3:.1f} us per step ({len(groups)} launches), {tf:.1f} TFLOP/s")
    return {"us_per_step": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "TFLOP/s": round(tf, 2),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "launches_per_step": len(groups),
            "kernel": ("dw4::decode_kernel (item table over q/k/v and gate/up)" if m == 1 else
                       "dw4::prefill2_kernel (item table over q/k/v and gate/up)")}


def chain_leg(mats, dev, steps: int, warmup: int, layers: int) -> dict:
    """The 56 projections of the decode leg as ONE dw4_gemm_chain launch per
    step, in two forms:

    * ``dependent``: each layer's data flow (q, k, v read the layer input; o
      reads v's output with the layer input as residual; gate and up read
      o's output; down reads up's output with o's output as residual and
      writes the next layer's input), so every link waits for the link it
      reads to complete on all workgroups;
    * ``independent``: every link reads a fixed activation (no waits), the
      same work as the per-launch decode leg.

    Both move the same algorithmic bytes as the decode leg."""
    import torch
    from gptq_synth import algorithmic_bytes
    from hip_extends.chain import ChainStep, Q4Chain

    f16 = dict(dtype=torch.float16, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    nbytes = sum(algorithmic_bytes(1, k, n, GROUP, False) for _, k, n, _ in mats)
    xs = {k: torch.randn(1, k, device=dev, generator=gen).to(torch.float16)
          for k in sorted({t[1] for t in mats})}
    ind = [ChainStep(q4, xs[k], torch.empty(1, n, **f16)) for _, k, n, q4 in mats]
    hidden = mats[0][1]
    hs = [torch.randn(1, hidden, device=dev, generator=gen).to(torch.float16)
          for _ in range(layers + 1)]
    dep, down = [], -1
    for li in range(layers):
        w = {name.split("_")[0]: (q4, n) for name, _, n, q4 in mats[7 * li:7 * li + 7]}
        out = {name: torch.empty(1, n, **f16) for name, (_, n) in w.items()}
        base = len(dep)
        dep += [ChainStep(w["q"][0], hs[li], out["q"], down),
                ChainStep(w["k"][0], hs[li], out["k"], down),
                ChainStep(w["v"][0], hs[li], out["v"], down),
                ChainStep(w["o"][0], out["v"], out["o"], base + 2, residual=hs[li]),
                ChainStep(w["gate"][0], out["o"], out["gate"], base + 3),
                ChainStep(w["up"][0], out["o"], out["up"], base + 3),
                ChainStep(w["down"][0], out["up"], hs[li + 1], base + 5, residual=out["o"])]
        down = base + 6
    res = {"kernel": "dw4::chain_kernel", "links": len(mats), "launches_per_step": 1,
           "algorithmic_bytes_per_step": nbytes}
    for name, links in (("dependent", dep), ("independent", ind)):
        chain = Q4Chain(links, 1)
        chain.run()
        torch.cuda.synchronize(dev)
        ms = time_callable(chain.run, steps, warmup, dev)
        if chain.timed_out():
            raise RuntimeError(f"chain leg ({name}): a dependency wait gave up")
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"chain ({name}) M=1: {ms * 1e3:.1f} us per step, {gbs:.1f} GB/s "
            f"(ring {chain.plan.ring}, {chain.plan.workgroups} workgroups)")
        res[name] = {"us_per_step": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "ring": chain.plan.ring,
                     "workgroups": chain.plan.workgroups, "waves": chain.plan.waves}
        del chain
    return res


def time_transpose(mats, m: int, steps: int, warmup: int, dev, dense: bool = False) -> float:
    """ms per pass of the PEFT-backward product g @ W^T over `mats` at M=m:
    the packed kernel, or (dense=True) the reference's route: bit-exact
    dequantisation into the shared fp16 buffer, then a library GEMM."""
    import torch

    gen = torch.Generator(device=dev)
    gen.manual_seed(m + 7)
    gs = {n: torch.randn(m, n, device=dev, generator=gen).to(torch.float16)
          for n in sorted({t[2] for t in mats})}
    for _, k, n, q4 in mats:  # size the workspaces before capture
        q4._transpose_native(gs[n], None)
        if dense:
            q4._dense_weight(None)

    def one_pass():
        for _, k, n, q4 in mats:
            if dense:
                torch.matmul(gs[n], q4._dense_weight(None).t())
            else:
                q4._transpose_native(gs[n], None)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        one_pass()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        one_pass()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize(dev)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize(dev)
    return start.elapsed_time(end) / steps


def sweep(mats, dev, steps: int, warmup: int,
          shapes=((4096, 4096), (4096, 11008), (11008, 4096)),
          ms_list=(1, 2, 4, 8, 16, 64, 256, 1024, 2048), act_order: bool = False,
          tag: str = "") -> list:
    """Per-shape, per-M lines (JSON on stderr): mean per launch over the
    rotated matrices of that shape, and the median / p10 / p90 of single
    graph replays (each replay = one launch per matrix of the shape).
    Returns the lines as dicts."""
    from gptq_synth import algorithmic_bytes, flops
    out = []
    for (k, n) in shapes:
        for m in ms_list:
            reps = []
            ms, _, sel = time_graph(mats, m, steps, warmup, dev,
                                    select=lambda t, k=k, n=n: t[1] == k and t[2] == n,
                                    per_replay=reps)
            per = ms / len(sel) * 1e3
            q = sorted(r / len(sel) * 1e3 for r in reps)
            pct = lambda f: round(q[min(len(q) - 1, int(f * len(q)))], 3)
            b = algorithmic_bytes(m, k, n, GROUP, act_order)
            f = flops(m, k, n)
            bound = "hbm" if b / HBM_PEAK_GBS * 1e-3 >= f / MFMA_FP16_PEAK_TFLOPS * 1e-6 else "mfma"
            frac = (b / per / 1e3 / HBM_PEAK_GBS) if bound == "hbm" else \
                (f / per / 1e6 / MFMA_FP16_PEAK_TFLOPS)
            rec = {"config": tag, "shape": f"{k}x{n}", "m": m, "act_order": act_order,
                   "matrices": len(sel), "us": round(per, 3), "median_us": pct(0.5),
                   "p10_us": pct(0.1), "p90_us": pct(0.9),
                   "GB/s": round(b / per / 1e3, 1), "TFLOP/s": round(f / per / 1e6, 2),
                   "bound": bound, "frac": round(frac, 4)}
            log(json.dumps(rec))
            out.append(rec)
    return out


def bf16_sweep(dev, steps: int, warmup: int,
               plan=(((4096, 4096), False), ((4096, 11008), False), ((11008, 4096), False),
                     ((5120, 5120), True)),
               ms_list=(1, 8, 16, 17, 32, 48, 64)) -> list:
    """bf16 activations through Q4MatrixV2.matmul: the packed-weight bf16
    decode launch (dw4_gemm_bf16) against the dense route (bf16
    dequantisation, then a bf16 library GEMM; must_blas), microseconds per
    call.  Each shape rotates over distinct matrices totalling at least
    256 MB (so no call finds its weights in the Infinity Cache), every call
    writing a preallocated output, captured in one HIP graph per (shape, M,
    route) and replayed steps times after warmup replays.  JSON lines on
    stderr; returns them."""
    import torch
    from gptq_synth import algorithmic_bytes

    out = []
    for (k, n), act in plan:
        count = max(4, -(-(256 << 20) // (k * n // 2)))
        mats, cache = build_matrices(dev, count, 64, seed0=500, shapes={"p": (k, n)},
                                     act_order=act)
        for m in ms_list:
            gen = torch.Generator(device=dev)
            gen.manual_seed(m)
            x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            us = {}
            for route, dense in (("native", False), ("dense", True)):
                def one():
                    for _, _, _, q4 in mats:
                        q4.matmul(x, output=y, must_blas=dense)

                side = torch.cuda.Stream(device=dev)
                side.wait_stream(torch.cuda.current_stream(dev))
                with torch.cuda.stream(side):
                    one()  # first calls (library handles, dequantisation buffers) outside capture
                torch.cuda.current_stream(dev).wait_stream(side)
                torch.cuda.synchronize(dev)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    one()
                for _ in range(warmup):
                    g.replay()
                torch.cuda.synchronize(dev)
                s = torch.cuda.current_stream(dev)
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(s)
                for _ in range(steps):
                    g.replay()
                b.record(s)
                torch.cuda.synchronize(dev)
                us[route] = a.elapsed_time(b) / steps * 1e3 / len(mats)
                del g
            nbytes = algorithmic_bytes(m, k, n, GROUP, act)
            rec = {"shape": f"{k}x{n}", "act_order": act, "m": m, "matrices": len(mats),
                   "native_us": round(us["native"], 2), "dense_us": round(us["dense"], 2),
                   "speedup": round(us["dense"] / us["native"], 2),
                   "native_GB/s": round(nbytes / us["native"] / 1e3, 1)}
            log(json.dumps(rec))
            out.append(rec)
        del mats, cache
        torch.cuda.empty_cache()
    return out


# The benchmark's configurations 1-4 as the default run measures them: (tag,
# shape, act-order, symmetric zeros, M values).  Configuration 5 is the stage
# leg.
CONFIG_PLAN = (
    ("C1", (4096, 4096), False, True, (1,)),
    ("C2", (4096, 4096), False, False, (1, 2, 4, 8, 16)),
    ("C3", (4096, 4096), False, False, (16, 64, 256, 1024, 2048)),
    ("C2", (4096, 11008), False, False, (1, 2, 4, 8, 16)),
    ("C3", (4096, 11008), False, False, (16, 64, 256, 1024, 2048)),
    ("C2", (11008, 4096), False, False, (1, 2, 4, 8, 16)),
    ("C3", (11008, 4096), False, False, (16, 64, 256, 1024, 2048)),
    ("C4", (5120, 5120), True, False, (1, 8, 64)),
    ("C4", (5120, 13824), True, False, (1, 8, 64)),
    ("C4", (13824, 5120), True, False, (1, 8, 64)),
)


def config_points(dev, steps: int) -> dict:
    """Configs 1-4, one entry per (shape, M): [shape, M, us per launch, GB/s,
    TFLOP/s, bound, fraction of that bound's peak].  Each shape rotates over
    distinct matrices totalling >= 512 MB, so the 256 MB Infinity Cache
    cannot serve the weights between launches."""
    import torch
    from gptq_synth import algorithmic_bytes
    res: dict = {}
    built = {}
    for tag, (k, n), act, sym, ms_list in CONFIG_PLAN:
        key = (k, n, act, sym)
        if key not in built:
            built.clear()
            torch.cuda.empty_cache()
            count = -(-(512 << 20) // algorithmic_bytes(1, k, n, GROUP, act))
            built[key] = build_matrices(dev, count, 2048, seed0=7000 + k + n + 17 * sym,
                                        shapes={f"{k}x{n}": (k, n)}, act_order=act,
                                        symmetric=sym)
        sm, _ = built[key]
        for r in sweep(sm, dev, steps, 3, shapes=((k, n),), ms_list=ms_list, act_order=act,
                       tag=tag):
            res.setdefault(tag, []).append([r["shape"], r["m"], r["us"], r["GB/s"],
                                            r["TFLOP/s"], r["bound"], r["frac"]])
    built.clear()
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--prefill-m", type=int, default=256)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-merged", action="store_true",
                    help="skip the merged-projection (4 GEMMs per layer) leg")
    ap.add_argument("--only-prefill", action="store_true",
                    help="run only the M=--prefill-m leg (for hardware-counter passes)")
    ap.add_argument("--sweep", action="store_true", help="per-shape/per-M table on stderr")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config points (configs 1-4) of the JSON line")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline decode step and print its line (for counter "
                         "passes)")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip the one-launch decode chain leg")
    ap.add_argument("--no-transpose", action="store_true",
                    help="skip the transposed (PEFT backward) leg")
    ap.add_argument("--no-stage", action="store_true",
                    help="skip the decoder-stage leg (GEMMs + RoPE + KV cache + paged attention)")
    ap.add_argument("--stage-batch", type=int, default=8)
    ap.add_argument("--stage-context", type=int, default=512)
    ap.add_argument("--stage-steps", type=int, default=128)
    ap.add_argument("--stage-block-size", type=int, default=16)
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="only time the calibration streaming read in the decode launch "
                         "shapes and exit")
    ap.add_argument("--crossover", action="store_true",
                    help="only time the 56-matrix pass native vs dense routes over M and exit")
    ap.add_argument("--bf16-sweep", action="store_true",
                    help="only time bf16 activations through the packed-weight bf16 decode "
                         "launch against the dense route over shapes and M, and exit")
    ap.add_argument("--peaks", action="store_true",
                    help="only time a large fp16 library GEMM, a 1 GiB copy and a 1 GiB "
                         "streaming read on this box, print them and exit")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run 5 plain device copies of this many bytes (the known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE) and exit")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the W4A16 GEMM path has no multi-GPU leg in this build", file=sys.stderr)
        return 2

    import torch
    from gptq_synth import LLAMA2_7B_SHAPES, algorithmic_bytes, flops

    dev = torch.device("cuda", 0)
    if args.copy_bytes:
        src = torch.ones(args.copy_bytes // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        log(f"copied {args.copy_bytes} bytes 5 times")
        return 0
    if args.stream_ceiling:
        stream_ceiling(dev, args.steps)
        return 0
    if args.peaks:
        device_peaks(dev, args.steps)
        return 0
    if args.bf16_sweep:
        bf16_sweep(dev, args.steps, args.warmup)
        return 0
    log(f"building {args.layers} layers x {len(LLAMA2_7B_SHAPES)} projections")
    mats, _cache = build_matrices(dev, args.layers, max(args.prefill_m, 1))
    weight_bytes = sum(q4.qweight.numel() * 4 + q4.scales.numel() * 2 + q4.qzeros.numel() * 4
                       for _, _, _, q4 in mats)

    torch.cuda.synchronize(dev)
    if args.crossover:
        crossover(mats, dev, args.steps)
        return 0
    if args.only_prefill:
        grouped_leg(mats, dev, args.steps, args.warmup, args.prefill_m)
        return 0
    step_bytes = sum(algorithmic_bytes(1, k, n, GROUP, False) for _, k, n, _ in mats)
    grouped = grouped_leg(mats, dev, args.steps, args.warmup)
    ms = grouped["us_per_step"] * 1e-3
    launches = grouped["launches_per_step"]
    gbs = step_bytes / (ms * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded random GPTQ int4 weights, N(0,1) fp16 activations)",
        "config": {
            "workload": ("llama2-7b 8-layer stage decode, 7 GPTQ projections per layer "
                         "(4x 4096x4096, 2x 4096x11008, 1x 11008x4096), M=1, group 128, "
                         "asymmetric zeros; 56 distinct weight matrices per step, each with its "
                         "own output, launched in the layer's data-flow order: q/k/v in one "
                         "grouped launch (they share the layer input), o, gate/up in one grouped "
                         "launch (they share o's output), down"),
            "m": 1, "layers": args.layers, "group_size": GROUP,
            "weight_bytes": weight_bytes, "algorithmic_bytes_per_step": step_bytes,
            "matrices_per_step": len(mats), "launches_per_step": launches, "hip_graph": True,
        },
        "device": device_info(dev),
        # Dominant (only) kernel of the step: dw4::decode_kernel (single-matrix
        # and item-table forms).  Algorithmic bytes per launch (mean over the
        # step's launches) / mean launch duration (HIP events around the graph
        # replays on the replay stream / launches).
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "dw4::decode_kernel",
            "bytes_per_launch": step_bytes // launches,
            "avg_launch_us": round(ms * 1e3 / launches, 3),
        },
    }

    # Measured HBM bytes per launch (two calibrated rocprofv3 counter passes
    # over this step), used only while the decode kernel's sources are the
    # ones it was measured on.
    traffic_file = os.path.join(REPO, "profiles", "decode_traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            rec = json.load(f)
        if rec.get("source_sha256") == decode_source_sha256() and \
                rec.get("launches_per_step") == launches:
            result["roofline"]["traffic"] = rec.get("hbm_bytes_per_launch")
        else:
            result["roofline"]["traffic_note"] = ("profiles/decode_traffic.json was measured on "
                                                  "other decode kernel sources or another step")
    if args.headline_only:
        print(json.dumps(result), flush=True)
        return 0

    # the same step with one launch per projection (56 launches)
    pms, wall, _ = time_graph(mats, 1, args.steps, args.warmup, dev)
    pg = step_bytes / (pms * 1e-3) / 1e9
    log(f"decode M=1, one launch per projection: {pms * 1e3:.1f} us per step ({len(mats)} "
        f"launches), {pg:.1f} GB/s, wall {wall:.3f} s")
    result["per_projection_launches"] = {"us_per_step": round(pms * 1e3, 2), "GB/s": round(pg, 1),
                                         "frac": round(pg / HBM_PEAK_GBS, 4),
                                         "launches_per_step": len(mats)}

    if not args.no_chain:
        result["chain"] = chain_leg(mats, dev, args.steps, args.warmup, args.layers)

    if not args.no_prefill:
        # the same 56 GEMMs at M=256 in the same data-flow launches (q/k/v
        # and gate/up grouped), and with one launch per projection
        m = args.prefill_m
        pg = grouped_leg(mats, dev, max(5, args.steps // 5), max(2, args.warmup // 5), m)
        pms = pg["us_per_step"] * 1e-3
        tf = pg["TFLOP/s"]
        ppms, _, _ = time_graph(mats, m, max(5, args.steps // 5), max(2, args.warmup // 5), dev)
        ptf = sum(flops(m, k, n) for _, k, n, _ in mats) / (ppms * 1e-3) / 1e12
        log(f"prefill M={m}, one launch per projection: {ppms * 1e3:.1f} us per step, "
            f"{ptf:.1f} TFLOP/s")
        result["prefill"] = {"m": m, "value": round(tf, 2), "unit": "TFLOP/s",
                             "ms_per_step": round(pms, 5),
                             "frac": round(tf / MFMA_FP16_PEAK_TFLOPS, 4),
                             "peak": MFMA_FP16_PEAK_TFLOPS, "bound": "mfma",
                             "launches_per_step": pg["launches_per_step"],
                             "per_projection_launches": {
                                 "value": round(ptf, 2), "ms_per_step": round(ppms, 5),
                                 "frac": round(ptf / MFMA_FP16_PEAK_TFLOPS, 4),
                                 "launches_per_step": len(mats)}}

    if args.sweep:
        # each shape rotates over distinct matrices totalling >= 512 MB, so the
        # 256 MB Infinity Cache cannot serve the weights between launches
        plan = [((4096, 4096), False, (1, 2, 4, 8, 16, 64, 256, 1024, 2048), "C2/C3 (7B)"),
                ((4096, 11008), False, (1, 2, 4, 8, 16, 64, 256, 1024, 2048), "C2/C3 (7B)"),
                ((11008, 4096), False, (1, 2, 4, 8, 16, 64, 256, 1024, 2048), "C2/C3 (7B)"),
                ((5120, 5120), True, (1, 8, 64), "C4 (13B act-order)"),
                ((5120, 13824), True, (1, 8, 64), "C4 (13B act-order)"),
                ((13824, 5120), True, (1, 8, 64), "C4 (13B act-order)")]
        for (k, n), act, ms_list, tag in plan:
            count = -(-(512 << 20) // algorithmic_bytes(1, k, n, GROUP, act))
            sm, sc = build_matrices(dev, count, max(ms_list), seed0=7000 + k + n,
                                    shapes={f"{k}x{n}": (k, n)}, act_order=act)
            sweep(sm, dev, max(5, args.steps // 5), 3, shapes=((k, n),), ms_list=ms_list,
                  act_order=act, tag=tag)
            del sm, sc
            torch.cuda.empty_cache()

    if not args.no_configs and not args.sweep:
        result["configs"] = config_points(dev, max(5, args.steps // 5))
        result["configs_columns"] = ["shape", "m", "us_per_launch", "GB/s", "TFLOP/s", "bound",
                                     "frac_of_bound_peak"]

    if not args.no_transpose:
        # PEFT backward through the same 56 frozen matrices at M=16
        m = 16
        tms = time_transpose(mats, m, max(5, args.steps // 5), 3, dev)
        dms = time_transpose(mats, m, max(5, args.steps // 5), 3, dev, dense=True)
        tbytes = sum(algorithmic_bytes(m, k, n, GROUP, False) for _, k, n, _ in mats)
        tg = tbytes / (tms * 1e-3) / 1e9
        log(f"transposed M={m}: {tms * 1e3:.1f} us per step packed, {dms * 1e3:.1f} us "
            f"dequantise + dense, {tg:.1f} GB/s")
        result["transpose"] = {"m": m, "value": round(tg, 2), "unit": "GB/s",
                               "ms_per_step": round(tms, 5), "frac": round(tg / HBM_PEAK_GBS, 4),
                               "dense_route_ms_per_step": round(dms, 5),
                               "kernel": "dw4::gemm_t_kernel",
                               "workload": "g @ W^T (the activation gradient) through the 56 "
                                           "matrices of the decode leg at M=16"}

    if not args.no_merged:
        # Same weight bytes with q/k/v and gate/up merged (4 GEMMs per layer),
        # as the reference's Marlin loader runs a decoder stage.
        from gptq_synth import LLAMA2_7B_MERGED_SHAPES
        del _cache
        mats.clear()
        torch.cuda.empty_cache()
        mmats, _mcache = build_matrices(dev, args.layers, max(args.prefill_m, 1),
                                        shapes=LLAMA2_7B_MERGED_SHAPES)
        mms, _, _ = time_graph(mmats, 1, args.steps, args.warmup, dev)
        mbytes = sum(algorithmic_bytes(1, k, n, GROUP, False) for _, k, n, _ in mmats)
        mg = mbytes / (mms * 1e-3) / 1e9
        log(f"merged decode M=1: {mms * 1e3:.1f} us per step ({len(mmats)} GEMMs), {mg:.1f} GB/s")
        merged = {"value": round(mg, 2), "unit": "GB/s", "ms_per_step": round(mms, 5),
                  "launches_per_step": len(mmats), "frac": round(mg / HBM_PEAK_GBS, 4),
                  "workload": "same 8 layers with q/k/v merged (4096x12288) and gate/up merged "
                              "(4096x22016): 4 GEMMs per layer"}
        if not args.no_prefill:
            m = args.prefill_m
            pms, _, _ = time_graph(mmats, m, max(5, args.steps // 5), max(2, args.warmup // 5), dev)
            tf = sum(flops(m, k, n) for _, k, n, _ in mmats) / (pms * 1e-3) / 1e12
            log(f"merged prefill M={m}: {pms * 1e3:.1f} us per step, {tf:.1f} TFLOP/s")
            merged["prefill"] = {"m": m, "value": round(tf, 2), "unit": "TFLOP/s",
                                 "ms_per_step": round(pms, 5),
                                 "frac": round(tf / MFMA_FP16_PEAK_TFLOPS, 4)}
        result["merged"] = merged
        if args.sweep:
            sweep(mmats, dev, max(5, args.steps // 5), 3,
                  shapes=((4096, 12288), (4096, 22016)), ms_list=(1, 2, 4, 8, 16, 64, 256),
                  tag="merged (8 layers; q/k/v set 210 MB)")
        del mmats, _mcache

    if not args.no_stage:
        mats.clear()
        torch.cuda.empty_cache()
        st = stage_leg(dev, args.layers, args.stage_batch, args.stage_context, args.stage_steps,
                       args.stage_block_size,
                       # warmup replays advance the context too: at most the
                       # timed steps, which the KV cache is sized for
                       min(max(2, args.warmup // 2), args.stage_steps))
        log(f"stage decode batch {st['batch']}: {st['ms_per_step'] * 1e3:.1f} us per step, "
            f"{st['tokens_per_s']:.0f} tokens/s, {st['hbm_gbs']:.0f} GB/s (weights + KV)")
        result["stage"] = st

    if not args.no_cpu:
        log("timing CPU baseline")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
